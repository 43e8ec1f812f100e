/* hk -- expert-GEMV shims for the reference's two MoE offload contracts,
 * exported by libhk.so next to hk.h.
 *
 * Both contracts take HOST pointers (the caller runs the model on the CPU and
 * offloads expert projections), quantise every weight to int8 with one
 * float32 scale per output row (scale = max|w| / 127, 1 for an all-zero row;
 * q = round-half-even(w / scale)), round the activations to bf16, and
 * return float32.
 *
 * 1. GGML MUL_MAT_ID (ollama-xdna/backend/ggml-xdna.cpp).  The GGML backend
 *    declares the op supported for at most 8 ids and rows/columns of at most
 *    2048 (supports_experts, :1681-1716) and computes
 *      out[slot][r] = bf16((sum_c q_e[r][c] * bf16(in[slot or 0][c])) * s_e[r])
 *    for e = ids[slot] (compute_experts, :1301-1441; the requantisation is
 *    pack_expert, :692-735).  A GGML backend shim calls
 *    hk_ggml_experts_supported from supports_op, hk_ggml_experts_create once
 *    per weight tensor (dequantising it to float32 with ggml's to_float first)
 *    and hk_ggml_mul_mat_id from graph_compute.  Q4_K and Q6_K tensors go to
 *    hk_ggml_quant_create unchanged instead, and dense single-row MUL_MATs to
 *    hk_ggml_dense_create / hk_ggml_quant_create and hk_ggml_mul_mat.
 *
 * 2. Colibri coli_cuda_* (colibri-xdna/backend/backend_xdna.cpp).  The
 *    symbols below keep Colibri's names and signatures, so a Colibri build
 *    links libhk.so in place of its XDNA backend.  Tensors are uploaded in
 *    format 0 (float32), 1 (int8 x per-row scale), 2 (int4 x per-row scale)
 *    or 4 (int4 x per-group scale) and requantised as above (:122-157).
 *    Projections run in 2048-column tiles; each tile's result is rounded to
 *    bf16 and the tiles are summed in float32 (:159-206).  An expert group
 *    (at most 8 experts of one shape, one row each) computes
 *      y_i = down_i( silu(gate_i(x_i)) * up_i(x_i) ),  silu(g) = g / (1 + e^-g)
 *    with the SwiGLU in float32 (:316-348).  These functions return 1 on
 *    success and 0 to ask the caller to fall back to the CPU, as Colibri's
 *    do.
 */
#ifndef HK_EXPERTS_H
#define HK_EXPERTS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- GGML MUL_MAT_ID and MUL_MAT ---- */

typedef struct hk_ggml_experts hk_ggml_experts;

/* ggml_type values of the two block formats the reference's native kernels
 * take (upstream ggml's enum ggml_type). */
#define HK_GGML_Q4_K 12
#define HK_GGML_Q6_K 14

/* 1 when the shapes fit the contract (ggml-xdna.cpp:1681-1716: 0 < in, out
 * <= 2048; n_experts >= 8; 1 <= n_ids <= 8; input_rows 1 or n_ids), else 0.
 * Type and contiguity checks stay with the caller. */
int hk_ggml_experts_supported(int64_t in_dim, int64_t out_dim, int64_t n_experts, int64_t n_ids,
                              int64_t input_rows);

/* Requantise float32 weights [n_experts][out_dim][in_dim] (host) to int8 +
 * per-row scale on the device (ggml-xdna.cpp:692-735).  Returns an HK_*
 * code (hk.h). */
int hk_ggml_experts_create(const float* weights, int64_t n_experts, int64_t out_dim, int64_t in_dim,
                           hk_ggml_experts** out);

/* out[slot][:] for slot < n_ids (host float32 [n_ids][out_dim]) from input
 * (host float32 [input_rows][in_dim]; row 0 for every slot when input_rows
 * is 1) and ids (host int32 [n_ids]); HK_ERR_INVALID for an id outside
 * [0, n_experts) (ggml-xdna.cpp:1301-1441).  Takes sets from
 * hk_ggml_experts_create and hk_ggml_quant_create (dims <= 2048). */
int hk_ggml_mul_mat_id(hk_ggml_experts* set, const float* input, int64_t input_rows, const int32_t* ids,
                       int64_t n_ids, float* out);

void hk_ggml_experts_destroy(hk_ggml_experts* set);

/* 1 when a dense single-row MUL_MAT fits the reference's dense offload
 * (supports_dense_qwen, ggml-xdna.cpp:1718-1748: out_dim <= 32768, one input
 * row), else 0. */
int hk_ggml_dense_supported(int64_t in_dim, int64_t out_dim, int64_t input_rows);

/* 1 when `ggml_type` is Q4_K or Q6_K and in_dim is a multiple of 256: the
 * native-block path (supports_native_experts / supports_native_dense,
 * ggml-xdna.cpp:967-993), else 0. */
int hk_ggml_quant_supported(int ggml_type, int64_t in_dim);

/* Dense MUL_MAT weights, float32 [out_dim][in_dim] (host), requantised to
 * int8 with one scale per (row, 2048-column tile): the reference's dense
 * tiles (pack_dense_tile, ggml-xdna.cpp:768-832).  Use with hk_ggml_mul_mat. */
int hk_ggml_dense_create(const float* weights, int64_t out_dim, int64_t in_dim, hk_ggml_experts** out);

/* GGML Q4_K or Q6_K weights as the tensor holds them: n_experts x out_dim
 * rows of in_dim / 256 blocks (144 or 210 bytes each), back to back (host).
 * They stay in block form on the device and are dequantised inside the dot
 * product (npu_llm/kernels/project_q4k_bf16.cc:76-117,
 * project_q6k_bf16.cc:53-99): per 2048-column tile bf16(sum_c w_c * bf16(x_c)),
 * tiles summed in float32.  With n_experts > 1 and dims <= 2048 the set
 * serves hk_ggml_mul_mat_id (compute_experts_native, ggml-xdna.cpp:1180-1299);
 * with one matrix of up to 32768 rows, hk_ggml_mul_mat (compute_dense_native,
 * :1101-1178). */
int hk_ggml_quant_create(int ggml_type, const void* blocks, int64_t n_experts, int64_t out_dim, int64_t in_dim,
                         hk_ggml_experts** out);

/* out[out_dim] = W @ input[in_dim] for a dense set (host float32):
 * ggml-xdna.cpp:1444-1538 (W8 tiles) and :1101-1178 (Q4_K / Q6_K). */
int hk_ggml_mul_mat(hk_ggml_experts* set, const float* input, float* out);

/* Measurement hook with no counterpart in the reference: after a successful
 * hk_ggml_mul_mat_id call on `set`, launches its kernel `launches` more times
 * back to back over the input that call left in device memory, launch i with
 * the n_ids expert ids ids[i * n_ids ...] (host int32 [launches][n_ids], n_ids
 * of that call), so a timing can rotate through more experts than the
 * caches hold.  The launches are captured into a HIP graph on a stream of
 * their own and replayed between two events (with HK_EAGER=1 in the
 * environment they are launched directly); stores the average time per
 * launch in *ms_per_launch.  The output of that call is overwritten. */
int hk_ggml_mul_mat_id_repeat(hk_ggml_experts* set, const int32_t* ids, int64_t launches, float* ms_per_launch);

/* ---- Colibri ---- */

typedef struct ColiCudaTensor ColiCudaTensor;

/* backend_xdna.cpp:219-239: device 0 is this process's current HIP device. */
int coli_cuda_init(const int* devices, int count);
void coli_cuda_shutdown(void);
int coli_cuda_available_device_count(void);
int coli_cuda_device_count(void);
int coli_cuda_device_at(int index);

/* backend_xdna.cpp:273-303 */
int coli_cuda_tensor_upload_g(ColiCudaTensor** out, const void* weights, const float* scales, int fmt,
                              int input, int output, int device, int group);
int coli_cuda_tensor_upload(ColiCudaTensor** out, const void* weights, const float* scales, int fmt,
                            int input, int output, int device);
void coli_cuda_tensor_free(ColiCudaTensor* tensor);
int coli_cuda_tensor_device(const ColiCudaTensor* tensor);
int coli_cuda_tensor_update(ColiCudaTensor* tensor, const void* weights, const float* scales);

/* backend_xdna.cpp:305-314: one row (rows must be 1); uploads *tensor from
 * weights/scales/fmt on first use. */
int coli_cuda_matmul(ColiCudaTensor** tensor, float* output, const float* input, const void* weights,
                     const float* scales, int fmt, int rows, int input_size, int output_size, int device,
                     int group);

/* backend_xdna.cpp:316-358: inputs and outputs are the experts' vectors
 * back to back. */
int coli_cuda_expert_group_pinned(ColiCudaTensor* const* gate, ColiCudaTensor* const* up,
                                  ColiCudaTensor* const* down, const int* rows, int count, float* output,
                                  const float* input, int pinned);
int coli_cuda_expert_group(ColiCudaTensor* const* gate, ColiCudaTensor* const* up, ColiCudaTensor* const* down,
                           const int* rows, int count, float* output, const float* input);
int coli_cuda_expert_mlp(ColiCudaTensor* gate, ColiCudaTensor* up, ColiCudaTensor* down, float* output,
                         const float* input, int rows);

#ifdef __cplusplus
}
#endif

#endif /* HK_EXPERTS_H */
