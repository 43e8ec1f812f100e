/* hk -- MI355X (gfx950) decode engine: the C ABI of libhk.so.
 *
 * Plain C types only: device pointers are `const void*` / typed pointers into
 * HIP device memory, streams are `void*` (a hipStream_t, NULL = the default
 * stream), host buffers are ordinary pointers.  Every function returns 0 on
 * success or one of the HK_ERR_* codes; hk_last_error() then holds a message
 * for the calling thread.  Calls on one engine must be serialised by the
 * caller (the reference serialises its decoder behind one lock,
 * npu_llm/api_server.py:559, 657); the engine also takes its own mutex.
 *
 * BF16 tensors are uint16 bit patterns.  Weight tensors use the reference's
 * package layout (npu_llm/tools/convert_smollm2.py:220-311): qkv rows are
 * q heads, k heads, v heads; gate_up rows are gate then up; row-major [M, K];
 * int8 weights carry a float32 scale per output row (convert_smollm2.py:81-86).
 */
#ifndef HK_H
#define HK_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HK_OK 0
#define HK_ERR_INVALID 1     /* bad argument: the reference raises ValueError */
#define HK_ERR_HIP 2         /* HIP runtime error: the reference's RuntimeError */
#define HK_ERR_UNSUPPORTED 3 /* shape or device this build does not handle */

#define HK_MODEL_QKV_BIAS 1u /* layers carry a float32 qkv bias */
#define HK_MODEL_W8 2u       /* layer projections are int8 + per-row scale */

typedef struct hk_engine hk_engine;

/* Model shape; fields as in the package metadata.json
 * (npu_llm/tools/convert_smollm2.py:188-210). */
typedef struct hk_model_desc {
  int32_t layers;
  int32_t hidden;       /* hidden_size */
  int32_t intermediate; /* intermediate_size */
  int32_t q_heads;      /* attention_heads */
  int32_t kv_heads;
  int32_t head_dim;     /* must be 64 */
  int32_t vocab;        /* vocab_size */
  int32_t max_context;  /* KV slots allocated per layer and head */
  float rms_eps;        /* rms_norm_eps, as float32 */
  uint32_t flags;       /* HK_MODEL_* */
} hk_model_desc;

/* Device pointers of one decoder layer (names as in the package manifest). */
typedef struct hk_layer_weights {
  const void* qkv;          /* [(Hq + 2 Hkv) * D, H] bf16 or int8 */
  const float* qkv_scale;   /* [(Hq + 2 Hkv) * D] (W8) */
  const float* qkv_bias;    /* [(Hq + 2 Hkv) * D] float32 (HK_MODEL_QKV_BIAS) */
  const void* o_proj;       /* [H, Hq * D] */
  const float* o_scale;
  const void* gate_up;      /* [2 I, H]: gate rows then up rows */
  const float* gate_up_scale;
  const void* down_proj;    /* [H, I] */
  const float* down_scale;
  const uint16_t* input_norm;     /* [H] bf16 */
  const uint16_t* post_attn_norm; /* [H] bf16 */
} hk_layer_weights;

typedef struct hk_model_weights {
  const uint16_t* token_embedding; /* [V, H] bf16 */
  const uint16_t* lm_head;         /* [V, H] bf16 (the embedding when tied) */
  const uint16_t* final_norm;      /* [H] bf16 */
  const float* rope_cos;           /* [max_context, D/2]: np.cos(f32(p) * inv_freq) */
  const float* rope_sin;           /* [max_context, D/2]: np.sin(f32(p) * inv_freq) */
  const hk_layer_weights* layers;  /* host array of `layers` entries */
} hk_model_weights;

/* Version of this ABI (bumped on any incompatible change). */
int32_t hk_abi_version(void);

/* Message for the last failing call on this thread ("" if none). */
const char* hk_last_error(void);

/* Select the HIP device and check it is a gfx950 (MI355X).
 * Replaces set_current_device(from_name("npu", n_cols=4)),
 * npu_llm/runtime/generate.py:131-132. */
int hk_init(int32_t device_ordinal);

/* Build a decode engine over caller-owned device weights (the caller keeps
 * them alive until hk_engine_destroy).  The engine allocates its own KV cache,
 * activations, logits and a stream.  Replaces QwenDecoderEngine.__init__
 * (npu_llm/runtime/qwen_engine.py:41-63) and DecoderEngine.__init__
 * (npu_llm/runtime/engine.py:32-49). */
int hk_engine_create(const hk_model_desc* desc, const hk_model_weights* weights,
                     hk_engine** out);

/* One decode step at `position`: every layer for one token, KV appended at
 * slot `position`, attention over slots 0..position.  The token's embedding
 * row comes from the device table, or from `embedding_host` ([H] bf16) when
 * that is non-NULL.  With `want_logits` the final RMSNorm, LM head and argmax
 * run too; `logits_host` ([V] float32) and `next_token_host` receive them.
 * Without outputs the call returns without waiting for the GPU.
 * Replaces QwenDecoderEngine.step (npu_llm/runtime/qwen_engine.py:77-94) and
 * the device program qwen_engine(...) (npu_llm/designs/qwen_engine.py:72-81).
 * HK_ERR_INVALID if position is outside [0, max_context) or token outside
 * [0, vocab) (the reference's ValueError, qwen_engine.py:84-85). */
int hk_engine_step(hk_engine* engine, int32_t token, int32_t position, int32_t want_logits,
                   const uint16_t* embedding_host, float* logits_host,
                   int32_t* next_token_host);

/* Greedy decode of `n_steps` tokens without host round trips: step i feeds
 * the argmax of step i-1, starting from `token` at `position`.  Writes the
 * n_steps emitted token ids to `tokens_host`.  Equivalent to n_steps calls of
 * hk_engine_step with argmax selection (npu_llm/runtime/generate.py:1130-1158
 * with the greedy sampler). */
int hk_engine_generate(hk_engine* engine, int32_t token, int32_t position, int32_t n_steps,
                       int32_t* tokens_host);

/* Batched prefill of `n` prompt tokens at slots start..start+n-1: every layer
 * runs on all tokens at once (MFMA bf16 GEMMs, causal GQA attention), the KV
 * cache gets all n slots, and, when `logits_host` or `next_token_host` is
 * non-NULL, the final norm + LM head + argmax run for the last token.  The
 * result equals n hk_engine_step calls (logits at the last one only) up to
 * float32 summation order.  Replaces the reference's per-position prefill
 * loop (npu_llm/runtime/generate.py:1110-1125) and the engine's lm_head=False
 * dispatches (npu_llm/designs/qwen_engine.py:213-219).  Prompts longer than
 * 4096 tokens (or the context length) run in chunks of that many. */
int hk_engine_prefill(hk_engine* engine, const int32_t* tokens_host, int32_t n, int32_t start,
                      float* logits_host, int32_t* next_token_host);

/* Final-RMSNorm output ([H] bf16) of the hidden state left by the last step:
 * the value DecoderEngine.step returns (npu_llm/runtime/engine.py:65-82). */
int hk_engine_final_hidden(hk_engine* engine, uint16_t* hidden_host);

/* Copy KV-cache slot `slot` of layer `layer` to the host: k_host and v_host
 * each receive [kv_heads, 64] bf16.  The reference keeps this cache on the
 * host and reads it back as a view (runtime/qwen_engine.py:60-63, 92-93). */
int hk_engine_read_kv(hk_engine* engine, int32_t layer, int32_t slot, uint16_t* k_host,
                      uint16_t* v_host);

/* Parts of one decode step, in launch order within a layer. */
#define HK_PART_QKV 0       /* RMSNorm + qkv projection + bias */
#define HK_PART_ATTENTION 1 /* RoPE + KV append + GQA attention */
#define HK_PART_O 2         /* o_proj + residual */
#define HK_PART_GATE_UP 3   /* RMSNorm + gate/up projection + SwiGLU */
#define HK_PART_DOWN 4      /* down_proj + residual */
#define HK_PART_HEAD 5      /* final RMSNorm + LM head + argmax */
#define HK_PART_STEP 6      /* the whole decode step as the engine runs it (one
                               persistent launch when the model shape has one) */

/* Enqueue one part of the step for `layer` on the engine stream, without
 * waiting, using the token/position of the last step.  For timing single
 * kernels with events on hk_engine_stream(); the head's token feedback is
 * switched off.  No reference counterpart: the NPU engine runs its step as
 * one opaque dispatch (designs/qwen_engine.py:72-341). */
int hk_engine_launch_part(hk_engine* engine, int32_t part, int32_t layer);

/* Enqueue `count` launches of one part, layer i % layers for launch i, as one
 * hipGraph (captured on first use per (part, count)), so host launch cost does
 * not pace the GPU when the launches are timed with events.  HK_PART_STEP
 * repeats the whole step at the last token/position, without token feedback;
 * a persistent step (one launch per step) is enqueued directly, without a
 * graph. */
int hk_engine_launch_part_repeat(hk_engine* engine, int32_t part, int32_t count);

/* Enqueue `count` GEMVs y = W_i @ x, W_i = weights[i % n_weights] (bf16, or
 * int8 with scales[i % n_weights] when `scales` is non-NULL), float32 output,
 * on `stream` -- a microbenchmark that rotates through distinct weight copies
 * so a cache cannot serve them.  The launches go out as one hipGraph,
 * captured on the first call per argument set (the 32 most recent sets are
 * kept), so host launch cost does not pace the GPU; HK_GEMV_REPEAT_GRAPH=0
 * launches them directly.  No counterpart in the reference. */
int hk_gemv_repeat(const void* const* weights, const float* const* scales, int32_t n_weights,
                   const uint16_t* x, float* y_f32, int32_t M, int32_t K, int32_t count,
                   void* stream);

/* Zero the KV cache (QwenDecoderEngine.reset, qwen_engine.py:65-66), and the
 * persistent step's tagged activations and partial sums. */
int hk_engine_reset(hk_engine* engine);

/* Test hook: advance the persistent step's epoch counter by `count`, as if
 * that many epochs (about 121 per Qwen2.5-0.5B step) had passed with no
 * launch, so tests can put a launch at any residue of the 16-bit activation
 * tags.  No effect on the per-kernel step.  No reference counterpart. */
int hk_engine_skip_epochs(hk_engine* engine, uint32_t count);

/* How a decode step at `position` runs, written to `kind_out`:
 * HK_STEP_KERNELS (one kernel per part, replayed as a hipGraph),
 * HK_STEP_PERSISTENT (one persistent launch over all CUs),
 * HK_STEP_XCD_SPLIT (one persistent launch with the attention block on XCD 0
 * and the MLP on the other XCDs; short contexts) or HK_STEP_XCD_SPLIT_LONG
 * (the same with the attention tasks on the MLP XCDs; contexts up to 4096 for
 * Qwen2.5-0.5B).  HK_ERR_INVALID for a position outside the context.  No
 * reference counterpart (the NPU engine has one dispatch form). */
#define HK_STEP_KERNELS 0
#define HK_STEP_PERSISTENT 1
#define HK_STEP_XCD_SPLIT 2
#define HK_STEP_XCD_SPLIT_LONG 3
int hk_engine_step_kind(hk_engine* engine, int32_t position, int32_t* kind_out);

/* The engine's HIP stream (hipStream_t), for timing with events. */
void* hk_engine_stream(hk_engine* engine);

/* Release everything the engine allocated; NULL is accepted
 * (QwenDecoderEngine.close, qwen_engine.py:96-102). */
void hk_engine_destroy(hk_engine* engine);

/* ---- single operations (device pointers; asynchronous on `stream`) ---- */

/* y = W @ x for bf16 W [M, K], bf16 x [K].  Outputs: `y_f32` receives the
 * unrounded float32 sums when non-NULL; otherwise `y` receives
 * bf16(f32(bf16(acc)) + bias) with `bias` (float32 [M]) or `residual`
 * (bf16 [M]) added when given (at most one).  Replaces the reference's BF16
 * projection (npu_llm/runtime/cpu_backend.py:64-69; designs/project_bf16.py). */
int hk_gemv_bf16(const uint16_t* W, const uint16_t* x, const float* bias,
                 const uint16_t* residual, uint16_t* y, float* y_f32, int32_t M, int32_t K,
                 void* stream);

/* W8 form: acc = sum_k f32(Wq[m,k]) * f32(x[k]); value = acc * scale[m]; then
 * as hk_gemv_bf16.  Replaces project_w8bf16_acc32 + project_dequant_bf16
 * (npu_llm/kernels/project_w8bf16.cc:14-38; designs/project.py:21-108). */
int hk_gemv_w8(const int8_t* Wq, const float* scale, const uint16_t* x, const float* bias,
               const uint16_t* residual, uint16_t* y, float* y_f32, int32_t M, int32_t K,
               void* stream);

/* Y[m, n] = epilogue(sum_k A[m, k] * W[n, k]) for bf16 A [M, K] (row stride
 * lda) and W [N, K]; float32 accumulation on the matrix cores; the epilogue
 * is bf16(acc), or bf16(f32(bf16(acc)) + bias[n]) / + residual[m, n] (row
 * stride N) when given.  The batched form of hk_gemv_bf16 used by prefill
 * (the reference has no batched projection: it prefills position by
 * position, npu_llm/runtime/generate.py:1110-1125).  K must be a multiple of 32. */
int hk_gemm_bf16(const uint16_t* A, int32_t lda, const uint16_t* W, const float* bias,
                 const uint16_t* residual, uint16_t* Y, int32_t M, int32_t N, int32_t K,
                 void* stream);

/* out = bf16((v * inv_rms) * gamma) (cpu_backend.py:71-76; designs/rmsnorm.py). */
int hk_rmsnorm(const uint16_t* x, const uint16_t* gamma, float eps, uint16_t* out, int32_t n,
               void* stream);

/* act[i] = bf16((g / (1 + exp(-clip(g, -80, 80)))) * u) over gate_up = [g | u]
 * (cpu_backend.py:154-165; designs/elementwise.py swiglu). */
int hk_swiglu(const uint16_t* gate_up, uint16_t* act, int32_t intermediate, void* stream);

/* index of the first maximum of x[0..n) (np.argmax, generate.py:709-714). */
int hk_argmax_f32(const float* x, int32_t n, int32_t* index_device, void* stream);

/* RoPE + KV append + GQA attention for one layer at `position`
 * (cpu_backend.py:95-129).  kcache/vcache: [kv_heads, max_context, 64] bf16;
 * cos/sin: [max_context, 32] float32; out: [q_heads * 64] bf16. */
int hk_attention_decode(const uint16_t* qkv, const float* rope_cos, const float* rope_sin,
                        uint16_t* kcache, uint16_t* vcache, int32_t position,
                        int32_t max_context, int32_t q_heads, int32_t kv_heads,
                        int32_t head_dim, uint16_t* out, void* stream);

/* hk_attention_decode without any allocation, for callers that cannot call
 * hipMalloc (code under HIP graph capture, tight serving loops, harnesses
 * that forbid it).  No counterpart in the reference.  Same arguments, results
 * and errors as hk_attention_decode; its scratch (the position word, one
 * split-KV ticket per query head and the split-KV partials) is a static
 * device array of 1 MiB + 4352 bytes per GPU, held until the process ends.
 * HK_ERR_INVALID when q_heads > 1024 or q_heads * ceil(max_context / 256) *
 * 264 bytes of partials exceed 1 MiB (Qwen2.5-0.5B's 14 heads: any context up
 * to 65536).  Calls on one GPU share the scratch: calls that overlap in time
 * on one GPU (several streams, or several host threads) race. */
int hk_attention_decode_noalloc(const uint16_t* qkv, const float* rope_cos, const float* rope_sin,
                                uint16_t* kcache, uint16_t* vcache, int32_t position,
                                int32_t max_context, int32_t q_heads, int32_t kv_heads,
                                int32_t head_dim, uint16_t* out, void* stream);

/* Wait for all work on `stream`. */
int hk_stream_sync(void* stream);

/* ---- routed-expert (MoE) block ----
 * Expert weights (device, bf16, caller-owned): router [E, H]; gate_up
 * [E + S, 2 I, H] (gate rows then up rows); down [E + S, H, I].  Routed experts
 * are 0..E-1, the S shared experts follow.  Per token: r = router @ x (f32),
 * p = softmax(r), the top_k experts by p (ties to the lower id) weighted by p,
 * each expert bf16(down @ bf16(silu(bf16(gate @ x)) * bf16(up @ x))), and
 * y = bf16(sum_k p_k e_k + sum_s e_s). */
typedef struct hk_moe hk_moe;

typedef struct hk_moe_desc {
  int32_t hidden;       /* H, multiple of 32 */
  int32_t intermediate; /* I, multiple of 32 */
  int32_t experts;      /* routed experts E, at most 64 */
  int32_t shared;       /* shared experts S, at most 8 */
  int32_t top_k;        /* at most 16 */
  int32_t max_tokens;   /* largest batch, at most 256 */
} hk_moe_desc;

/* The block also makes an MFMA-native copy of every expert's gate/up and down
 * weights (the same size again, owned by the block, freed by hk_moe_destroy);
 * the caller's weights must stay unchanged while the block is used. */
int hk_moe_create(const hk_moe_desc* desc, const uint16_t* router, const uint16_t* gate_up,
                  const uint16_t* down, hk_moe** out);

/* Router + top-k + experts + combine for x [tokens, H] -> y [tokens, H]
 * (device pointers).  ids_out [tokens, top_k] int32 and weights_out float32
 * (device, optional) receive the routing.  No reference counterpart for the
 * router (the reference routes in upstream ggml/Colibri); the expert part
 * replaces compute_experts (ollama-xdna/backend/ggml-xdna.cpp:1301-1441). */
int hk_moe_forward(hk_moe* moe, const uint16_t* x, int32_t tokens, uint16_t* y, int32_t* ids_out,
                   float* weights_out, void* stream);

/* Experts + combine with caller routing (device ids [tokens, top_k], weights
 * [tokens, top_k]): the GGML MUL_MAT_ID contract
 * (ollama-xdna/backend/ggml-xdna.cpp:1681-1716, 1301-1441) and Colibri's
 * expert group (colibri-xdna/backend/backend_xdna.cpp:316-348).  Ids outside
 * [0, experts) are rejected. */
int hk_moe_experts(hk_moe* moe, const uint16_t* x, int32_t tokens, const int32_t* ids,
                   const float* weights, uint16_t* y, void* stream);

void hk_moe_destroy(hk_moe* moe);

/* ---- device memory, streams and events (the engine's buffer plumbing) ----
 * They stand in for the reference's XRT buffer objects (iron.tensor /
 * iron.zeros, npu_llm/runtime/qwen_engine.py:52-59) so a host needs no other
 * GPU library.  Copies are synchronous. */
int hk_malloc(uint64_t bytes, void** device_ptr);
int hk_free(void* device_ptr);
int hk_memcpy_h2d(void* device_dst, const void* host_src, uint64_t bytes);
int hk_memcpy_d2h(void* host_dst, const void* device_src, uint64_t bytes);
int hk_memcpy_d2d(void* device_dst, const void* device_src, uint64_t bytes);
int hk_memset(void* device_dst, int32_t value, uint64_t bytes);
int hk_stream_create(void** stream);
int hk_stream_destroy(void* stream);
int hk_event_create(void** event);
int hk_event_destroy(void* event);
int hk_event_record(void* event, void* stream);
/* Milliseconds between two recorded events (waits for `end`). */
int hk_event_elapsed_ms(void* start, void* end, float* ms);

#ifdef __cplusplus
}
#endif

#endif /* HK_H */
