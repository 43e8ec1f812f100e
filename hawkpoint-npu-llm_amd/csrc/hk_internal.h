// Host-side declarations shared between the hk translation units: kernel
// argument blocks and the launch functions each .hip file exports.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

namespace hk {

// Per-thread error message behind hk_last_error().
void set_error(const std::string& message);
int fail(const std::string& message);           // set_error + return HK_ERR_INVALID
int hip_fail(hipError_t err, const char* what);  // set_error + return HK_ERR_HIP

// Argmax keys (see argmax_key in hk_common.h): a launch that reduces rows
// writes one partial key per workgroup; launch_argmax_finalize reduces them.
constexpr int kMaxPartialKeys = 4096;

// Decode-step control block, read by the kernels of a captured step so the
// same graph serves every position.
struct StepCtrl {
  int32_t token;     // token whose embedding row feeds layer 0; -1: hidden preloaded
  int32_t position;  // KV slot written and last slot attended
  int32_t n_out;     // tokens emitted so far by device-driven decode
  int32_t advance;   // 1: the LM head writes its argmax to `token` and bumps `position`
};

enum GemvEpilogue : int {
  EPI_BF16 = 0,        // y = bf16(acc)
  EPI_BIAS = 1,        // y = bf16(f32(bf16(acc)) + bias)
  EPI_RESID = 2,       // y = bf16(f32(bf16(acc)) + f32(resid))
  EPI_F32 = 3,         // yf = acc (unrounded)
  EPI_F32_ARGMAX = 4,  // yf = acc, plus one partial argmax key per workgroup
  EPI_SWIGLU = 5,      // rows i and M+i: y = bf16(silu(bf16(g)) * bf16(u))
};

enum GemvPrologue : int {
  PRO_PLAIN = 0,  // x as given
  PRO_NORM = 1,   // x = bf16((v * inv_rms) * gamma), the reference's RMSNorm
};

struct GemvArgs {
  const void* W;             // [rows, K] bf16 bits, or int8 when w8
  const float* scale;        // [rows] per-row dequant scale (w8)
  const uint16_t* x;         // [K] bf16 input
  const int32_t* x_index;    // optional: x = x_table + (*x_index) * K when *x_index >= 0
  const uint16_t* x_table;
  uint16_t* x_copy;          // optional: workgroup 0 stores the looked-up x row here
  const uint16_t* gamma;     // [K] RMSNorm gain (PRO_NORM)
  float eps;
  const float* bias;         // [M] (EPI_BIAS)
  const uint16_t* resid;     // [M] (EPI_RESID)
  uint16_t* y;               // [M] bf16 output
  float* yf;                 // [M] f32 output
  unsigned long long* keys;  // EPI_F32_ARGMAX: [gridDim.x] partial keys
  int M, K, vocab_limit;
  int pro, epi;
};

// Launches y = W @ x with the given prologue/epilogue.  Returns 0 or an
// hk error code (message via set_error).  `*blocks_out` (optional) receives
// the number of workgroups, i.e. of partial argmax keys written.
int launch_gemv(const GemvArgs& a, bool w8, hipStream_t stream, int* blocks_out = nullptr);


// Reduce `n` partial keys to the first-maximum index; write it to
// `token_out` (if set) and, when ctrl->advance, feed it back into `ctrl`
// and append it to `out_tokens` (capacity `out_cap`).
int launch_argmax_finalize(const unsigned long long* keys, int n, StepCtrl* ctrl,
                           int32_t* out_tokens, int out_cap, int32_t* token_out,
                           hipStream_t stream);

struct AttnArgs {
  const uint16_t* qkv;       // [(Hq + 2 Hkv) * 64] bf16: q heads, k heads, v heads
  const float* cos_tab;      // [max_ctx, 32]
  const float* sin_tab;      // [max_ctx, 32]
  uint16_t* kcache;          // this layer: [Hkv, max_ctx, 64] bf16
  uint16_t* vcache;          // this layer: [Hkv, max_ctx, 64] bf16
  const int32_t* position;   // device scalar
  uint16_t* out;             // [Hq * 64] bf16
  float* partial;            // [Hq, max_splits, 66] split-KV partials (contexts > 256)
  unsigned int* counters;    // [Hq] zero between launches
  int q_heads, kv_heads, max_ctx, max_splits;
};

constexpr int kHeadDim = 64;
constexpr int kAttnChunk = 256;  // slots per split-KV workgroup
constexpr int kMaxQPerKV = 16;
constexpr int kMaxContext = 65536;

// Split-KV workgroups per KV head for a context of `max_ctx` slots.
inline int attention_splits(int max_ctx) { return (max_ctx + kAttnChunk - 1) / kAttnChunk; }

int launch_attention_decode(const AttnArgs& a, hipStream_t stream);

// ---- whole decode step in one persistent launch (persistent.hip) ----
constexpr int kPersistentThreads = 512;  // one workgroup per CU
constexpr int kPersistentGrid = 256;     // workgroups (MI355X has 256 CUs)
constexpr int kPersistentChunk = 256;    // attention slots per task
constexpr int kFlagStride = 32;          // uint32 words between flags (one 128-byte line each)
constexpr int kPersistentMaxLayers = 128;

// Layer weights of the persistent step.  For a W8 model the four projection
// pointers hold int8 [rows, cols] and the *_scale pointers the float32 scale
// of each output row (gate_up_scale: 2 I, gate rows first); for bf16 they
// hold bf16 and the scales are null.
struct PersistentLayer {
  const uint16_t* qkv;
  const float* qkv_bias;  // null when the model has none
  const uint16_t* o;
  const uint16_t* gate_up;
  const uint16_t* down;
  const uint16_t* in_norm;
  const uint16_t* post_norm;
  // down_proj regrouped for the XCD split (null otherwise): for each group of
  // four intermediate rows g, [H / R][R][4] -- element (c, e, j) is
  // down[R c + e][4g + j], so one 16-byte chunk holds R / 4 outputs of all
  // four rows (R = 8 for bf16, 16 for int8; see launch_regroup_down)
  const uint16_t* down_x;
  const float* qkv_scale;
  const float* o_scale;
  const float* gate_up_scale;
  const float* down_scale;
  // W8 under the XCD split (null otherwise): the int8 QKV and O weights as
  // bf16 (each value exact), which XCD 0's stager waves load in place of
  // their int8 rows, so they need not widen them between their poll and the
  // hand-off (see launch_widen_i8)
  const uint16_t* qkv_wide;
  const uint16_t* o_wide;
};

struct PersistentArgs {
  const PersistentLayer* w;  // device array [layers]
  int layers, vocab, max_ctx, max_splits;
  int head;  // 1: final norm, LM head and argmax (with token feedback when ctrl->advance)
  float eps;
  const uint16_t* embed;
  const uint16_t* lm_head;
  const uint16_t* final_norm;
  const float* cos_tab;
  const float* sin_tab;
  uint16_t* kcache;  // [L][Hkv][max_ctx][64]
  uint16_t* vcache;
  uint16_t* h;  // plain bf16 hidden: layer-0 input when ctrl->token < 0; final hidden out
  // tagged activations, (tag << 16) | bf16 per element
  uint32_t* th;     // [H] layer output
  uint32_t* th1;    // [H] after attention + residual
  uint32_t* tqkv;   // [(Hq + 2 Hkv) * 64]
  uint32_t* tattn;  // [Hq * 64]
  uint32_t* tact;   // [I]
  uint32_t* pad;    // [kPersistentGrid * 8] per-wave sink for stores of rows a wave does not own
  float* logits;             // [vocab + kPersistentGrid * 8]: the tail is a per-wave sink
  unsigned long long* keys;  // [kPersistentGrid]
  // [Hq, max_splits, 66] split-KV partials as (tag << 32) | float words;
  // zero between launch sequences
  unsigned long long* partial;
  unsigned int* counters;    // [Hq], zero between launches
  StepCtrl* ctrl;
  int32_t* out_tokens;
  int32_t* result;
  // XCD split: per-workgroup and per-XCD partial down products, 64-bit words
  // (epoch tag << 32) | float bits; zero between launch sequences
  unsigned long long* wpart;  // [kPersistentGrid][H]
  unsigned long long* xpart;  // [8][H]
  unsigned int* progress;  // [kPersistentGrid * kFlagStride] last epoch per workgroup
  unsigned int* error;     // nonzero: a wait timed out; the launch was abandoned
  unsigned int spin_limit; // polls before a wait is abandoned
};

constexpr unsigned kPersistentSpinLimit = 1u << 20;

// Model shapes the persistent step is compiled for: 0 SmolLM2-135M, 1
// Qwen2.5-0.5B, 2 and 3 the same with W8 layer projections (-1: use the
// per-kernel step).
int persistent_shape(int hidden, int intermediate, int q_heads, int kv_heads, bool w8);
// 1 when the step of this shape can also run split by XCD (attention block on
// XCD 0, MLP on the others) on the current device; else 0 with the reason in
// hk_last_error().  Runs a small probe kernel on `stream` and waits for it.
int persistent_xcd_split(int shape, hipStream_t stream);
// Forms of the persistent step.  kStepSplit runs a layer's attention tasks
// (query heads x 256-slot chunks) on XCD 0, kStepSplitLong on the MLP
// workgroups of the other XCDs; each is correct for any position, and
// persistent_split_tasks_max(long_form) is the task count up to which it
// keeps one task per workgroup.
enum StepForm : int { kStepUndivided = 0, kStepSplit = 1, kStepSplitLong = 2 };
int persistent_split_tasks_max(bool long_form);
int launch_persistent_step(int shape, const PersistentArgs& a, hipStream_t stream,
                           int form = kStepUndivided);
// down_x for the XCD split from down [H, I] (bf16, or int8 when w8; I a
// multiple of 4, H of 8, or of 16 for int8).
int launch_regroup_down(const void* down, void* down_x, int H, int I, bool w8, hipStream_t stream);
// dst[i] = bf16(src[i]) for n int8 values (exact).
int launch_widen_i8(const void* src, void* dst, size_t n, hipStream_t stream);

// ---- batched prefill (prefill.hip) ----

struct PrefillGemmArgs {
  const uint16_t* A;      // [M, lda] bf16 activations (tokens x K)
  const uint16_t* W;      // [N, K] bf16 weights (SwiGLU: [2N, K], gate rows then up rows)
  const float* bias;      // [N] (EPI_BIAS)
  // W8: W holds int8 [N, K] (SwiGLU [2N, K]) and scale the float32 scale of
  // each weight row, applied to the finished sum; null for bf16 weights
  const float* scale;
  const uint16_t* resid;  // [M, ldr] (EPI_RESID)
  uint16_t* Y;            // [M, ldy] bf16 output
  int M, N, K, lda, ldr, ldy;
  int epi;                // EPI_BF16, EPI_BIAS, EPI_RESID or EPI_SWIGLU
  // Grouped mode (routed experts), on when grp_count is set: workgroup z of
  // the third grid dimension computes group z < *n_groups with weights
  // W + grp_expert[z] * w_stride, grp_count[z] rows whose output rows are
  // grp_offset[z] + m and whose A rows are a_rows[grp_offset[z] + m] (or
  // grp_offset[z] + m when a_rows is null).
  const int32_t* a_rows;
  const int32_t* grp_expert;
  const int32_t* grp_count;
  const int32_t* grp_offset;
  const int32_t* n_groups;
  long long w_stride;
  int max_groups;         // grid size in z
  int max_rows;           // rows per group bound (grid size in y = ceil / 64)
  // Optional float32 workspace: when the GEMM has too few tiles to fill the
  // GPU (short prompts, narrow outputs), K is split across workgroups that
  // write partial sums here, and a second kernel adds them up in order and
  // applies the epilogue.  Without it (or when it is too small) the GEMM runs
  // unsplit.
  float* split_ws;
  size_t split_ws_floats;
  // Prompts of at most kSlabMaxTokens tokens run on the slab GEMM (one
  // workgroup per 16 outputs over all of K; no workspace).  With `gamma` (K at
  // most kSlabNormMaxK) the A rows are RMSNorm inputs, normalised as they are
  // loaded: A = bf16((x * inv_rms) * gamma) with inv_rms = 1 / sqrt(mean(x^2) + eps).
  const uint16_t* gamma;
  float eps;
  // Slab GEMM only: A, and Y with the residual, k-blocked with M rows --
  // element (m, k) at ((k / 8) M + m) 8 + k % 8 -- so that the 16 token rows
  // of an MFMA fragment are one 256-byte run (lda, ldy, ldr unused).  A only
  // with kblock = 1, all three with kblock = 2.
  int kblock;
  // The QKV projection (slab GEMM, or 128-token tiles when
  // prefill_rope_fusable): with rope.on the epilogue applies RoPE and writes
  // the rotated queries to rope.qrot and the rotated keys and the values to
  // the caches at slots rope.start.. (rope_append_kernel's job; Y is not
  // written).  The slabs then take the rows of each RoPE pair together
  // (rope_row); a 128-token tile holds whole heads.  N = (q_heads + 2
  // kv_heads) * 64.
  // Slab GEMM only: the MFMA-native copy of W (launch_repack_mfma), or null
  const void* Wn;
  // Long-K slab GEMM without RoPE, norm or SwiGLU only (the down
  // projection): with slab_ws, K is split kSlabParts ways over workgroups of
  // one XCD (workgroup i runs on XCD i % 8).  Parts 1.. publish their float32
  // partial sums as tagged words (slab_tag << 32 | bits) into slab_ws, which
  // holds ceil(N / 16) * kSlabParts * kSlabMaxTokens * 16 of them; part 0
  // polls them from the XCD's L2, adds the parts in order and applies the
  // epilogue.  slab_tag is nonzero and new for every launch; a wait that
  // gives up after slab_spin polls, or a workgroup found on another XCD,
  // sets *slab_error.
  unsigned long long* slab_ws;
  unsigned slab_tag, slab_spin;
  unsigned* slab_error;
  struct {
    const float* cos_tab;  // [max_ctx, 32]
    const float* sin_tab;
    uint16_t* qrot;        // [M, q_heads * 64]
    uint16_t* kcache;      // this layer: [kv_heads, max_ctx, 64]
    uint16_t* vcache;
    int start, q_heads, kv_heads, max_ctx, on;
  } rope;
};

constexpr int kSlabMaxTokens = 64;
constexpr int kSlabParts = 4;  // K split of the slab GEMM with slab_ws
constexpr int kSlabNormMaxK = 1024;
// compute units of the current device
int cu_count();

constexpr int kSplitTarget = 256;  // workgroups the split aims for
// float32 workspace the split-K path needs for an M x N GEMM (2N outputs
// with SwiGLU) with K columns: one M x outputs slice per K part (0 when
// the GEMM is not split).
size_t split_ws_need(int M, int N, int K, bool pair);

int launch_prefill_gemm(const PrefillGemmArgs& a, hipStream_t stream);

struct PrefillAttnArgs {
  const uint16_t* qkv;      // [n, ld_qkv] bf16 rows: q heads, k heads, v heads
  int ld_qkv;
  const float* cos_tab;     // [max_ctx, 32]
  const float* sin_tab;
  uint16_t* qrot;           // [n, q_heads * 64] rotated queries (written)
  uint16_t* kcache;         // this layer: [Hkv, max_ctx, 64]
  uint16_t* vcache;
  uint16_t* out;            // [n, ld_out] bf16 attention output
  int ld_out;
  int out_kblock;           // nonzero: out k-blocked with n rows (see PrefillGemmArgs::kblock)
  int rope_done;            // nonzero: qrot and the caches are written already (the QKV GEMM's RoPE)
  int n, start, q_heads, kv_heads, max_ctx;
  int period;               // set by launch_prefill_attention: the CU count
};

// Whether a QKV GEMM of M > 64 tokens and K inputs can apply RoPE and the KV
// append in its epilogue (PrefillGemmArgs::rope; the 128-token tiles).
bool prefill_rope_fusable(int M, int K);
// rope_append (unless rope_done) then causal attention for tokens start..start+n-1.
int launch_prefill_attention(const PrefillAttnArgs& a, hipStream_t stream);
int launch_embed_rows(const int32_t* tokens, int n, int vocab, const uint16_t* table, int H,
                      uint16_t* X, hipStream_t stream, int kb_rows = 0);
int launch_rmsnorm_rows(const uint16_t* X, int ldx, const uint16_t* gamma, float eps, uint16_t* out,
                        int ldo, int rows, int H, hipStream_t stream);
// dst = the MFMA-native copy of the row-major [R, K] matrix src (weights of
// weight_bytes bytes) for the slab GEMM: piece (16 s + r, c) of 8 weights at
// (s (K / 8) + c) 16 + r; rope: the rows of slab s are the QKV GEMM's RoPE
// order, so the copy serves a GEMM with rope.on.
int launch_repack_mfma(const void* src, void* dst, int R, int K, int weight_bytes, int rope, hipStream_t stream);

// Standalone RMSNorm: out = bf16((v * inv_rms) * gamma).
int launch_rmsnorm(const uint16_t* x, const uint16_t* gamma, float eps, uint16_t* out,
                   int n, hipStream_t stream);
// Elementwise SwiGLU over a [2I] gate|up vector.
int launch_swiglu(const uint16_t* gate_up, uint16_t* act, int inter, hipStream_t stream);
// Argmax over n float32 values (first maximum); `keys` holds kMaxPartialKeys.
int launch_argmax(const float* x, int n, unsigned long long* keys, int32_t* out_index,
                  hipStream_t stream);

}  // namespace hk
