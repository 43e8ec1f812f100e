// The decode engine and the C ABI of libhk.so (declared in include/hk.h).
//
// One decode step (npu_llm/runtime/cpu_backend.py:131-181 per layer, plus the
// head) is five kernels per layer and one for the head:
//   qkv     RMSNorm prologue + GEMV + bias           (gemv.hip)
//   attn    RoPE + KV append + GQA attention         (attention.hip)
//   o       GEMV + residual                          (gemv.hip)
//   gate_up RMSNorm prologue + paired GEMV + SwiGLU  (gemv.hip)
//   down    GEMV + residual                          (gemv.hip)
//   head    RMSNorm prologue + GEMV (f32 logits) + argmax with token feedback
// The kernels read the token and position from a device control block, so
// one captured hipGraph per variant (with / without the head) serves every
// position; the host only rewrites the control block between replays.
#include <algorithm>
#include <array>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/hk.h"
#include "hk_common.h"
#include "hk_internal.h"

namespace hk {

static thread_local std::string g_error;

void set_error(const std::string& message) { g_error = message; }

int fail(const std::string& message) {
  set_error(message);
  return HK_ERR_INVALID;
}

int hip_fail(hipError_t err, const char* what) {
  set_error(std::string(what) + ": " + hipGetErrorString(err));
  return HK_ERR_HIP;
}

namespace {

#define HK_CHECK(expr)                                   \
  do {                                                   \
    const hipError_t err_ = (expr);                      \
    if (err_ != hipSuccess) return hip_fail(err_, #expr); \
  } while (0)

#define HK_TRY(expr)              \
  do {                            \
    const int rc_ = (expr);       \
    if (rc_ != 0) return rc_;     \
  } while (0)

__global__ void set_ctrl_kernel(StepCtrl* ctrl, int32_t token, int32_t position, int32_t advance) {
  ctrl->token = token;
  ctrl->position = position;
  ctrl->n_out = 0;
  ctrl->advance = advance;
}

__global__ void store_i32_kernel(int32_t* dst, int32_t value) { *dst = value; }

// Zero n 32-bit words (a kernel rather than hipMemsetAsync, so that a
// captured step graph can hold it).
__global__ void clear_words_kernel(uint32_t* p, int n) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = 0u;
}

// Advance every workgroup's epoch of the persistent step by `count`.
__global__ void skip_epochs_kernel(unsigned int* progress, int n, int stride, unsigned int count) {
  for (int i = threadIdx.x; i < n; i += blockDim.x) progress[(size_t)i * stride] += count;
}

// Scratch shared by the single-operation entry points on one device.
struct OpScratch {
  int device = -1;
  unsigned long long* keys = nullptr;
  int32_t* position = nullptr;
  float* partial = nullptr;
  unsigned int* counters = nullptr;
  size_t partial_floats = 0;
  int counter_slots = 0;
};
std::mutex g_op_mutex;
std::vector<OpScratch> g_op_scratch;

int op_scratch(OpScratch** out, size_t partial_floats, int counter_slots) {
  int dev = 0;
  HK_CHECK(hipGetDevice(&dev));
  if ((int)g_op_scratch.size() <= dev) g_op_scratch.resize(dev + 1);
  OpScratch& s = g_op_scratch[dev];
  if (s.keys == nullptr) {
    HK_CHECK(hipMalloc(&s.keys, kMaxPartialKeys * sizeof(unsigned long long)));
    HK_CHECK(hipMalloc(&s.position, sizeof(int32_t)));
  }
  if (partial_floats > s.partial_floats) {
    if (s.partial) HK_CHECK(hipFree(s.partial));
    HK_CHECK(hipMalloc(&s.partial, partial_floats * sizeof(float)));
    s.partial_floats = partial_floats;
  }
  if (counter_slots > s.counter_slots) {
    if (s.counters) HK_CHECK(hipFree(s.counters));
    HK_CHECK(hipMalloc(&s.counters, counter_slots * sizeof(unsigned int)));
    HK_CHECK(hipMemset(s.counters, 0, counter_slots * sizeof(unsigned int)));
    s.counter_slots = counter_slots;
  }
  s.device = dev;
  *out = &s;
  return 0;
}

int gemv_common(const void* W, const float* scale, const uint16_t* x, const float* bias,
                const uint16_t* residual, uint16_t* y, float* y_f32, int32_t M, int32_t K,
                bool w8, void* stream) {
  if (W == nullptr || x == nullptr) return fail("gemv: null weight or input pointer");
  if (bias != nullptr && residual != nullptr) return fail("gemv: give bias or residual, not both");
  GemvArgs a = {};
  a.W = W;
  a.scale = scale;
  a.x = x;
  a.y = y;
  a.yf = y_f32;
  a.bias = bias;
  a.resid = residual;
  a.M = M;
  a.K = K;
  a.pro = PRO_PLAIN;
  if (y_f32 != nullptr) {
    if (bias || residual) return fail("gemv: float32 output takes no bias or residual");
    a.epi = EPI_F32;
  } else {
    a.epi = bias ? EPI_BIAS : residual ? EPI_RESID : EPI_BF16;
  }
  return launch_gemv(a, w8, static_cast<hipStream_t>(stream));
}

}  // namespace
}  // namespace hk

using namespace hk;

struct hk_engine {
  std::mutex mu;
  hk_model_desc d{};
  std::vector<hk_layer_weights> layers;
  hk_model_weights w{};
  int device = 0;
  hipStream_t stream = nullptr;
  bool w8 = false;
  int qkv_rows = 0;
  int max_splits = 0;
  // device state
  uint16_t* h = nullptr;       // residual stream (layer input / down output)
  uint16_t* h1 = nullptr;      // after attention + residual
  uint16_t* qkv = nullptr;
  uint16_t* attn = nullptr;
  uint16_t* act = nullptr;
  uint16_t* normed = nullptr;  // final RMSNorm output for hk_engine_final_hidden
  float* logits = nullptr;
  uint16_t* kcache = nullptr;  // [L][Hkv][max_ctx][64]
  uint16_t* vcache = nullptr;
  float* partial = nullptr;
  unsigned int* counters = nullptr;
  unsigned long long* keys = nullptr;  // [kMaxPartialKeys] LM-head argmax partials
  StepCtrl* ctrl = nullptr;
  int32_t* out_tokens = nullptr;  // [max_ctx]
  int32_t* result = nullptr;      // [3]: last argmax token, persistent-step error word, prefill split error word
  // whole step in one persistent launch (persistent.hip); -1: per-kernel graph
  int pshape = -1;
  // the step may also run split by XCD (attention block on XCD 0); it does so
  // while the context is short enough for one attention task per workgroup
  // there, judged by next_pos, the position the next launch decodes
  bool xcd_split = false;
  int next_pos = 0;
  std::vector<uint16_t*> down_x;         // per layer, down_proj regrouped for the split
  std::vector<uint16_t*> wide;           // W8 split: per layer, QKV then O as bf16 (PersistentLayer::qkv_wide)
  unsigned long long* wpart = nullptr;   // the split's partial down products
  unsigned long long* xpart = nullptr;
  PersistentLayer* players = nullptr;  // device copy of the layer pointers
  unsigned int spin_limit = kPersistentSpinLimit;
  unsigned int* psync = nullptr;       // per-workgroup epochs
  uint32_t* ptag = nullptr;            // tagged activations: h, h1, qkv, attn, act
  // a split launch ran since the last undivided one: the split never writes
  // act[H..I), so those words may hold tags of an old undivided launch that
  // recur after the 16-bit tags wrap; the next undivided launch clears act first
  bool act_stale = false;
  hipGraphExec_t graph[2] = {nullptr, nullptr};
  std::map<long long, hipGraphExec_t> repeat_graphs;  // timing graphs by (part, count)
  bool use_graph = true;
  // batched-prefill workspace, allocated on first use for kPrefillRows tokens
  int pf_rows = 0;
  uint16_t* pf_x = nullptr;    // layer input / down output [rows, H]
  uint16_t* pf_h1 = nullptr;   // after attention + residual [rows, H]
  uint16_t* pf_xn = nullptr;   // normalised rows [rows, H]
  uint16_t* pf_qkv = nullptr;  // [rows, qkv_rows]
  uint16_t* pf_q = nullptr;    // rotated queries [rows, Hq * 64]
  uint16_t* pf_att = nullptr;  // attention output [rows, Hq * 64]
  uint16_t* pf_act = nullptr;  // SwiGLU output [rows, I]
  int32_t* pf_tokens = nullptr;
  float* pf_split = nullptr;   // split-K partial sums of GEMMs with few tiles
  size_t pf_split_floats = 0;
  // per layer, MFMA-native copies of qkv (RoPE order), o, gate_up and down
  // for the slab GEMMs of chunks up to 64 tokens (empty: row-major weights)
  std::vector<std::array<void*, 4>> pf_native;
  // the down slab GEMM of short prompts with K split inside an XCD
  // (PrefillGemmArgs::slab_ws): on where the XCD split's placement check
  // passed, unless HK_SLAB_SPLIT=0; off for good after a wait gave up
  bool slab_split = false;
  unsigned long long* slab_ws = nullptr;
  unsigned slab_tag = 0;
};

namespace {

size_t kv_layer_elems(const hk_engine* e) {
  return (size_t)e->d.kv_heads * (size_t)e->d.max_context * kHeadDim;
}

// Launch one part of the step for layer `l` (the head ignores `l`).
int launch_part(hk_engine* e, int part, int l) {
  const hk_model_desc& d = e->d;
  const hipStream_t s = e->stream;
  const hk_layer_weights& lw = e->layers[l];
  switch (part) {
    case HK_PART_QKV: {
      GemvArgs q = {};
      q.W = lw.qkv;
      q.scale = lw.qkv_scale;
      q.x = e->h;
      if (l == 0) {
        q.x_index = &e->ctrl->token;
        q.x_table = e->w.token_embedding;
        q.x_copy = e->h;
        q.vocab_limit = d.vocab;
      }
      q.gamma = lw.input_norm;
      q.eps = d.rms_eps;
      q.bias = lw.qkv_bias;
      q.y = e->qkv;
      q.M = e->qkv_rows;
      q.K = d.hidden;
      q.pro = PRO_NORM;
      q.epi = lw.qkv_bias ? EPI_BIAS : EPI_BF16;
      return launch_gemv(q, e->w8, s);
    }
    case HK_PART_ATTENTION: {
      AttnArgs at = {};
      at.qkv = e->qkv;
      at.cos_tab = e->w.rope_cos;
      at.sin_tab = e->w.rope_sin;
      at.kcache = e->kcache + (size_t)l * kv_layer_elems(e);
      at.vcache = e->vcache + (size_t)l * kv_layer_elems(e);
      at.position = &e->ctrl->position;
      at.out = e->attn;
      at.partial = e->partial;
      at.counters = e->counters;
      at.q_heads = d.q_heads;
      at.kv_heads = d.kv_heads;
      at.max_ctx = d.max_context;
      at.max_splits = e->max_splits;
      return launch_attention_decode(at, s);
    }
    case HK_PART_O: {
      GemvArgs o = {};
      o.W = lw.o_proj;
      o.scale = lw.o_scale;
      o.x = e->attn;
      o.resid = e->h;
      o.y = e->h1;
      o.M = d.hidden;
      o.K = d.q_heads * kHeadDim;
      o.pro = PRO_PLAIN;
      o.epi = EPI_RESID;
      return launch_gemv(o, e->w8, s);
    }
    case HK_PART_GATE_UP: {
      GemvArgs g = {};
      g.W = lw.gate_up;
      g.scale = lw.gate_up_scale;
      g.x = e->h1;
      g.gamma = lw.post_attn_norm;
      g.eps = d.rms_eps;
      g.y = e->act;
      g.M = d.intermediate;
      g.K = d.hidden;
      g.pro = PRO_NORM;
      g.epi = EPI_SWIGLU;
      return launch_gemv(g, e->w8, s);
    }
    case HK_PART_DOWN: {
      GemvArgs dn = {};
      dn.W = lw.down_proj;
      dn.scale = lw.down_scale;
      dn.x = e->act;
      dn.resid = e->h1;
      dn.y = e->h;
      dn.M = d.hidden;
      dn.K = d.intermediate;
      dn.pro = PRO_PLAIN;
      dn.epi = EPI_RESID;
      return launch_gemv(dn, e->w8, s);
    }
    case HK_PART_HEAD: {
      GemvArgs hd = {};
      hd.W = e->w.lm_head;
      hd.x = e->h;
      hd.gamma = e->w.final_norm;
      hd.eps = d.rms_eps;
      hd.yf = e->logits;
      hd.keys = e->keys;
      hd.M = d.vocab;
      hd.K = d.hidden;
      hd.pro = PRO_NORM;
      hd.epi = EPI_F32_ARGMAX;
      int blocks = 0;
      HK_TRY(launch_gemv(hd, false, s, &blocks));
      return launch_argmax_finalize(e->keys, blocks, e->ctrl, e->out_tokens, d.max_context,
                                    e->result, s);
    }
    default:
      return fail("unknown step part");
  }
}

// The form of a persistent launch at `position`: split by XCD with the
// attention tasks on XCD 0 while they fit its workgroups, on the MLP
// workgroups while they fit those, else undivided.
int form_at(const hk_engine* e, int position) {
  if (!e->xcd_split) return kStepUndivided;
  const int tasks = e->d.q_heads * (position / kPersistentChunk + 1);
  if (tasks <= persistent_split_tasks_max(false)) return kStepSplit;
  if (tasks <= persistent_split_tasks_max(true)) return kStepSplitLong;
  return kStepUndivided;
}
int step_form(const hk_engine* e) { return form_at(e, e->next_pos); }

int launch_persistent(hk_engine* e, bool head) {
  const hk_model_desc& d = e->d;
  PersistentArgs a = {};
  a.w = e->players;
  a.layers = d.layers;
  a.vocab = d.vocab;
  a.max_ctx = d.max_context;
  a.max_splits = e->max_splits;
  a.head = head ? 1 : 0;
  a.eps = d.rms_eps;
  a.embed = e->w.token_embedding;
  a.lm_head = e->w.lm_head;
  a.final_norm = e->w.final_norm;
  a.cos_tab = e->w.rope_cos;
  a.sin_tab = e->w.rope_sin;
  a.kcache = e->kcache;
  a.vcache = e->vcache;
  a.h = e->h;
  a.th = e->ptag;
  a.th1 = a.th + d.hidden;
  a.tqkv = a.th1 + d.hidden;
  a.tattn = a.tqkv + e->qkv_rows;
  a.tact = a.tattn + (size_t)d.q_heads * kHeadDim;
  a.pad = a.tact + d.intermediate;
  a.logits = e->logits;
  a.keys = e->keys;
  a.partial = reinterpret_cast<unsigned long long*>(e->partial);
  a.counters = e->counters;
  a.ctrl = e->ctrl;
  a.out_tokens = e->out_tokens;
  a.result = e->result;
  a.wpart = e->wpart;
  a.xpart = e->xpart;
  a.progress = e->psync;
  a.error = reinterpret_cast<unsigned int*>(e->result + 1);
  a.spin_limit = e->spin_limit;
  const int form = step_form(e);
  if (form != kStepUndivided) {
    e->act_stale = true;
  } else if (e->act_stale) {
    hipLaunchKernelGGL(clear_words_kernel, dim3(8), dim3(256), 0, e->stream, a.tact, (int)d.intermediate);
    HK_CHECK(hipGetLastError());
    e->act_stale = false;
  }
  return launch_persistent_step(e->pshape, a, e->stream, form);
}

size_t psync_words(const hk_engine*) { return (size_t)kPersistentGrid * kFlagStride; }

size_t partial_floats(const hk_engine* e) { return (size_t)e->d.q_heads * e->max_splits * (kHeadDim + 2) * 2; }

size_t ptag_words(const hk_engine* e) {
  const hk_model_desc& d = e->d;
  return 2 * (size_t)d.hidden + e->qkv_rows + (size_t)d.q_heads * kHeadDim + d.intermediate +
         (size_t)kPersistentGrid * (kPersistentThreads / 64);
}

// After a synchronised copy of `result` (token, error word): an error means a
// persistent launch was abandoned; clear its flags so the next step starts
// clean, and report it.
int check_persistent(hk_engine* e, const int32_t* result_host) {
  if (e->pshape < 0 || result_host[1] == 0) return 0;
  // a split launch also leaves when a workgroup finds itself on another XCD
  // than the split assumes: later steps run undivided
  e->xcd_split = false;
  HK_CHECK(hipStreamSynchronize(e->stream));
  HK_CHECK(hipMemset(e->psync, 0, psync_words(e) * sizeof(unsigned int)));
  HK_CHECK(hipMemset(e->ptag, 0, ptag_words(e) * sizeof(uint32_t)));
  if (e->wpart) HK_CHECK(hipMemset(e->wpart, 0, (size_t)kPersistentGrid * e->d.hidden * 8));
  if (e->xpart) HK_CHECK(hipMemset(e->xpart, 0, (size_t)8 * e->d.hidden * 8));
  HK_CHECK(hipMemset(e->partial, 0, partial_floats(e) * sizeof(float)));
  HK_CHECK(hipMemset(e->counters, 0, e->d.q_heads * sizeof(unsigned int)));
  HK_CHECK(hipMemset(e->result, 0, 3 * sizeof(int32_t)));
  HK_CHECK(hipDeviceSynchronize());
  set_error("decode step abandoned: a workgroup of the persistent step waited too long for "
            "another (is another kernel occupying the GPU?); its outputs and KV slot are invalid");
  return HK_ERR_HIP;
}

int enqueue_step(hk_engine* e, bool head) {
  for (int l = 0; l < e->d.layers; ++l)
    for (int part = HK_PART_QKV; part <= HK_PART_DOWN; ++part) HK_TRY(launch_part(e, part, l));
  if (head) HK_TRY(launch_part(e, HK_PART_HEAD, 0));
  return 0;
}

int run_step(hk_engine* e, bool head) {
  if (e->pshape >= 0) return launch_persistent(e, head);
  if (!e->use_graph) return enqueue_step(e, head);
  hipGraphExec_t& exec = e->graph[head ? 1 : 0];
  if (exec == nullptr) {
    hipGraph_t graph = nullptr;
    HK_CHECK(hipStreamBeginCapture(e->stream, hipStreamCaptureModeThreadLocal));
    const int rc = enqueue_step(e, head);
    const hipError_t end = hipStreamEndCapture(e->stream, &graph);
    if (rc != 0) {
      if (graph) (void)hipGraphDestroy(graph);
      return rc;
    }
    if (end != hipSuccess) return hip_fail(end, "hipStreamEndCapture");
    const hipError_t inst = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    if (inst != hipSuccess) {
      exec = nullptr;
      return hip_fail(inst, "hipGraphInstantiate");
    }
  }
  HK_CHECK(hipGraphLaunch(exec, e->stream));
  return 0;
}

// Turn off token feedback without touching token/position (for timing the
// head on its own).
__global__ void ctrl_no_advance_kernel(StepCtrl* ctrl) { ctrl->advance = 0; }

int set_ctrl_keep(hk_engine* e) {
  hipLaunchKernelGGL(ctrl_no_advance_kernel, dim3(1), dim3(1), 0, e->stream, e->ctrl);
  HK_CHECK(hipGetLastError());
  return 0;
}

int set_ctrl(hk_engine* e, int32_t token, int32_t position, int32_t advance) {
  e->next_pos = position;
  hipLaunchKernelGGL(set_ctrl_kernel, dim3(1), dim3(1), 0, e->stream, e->ctrl, token, position,
                     advance);
  HK_CHECK(hipGetLastError());
  return 0;
}

void free_engine(hk_engine* e) {
  for (auto& g : e->graph)
    if (g) (void)hipGraphExecDestroy(g);
  for (auto& kv : e->repeat_graphs) (void)hipGraphExecDestroy(kv.second);
  void* bufs[] = {e->h,       e->h1,       e->qkv,      e->attn,       e->act,
                  e->normed,  e->logits,   e->kcache,   e->vcache,     e->partial,
                  e->counters, e->keys,    e->ctrl,     e->out_tokens, e->result,
                  e->pf_x,    e->pf_h1,    e->pf_xn,    e->pf_qkv,     e->pf_q,
                  e->pf_att,  e->pf_act,   e->pf_tokens, e->pf_split, e->players, e->psync, e->ptag,
                  e->wpart,   e->xpart};
  for (void* p : bufs)
    if (p) (void)hipFree(p);
  for (uint16_t* p : e->down_x)
    if (p) (void)hipFree(p);
  for (uint16_t* p : e->wide)
    if (p) (void)hipFree(p);
  for (auto& m : e->pf_native)
    for (void* p : m)
      if (p) (void)hipFree(p);
  if (e->stream) (void)hipStreamDestroy(e->stream);
  delete e;
}

template <typename T>
int dalloc(T** p, size_t count) {
  HK_CHECK(hipMalloc(reinterpret_cast<void**>(p), count * sizeof(T)));
  return 0;
}

// Tokens per prefill chunk: a whole 4096-token prompt is one chunk, so every
// GEMM has (tokens / 64) x (outputs / 64) tiles to spread over the CUs.
constexpr int kPrefillRows = 4096;

// Frees the prefill row buffers (null ones are skipped) and marks the
// workspace absent, so the next prefill allocates it from nothing.
void free_prefill_buffers(hk_engine* e) {
  auto drop = [](auto*& p) {
    if (p) (void)hipFree(p);
    p = nullptr;
  };
  drop(e->pf_x), drop(e->pf_h1), drop(e->pf_xn), drop(e->pf_qkv), drop(e->pf_q);
  drop(e->pf_att), drop(e->pf_act), drop(e->pf_tokens), drop(e->pf_split), drop(e->slab_ws);
  e->pf_rows = 0;
}

int alloc_prefill_buffers(hk_engine* e, int rows) {
  const hk_model_desc& d = e->d;
  const size_t r = rows;
  HK_TRY(dalloc(&e->pf_x, r * d.hidden));
  HK_TRY(dalloc(&e->pf_h1, r * d.hidden));
  HK_TRY(dalloc(&e->pf_xn, r * d.hidden));
  HK_TRY(dalloc(&e->pf_qkv, r * e->qkv_rows));
  HK_TRY(dalloc(&e->pf_q, r * d.q_heads * kHeadDim));
  HK_TRY(dalloc(&e->pf_att, r * d.q_heads * kHeadDim));
  HK_TRY(dalloc(&e->pf_act, r * d.intermediate));
  HK_TRY(dalloc(&e->pf_tokens, r));
  // the largest split workspace any chunk length up to `rows` asks for
  const int QD = d.q_heads * kHeadDim;
  e->pf_split_floats = 1;
  for (int m = 1; m <= rows; ++m)
    e->pf_split_floats = std::max({e->pf_split_floats, split_ws_need(m, e->qkv_rows, d.hidden, false),
                                   split_ws_need(m, d.hidden, QD, false),
                                   split_ws_need(m, d.intermediate, d.hidden, true),
                                   split_ws_need(m, d.hidden, d.intermediate, false)});
  HK_TRY(dalloc(&e->pf_split, e->pf_split_floats));
  // tagged partial sums of the K-split down slabs (N = hidden); tag 0 never
  // matches a launch's
  const size_t slab_words = (size_t)((d.hidden + 15) / 16) * kSlabParts * kSlabMaxTokens * 16;
  HK_TRY(dalloc(&e->slab_ws, slab_words));
  HK_CHECK(hipMemset(e->slab_ws, 0, slab_words * sizeof(unsigned long long)));
  return 0;
}

// The row buffers of a prefill chunk, allocated on the first prefill.  On a
// failure nothing stays allocated, so a retry starts over instead of
// overwriting (and leaking) what an earlier attempt got.
int prefill_workspace(hk_engine* e) {
  if (e->pf_rows) return 0;
  const int rows = std::min(kPrefillRows, (int)e->d.max_context);
  const int rc = alloc_prefill_buffers(e, rows);
  if (rc != 0) {
    free_prefill_buffers(e);
    return rc;
  }
  e->pf_rows = rows;
  return 0;
}

void free_native_copies(hk_engine* e) {
  for (auto& m : e->pf_native)
    for (void*& p : m) {
      if (p) (void)hipFree(p);
      p = nullptr;
    }
  e->pf_native.clear();
}

// The MFMA-native weight copies the slab GEMMs read (chunks of at most
// kSlabMaxTokens tokens), made the first time such a chunk runs: an engine
// that only prefills long prompts never holds them.  Every matrix of an
// engine shape has whole 16-row slabs (64-wide heads, hidden and
// intermediate sizes multiples of 16).  On a failure every copy is freed, so
// prefill_chunk then reads the row-major weights and a later chunk retries.
int native_copies(hk_engine* e) {
  const hk_model_desc& d = e->d;
  if (!e->pf_native.empty() || d.hidden % 16 != 0 || d.intermediate % 16 != 0) return 0;
  const int wb = e->w8 ? 1 : 2, QD = d.q_heads * kHeadDim;
  e->pf_native.assign(d.layers, {nullptr, nullptr, nullptr, nullptr});
  for (int l = 0; l < d.layers; ++l) {
    const hk_layer_weights& lw = e->layers[l];
    const struct { const void* src; int R, K, rope; } m[4] = {
        {lw.qkv, e->qkv_rows, d.hidden, 1}, {lw.o_proj, d.hidden, QD, 0},
        {lw.gate_up, 2 * d.intermediate, d.hidden, 0}, {lw.down_proj, d.hidden, d.intermediate, 0}};
    for (int i = 0; i < 4; ++i) {
      const hipError_t err = hipMalloc(&e->pf_native[l][i], (size_t)m[i].R * m[i].K * wb);
      int rc = err == hipSuccess ? 0 : hip_fail(err, "hipMalloc");
      if (rc == 0) rc = launch_repack_mfma(m[i].src, e->pf_native[l][i], m[i].R, m[i].K, wb, m[i].rope, e->stream);
      if (rc != 0) {
        if (err != hipSuccess) e->pf_native[l][i] = nullptr;
        free_native_copies(e);
        return rc;
      }
    }
  }
  return 0;
}

// All layers for tokens[0..n) (already on the device) at slots start..start+n-1.
int prefill_chunk(hk_engine* e, const int32_t* tokens_dev, int n, int start) {
  const hk_model_desc& d = e->d;
  const hipStream_t s = e->stream;
  const int H = d.hidden, I = d.intermediate, QD = d.q_heads * kHeadDim;
  // chunks of up to 64 tokens run the slab GEMMs, which apply the RMSNorms
  // to their A operand as they load it (hidden sizes up to 1024); their
  // activations (x, the attention output, h1, act) are then k-blocked, so
  // the 16 token rows of an MFMA fragment are one 256-byte run
  const bool fused_norm = n <= kSlabMaxTokens && H <= kSlabNormMaxK;
  const int kb = fused_norm ? 2 : 0;
  const bool slab = n <= kSlabMaxTokens, native = !e->pf_native.empty();
  HK_TRY(launch_embed_rows(tokens_dev, n, d.vocab, e->w.token_embedding, H, e->pf_x, s, fused_norm ? n : 0));
  for (int l = 0; l < d.layers; ++l) {
    const hk_layer_weights& lw = e->layers[l];
    if (!fused_norm) HK_TRY(launch_rmsnorm_rows(e->pf_x, H, lw.input_norm, d.rms_eps, e->pf_xn, H, n, H, s));
    PrefillGemmArgs q = {};
    q.A = fused_norm ? e->pf_x : e->pf_xn;
    q.gamma = fused_norm ? lw.input_norm : nullptr;
    q.eps = d.rms_eps;
    q.lda = H;
    q.W = static_cast<const uint16_t*>(lw.qkv);
    q.Wn = fused_norm && native ? e->pf_native[l][0] : nullptr;
    q.scale = e->w8 ? lw.qkv_scale : nullptr;
    q.bias = lw.qkv_bias;
    q.Y = e->pf_qkv;
    q.ldy = e->qkv_rows;
    q.M = n;
    q.N = e->qkv_rows;
    q.K = H;
    q.epi = lw.qkv_bias ? EPI_BIAS : EPI_BF16;
    q.kblock = fused_norm ? 1 : 0;
    // RoPE and the KV append in the QKV epilogue (no q/k/v rows, no
    // rope_append launch): the slab GEMMs with the fused norm, and the
    // 128-token tiles
    const bool rope_fused = fused_norm || prefill_rope_fusable(n, H);
    if (rope_fused) {
      q.rope.cos_tab = e->w.rope_cos;
      q.rope.sin_tab = e->w.rope_sin;
      q.rope.qrot = e->pf_q;
      q.rope.kcache = e->kcache + (size_t)l * kv_layer_elems(e);
      q.rope.vcache = e->vcache + (size_t)l * kv_layer_elems(e);
      q.rope.start = start;
      q.rope.q_heads = d.q_heads;
      q.rope.kv_heads = d.kv_heads;
      q.rope.max_ctx = d.max_context;
      q.rope.on = 1;
    }
    q.split_ws = e->pf_split;
    q.split_ws_floats = e->pf_split_floats;
    HK_TRY(launch_prefill_gemm(q, s));
    PrefillAttnArgs at = {};
    at.qkv = e->pf_qkv;
    at.ld_qkv = e->qkv_rows;
    at.cos_tab = e->w.rope_cos;
    at.sin_tab = e->w.rope_sin;
    at.qrot = e->pf_q;
    at.kcache = e->kcache + (size_t)l * kv_layer_elems(e);
    at.vcache = e->vcache + (size_t)l * kv_layer_elems(e);
    at.out = e->pf_att;
    at.ld_out = QD;
    at.out_kblock = kb;
    at.rope_done = rope_fused ? 1 : 0;
    at.n = n;
    at.start = start;
    at.q_heads = d.q_heads;
    at.kv_heads = d.kv_heads;
    at.max_ctx = d.max_context;
    HK_TRY(launch_prefill_attention(at, s));
    PrefillGemmArgs o = {};
    o.A = e->pf_att;
    o.lda = QD;
    o.W = static_cast<const uint16_t*>(lw.o_proj);
    o.Wn = slab && native ? e->pf_native[l][1] : nullptr;
    o.scale = e->w8 ? lw.o_scale : nullptr;
    o.resid = e->pf_x;
    o.ldr = H;
    o.Y = e->pf_h1;
    o.ldy = H;
    o.M = n;
    o.N = H;
    o.K = QD;
    o.epi = EPI_RESID;
    o.kblock = kb;
    o.split_ws = e->pf_split;
    o.split_ws_floats = e->pf_split_floats;
    HK_TRY(launch_prefill_gemm(o, s));
    if (!fused_norm) HK_TRY(launch_rmsnorm_rows(e->pf_h1, H, lw.post_attn_norm, d.rms_eps, e->pf_xn, H, n, H, s));
    PrefillGemmArgs g = {};
    g.A = fused_norm ? e->pf_h1 : e->pf_xn;
    g.gamma = fused_norm ? lw.post_attn_norm : nullptr;
    g.eps = d.rms_eps;
    g.lda = H;
    g.W = static_cast<const uint16_t*>(lw.gate_up);
    g.Wn = slab && native ? e->pf_native[l][2] : nullptr;
    g.scale = e->w8 ? lw.gate_up_scale : nullptr;
    g.Y = e->pf_act;
    g.ldy = I;
    g.M = n;
    g.N = I;
    g.K = H;
    g.epi = EPI_SWIGLU;
    g.kblock = kb;
    g.split_ws = e->pf_split;
    g.split_ws_floats = e->pf_split_floats;
    HK_TRY(launch_prefill_gemm(g, s));
    PrefillGemmArgs dn = {};
    dn.A = e->pf_act;
    dn.lda = I;
    dn.W = static_cast<const uint16_t*>(lw.down_proj);
    dn.Wn = slab && native ? e->pf_native[l][3] : nullptr;
    dn.scale = e->w8 ? lw.down_scale : nullptr;
    dn.resid = e->pf_h1;
    dn.ldr = H;
    dn.Y = e->pf_x;
    dn.ldy = H;
    dn.M = n;
    dn.N = H;
    dn.K = I;
    dn.epi = EPI_RESID;
    dn.kblock = kb;
    dn.split_ws = e->pf_split;
    dn.split_ws_floats = e->pf_split_floats;
    if (slab && e->slab_split && e->slab_ws) {  // K split inside an XCD, a new tag per launch
      if (++e->slab_tag == 0) e->slab_tag = 1;
      dn.slab_ws = e->slab_ws;
      dn.slab_tag = e->slab_tag;
      dn.slab_spin = e->spin_limit;
      dn.slab_error = reinterpret_cast<unsigned*>(e->result + 2);
    }
    HK_TRY(launch_prefill_gemm(dn, s));
  }
  return 0;
}

// ---- static scratch of hk_attention_decode_noalloc ----
// Layout: [0, 256) the position word; [256, 256 + 4 kScratchTickets) the
// per-head split-KV tickets; then the split-KV partials, [q_heads][splits][66]
// floats.  Every GPU holds its own copy until the process ends; calls on one
// GPU share it.
constexpr size_t kScratchTicketsOffset = 256;
constexpr int kScratchTickets = 1024;
constexpr size_t kScratchPartialOffset = kScratchTicketsOffset + 4 * kScratchTickets;
constexpr size_t kScratchPartialBytes = size_t(1) << 20;
constexpr size_t kScratchBytes = kScratchPartialOffset + kScratchPartialBytes;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_scratch_mutex;
std::vector<void*> g_scratch_address;  // device address of `scratch` per device

// Device address of `scratch` on the current device, looked up once per
// device (the array's name in host code is not a device address).
int scratch_address(void** out) {
  int dev = 0;
  HK_CHECK(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if ((int)g_scratch_address.size() <= dev) g_scratch_address.resize(dev + 1, nullptr);
  if (g_scratch_address[dev] == nullptr) {
    void* ptr = nullptr;
    const hipError_t err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (err != hipSuccess) return hip_fail(err, "hipGetSymbolAddress(scratch)");
    if (ptr == nullptr) return fail("hipGetSymbolAddress(scratch) returned null");
    g_scratch_address[dev] = ptr;
  }
  *out = g_scratch_address[dev];
  return 0;
}

// Position word and cleared tickets for one attention call.
__global__ void attention_scratch_kernel(int32_t* position_word, int32_t position, unsigned int* tickets, int n) {
  if (threadIdx.x == 0) *position_word = position;
  for (int i = threadIdx.x; i < n; i += blockDim.x) tickets[i] = 0u;
}

// Argument checks shared by both attention entry points.
int check_attention_args(const uint16_t* qkv, const float* rope_cos, const float* rope_sin,
                         const uint16_t* kcache, const uint16_t* vcache, int32_t position,
                         int32_t max_context, int32_t q_heads, int32_t kv_heads, int32_t head_dim,
                         const uint16_t* out) {
  if (!qkv || !rope_cos || !rope_sin || !kcache || !vcache || !out)
    return fail("hk_attention_decode: null pointer");
  if (head_dim != kHeadDim) {
    set_error("hk_attention_decode: only head_dim 64 is supported");
    return HK_ERR_UNSUPPORTED;
  }
  if (max_context <= 0 || position < 0 || position >= max_context)
    return fail("hk_attention_decode: position outside the context");
  if (kv_heads <= 0 || q_heads <= 0 || q_heads % kv_heads != 0)
    return fail("hk_attention_decode: q_heads must be a multiple of kv_heads");
  if (max_context > kMaxContext) return fail("hk_attention_decode: context above 65536 slots");
  return 0;
}

}  // namespace

extern "C" {

int32_t hk_abi_version(void) { return 1; }

const char* hk_last_error(void) { return g_error.c_str(); }

int hk_init(int32_t device_ordinal) {
  int count = 0;
  HK_CHECK(hipGetDeviceCount(&count));
  if (device_ordinal < 0 || device_ordinal >= count)
    return fail("hk_init: device ordinal out of range");
  HK_CHECK(hipSetDevice(device_ordinal));
  hipDeviceProp_t prop;
  HK_CHECK(hipGetDeviceProperties(&prop, device_ordinal));
  if (std::string(prop.gcnArchName).rfind("gfx950", 0) != 0) {
    set_error(std::string("hk_init: libhk.so is built for gfx950 (MI355X); device is ") +
              prop.gcnArchName);
    return HK_ERR_UNSUPPORTED;
  }
  void* unused = nullptr;
  return scratch_address(&unused);  // resolved once per device, here or at first use
}

int hk_engine_create(const hk_model_desc* desc, const hk_model_weights* weights,
                     hk_engine** out) {
  if (!desc || !weights || !out) return fail("hk_engine_create: null argument");
  *out = nullptr;
  const hk_model_desc& d = *desc;
  if (d.layers <= 0 || d.hidden <= 0 || d.intermediate <= 0 || d.vocab <= 0 || d.max_context <= 0)
    return fail("hk_engine_create: sizes must be positive");
  if (d.max_context > kMaxContext) return fail("hk_engine_create: max_context above 65536");
  if (d.head_dim != kHeadDim) {
    set_error("hk_engine_create: only head_dim 64 is supported");
    return HK_ERR_UNSUPPORTED;
  }
  if (d.kv_heads <= 0 || d.q_heads % d.kv_heads != 0 || d.q_heads / d.kv_heads > kMaxQPerKV)
    return fail("hk_engine_create: q_heads must be a multiple of kv_heads (ratio <= 16)");
  const bool w8 = (d.flags & HK_MODEL_W8) != 0;
  const int align = w8 ? 16 : 8;
  if (d.hidden % align || d.intermediate % align || (d.q_heads * kHeadDim) % align)
    return fail("hk_engine_create: hidden/intermediate sizes must be multiples of 8 (16 for W8)");
  if (!weights->token_embedding || !weights->lm_head || !weights->final_norm ||
      !weights->rope_cos || !weights->rope_sin || !weights->layers)
    return fail("hk_engine_create: missing model tensor");
  for (int l = 0; l < d.layers; ++l) {
    const hk_layer_weights& lw = weights->layers[l];
    if (!lw.qkv || !lw.o_proj || !lw.gate_up || !lw.down_proj || !lw.input_norm ||
        !lw.post_attn_norm)
      return fail("hk_engine_create: missing layer tensor in layer " + std::to_string(l));
    if (w8 && (!lw.qkv_scale || !lw.o_scale || !lw.gate_up_scale || !lw.down_scale))
      return fail("hk_engine_create: W8 layer without scales in layer " + std::to_string(l));
    if ((d.flags & HK_MODEL_QKV_BIAS) && !lw.qkv_bias)
      return fail("hk_engine_create: qkv bias missing in layer " + std::to_string(l));
  }

  hk_engine* e = new hk_engine();
  e->d = d;
  e->w8 = w8;
  e->layers.assign(weights->layers, weights->layers + d.layers);
  if (!(d.flags & HK_MODEL_QKV_BIAS))
    for (auto& lw : e->layers) lw.qkv_bias = nullptr;
  e->w = *weights;
  e->w.layers = e->layers.data();
  e->qkv_rows = (d.q_heads + 2 * d.kv_heads) * kHeadDim;
  e->max_splits = attention_splits(d.max_context);
  const char* env = getenv("HK_EAGER");
  e->use_graph = !(env && env[0] == '1');

  int rc = 0;
  auto body = [&]() -> int {
    HK_CHECK(hipGetDevice(&e->device));
    HK_CHECK(hipStreamCreateWithFlags(&e->stream, hipStreamNonBlocking));
    HK_TRY(dalloc(&e->h, d.hidden));
    HK_TRY(dalloc(&e->h1, d.hidden));
    HK_TRY(dalloc(&e->qkv, e->qkv_rows));
    HK_TRY(dalloc(&e->attn, (size_t)d.q_heads * kHeadDim));
    HK_TRY(dalloc(&e->act, d.intermediate));
    HK_TRY(dalloc(&e->normed, d.hidden));
    // the tail past vocab is the persistent step's per-wave store sink
    HK_TRY(dalloc(&e->logits, (size_t)d.vocab + kPersistentGrid * (kPersistentThreads / 64)));
    const size_t kv = (size_t)d.layers * kv_layer_elems(e);
    HK_TRY(dalloc(&e->kcache, kv));
    HK_TRY(dalloc(&e->vcache, kv));
    // split-KV partials: floats for the per-kernel attention, 64-bit tagged
    // words for the persistent step (twice the floats), zero to start
    HK_TRY(dalloc(&e->partial, partial_floats(e)));
    HK_CHECK(hipMemset(e->partial, 0, partial_floats(e) * sizeof(float)));
    HK_TRY(dalloc(&e->counters, d.q_heads));
    HK_TRY(dalloc(&e->keys, kMaxPartialKeys));
    HK_TRY(dalloc(&e->ctrl, 1));
    HK_TRY(dalloc(&e->out_tokens, d.max_context));
    HK_TRY(dalloc(&e->result, 3));
    HK_CHECK(hipMemset(e->kcache, 0, kv * sizeof(uint16_t)));
    HK_CHECK(hipMemset(e->vcache, 0, kv * sizeof(uint16_t)));
    HK_CHECK(hipMemset(e->h, 0, d.hidden * sizeof(uint16_t)));
    HK_CHECK(hipMemset(e->counters, 0, d.q_heads * sizeof(unsigned int)));
    HK_CHECK(hipMemset(e->ctrl, 0, sizeof(StepCtrl)));
    HK_CHECK(hipMemset(e->result, 0, 3 * sizeof(int32_t)));
    const char* pers = getenv("HK_PERSISTENT");
    if (!(pers && pers[0] == '0') && d.layers <= kPersistentMaxLayers)
      e->pshape = persistent_shape(d.hidden, d.intermediate, d.q_heads, d.kv_heads, w8);
    // polls a persistent-step wait may take before the launch is abandoned
    // (a small value forces the abandon path, for tests of it)
    if (const char* spin = getenv("HK_PERSISTENT_SPIN"))
      e->spin_limit = (unsigned int)strtoul(spin, nullptr, 10);
    // HK_XCD_SPLIT: 0 off, 1 required (creation fails with the reason when
    // the device cannot run it), unset: on where the device allows it
    const char* split = getenv("HK_XCD_SPLIT");
    if (e->pshape >= 0 && !(split && split[0] == '0')) {
      e->xcd_split = persistent_xcd_split(e->pshape, e->stream) == 1;
      if (!e->xcd_split && split && split[0] == '1') return HK_ERR_INVALID;
    }
    // HK_SLAB_SPLIT=0: the down slabs of short prompts unsplit; they rely on
    // the workgroup placement the XCD split checked
    const char* slab_split = getenv("HK_SLAB_SPLIT");
    e->slab_split = e->xcd_split && !(slab_split && slab_split[0] == '0');
    if (e->pshape >= 0) {
      std::vector<PersistentLayer> pl(d.layers);
      for (int l = 0; l < d.layers; ++l) {
        const hk_layer_weights& lw = e->layers[l];
        pl[l] = {static_cast<const uint16_t*>(lw.qkv),     lw.qkv_bias,
                 static_cast<const uint16_t*>(lw.o_proj),  static_cast<const uint16_t*>(lw.gate_up),
                 static_cast<const uint16_t*>(lw.down_proj), lw.input_norm, lw.post_attn_norm,
                 nullptr, lw.qkv_scale, lw.o_scale, lw.gate_up_scale, lw.down_scale, nullptr, nullptr};
      }
      if (e->xcd_split) {
        // the split fuses down_proj into the gate/up workgroups: a regrouped
        // copy per layer (H x I weights each, bf16 or int8) and the
        // partial-sum words
        e->down_x.assign(d.layers, nullptr);
        for (int l = 0; l < d.layers; ++l) {
          HK_TRY(dalloc(&e->down_x[l], (size_t)d.hidden * d.intermediate / (w8 ? 2 : 1)));
          HK_TRY(launch_regroup_down(e->layers[l].down_proj, e->down_x[l], d.hidden, d.intermediate, w8,
                                     e->stream));
          pl[l].down_x = e->down_x[l];
        }
        if (w8) {
          // XCD 0's stager waves read their QKV and O rows as bf16 (exact
          // copies of the int8 values): QKV rows x hidden, then hidden x
          // attention width, per layer
          const size_t nq = (size_t)e->qkv_rows * d.hidden, no = (size_t)d.hidden * d.q_heads * kHeadDim;
          e->wide.assign(d.layers, nullptr);
          for (int l = 0; l < d.layers; ++l) {
            HK_TRY(dalloc(&e->wide[l], nq + no));
            HK_TRY(launch_widen_i8(e->layers[l].qkv, e->wide[l], nq, e->stream));
            HK_TRY(launch_widen_i8(e->layers[l].o_proj, e->wide[l] + nq, no, e->stream));
            pl[l].qkv_wide = e->wide[l];
            pl[l].o_wide = e->wide[l] + nq;
          }
        }
        HK_TRY(dalloc(&e->wpart, (size_t)kPersistentGrid * d.hidden));
        HK_CHECK(hipMemset(e->wpart, 0, (size_t)kPersistentGrid * d.hidden * 8));
        HK_TRY(dalloc(&e->xpart, (size_t)8 * d.hidden));
        HK_CHECK(hipMemset(e->xpart, 0, (size_t)8 * d.hidden * 8));
        HK_CHECK(hipStreamSynchronize(e->stream));
      }
      HK_TRY(dalloc(&e->players, d.layers));
      HK_CHECK(hipMemcpy(e->players, pl.data(), d.layers * sizeof(PersistentLayer),
                         hipMemcpyHostToDevice));
      HK_TRY(dalloc(&e->psync, psync_words(e)));
      HK_CHECK(hipMemset(e->psync, 0, psync_words(e) * sizeof(unsigned int)));
      HK_TRY(dalloc(&e->ptag, ptag_words(e)));
      HK_CHECK(hipMemset(e->ptag, 0, ptag_words(e) * sizeof(uint32_t)));
    }
    HK_CHECK(hipDeviceSynchronize());
    return 0;
  };
  rc = body();
  if (rc != 0) {
    free_engine(e);
    return rc;
  }
  *out = e;
  return 0;
}

int hk_engine_step(hk_engine* e, int32_t token, int32_t position, int32_t want_logits,
                   const uint16_t* embedding_host, float* logits_host, int32_t* next_token_host) {
  if (!e) return fail("hk_engine_step: null engine");
  std::lock_guard<std::mutex> lock(e->mu);
  if (position < 0 || position >= e->d.max_context)
    return fail("position outside the " + std::to_string(e->d.max_context) + "-token context");
  if (embedding_host == nullptr && (token < 0 || token >= e->d.vocab))
    return fail("token id outside the vocabulary");
  if (!want_logits && (logits_host || next_token_host))
    return fail("hk_engine_step: outputs requested without want_logits");
  HK_CHECK(hipSetDevice(e->device));
  if (embedding_host != nullptr) {
    HK_CHECK(hipMemcpyAsync(e->h, embedding_host, e->d.hidden * sizeof(uint16_t),
                            hipMemcpyHostToDevice, e->stream));
    HK_TRY(set_ctrl(e, -1, position, 0));
  } else {
    HK_TRY(set_ctrl(e, token, position, 0));
  }
  HK_TRY(run_step(e, want_logits != 0));
  if (logits_host)
    HK_CHECK(hipMemcpyAsync(logits_host, e->logits, (size_t)e->d.vocab * sizeof(float),
                            hipMemcpyDeviceToHost, e->stream));
  if (embedding_host || logits_host || next_token_host) {
    int32_t result[2] = {0, 0};
    HK_CHECK(hipMemcpyAsync(result, e->result, sizeof(result), hipMemcpyDeviceToHost, e->stream));
    HK_CHECK(hipStreamSynchronize(e->stream));
    HK_TRY(check_persistent(e, result));
    if (next_token_host) *next_token_host = result[0];
  }
  return 0;
}

int hk_engine_generate(hk_engine* e, int32_t token, int32_t position, int32_t n_steps,
                       int32_t* tokens_host) {
  if (!e || !tokens_host) return fail("hk_engine_generate: null argument");
  std::lock_guard<std::mutex> lock(e->mu);
  if (n_steps <= 0) return fail("hk_engine_generate: n_steps must be positive");
  if (position < 0 || (int64_t)position + n_steps > e->d.max_context)
    return fail("position outside the " + std::to_string(e->d.max_context) + "-token context");
  if (token < 0 || token >= e->d.vocab) return fail("token id outside the vocabulary");
  HK_CHECK(hipSetDevice(e->device));
  HK_TRY(set_ctrl(e, token, position, 1));
  for (int i = 0; i < n_steps; ++i) {
    e->next_pos = position + i;
    HK_TRY(run_step(e, true));
  }
  e->next_pos = position + n_steps;
  int32_t result[2] = {0, 0};
  HK_CHECK(hipMemcpyAsync(tokens_host, e->out_tokens, (size_t)n_steps * sizeof(int32_t),
                          hipMemcpyDeviceToHost, e->stream));
  HK_CHECK(hipMemcpyAsync(result, e->result, sizeof(result), hipMemcpyDeviceToHost, e->stream));
  HK_CHECK(hipStreamSynchronize(e->stream));
  return check_persistent(e, result);
}

int hk_engine_prefill(hk_engine* e, const int32_t* tokens_host, int32_t n, int32_t start,
                      float* logits_host, int32_t* next_token_host) {
  if (!e || !tokens_host) return fail("hk_engine_prefill: null argument");
  std::lock_guard<std::mutex> lock(e->mu);
  if (n <= 0) return fail("hk_engine_prefill: n must be positive");
  if (start < 0 || (int64_t)start + n > e->d.max_context)
    return fail("position outside the " + std::to_string(e->d.max_context) + "-token context");
  for (int i = 0; i < n; ++i)
    if (tokens_host[i] < 0 || tokens_host[i] >= e->d.vocab) return fail("token id outside the vocabulary");
  HK_CHECK(hipSetDevice(e->device));
  const bool want = logits_host != nullptr || next_token_host != nullptr;
  if ((e->d.hidden % 32) || (e->d.intermediate % 32) || ((e->d.q_heads * kHeadDim) % 32)) {
    // shapes off the MFMA tile use the decode step per position
    for (int i = 0; i < n; ++i) {
      const bool last = want && i == n - 1;
      HK_TRY(set_ctrl(e, tokens_host[i], start + i, 0));
      HK_TRY(run_step(e, last));
    }
  } else {
    HK_TRY(prefill_workspace(e));
    for (int c0 = 0; c0 < n; c0 += e->pf_rows) {
      const int m = std::min(e->pf_rows, n - c0);
      if (m <= kSlabMaxTokens) HK_TRY(native_copies(e));
      HK_CHECK(hipMemcpyAsync(e->pf_tokens, tokens_host + c0, m * sizeof(int32_t),
                              hipMemcpyHostToDevice, e->stream));
      HK_TRY(prefill_chunk(e, e->pf_tokens, m, start + c0));
      if (c0 + m == n && want) {
        if (m <= kSlabMaxTokens && e->d.hidden <= kSlabNormMaxK)  // k-blocked x: 16-byte pieces m * 16 bytes apart
          HK_CHECK(hipMemcpy2DAsync(e->h, 16, e->pf_x + (size_t)(m - 1) * 8, (size_t)m * 16, 16, e->d.hidden / 8,
                                    hipMemcpyDeviceToDevice, e->stream));
        else
          HK_CHECK(hipMemcpyAsync(e->h, e->pf_x + (size_t)(m - 1) * e->d.hidden,
                                  e->d.hidden * sizeof(uint16_t), hipMemcpyDeviceToDevice, e->stream));
        HK_TRY(set_ctrl(e, -1, start + n - 1, 0));
        HK_TRY(launch_part(e, HK_PART_HEAD, 0));
      }
      HK_CHECK(hipStreamSynchronize(e->stream));  // pf_tokens is reused by the next chunk
    }
  }
  if (logits_host)
    HK_CHECK(hipMemcpyAsync(logits_host, e->logits, (size_t)e->d.vocab * sizeof(float),
                            hipMemcpyDeviceToHost, e->stream));
  int32_t result[3] = {0, 0, 0};  // token, (step error), split-slab error
  HK_CHECK(hipMemcpyAsync(result, e->result, sizeof(result), hipMemcpyDeviceToHost, e->stream));
  HK_CHECK(hipStreamSynchronize(e->stream));
  if (result[2] != 0) {
    // a K-split slab waited too long for one of its parts, or found a part
    // on another XCD: this prefill's KV slots and logits are invalid; later
    // prefills run the slabs unsplit
    e->slab_split = false;
    HK_CHECK(hipMemset(e->result + 2, 0, sizeof(int32_t)));
    HK_CHECK(hipDeviceSynchronize());
    set_error("prefill abandoned: a K-split GEMM waited too long for one of its parts (is another kernel "
              "occupying the GPU?); its KV slots and logits are invalid");
    return HK_ERR_HIP;
  }
  if (next_token_host) *next_token_host = result[0];
  return 0;
}

int hk_engine_final_hidden(hk_engine* e, uint16_t* hidden_host) {
  if (!e || !hidden_host) return fail("hk_engine_final_hidden: null argument");
  std::lock_guard<std::mutex> lock(e->mu);
  HK_CHECK(hipSetDevice(e->device));
  HK_TRY(launch_rmsnorm(e->h, e->w.final_norm, e->d.rms_eps, e->normed, e->d.hidden, e->stream));
  HK_CHECK(hipMemcpyAsync(hidden_host, e->normed, e->d.hidden * sizeof(uint16_t),
                          hipMemcpyDeviceToHost, e->stream));
  HK_CHECK(hipStreamSynchronize(e->stream));
  return 0;
}

int hk_engine_launch_part(hk_engine* e, int32_t part, int32_t layer) {
  if (!e) return fail("hk_engine_launch_part: null engine");
  std::lock_guard<std::mutex> lock(e->mu);
  if (part < HK_PART_QKV || part > HK_PART_STEP) return fail("hk_engine_launch_part: unknown part");
  if (layer < 0 || layer >= e->d.layers) return fail("hk_engine_launch_part: layer out of range");
  HK_CHECK(hipSetDevice(e->device));
  if (part >= HK_PART_HEAD) HK_TRY(set_ctrl_keep(e));
  if (part == HK_PART_STEP) return run_step(e, true);
  return launch_part(e, part, layer);
}

int hk_engine_launch_part_repeat(hk_engine* e, int32_t part, int32_t count) {
  if (!e) return fail("hk_engine_launch_part_repeat: null engine");
  std::lock_guard<std::mutex> lock(e->mu);
  if (part < HK_PART_QKV || part > HK_PART_STEP) return fail("hk_engine_launch_part_repeat: unknown part");
  if (count <= 0 || count > 100000) return fail("hk_engine_launch_part_repeat: count out of range");
  HK_CHECK(hipSetDevice(e->device));
  if (part >= HK_PART_HEAD) HK_TRY(set_ctrl_keep(e));
  if (part == HK_PART_STEP && e->pshape >= 0) {
    // one persistent launch per step: launched back to back, the GPU never
    // waits for the host, so no graph is needed (and profilers that trace
    // kernels see ordinary launches)
    for (int i = 0; i < count; ++i) HK_TRY(launch_persistent(e, true));
    return 0;
  }
  const long long key = (long long)part << 32 | (unsigned)count |
                        (part == HK_PART_STEP && e->pshape >= 0 ? (long long)step_form(e) << 60 : 0);
  auto it = e->repeat_graphs.find(key);
  if (it == e->repeat_graphs.end()) {
    hipGraph_t graph = nullptr;
    HK_CHECK(hipStreamBeginCapture(e->stream, hipStreamCaptureModeThreadLocal));
    int rc = 0;
    for (int i = 0; i < count && rc == 0; ++i) {
      if (part != HK_PART_STEP)
        rc = launch_part(e, part, i % e->d.layers);
      else
        rc = e->pshape >= 0 ? launch_persistent(e, true) : enqueue_step(e, true);
    }
    const hipError_t end = hipStreamEndCapture(e->stream, &graph);
    if (rc != 0) {
      if (graph) (void)hipGraphDestroy(graph);
      return rc;
    }
    if (end != hipSuccess) return hip_fail(end, "hipStreamEndCapture");
    hipGraphExec_t exec = nullptr;
    const hipError_t inst = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    if (inst != hipSuccess) return hip_fail(inst, "hipGraphInstantiate");
    it = e->repeat_graphs.emplace(key, exec).first;
  }
  HK_CHECK(hipGraphLaunch(it->second, e->stream));
  return 0;
}

namespace {
// hk_gemv_repeat's captured graphs, one per argument set (a timed call is a
// replay of the graph its untimed twin captured), at most kGemvGraphs kept.
struct GemvRepeat {
  std::vector<const void*> w;
  std::vector<const float*> s;
  const uint16_t* x;
  float* y;
  int M, K, count, device;
  hipGraphExec_t exec;
};
constexpr size_t kGemvGraphs = 32;
std::mutex gemv_graph_mu;
std::vector<GemvRepeat> gemv_graphs;
}  // namespace

int hk_gemv_repeat(const void* const* weights, const float* const* scales, int32_t n_weights,
                   const uint16_t* x, float* y_f32, int32_t M, int32_t K, int32_t count,
                   void* stream) {
  if (!weights || !x || !y_f32 || n_weights <= 0 || count <= 0 || count > 100000)
    return fail("hk_gemv_repeat: bad argument");
  auto enqueue = [&](hipStream_t s) {
    for (int i = 0; i < count; ++i) {
      const int j = i % n_weights;
      const int rc = gemv_common(weights[j], scales ? scales[j] : nullptr, x, nullptr, nullptr, nullptr, y_f32,
                                 M, K, scales != nullptr, s);
      if (rc != 0) return rc;
    }
    return 0;
  };
  // HK_GEMV_REPEAT_GRAPH=0: direct launches (kernel tracers that do not
  // follow graph launches); otherwise one captured graph, so the host's
  // launch cost (about 2.5 us per launch) does not pace kernels that take
  // about as long
  static const bool direct = [] {
    const char* e = getenv("HK_GEMV_REPEAT_GRAPH");
    return e && e[0] == '0';
  }();
  if (direct) return enqueue(static_cast<hipStream_t>(stream));
  int device = 0;
  HK_CHECK(hipGetDevice(&device));
  std::lock_guard<std::mutex> lock(gemv_graph_mu);
  std::vector<const void*> w(weights, weights + n_weights);
  std::vector<const float*> sc;
  if (scales) sc.assign(scales, scales + n_weights);
  GemvRepeat* hit = nullptr;
  for (GemvRepeat& g : gemv_graphs)
    if (g.w == w && g.s == sc && g.x == x && g.y == y_f32 && g.M == M && g.K == K && g.count == count &&
        g.device == device)
      hit = &g;
  if (!hit) {
    if (gemv_graphs.size() >= kGemvGraphs) {  // the oldest goes (after any replay of it has ended)
      HK_CHECK(hipDeviceSynchronize());
      (void)hipGraphExecDestroy(gemv_graphs.front().exec);
      gemv_graphs.erase(gemv_graphs.begin());
    }
    hipStream_t cs = nullptr;
    HK_CHECK(hipStreamCreateWithFlags(&cs, hipStreamNonBlocking));
    hipGraph_t graph = nullptr;
    hipError_t err = hipStreamBeginCapture(cs, hipStreamCaptureModeThreadLocal);
    int rc = err == hipSuccess ? enqueue(cs) : hip_fail(err, "hipStreamBeginCapture");
    if (err == hipSuccess) {
      const hipError_t end = hipStreamEndCapture(cs, &graph);
      if (rc == 0 && end != hipSuccess) rc = hip_fail(end, "hipStreamEndCapture");
    }
    (void)hipStreamDestroy(cs);
    hipGraphExec_t exec = nullptr;
    if (rc == 0) {
      const hipError_t inst = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
      if (inst != hipSuccess) rc = hip_fail(inst, "hipGraphInstantiate");
    }
    if (graph) (void)hipGraphDestroy(graph);
    if (rc != 0) return rc;
    gemv_graphs.push_back({std::move(w), std::move(sc), x, y_f32, M, K, count, device, exec});
    hit = &gemv_graphs.back();
  }
  HK_CHECK(hipGraphLaunch(hit->exec, static_cast<hipStream_t>(stream)));
  return 0;
}

int hk_engine_read_kv(hk_engine* e, int32_t layer, int32_t slot, uint16_t* k_host,
                      uint16_t* v_host) {
  if (!e || !k_host || !v_host) return fail("hk_engine_read_kv: null argument");
  std::lock_guard<std::mutex> lock(e->mu);
  if (layer < 0 || layer >= e->d.layers) return fail("hk_engine_read_kv: layer out of range");
  if (slot < 0 || slot >= e->d.max_context) return fail("hk_engine_read_kv: slot out of range");
  HK_CHECK(hipSetDevice(e->device));
  HK_CHECK(hipStreamSynchronize(e->stream));
  const size_t row = kHeadDim * sizeof(uint16_t);
  for (int g = 0; g < e->d.kv_heads; ++g) {
    const size_t off = (size_t)layer * kv_layer_elems(e) + ((size_t)g * e->d.max_context + slot) * kHeadDim;
    HK_CHECK(hipMemcpy(k_host + g * kHeadDim, e->kcache + off, row, hipMemcpyDeviceToHost));
    HK_CHECK(hipMemcpy(v_host + g * kHeadDim, e->vcache + off, row, hipMemcpyDeviceToHost));
  }
  return 0;
}

int hk_engine_reset(hk_engine* e) {
  if (!e) return fail("hk_engine_reset: null engine");
  std::lock_guard<std::mutex> lock(e->mu);
  HK_CHECK(hipSetDevice(e->device));
  const size_t kv = (size_t)e->d.layers * kv_layer_elems(e) * sizeof(uint16_t);
  HK_CHECK(hipMemsetAsync(e->kcache, 0, kv, e->stream));
  HK_CHECK(hipMemsetAsync(e->vcache, 0, kv, e->stream));
  // the persistent step's tagged words start over too: zero never matches a
  // tag, so no word written before the reset can satisfy a later poll
  if (e->ptag) HK_CHECK(hipMemsetAsync(e->ptag, 0, ptag_words(e) * sizeof(uint32_t), e->stream));
  if (e->wpart) HK_CHECK(hipMemsetAsync(e->wpart, 0, (size_t)kPersistentGrid * e->d.hidden * 8, e->stream));
  if (e->xpart) HK_CHECK(hipMemsetAsync(e->xpart, 0, (size_t)8 * e->d.hidden * 8, e->stream));
  HK_CHECK(hipMemsetAsync(e->partial, 0, partial_floats(e) * sizeof(float), e->stream));
  e->act_stale = false;
  HK_CHECK(hipStreamSynchronize(e->stream));
  return 0;
}

int hk_engine_skip_epochs(hk_engine* e, uint32_t count) {
  if (!e) return fail("hk_engine_skip_epochs: null engine");
  std::lock_guard<std::mutex> lock(e->mu);
  if (e->pshape < 0) return 0;
  HK_CHECK(hipSetDevice(e->device));
  hipLaunchKernelGGL(skip_epochs_kernel, dim3(1), dim3(256), 0, e->stream, e->psync, kPersistentGrid,
                     kFlagStride, (unsigned int)count);
  HK_CHECK(hipGetLastError());
  HK_CHECK(hipStreamSynchronize(e->stream));
  return 0;
}

void* hk_engine_stream(hk_engine* e) { return e ? (void*)e->stream : nullptr; }

int hk_engine_step_kind(hk_engine* e, int32_t position, int32_t* kind_out) {
  if (!e || !kind_out) return fail("hk_engine_step_kind: null argument");
  if (position < 0 || position >= e->d.max_context)
    return fail("position outside the " + std::to_string(e->d.max_context) + "-token context");
  static const int32_t kinds[] = {HK_STEP_PERSISTENT, HK_STEP_XCD_SPLIT, HK_STEP_XCD_SPLIT_LONG};
  *kind_out = e->pshape < 0 ? HK_STEP_KERNELS : kinds[form_at(e, position)];
  return HK_OK;
}

void hk_engine_destroy(hk_engine* e) {
  if (!e) return;
  {
    std::lock_guard<std::mutex> lock(e->mu);
    (void)hipSetDevice(e->device);
    if (e->stream) (void)hipStreamSynchronize(e->stream);
  }
  free_engine(e);
}

int hk_gemv_bf16(const uint16_t* W, const uint16_t* x, const float* bias,
                 const uint16_t* residual, uint16_t* y, float* y_f32, int32_t M, int32_t K,
                 void* stream) {
  return gemv_common(W, nullptr, x, bias, residual, y, y_f32, M, K, false, stream);
}

int hk_gemv_w8(const int8_t* Wq, const float* scale, const uint16_t* x, const float* bias,
               const uint16_t* residual, uint16_t* y, float* y_f32, int32_t M, int32_t K,
               void* stream) {
  return gemv_common(Wq, scale, x, bias, residual, y, y_f32, M, K, true, stream);
}

int hk_gemm_bf16(const uint16_t* A, int32_t lda, const uint16_t* W, const float* bias,
                 const uint16_t* residual, uint16_t* Y, int32_t M, int32_t N, int32_t K,
                 void* stream) {
  if (!A || !W || !Y) return fail("hk_gemm_bf16: null pointer");
  if (bias && residual) return fail("hk_gemm_bf16: give bias or residual, not both");
  if (lda < K) return fail("hk_gemm_bf16: lda below K");
  PrefillGemmArgs a = {};
  a.A = A;
  a.lda = lda;
  a.W = W;
  a.bias = bias;
  a.resid = residual;
  a.ldr = N;
  a.Y = Y;
  a.ldy = N;
  a.M = M;
  a.N = N;
  a.K = K;
  a.epi = bias ? EPI_BIAS : residual ? EPI_RESID : EPI_BF16;
  return launch_prefill_gemm(a, static_cast<hipStream_t>(stream));
}

int hk_rmsnorm(const uint16_t* x, const uint16_t* gamma, float eps, uint16_t* out, int32_t n,
               void* stream) {
  if (!x || !gamma || !out) return fail("hk_rmsnorm: null pointer");
  return launch_rmsnorm(x, gamma, eps, out, n, static_cast<hipStream_t>(stream));
}

int hk_swiglu(const uint16_t* gate_up, uint16_t* act, int32_t intermediate, void* stream) {
  if (!gate_up || !act) return fail("hk_swiglu: null pointer");
  return launch_swiglu(gate_up, act, intermediate, static_cast<hipStream_t>(stream));
}

int hk_argmax_f32(const float* x, int32_t n, int32_t* index_device, void* stream) {
  if (!x || !index_device) return fail("hk_argmax_f32: null pointer");
  std::lock_guard<std::mutex> lock(g_op_mutex);
  OpScratch* s = nullptr;
  HK_TRY(op_scratch(&s, 0, 0));
  return launch_argmax(x, n, s->keys, index_device, static_cast<hipStream_t>(stream));
}

int hk_attention_decode(const uint16_t* qkv, const float* rope_cos, const float* rope_sin,
                        uint16_t* kcache, uint16_t* vcache, int32_t position,
                        int32_t max_context, int32_t q_heads, int32_t kv_heads,
                        int32_t head_dim, uint16_t* out, void* stream) {
  HK_TRY(check_attention_args(qkv, rope_cos, rope_sin, kcache, vcache, position, max_context, q_heads,
                              kv_heads, head_dim, out));
  const hipStream_t st = static_cast<hipStream_t>(stream);
  std::lock_guard<std::mutex> lock(g_op_mutex);
  const int splits = attention_splits(max_context);
  OpScratch* s = nullptr;
  HK_TRY(op_scratch(&s, (size_t)q_heads * splits * (kHeadDim + 2), q_heads));
  hipLaunchKernelGGL(store_i32_kernel, dim3(1), dim3(1), 0, st, s->position, position);
  HK_CHECK(hipGetLastError());
  AttnArgs a = {};
  a.qkv = qkv;
  a.cos_tab = rope_cos;
  a.sin_tab = rope_sin;
  a.kcache = kcache;
  a.vcache = vcache;
  a.position = s->position;
  a.out = out;
  a.partial = s->partial;
  a.counters = s->counters;
  a.q_heads = q_heads;
  a.kv_heads = kv_heads;
  a.max_ctx = max_context;
  a.max_splits = splits;
  return launch_attention_decode(a, st);
}

int hk_attention_decode_noalloc(const uint16_t* qkv, const float* rope_cos, const float* rope_sin,
                                uint16_t* kcache, uint16_t* vcache, int32_t position,
                                int32_t max_context, int32_t q_heads, int32_t kv_heads,
                                int32_t head_dim, uint16_t* out, void* stream) {
  HK_TRY(check_attention_args(qkv, rope_cos, rope_sin, kcache, vcache, position, max_context, q_heads,
                              kv_heads, head_dim, out));
  const int splits = attention_splits(max_context);
  const size_t partial_bytes = (size_t)q_heads * splits * (kHeadDim + 2) * sizeof(float);
  if (q_heads > kScratchTickets || partial_bytes > kScratchPartialBytes)
    return fail("hk_attention_decode_noalloc: q_heads x ceil(max_context / 256) x 264 bytes of split-KV "
                "partials exceed its 1 MiB static scratch (" + std::to_string(partial_bytes) + " bytes asked)");
  void* base = nullptr;
  HK_TRY(scratch_address(&base));
  unsigned char* b = static_cast<unsigned char*>(base);
  int32_t* position_word = reinterpret_cast<int32_t*>(b);
  unsigned int* tickets = reinterpret_cast<unsigned int*>(b + kScratchTicketsOffset);
  const hipStream_t st = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(attention_scratch_kernel, dim3(1), dim3(256), 0, st, position_word, position, tickets,
                     (int)q_heads);
  HK_CHECK(hipGetLastError());
  AttnArgs a = {};
  a.qkv = qkv;
  a.cos_tab = rope_cos;
  a.sin_tab = rope_sin;
  a.kcache = kcache;
  a.vcache = vcache;
  a.position = position_word;
  a.out = out;
  a.partial = reinterpret_cast<float*>(b + kScratchPartialOffset);
  a.counters = tickets;
  a.q_heads = q_heads;
  a.kv_heads = kv_heads;
  a.max_ctx = max_context;
  a.max_splits = splits;
  return launch_attention_decode(a, st);
}

int hk_stream_sync(void* stream) {
  HK_CHECK(hipStreamSynchronize(static_cast<hipStream_t>(stream)));
  return 0;
}

int hk_malloc(uint64_t bytes, void** device_ptr) {
  if (!device_ptr) return fail("hk_malloc: null output");
  *device_ptr = nullptr;
  if (bytes == 0) return fail("hk_malloc: zero bytes");
  HK_CHECK(hipMalloc(device_ptr, bytes));
  return 0;
}

int hk_free(void* device_ptr) {
  if (device_ptr) HK_CHECK(hipFree(device_ptr));
  return 0;
}

int hk_memcpy_h2d(void* device_dst, const void* host_src, uint64_t bytes) {
  if (bytes == 0) return 0;
  if (!device_dst || !host_src) return fail("hk_memcpy_h2d: null pointer");
  HK_CHECK(hipMemcpy(device_dst, host_src, bytes, hipMemcpyHostToDevice));
  return 0;
}

int hk_memcpy_d2h(void* host_dst, const void* device_src, uint64_t bytes) {
  if (bytes == 0) return 0;
  if (!host_dst || !device_src) return fail("hk_memcpy_d2h: null pointer");
  HK_CHECK(hipMemcpy(host_dst, device_src, bytes, hipMemcpyDeviceToHost));
  return 0;
}

int hk_memcpy_d2d(void* device_dst, const void* device_src, uint64_t bytes) {
  if (bytes == 0) return 0;
  if (!device_dst || !device_src) return fail("hk_memcpy_d2d: null pointer");
  HK_CHECK(hipMemcpy(device_dst, device_src, bytes, hipMemcpyDeviceToDevice));
  return 0;
}

int hk_memset(void* device_dst, int32_t value, uint64_t bytes) {
  if (bytes == 0) return 0;
  if (!device_dst) return fail("hk_memset: null pointer");
  HK_CHECK(hipMemset(device_dst, value, bytes));
  HK_CHECK(hipDeviceSynchronize());
  return 0;
}

int hk_stream_create(void** stream) {
  if (!stream) return fail("hk_stream_create: null output");
  hipStream_t s = nullptr;
  HK_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  *stream = s;
  return 0;
}

int hk_stream_destroy(void* stream) {
  if (stream) HK_CHECK(hipStreamDestroy(static_cast<hipStream_t>(stream)));
  return 0;
}

int hk_event_create(void** event) {
  if (!event) return fail("hk_event_create: null output");
  hipEvent_t ev = nullptr;
  HK_CHECK(hipEventCreate(&ev));
  *event = ev;
  return 0;
}

int hk_event_destroy(void* event) {
  if (event) HK_CHECK(hipEventDestroy(static_cast<hipEvent_t>(event)));
  return 0;
}

int hk_event_record(void* event, void* stream) {
  if (!event) return fail("hk_event_record: null event");
  HK_CHECK(hipEventRecord(static_cast<hipEvent_t>(event), static_cast<hipStream_t>(stream)));
  return 0;
}

int hk_event_elapsed_ms(void* start, void* end, float* ms) {
  if (!start || !end || !ms) return fail("hk_event_elapsed_ms: null argument");
  HK_CHECK(hipEventSynchronize(static_cast<hipEvent_t>(end)));
  HK_CHECK(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(end)));
  return 0;
}

}  // extern "C"
