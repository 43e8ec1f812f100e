// Routed-expert (MoE) block for 1..max_tokens tokens.
//
// The reference offloads expert projections given expert ids (GGML
// MUL_MAT_ID, ollama-xdna/backend/ggml-xdna.cpp:1301-1441; Colibri expert
// group, colibri-xdna/backend/backend_xdna.cpp:316-348: gate, up, silu(g)*u,
// down).  This file adds the router and the combine around them:
//   router_topk   r = W_router @ x (float32), p = softmax(r), top-k by p with
//                 ties to the lower expert id (one wave per token, lane = expert)
//   route_plan    groups the (token, expert) pairs by expert: routed experts in
//                 id order, then the shared experts (every token, weight 1)
//   grouped GEMM  (prefill.hip, grouped mode) gate/up + SwiGLU, then down, each
//                 expert's weights streamed once for all of its tokens
//   combine       y = bf16(sum_k p_k * e_k + sum_s e_s) in float32, rank order
// Rounding points follow the dense layer: bf16 after gate/up, after SwiGLU and
// after down.
#include <algorithm>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/hk.h"
#include "hk_common.h"
#include "hk_internal.h"

namespace hk {
namespace {

#define MOE_CHECK(expr)                                   \
  do {                                                    \
    const hipError_t err_ = (expr);                       \
    if (err_ != hipSuccess) return hip_fail(err_, #expr); \
  } while (0)
#define MOE_TRY(expr)         \
  do {                        \
    const int rc_ = (expr);   \
    if (rc_ != 0) return rc_; \
  } while (0)

constexpr int kThreads = 256;
constexpr int kMaxRouted = 64;   // one lane per routed expert
constexpr int kMaxShared = 8;
constexpr int kMaxTopK = 16;

__global__ __launch_bounds__(kThreads) void router_topk_kernel(const uint16_t* x, const uint16_t* router,
                                                               int H, int E, int K, int32_t* ids,
                                                               float* weights) {
  extern __shared__ float xs[];
  __shared__ float logits[kMaxRouted];
  const int t = blockIdx.x;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const uint16_t* xt = x + (size_t)t * H;
  for (int i = tid; i < H; i += kThreads) xs[i] = bf16_to_f32(xt[i]);
  __syncthreads();
  const int CH = H / 8;
  for (int e = wave; e < E; e += kThreads / 64) {
    const uint16_t* w = router + (size_t)e * H;
    float a0 = 0.f, a1 = 0.f;
    for (int c = lane; c < CH; c += 64) {
      const u32x4 v = load16(w + c * 8);
      const float* xv = xs + c * 8;
      a0 = fmaf(bf_lo(v.x), xv[0], a0);
      a1 = fmaf(bf_hi(v.x), xv[1], a1);
      a0 = fmaf(bf_lo(v.y), xv[2], a0);
      a1 = fmaf(bf_hi(v.y), xv[3], a1);
      a0 = fmaf(bf_lo(v.z), xv[4], a0);
      a1 = fmaf(bf_hi(v.z), xv[5], a1);
      a0 = fmaf(bf_lo(v.w), xv[6], a0);
      a1 = fmaf(bf_hi(v.w), xv[7], a1);
    }
    const float r = group_sum<64>(a0 + a1);
    if (lane == 0) logits[e] = r;
  }
  __syncthreads();
  if (wave != 0) return;
  const bool live = lane < E;
  const float r = live ? logits[lane] : -INFINITY;
  const float m = group_max<64>(r);
  const float ex = live ? expf(r - m) : 0.0f;
  const float s = group_sum<64>(ex);
  const float p = ex / s;
  bool alive = live;
  for (int k = 0; k < K; ++k) {
    unsigned long long key = alive ? argmax_key(p, (uint32_t)lane) : 0ull;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) key = umax64(key, shfl_xor_u64(key, off));
    const int idx = (int)argmax_key_index(key);
    const float pw = __shfl(p, idx, 64);
    if (lane == 0) {
      ids[t * K + k] = idx;
      weights[t * K + k] = pw;
    }
    if (lane == idx) alive = false;
  }
}

// Serial grouping of T*(K+S) pairs (a few hundred at most) by one thread.
__global__ void route_plan_kernel(const int32_t* ids, int T, int K, int E, int S, int32_t* grp_expert,
                                  int32_t* grp_count, int32_t* grp_offset, int32_t* n_groups,
                                  int32_t* a_rows, int32_t* pair_slot) {
  __shared__ int counts[kMaxRouted + kMaxShared];
  __shared__ int cursor[kMaxRouted + kMaxShared];
  if (threadIdx.x != 0) return;
  const int total = E + S;
  for (int e = 0; e < total; ++e) counts[e] = 0;
  for (int i = 0; i < T * K; ++i) {
    int e = ids[i];
    e = e < 0 ? 0 : (e >= E ? E - 1 : e);
    counts[e] += 1;
  }
  for (int s = 0; s < S; ++s) counts[E + s] = T;
  int n = 0, off = 0;
  for (int e = 0; e < total; ++e) {
    cursor[e] = off;
    if (counts[e] == 0) continue;
    grp_expert[n] = e;
    grp_count[n] = counts[e];
    grp_offset[n] = off;
    off += counts[e];
    ++n;
  }
  *n_groups = n;
  const int per = K + S;
  for (int t = 0; t < T; ++t) {
    for (int k = 0; k < K; ++k) {
      int e = ids[t * K + k];
      e = e < 0 ? 0 : (e >= E ? E - 1 : e);
      const int slot = cursor[e]++;
      a_rows[slot] = t;
      pair_slot[t * per + k] = slot;
    }
    for (int s = 0; s < S; ++s) {
      const int slot = cursor[E + s]++;
      a_rows[slot] = t;
      pair_slot[t * per + K + s] = slot;
    }
  }
}

__global__ __launch_bounds__(kThreads) void combine_kernel(const uint16_t* out, const int32_t* pair_slot,
                                                           const float* weights, int H, int K, int S,
                                                           uint16_t* y) {
  const int t = blockIdx.x;
  const int per = K + S;
  for (int d = threadIdx.x; d < H; d += kThreads) {
    float acc = 0.0f;
    for (int k = 0; k < K; ++k) {
      const float v = bf16_to_f32(out[(size_t)pair_slot[t * per + k] * H + d]);
      acc = acc + weights[t * K + k] * v;
    }
    for (int s = 0; s < S; ++s) acc = acc + bf16_to_f32(out[(size_t)pair_slot[t * per + K + s] * H + d]);
    y[(size_t)t * H + d] = (uint16_t)f32_to_bf16(acc);
  }
}

}  // namespace
}  // namespace hk

using namespace hk;

struct hk_moe {
  std::mutex mu;
  hk_moe_desc d{};
  const uint16_t* router = nullptr;
  const uint16_t* gate_up = nullptr;
  const uint16_t* down = nullptr;
  int32_t* ids = nullptr;        // [max_tokens * top_k]
  float* weights = nullptr;      // [max_tokens * top_k]
  int32_t* grp_expert = nullptr;
  int32_t* grp_count = nullptr;
  int32_t* grp_offset = nullptr;
  int32_t* n_groups = nullptr;
  int32_t* a_rows = nullptr;     // [pairs]
  int32_t* pair_slot = nullptr;  // [max_tokens * (top_k + shared)]
  uint16_t* act = nullptr;       // [pairs, I]
  uint16_t* out = nullptr;       // [pairs, H]
};

namespace {

void moe_free(hk_moe* m) {
  void* bufs[] = {m->ids, m->weights, m->grp_expert, m->grp_count, m->grp_offset, m->n_groups,
                  m->a_rows, m->pair_slot, m->act, m->out};
  for (void* p : bufs)
    if (p) (void)hipFree(p);
  delete m;
}

int moe_run(hk_moe* m, const uint16_t* x, int T, const int32_t* ids, const float* weights,
            uint16_t* y, hipStream_t st) {
  const hk_moe_desc& d = m->d;
  const int K = d.top_k, S = d.shared, E = d.experts;
  hipLaunchKernelGGL(route_plan_kernel, dim3(1), dim3(64), 0, st, ids, T, K, E, S, m->grp_expert,
                     m->grp_count, m->grp_offset, m->n_groups, m->a_rows, m->pair_slot);
  MOE_CHECK(hipGetLastError());
  const int max_groups = std::min(E, T * K) + S;
  PrefillGemmArgs gu = {};
  gu.A = x;
  gu.lda = d.hidden;
  gu.W = m->gate_up;
  gu.w_stride = (long long)2 * d.intermediate * d.hidden;
  gu.Y = m->act;
  gu.ldy = d.intermediate;
  gu.M = T;
  gu.N = d.intermediate;
  gu.K = d.hidden;
  gu.epi = EPI_SWIGLU;
  gu.a_rows = m->a_rows;
  gu.grp_expert = m->grp_expert;
  gu.grp_count = m->grp_count;
  gu.grp_offset = m->grp_offset;
  gu.n_groups = m->n_groups;
  gu.max_groups = max_groups;
  gu.max_rows = T;
  MOE_TRY(launch_prefill_gemm(gu, st));
  PrefillGemmArgs dn = gu;
  dn.A = m->act;
  dn.lda = d.intermediate;
  dn.W = m->down;
  dn.w_stride = (long long)d.hidden * d.intermediate;
  dn.Y = m->out;
  dn.ldy = d.hidden;
  dn.N = d.hidden;
  dn.K = d.intermediate;
  dn.epi = EPI_BF16;
  dn.a_rows = nullptr;
  MOE_TRY(launch_prefill_gemm(dn, st));
  hipLaunchKernelGGL(combine_kernel, dim3(T), dim3(kThreads), 0, st, m->out, m->pair_slot, weights,
                     d.hidden, K, S, y);
  MOE_CHECK(hipGetLastError());
  return 0;
}

template <typename T>
int moe_alloc(T** p, size_t count) {
  MOE_CHECK(hipMalloc(reinterpret_cast<void**>(p), count * sizeof(T)));
  return 0;
}

}  // namespace

extern "C" {

int hk_moe_create(const hk_moe_desc* desc, const uint16_t* router, const uint16_t* gate_up,
                  const uint16_t* down, hk_moe** out) {
  if (!desc || !router || !gate_up || !down || !out) return fail("hk_moe_create: null argument");
  *out = nullptr;
  const hk_moe_desc& d = *desc;
  if (d.experts <= 0 || d.experts > kMaxRouted) return fail("hk_moe_create: 1..64 routed experts");
  if (d.shared < 0 || d.shared > kMaxShared) return fail("hk_moe_create: 0..8 shared experts");
  if (d.top_k <= 0 || d.top_k > d.experts || d.top_k > kMaxTopK) return fail("hk_moe_create: bad top_k");
  if (d.hidden <= 0 || d.hidden % 32 || d.intermediate <= 0 || d.intermediate % 32)
    return fail("hk_moe_create: hidden and intermediate must be positive multiples of 32");
  if (d.max_tokens <= 0 || d.max_tokens > 256) return fail("hk_moe_create: max_tokens must be 1..256");
  hk_moe* m = new hk_moe();
  m->d = d;
  m->router = router;
  m->gate_up = gate_up;
  m->down = down;
  const size_t pairs = (size_t)d.max_tokens * (d.top_k + d.shared);
  const size_t groups = (size_t)d.experts + d.shared;
  auto body = [&]() -> int {
    MOE_TRY(moe_alloc(&m->ids, (size_t)d.max_tokens * d.top_k));
    MOE_TRY(moe_alloc(&m->weights, (size_t)d.max_tokens * d.top_k));
    MOE_TRY(moe_alloc(&m->grp_expert, groups));
    MOE_TRY(moe_alloc(&m->grp_count, groups));
    MOE_TRY(moe_alloc(&m->grp_offset, groups));
    MOE_TRY(moe_alloc(&m->n_groups, 1));
    MOE_TRY(moe_alloc(&m->a_rows, pairs));
    MOE_TRY(moe_alloc(&m->pair_slot, pairs));
    MOE_TRY(moe_alloc(&m->act, pairs * d.intermediate));
    MOE_TRY(moe_alloc(&m->out, pairs * d.hidden));
    return 0;
  };
  const int rc = body();
  if (rc != 0) {
    moe_free(m);
    return rc;
  }
  *out = m;
  return 0;
}

int hk_moe_forward(hk_moe* m, const uint16_t* x, int32_t tokens, uint16_t* y, int32_t* ids_out,
                   float* weights_out, void* stream) {
  if (!m || !x || !y) return fail("hk_moe_forward: null argument");
  std::lock_guard<std::mutex> lock(m->mu);
  if (tokens <= 0 || tokens > m->d.max_tokens) return fail("hk_moe_forward: token count out of range");
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const hk_moe_desc& d = m->d;
  const size_t lds = (size_t)d.hidden * sizeof(float);
  if (lds > 65536) return fail("hk_moe_forward: hidden above 16384");
  hipLaunchKernelGGL(router_topk_kernel, dim3(tokens), dim3(kThreads), lds, st, x, m->router,
                     d.hidden, d.experts, d.top_k, m->ids, m->weights);
  MOE_CHECK(hipGetLastError());
  MOE_TRY(moe_run(m, x, tokens, m->ids, m->weights, y, st));
  const size_t nk = (size_t)tokens * d.top_k;
  if (ids_out)
    MOE_CHECK(hipMemcpyAsync(ids_out, m->ids, nk * sizeof(int32_t), hipMemcpyDeviceToDevice, st));
  if (weights_out)
    MOE_CHECK(hipMemcpyAsync(weights_out, m->weights, nk * sizeof(float), hipMemcpyDeviceToDevice, st));
  return 0;
}

int hk_moe_experts(hk_moe* m, const uint16_t* x, int32_t tokens, const int32_t* ids,
                   const float* weights, uint16_t* y, void* stream) {
  if (!m || !x || !ids || !weights || !y) return fail("hk_moe_experts: null argument");
  std::lock_guard<std::mutex> lock(m->mu);
  if (tokens <= 0 || tokens > m->d.max_tokens) return fail("hk_moe_experts: token count out of range");
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const size_t nk = (size_t)tokens * m->d.top_k;
  std::vector<int32_t> host(nk);
  MOE_CHECK(hipMemcpyAsync(host.data(), ids, nk * sizeof(int32_t), hipMemcpyDeviceToHost, st));
  MOE_CHECK(hipStreamSynchronize(st));
  for (int32_t e : host)
    if (e < 0 || e >= m->d.experts) return fail("hk_moe_experts: expert id out of range");
  return moe_run(m, x, tokens, ids, weights, y, st);
}

void hk_moe_destroy(hk_moe* m) {
  if (m) moe_free(m);
}

}  // extern "C"
