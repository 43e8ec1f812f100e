// Routed-expert (MoE) block for 1..max_tokens tokens.
//
// The reference offloads expert projections given expert ids (GGML
// MUL_MAT_ID, ollama-xdna/backend/ggml-xdna.cpp:1301-1441; Colibri expert
// group, colibri-xdna/backend/backend_xdna.cpp:316-348: gate, up, silu(g)*u,
// down).  This file adds the router and the combine around them:
//   router        r = W_router @ x (float32), 16 experts of one token per
//                 workgroup (router_logits); then p = softmax(r), top-k by p
//                 with ties to the lower expert id (one wave per token, lane =
//                 expert) and the plan, in one workgroup (topk_plan)
//   route_plan    groups the (token, expert) pairs by expert: routed experts in
//                 id order, then the shared experts (every token, weight 1)
//   expert GEMMs  gate/up + SwiGLU, then down, each expert's weights streamed
//                 once for all of its tokens: up to 16 rows per expert on
//                 expert_slab (one workgroup per 16 outputs of an expert, K
//                 split over its waves, every weight fragment requested at
//                 once); more rows on prefill.hip's grouped GEMM
//   combine       y = bf16(sum_k p_k * e_k + sum_s e_s) in float32, rank order,
//                 one thread per output element
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

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kMaxRouted = 64;   // one lane per routed expert
constexpr int kMaxShared = 8;
constexpr int kMaxTopK = 16;

constexpr int kRouterRows = 16;  // routed experts per router_logits workgroup
constexpr int kPlanThreads = 1024;  // topk_plan: one wave per token, 16 at a time
constexpr int kMaxTokens = 256;

// r[t][e] = W_router[e] . x[t] in float32 for the kRouterRows experts e0.. of
// token t = blockIdx.x: wave w takes experts e0 + 4 w .. + 3 and requests
// every lane's chunks of the four rows at once.  Per expert row the lane sums
// its chunks c = lane + 64 j in order into two accumulators (even and odd
// elements), and the 64 lanes are added by group_sum.
__global__ __launch_bounds__(kThreads) void router_logits_kernel(const uint16_t* x, const uint16_t* router,
                                                                 int H, int E, float* logits) {
  constexpr int R = kRouterRows / (kThreads / 64);  // rows per wave
  constexpr int J = 4;                               // chunks per lane per round
  const int t = blockIdx.x;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int e0 = blockIdx.y * kRouterRows + wave * R;
  const int CH = H / 8;
  const uint16_t* xt = x + (size_t)t * H;
  float a0[R], a1[R];
#pragma unroll
  for (int r = 0; r < R; ++r) a0[r] = a1[r] = 0.0f;
  const u32x4 zero = {0u, 0u, 0u, 0u};
  for (int c0 = 0; c0 < CH; c0 += 64 * J) {
    u32x4 xv[J], wv[R][J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int c = c0 + lane + 64 * j;
      xv[j] = c < CH ? load16(xt + c * 8) : zero;
#pragma unroll
      for (int r = 0; r < R; ++r) wv[r][j] = c < CH && e0 + r < E ? load16(router + (size_t)(e0 + r) * H + c * 8) : zero;
    }
#pragma unroll
    for (int j = 0; j < J; ++j)
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const u32x4 v = wv[r][j], xx = xv[j];
        a0[r] = fmaf(bf_lo(v.x), bf_lo(xx.x), a0[r]);
        a1[r] = fmaf(bf_hi(v.x), bf_hi(xx.x), a1[r]);
        a0[r] = fmaf(bf_lo(v.y), bf_lo(xx.y), a0[r]);
        a1[r] = fmaf(bf_hi(v.y), bf_hi(xx.y), a1[r]);
        a0[r] = fmaf(bf_lo(v.z), bf_lo(xx.z), a0[r]);
        a1[r] = fmaf(bf_hi(v.z), bf_hi(xx.z), a1[r]);
        a0[r] = fmaf(bf_lo(v.w), bf_lo(xx.w), a0[r]);
        a1[r] = fmaf(bf_hi(v.w), bf_hi(xx.w), a1[r]);
      }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const float v = group_sum<64>(a0[r] + a1[r]);
    if (lane == 0 && e0 + r < E) logits[t * E + e0 + r] = v;
  }
}

// p = softmax(r) over the routed experts and the top K by p (ties to the
// lower expert id) of token t, on one wave (lane = expert).
__device__ __forceinline__ void topk_wave(const float* logits, int t, int E, int K, int lane, int32_t* ids,
                                          float* weights, int32_t* ids_lds) {
  const bool live = lane < E;
  const float r = live ? logits[t * E + lane] : -INFINITY;
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
      ids_lds[t * K + k] = idx;
    }
    if (lane == idx) alive = false;
  }
}

// The grouping of the T*(K+S) (token, expert) pairs by expert, from the ids
// in LDS, on the calling workgroup (nt threads; every thread calls it):
// counts by LDS atomics; the offsets and the non-empty groups on wave 0 (lane
// e: routed expert e, a prefix sum across lanes, the group index from a
// ballot; the shared experts follow the routed pairs); then routed expert
// e's slots by thread e, which walks the pairs in token order (an expert
// appears at most once per token from the router; repeated caller ids take
// consecutive slots), and shared expert s's slots (one per token) by thread
// E + s.  Within an expert the slots follow token order, so the plan does not
// depend on timing.
// `tokens` (distinct: every token names an expert at most once, T <= 64):
// routed expert e's tokens as a bit mask, and pair (t, k)'s slot is e's
// offset plus the number of e's tokens before t, all pairs at once.
__device__ void plan_pairs(const int32_t* ids, int T, int K, int E, int S, int nt, int* counts, int* offs,
                           unsigned long long* tokens, bool distinct, int32_t* grp_expert, int32_t* grp_count,
                           int32_t* grp_offset, int32_t* n_groups, int32_t* a_rows, int32_t* pair_slot) {
  static_assert(kMaxRouted <= 64, "one lane per routed expert");
  const int tid = threadIdx.x;
  const int total = E + S, per = K + S;
  auto clamp = [&](int e) { return e < 0 ? 0 : (e >= E ? E - 1 : e); };
  distinct = distinct && T <= 64;
  for (int e = tid; e < E; e += nt) {
    counts[e] = 0;
    tokens[e] = 0ull;
  }
  __syncthreads();
  for (int i = tid; i < T * K; i += nt) {
    const int e = clamp(ids[i]);
    atomicAdd(&counts[e], 1);
    if (distinct) atomicOr(&tokens[e], 1ull << (i / K));
  }
  __syncthreads();
  if (tid < 64) {
    const int lane = tid;
    const int c = lane < E ? counts[lane] : 0;
    int incl = c;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int v = __shfl_up(incl, d, 64);
      if (lane >= d) incl += v;
    }
    const unsigned long long nonempty = __ballot(c > 0);
    const int g = __popcll(nonempty & ((1ull << lane) - 1ull));
    const int nr = __popcll(nonempty);
    if (lane < E) {
      offs[lane] = incl - c;
      if (c > 0) {
        grp_expert[g] = lane;
        grp_count[g] = c;
        grp_offset[g] = incl - c;
      }
    }
    if (lane < S) {  // shared expert lane: every token, after the routed pairs
      offs[E + lane] = T * K + lane * T;
      grp_expert[nr + lane] = E + lane;
      grp_count[nr + lane] = T;
      grp_offset[nr + lane] = T * K + lane * T;
    }
    if (lane == 0) *n_groups = nr + S;
  }
  __syncthreads();
  if (distinct) {
    for (int i = tid; i < T * (K + S); i += nt) {
      const int t = i / per, k = i % per;
      int slot;
      if (k < K) {
        const int e = clamp(ids[t * K + k]);
        slot = offs[e] + __popcll(tokens[e] & ((1ull << t) - 1ull));
      } else {
        slot = offs[E + k - K] + t;
      }
      a_rows[slot] = t;
      pair_slot[t * per + k] = slot;
    }
    return;
  }
  for (int e = tid; e < total; e += nt) {
    int slot = offs[e];
    if (e < E) {
#pragma unroll 8
      for (int i = 0; i < T * K; ++i)
        if (clamp(ids[i]) == e) {
          a_rows[slot] = i / K;
          pair_slot[(i / K) * per + i % K] = slot;
          ++slot;
        }
    } else {
      for (int t = 0; t < T; ++t, ++slot) {
        a_rows[slot] = t;
        pair_slot[t * per + K + (e - E)] = slot;
      }
    }
  }
}

// Top-k of every token (wave w takes tokens w, w + 16, ...), then the plan.
__global__ __launch_bounds__(kPlanThreads) void topk_plan_kernel(const float* logits, int T, int E, int K, int S,
                                                                 int32_t* ids, float* weights, int32_t* grp_expert,
                                                                 int32_t* grp_count, int32_t* grp_offset,
                                                                 int32_t* n_groups, int32_t* a_rows,
                                                                 int32_t* pair_slot) {
  __shared__ int32_t sids[kMaxTokens * kMaxTopK];
  __shared__ int counts[kMaxRouted + kMaxShared];
  __shared__ int offs[kMaxRouted + kMaxShared];
  __shared__ unsigned long long tokens[kMaxRouted];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  for (int t = wave; t < T; t += kPlanThreads / 64) topk_wave(logits, t, E, K, lane, ids, weights, sids);
  __syncthreads();
  // (the top-k of a token names each expert once)
  plan_pairs(sids, T, K, E, S, kPlanThreads, counts, offs, tokens, true, grp_expert, grp_count, grp_offset,
             n_groups, a_rows, pair_slot);
}

// The plan for caller-supplied ids (hk_moe_experts): the ids are copied to
// LDS, then grouped.
__global__ __launch_bounds__(kThreads) void route_plan_kernel(const int32_t* ids, int T, int K, int E, int S,
                                                              int32_t* grp_expert, int32_t* grp_count,
                                                              int32_t* grp_offset, int32_t* n_groups,
                                                              int32_t* a_rows, int32_t* pair_slot) {
  __shared__ int32_t sids[kMaxTokens * kMaxTopK];
  __shared__ int counts[kMaxRouted + kMaxShared];
  __shared__ int offs[kMaxRouted + kMaxShared];
  __shared__ unsigned long long tokens[kMaxRouted];
  for (int i = threadIdx.x; i < T * K; i += kThreads) sids[i] = ids[i];
  __syncthreads();
  // (caller ids may name an expert twice for one token: the serial slots)
  plan_pairs(sids, T, K, E, S, kThreads, counts, offs, tokens, false, grp_expert, grp_count, grp_offset, n_groups,
             a_rows, pair_slot);
}

// y[t][d] = bf16(sum_k p_k e_k[d] + sum_s e_s[d]) in float32, ranks in order;
// one thread per (t, d): every expert output of the element requested at once.
__global__ __launch_bounds__(kThreads) void combine_kernel(const uint16_t* out, const int32_t* pair_slot,
                                                           const float* weights, int H, int K, int S,
                                                           uint16_t* y) {
  const int t = blockIdx.x;
  const int d = blockIdx.y * kThreads + threadIdx.x;
  if (d >= H) return;
  const int per = K + S;
  float v[kMaxTopK + kMaxShared];
#pragma unroll
  for (int k = 0; k < kMaxTopK + kMaxShared; ++k)
    v[k] = k < per ? bf16_to_f32(out[(size_t)pair_slot[t * per + k] * H + d]) : 0.0f;
  float acc = 0.0f;
  for (int k = 0; k < K; ++k) acc = acc + weights[t * K + k] * v[k];
  for (int s = 0; s < S; ++s) acc = acc + v[K + s];
  y[(size_t)t * H + d] = (uint16_t)f32_to_bf16(acc);
}

// SwiGLU of the bf16 gate and up sums, as in the dense layer's GEMMs.
__device__ __forceinline__ float silu_mul(float g, float u) {
  const float clipped = fminf(fmaxf(g, -80.0f), 80.0f);
  return (g / (1.0f + expf(-clipped))) * u;
}

constexpr int kSlabThreads = 512;               // expert_slab: 8 waves
constexpr int kSlabWavesE = kSlabThreads / 64;
constexpr int kSlabBatchE = 8;                  // K steps per wave requested at once
constexpr int kSlabMaxRowsE = 16;               // rows per expert group on expert_slab

// Expert GEMM for groups of at most 16 rows (the decode batch).  Workgroup
// (s, z) computes outputs 16 s .. + 15 of group z's expert (the MFMA-native
// copy Wn + expert * w_stride) for the group's rows: wave w takes the 32-column K steps w, w +
// 8, ..., requests the weight fragments (and the up rows' for SwiGLU) and the
// row fragments of up to kSlabBatchE of them at once, and multiplies on MFMA
// 16x16x32 (rows x outputs); the waves' partial sums meet in LDS and are added
// in wave order.  Row i of the group reads A row a_rows[offset + i] (or offset
// + i) and writes output row offset + i.  Epilogue as the dense layer:
// SwiGLU bf16(silu(bf16(g)) * bf16(u)), else bf16.
// TWO (without SwiGLU): the workgroup takes outputs 32 s .. + 31, the second
// 16 in place of the up rows (one row fragment, two weight fragments per K step).
template <bool PAIR, bool TWO = false>
__global__ __launch_bounds__(kSlabThreads) void expert_slab_kernel(PrefillGemmArgs a) {
  static_assert(!(PAIR && TWO), "SwiGLU pairs take one slab");
  constexpr bool U = PAIR || TWO;  // a second weight fragment per step
  __shared__ f32x4 red[U ? 2 : 1][kSlabWavesE][64];
  const int z = blockIdx.y;
  if (z >= *a.n_groups) return;
  const int count = min(a.grp_count[z], kSlabMaxRowsE);
  const int off = a.grp_offset[z];
  const int n0 = blockIdx.x * (TWO ? 32 : 16);
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int fr = lane & 15, fk = (lane >> 4) * 8;
  const int N = a.N, K = a.K;
  // the expert's MFMA-native copy (Wn: [rows / 16][K / 8][16] pieces of 8
  // weights, a fragment's 16 rows one 256-byte run, a wave's K step one 1 KiB
  // run)
  const uint16_t* W = static_cast<const uint16_t*>(a.Wn) + (size_t)a.grp_expert[z] * (size_t)a.w_stride;
  const __amdgpu_buffer_rsrc_t wr = rsrc(W, (PAIR ? 2 : 1) * N * K * 2);
  // this lane's piece of its weight row (and up row) and its A row at column
  // fk; rows past the ends read zero
  auto piece = [&](int n) { return (unsigned)((((n >> 4) * (K >> 3) + (fk >> 3)) * 16 + (n & 15)) * 16); };
  const unsigned wofs = n0 + fr < N ? piece(n0 + fr) : 0x7ffffff0u;
  const unsigned uofs = PAIR ? (n0 + fr < N ? piece(N + n0 + fr) : 0x7ffffff0u)
                             : (n0 + 16 + fr < N ? piece(n0 + 16 + fr) : 0x7ffffff0u);
  const int arow = fr < count ? (a.a_rows ? a.a_rows[off + fr] : off + fr) : -1;
  const __amdgpu_buffer_rsrc_t ar = rsrc(a.A + (size_t)(arow < 0 ? 0 : arow) * a.lda, arow < 0 ? 0 : K * 2);
  const unsigned aofs = (unsigned)fk * 2u;
  const int steps = K / 32;
  const int mine = steps > wave ? (steps - wave + kSlabWavesE - 1) / kSlabWavesE : 0;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f}, accu = {0.f, 0.f, 0.f, 0.f};
  for (int j0 = 0; j0 < mine; j0 += kSlabBatchE) {
    u32x4 w[kSlabBatchE], u[U ? kSlabBatchE : 1], x[kSlabBatchE];
#pragma unroll
    for (int i = 0; i < kSlabBatchE; ++i) {
      const bool live = j0 + i < mine;
      const int st = wave + kSlabWavesE * (j0 + i);
      const unsigned k0b = (unsigned)(32 * st) * 2u;  // bytes along an A row
      const unsigned k0w = (unsigned)st * 4u * 256u;  // four k groups of 16 pieces in the native copy
      w[i] = __builtin_amdgcn_raw_buffer_load_b128(wr, live ? wofs + k0w : 0x7ffffff0u, 0, 2);
      if constexpr (U) u[i] = __builtin_amdgcn_raw_buffer_load_b128(wr, live ? uofs + k0w : 0x7ffffff0u, 0, 2);
      x[i] = __builtin_amdgcn_raw_buffer_load_b128(ar, live ? aofs + k0b : 0x7ffffff0u, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < kSlabBatchE; ++i) {
      const bf16x8 xa = __builtin_bit_cast(bf16x8, x[i]);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa, __builtin_bit_cast(bf16x8, w[i]), acc, 0, 0, 0);
      if constexpr (U)
        accu = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa, __builtin_bit_cast(bf16x8, u[i]), accu, 0, 0, 0);
    }
  }
  red[0][wave][lane] = acc;
  if constexpr (U) red[1][wave][lane] = accu;
  __syncthreads();
  if (wave != 0) return;
  // D layout: lane holds rows 4 (lane / 16) + r, output lane % 16
  f32x4 g = red[0][0][lane], up = U ? red[1][0][lane] : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int w = 1; w < kSlabWavesE; ++w) {
    g += red[0][w][lane];
    if constexpr (U) up += red[1][w][lane];
  }
  const int n = n0 + fr;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int i = 4 * (lane >> 4) + r;
    if (i >= count) continue;
    uint16_t* y = a.Y + (size_t)(off + i) * a.ldy;
    if constexpr (PAIR) {
      if (n < N) y[n] = (uint16_t)f32_to_bf16(silu_mul(round_bf16(g[r]), round_bf16(up[r])));
    } else {
      if (n < N) y[n] = (uint16_t)f32_to_bf16(g[r]);
      if (TWO && n + 16 < N) y[n + 16] = (uint16_t)f32_to_bf16(up[r]);
    }
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
  uint16_t* gate_up_n = nullptr;  // MFMA-native copies of every expert (expert_slab_kernel)
  uint16_t* down_n = nullptr;
  float* logits = nullptr;       // [max_tokens * experts] router outputs
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
  void* bufs[] = {m->gate_up_n, m->down_n, m->logits, m->ids, m->weights, m->grp_expert, m->grp_count, m->grp_offset, m->n_groups,
                  m->a_rows, m->pair_slot, m->act, m->out};
  for (void* p : bufs)
    if (p) (void)hipFree(p);
  delete m;
}

// The experts and the combine after the plan (hk_moe_forward plans in
// topk_plan_kernel; `planned` false runs route_plan_kernel on `ids` first).
// `max_rows`: the most rows any expert gets (at most T when every token
// names an expert once).
int moe_run(hk_moe* m, const uint16_t* x, int T, const int32_t* ids, const float* weights,
            uint16_t* y, hipStream_t st, bool planned, int max_rows) {
  const hk_moe_desc& d = m->d;
  const int K = d.top_k, S = d.shared, E = d.experts;
  if (!planned) {
    hipLaunchKernelGGL(route_plan_kernel, dim3(1), dim3(kThreads), 0, st, ids, T, K, E, S, m->grp_expert,
                       m->grp_count, m->grp_offset, m->n_groups, m->a_rows, m->pair_slot);
    MOE_CHECK(hipGetLastError());
  }
  const int max_groups = std::min(E, T * K) + S;
  PrefillGemmArgs gu = {};
  gu.A = x;
  gu.lda = d.hidden;
  gu.W = m->gate_up;
  gu.Wn = m->gate_up_n;
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
  // at most 16 rows per group: the expert slabs (every group's rows in one
  // MFMA block); more: the grouped tile GEMM
  const bool slab = max_rows <= kSlabMaxRowsE;  // (hidden and intermediate are multiples of 32)
  if (slab) {
    hipLaunchKernelGGL(expert_slab_kernel<true>, dim3((d.intermediate + 15) / 16, max_groups), dim3(kSlabThreads),
                       0, st, gu);
    MOE_CHECK(hipGetLastError());
  } else {
    PrefillGemmArgs g = gu;
    g.Wn = nullptr;  // (the tile GEMM reads the row-major weights)
    MOE_TRY(launch_prefill_gemm(g, st));
  }
  PrefillGemmArgs dn = gu;
  dn.A = m->act;
  dn.lda = d.intermediate;
  dn.W = m->down;
  dn.Wn = m->down_n;
  dn.w_stride = (long long)d.hidden * d.intermediate;
  dn.Y = m->out;
  dn.ldy = d.hidden;
  dn.N = d.hidden;
  dn.K = d.intermediate;
  dn.epi = EPI_BF16;
  dn.a_rows = nullptr;
  if (slab) {
    hipLaunchKernelGGL((expert_slab_kernel<false, true>), dim3((d.hidden + 31) / 32, max_groups),
                       dim3(kSlabThreads), 0, st, dn);
    MOE_CHECK(hipGetLastError());
  } else {
    PrefillGemmArgs g = dn;
    g.Wn = nullptr;
    MOE_TRY(launch_prefill_gemm(g, st));
  }
  hipLaunchKernelGGL(combine_kernel, dim3(T, (d.hidden + kThreads - 1) / kThreads), dim3(kThreads), 0, st, m->out,
                     m->pair_slot, weights, d.hidden, K, S, y);
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
    // the MFMA-native copies, one repack per expert matrix
    const size_t gu_n = (size_t)2 * d.intermediate * d.hidden, dn_n = (size_t)d.hidden * d.intermediate;
    MOE_TRY(moe_alloc(&m->gate_up_n, groups * gu_n));
    MOE_TRY(moe_alloc(&m->down_n, groups * dn_n));
    for (size_t e = 0; e < groups; ++e) {
      MOE_TRY(launch_repack_mfma(gate_up + e * gu_n, m->gate_up_n + e * gu_n, 2 * d.intermediate, d.hidden, 2, 0,
                                 nullptr));
      MOE_TRY(launch_repack_mfma(down + e * dn_n, m->down_n + e * dn_n, d.hidden, d.intermediate, 2, 0, nullptr));
    }
    MOE_CHECK(hipStreamSynchronize(nullptr));
    MOE_TRY(moe_alloc(&m->logits, (size_t)d.max_tokens * d.experts));
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
  hipLaunchKernelGGL(router_logits_kernel, dim3(tokens, (d.experts + kRouterRows - 1) / kRouterRows),
                     dim3(kThreads), 0, st, x, m->router, d.hidden, d.experts, m->logits);
  MOE_CHECK(hipGetLastError());
  hipLaunchKernelGGL(topk_plan_kernel, dim3(1), dim3(kPlanThreads), 0, st, m->logits, tokens, d.experts, d.top_k,
                     d.shared, m->ids, m->weights, m->grp_expert, m->grp_count, m->grp_offset, m->n_groups,
                     m->a_rows, m->pair_slot);
  MOE_CHECK(hipGetLastError());
  MOE_TRY(moe_run(m, x, tokens, m->ids, m->weights, y, st, true, tokens));  // (top-k ids are distinct)
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
  std::vector<int> rows(m->d.experts, 0);
  int max_rows = tokens;  // the shared experts
  for (int32_t e : host) {
    if (e < 0 || e >= m->d.experts) return fail("hk_moe_experts: expert id out of range");
    max_rows = std::max(max_rows, ++rows[e]);  // a token may name an expert twice
  }
  return moe_run(m, x, tokens, ids, weights, y, st, false, max_rows);
}

void hk_moe_destroy(hk_moe* m) {
  if (m) moe_free(m);
}

}  // extern "C"
