// Whole decode step in one persistent launch (bf16 weights).
//
// The step of npu_llm/runtime/cpu_backend.py:131-181 is a chain of small
// dependent GEMVs (QKV, O, gate/up, down per layer, then the LM head).  As
// separate kernels each one pays a launch and a full HBM latency before its
// first byte arrives, so at batch 1 they run at 1-3 TB/s.  Here one
// workgroup per CU stays resident for the whole step and the phases are
// linked by flags instead of kernel boundaries:
//
//   Q  qkv = bf16(W_qkv @ rmsnorm(h) [+ bias])           cpu_backend.py:134-143
//   A  RoPE, KV append at slot p, GQA attention          :95-129
//   O  h1 = bf16(bf16(W_o @ attn) + h)                   :144-150
//   G  act = bf16(silu(bf16(W_g @ n)) * bf16(W_u @ n)), n = rmsnorm(h1)  :151-165
//   D  h = bf16(bf16(W_d @ act) + h1)                    :166-171
//   H  logits = W_lm @ rmsnorm(h) (f32), argmax           :173-181
//
// * Every wave owns at most one row group per GEMV phase, and issues the
//   loads of that group's weights as soon as it has finished the previous
//   phase -- before it waits for the previous phase's results -- so weight
//   streaming overlaps the dependency wait.  The LM head streams its rows
//   with a double buffer.
// * Dependencies: each workgroup publishes an epoch number after its outputs
//   of a phase are stored (progress[wg]); attention publishes one per query
//   head (headflag[h]).  A consumer waits only for the producers of what it
//   reads.  Epochs only grow (base + phase index, base = the epoch the
//   previous launch ended on), so flags are never reset between steps.
// * Cross-workgroup data (activations, split-KV partials, argmax keys) is
//   written and read with device-coherent (sc1) accesses: the eight XCDs have
//   separate L2 caches, and sc1 accesses bypass their incoherent state
//   without whole-cache write-back or invalidate fences.  Each producer waits
//   for its stores (s_waitcnt) before its flag is stored.
// * Every wait is bounded: after kSpinLimit polls, or once another workgroup
//   has flagged an error, the workgroup records the error and leaves; all
//   later waits then end at once, so the launch always drains.  The host
//   reports the error and resets the flags.
//
// Rounding points are those of the separate kernels (gemv.hip, attention.hip).
#include "hk_common.h"
#include "hk_internal.h"

namespace hk {
namespace {

constexpr int kPT = kPersistentThreads;  // threads per workgroup (one workgroup per CU)
constexpr int kPW = kPT / 64;             // waves per workgroup
constexpr int kPf = 16;                   // 16-byte weight chunks a lane holds across a wait
constexpr int kXMax = 8192;               // floats of x staged in LDS
constexpr int kChunk = kPersistentChunk;  // attention slots per task
constexpr int kHalf = kHeadDim / 2;
constexpr int kGroupsPV = kPT / kHalf;    // slot groups of the P @ V loop
constexpr int kPartStride = kHeadDim + 2;
constexpr unsigned kSpinLimit = 1u << 21;
constexpr int kSc1 = 16;                  // buffer-load cache policy: device scope (sc1)
static_assert(kChunk == kPT, "one thread per attention slot");

// ---- device-coherent accesses ----
__device__ __forceinline__ void st_c16(uint16_t* p, uint32_t v) {
  __hip_atomic_store(p, (uint16_t)v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ld_c16(const uint16_t* p) {
  return __hip_atomic_load(const_cast<uint16_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_c32(unsigned* p, unsigned v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned ld_c32(const unsigned* p) {
  return __hip_atomic_load(const_cast<unsigned*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_cf(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_cf(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_c64(unsigned long long* p, unsigned long long v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned long long ld_c64(const unsigned long long* p) {
  return __hip_atomic_load(const_cast<unsigned long long*>(p), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}
// 16 bytes at base + off, device-coherent; reads past `bytes` return zero.
__device__ __forceinline__ u32x4 ld_c128(const void* base, int bytes, int off) {
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes, 0x00020000);
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kSc1);
}

__device__ __forceinline__ bool reached(unsigned v, unsigned target) {
  return (int)(v - target) >= 0;
}

// ---- phase shapes ----
struct PhaseCfg {
  int lpr, nj;
};

// Lanes per row (64, 32, 16 or 8) so that a wave owns at most one row group of
// the phase at `waves` waves in the grid, with the group's chunks fitting in
// the kPf prefetch registers.
constexpr PhaseCfg pick_cfg(int M, int K, bool pair, int waves) {
  for (int lpr = 64; lpr >= 8; lpr /= 2) {
    const int rpw = 64 / lpr;
    const int groups = (M + rpw - 1) / rpw;
    const int nj = (K / 8 + lpr - 1) / lpr;
    if (groups <= waves && nj * (pair ? 2 : 1) <= kPf) return {lpr, nj};
  }
  return {0, 0};
}

template <int H_, int I_, int HQ_, int HKV_>
struct Shape {
  static constexpr int H = H_, I = I_, HQ = HQ_, HKV = HKV_;
  static constexpr int QPK = HQ / HKV;
  static constexpr int QKV = (HQ + 2 * HKV) * kHeadDim;
  static constexpr int AO = HQ * kHeadDim;
  static constexpr int kWaves = kPersistentGrid * kPW;
  static constexpr PhaseCfg q = pick_cfg(QKV, H, false, kWaves);
  static constexpr PhaseCfg o = pick_cfg(H, AO, false, kWaves);
  static constexpr PhaseCfg g = pick_cfg(I, H, true, kWaves);
  static constexpr PhaseCfg d = pick_cfg(H, I, false, kWaves);
  static constexpr int head_lpr = 16;
  static constexpr int head_nj = (H / 8 + head_lpr - 1) / head_lpr;
  static_assert(q.lpr && o.lpr && g.lpr && d.lpr, "no register plan for this shape");
  static_assert(head_nj <= kPf / 2, "LM head rows too long for the double buffer");
  static_assert(H <= kXMax && I <= kXMax && AO <= kXMax, "x staging too small");
  static_assert(H % 8 == 0 && I % 8 == 0, "rows are read in 16-byte chunks");
};

// producers of a phase: workgroups whose waves own row groups
__host__ __device__ constexpr int producers(PhaseCfg c, int M) {
  return ((M + 64 / c.lpr - 1) / (64 / c.lpr) + kPW - 1) / kPW;
}

struct PShared {
  float xs[kXMax];
  float red[2][kPW];
  unsigned long long keys[kPW];
  int abort;
  int ticket;
};

struct Ctx {
  const PersistentArgs* a;
  PShared* sm;
  int wg, wave, lane, gw;
};

// Wave 0 waits until flags[i * kFlagStride] has reached `target` for every i
// in the given ranges; the other waves wait at the workgroup barrier.
// Returns false when the launch is being abandoned.
__device__ bool wait_flags(Ctx& c, const unsigned* flags, int lo0, int hi0, int lo1, int hi1,
                           int lo2, int hi2, unsigned target) {
  if (c.wave == 0) {
    const int n0 = hi0 - lo0, n1 = hi1 - lo1, n2 = hi2 - lo2;
    const int total = n0 + n1 + n2;
    unsigned spins = 0;
    int abort = 0;
    for (;;) {
      bool ok = true;
      for (int i = c.lane; i < total; i += 64) {
        const int f = i < n0 ? lo0 + i : i < n0 + n1 ? lo1 + (i - n0) : lo2 + (i - n0 - n1);
        ok = ok && reached(ld_c32(flags + (size_t)f * kFlagStride), target);
      }
      if (__all(ok)) break;
      if (ld_c32(c.a->error) != 0u) {
        abort = 1;
        break;
      }
      if (++spins > kSpinLimit) {
        abort = 1;
        if (c.lane == 0) st_c32(c.a->error, 1u);
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    if (c.lane == 0) c.sm->abort = abort;
  }
  __syncthreads();
  return c.sm->abort == 0;
}

__device__ __forceinline__ bool wait_all(Ctx& c, const unsigned* flags, int n, unsigned target) {
  return wait_flags(c, flags, 0, n, 0, 0, 0, 0, target);
}

// Publish this workgroup's epoch once every thread's stores have completed.
__device__ __forceinline__ void publish(Ctx& c, unsigned* flag, unsigned epoch) {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) st_c32(flag, epoch);
}

// Stage K bf16 values into LDS as f32 (coherent loads when another workgroup
// wrote them), RMS-normalised with gamma when given (cpu_backend.py:71-76).
template <int K>
__device__ void stage_x(Ctx& c, const uint16_t* src, bool coherent, const uint16_t* gamma,
                        float eps) {
  constexpr int CH = K / 8;
  float* xs = c.sm->xs;
  float ss = 0.0f;
  for (int i = threadIdx.x; i < CH; i += kPT) {
    const u32x4 v = coherent ? ld_c128(src, K * 2, i * 16) : load16(src + i * 8);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float lo = bf_lo(w[q]), hi = bf_hi(w[q]);
      xs[i * 8 + 2 * q] = lo;
      xs[i * 8 + 2 * q + 1] = hi;
      ss += lo * lo;
      ss += hi * hi;
    }
  }
  if (gamma != nullptr) {
    ss = group_sum<64>(ss);
    if (c.lane == 0) c.sm->red[0][c.wave] = ss;
    __syncthreads();
    float total = c.sm->red[0][0];
#pragma unroll
    for (int w = 1; w < kPW; ++w) total += c.sm->red[0][w];
    const float inv = 1.0f / sqrtf(total / (float)K + eps);
    for (int i = threadIdx.x; i < CH; i += kPT) {
      const u32x4 gv = load16(gamma + i * 8);
      const uint32_t gw[4] = {gv.x, gv.y, gv.z, gv.w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        xs[i * 8 + 2 * q] = round_bf16((xs[i * 8 + 2 * q] * inv) * bf_lo(gw[q]));
        xs[i * 8 + 2 * q + 1] = round_bf16((xs[i * 8 + 2 * q + 1] * inv) * bf_hi(gw[q]));
      }
    }
  }
  __syncthreads();
}

// Issue the loads of this wave's row group (rows gw*RPW + sub) of W [M, K]
// (plus the paired rows M.. for gate/up) into pf.
template <int LPR, int NJ, bool PAIR>
__device__ __forceinline__ void prefetch(u32x4 (&pf)[kPf], const uint16_t* W, int M, int K,
                                         int group) {
  constexpr int RPW = 64 / LPR;
  const int lane = threadIdx.x & 63;
  const int l = lane % LPR, sub = lane / LPR;
  const int row = group * RPW + sub;
  const bool live = row < M;
  const int CH = K / 8;
  const char* wrow = reinterpret_cast<const char*>(W) + (size_t)(live ? row : 0) * K * 2;
  const size_t pair_off = (size_t)M * K * 2;
  const u32x4 zero = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int ch = l + j * LPR;
    const bool ok = live && ch < CH;
    pf[j] = ok ? load_stream16(wrow + (size_t)ch * 16) : zero;
    if constexpr (PAIR) pf[NJ + j] = ok ? load_stream16(wrow + pair_off + (size_t)ch * 16) : zero;
  }
}

__device__ __forceinline__ void fma8(const u32x4 w, const float* xs, int ch, float& a0, float& a1) {
  const float4* xv = reinterpret_cast<const float4*>(xs + ch * 8);
  const float4 p = xv[0], q = xv[1];
  a0 = fmaf(bf_lo(w.x), p.x, a0);
  a1 = fmaf(bf_hi(w.x), p.y, a1);
  a0 = fmaf(bf_lo(w.y), p.z, a0);
  a1 = fmaf(bf_hi(w.y), p.w, a1);
  a0 = fmaf(bf_lo(w.z), q.x, a0);
  a1 = fmaf(bf_hi(w.z), q.y, a1);
  a0 = fmaf(bf_lo(w.w), q.z, a0);
  a1 = fmaf(bf_hi(w.w), q.w, a1);
}

// Dot products of the prefetched row group with the staged x; every lane of
// the row's LPR lanes ends with the sums.
template <int LPR, int NJ, bool PAIR>
__device__ __forceinline__ void dot_group(const u32x4 (&pf)[kPf], const float* xs, int K,
                                          float& acc, float& accu) {
  const int l = (threadIdx.x & 63) % LPR;
  const int CH = K / 8;
  float a0 = 0.f, a1 = 0.f, b0 = 0.f, b1 = 0.f;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int ch = l + j * LPR;
    if (ch < CH) {
      fma8(pf[j], xs, ch, a0, a1);
      if constexpr (PAIR) fma8(pf[NJ + j], xs, ch, b0, b1);
    }
  }
  acc = group_sum<LPR>(a0 + a1);
  accu = PAIR ? group_sum<LPR>(b0 + b1) : 0.0f;
}

__device__ __forceinline__ float silu_mul(float g, float u) {
  const float clipped = fminf(fmaxf(g, -80.0f), 80.0f);
  const float denom = 1.0f + expf(-clipped);
  return (g / denom) * u;
}

// ---- attention task: query head h, slots [s * kChunk, ...] of layer l ----
template <class S>
__device__ bool attention_task(Ctx& c, int l, int h, int s, int p, unsigned ep_q, unsigned ep_a) {
  const PersistentArgs& a = *c.a;
  const int g = h / S::QPK;
  const int t0 = s * kChunk;
  const int n = min(kChunk, p + 1 - t0);
  const int nsplit = p / kChunk + 1;
  const bool holds_new = (s == nsplit - 1);
  const int tid = threadIdx.x;
  float* qs = c.sm->xs;                 // [64]
  float* knew = qs + kHeadDim;          // [64]
  float* pr = knew + kHeadDim;          // [kChunk]
  float* acc = pr + kChunk;             // [kGroupsPV][64]
  const size_t head_base = ((size_t)l * S::HKV + g) * a.max_ctx;
  const uint16_t* kc = a.kcache + head_base * kHeadDim;
  const uint16_t* vc = a.vcache + head_base * kHeadDim;

  // K row of this thread's slot: cache rows were written by earlier launches,
  // so these loads go out before the wait.
  const int slot = t0 + tid;
  const bool has_slot = tid < n && slot != p;
  u32x4 krow[kHeadDim / 8];
  {
    const uint16_t* src = kc + (size_t)(has_slot ? slot : 0) * kHeadDim;
#pragma unroll
    for (int ch = 0; ch < kHeadDim / 8; ++ch)
      krow[ch] = has_slot ? load16(src + ch * 8) : u32x4{0u, 0u, 0u, 0u};
  }

  // rows of q head h, k head g, v head g come from Q-phase producers
  constexpr int rows_per_wg = kPW * (64 / S::q.lpr);
  const int qr = h * kHeadDim, kr = (S::HQ + g) * kHeadDim, vr = (S::HQ + S::HKV + g) * kHeadDim;
  if (!wait_flags(c, a.progress, qr / rows_per_wg, (qr + kHeadDim - 1) / rows_per_wg + 1,
                  kr / rows_per_wg, (kr + kHeadDim - 1) / rows_per_wg + 1, vr / rows_per_wg,
                  (vr + kHeadDim - 1) / rows_per_wg + 1, ep_q))
    return false;

  const uint16_t* qkv = a.qkv;
  const uint16_t* vnew = qkv + vr;
  // V words of this thread's slot group for the P @ V loop (slot p from
  // qkv); they arrive while the scores and the softmax are formed
  const int dp = tid & (kHalf - 1);
  const int gi = tid / kHalf;
  uint32_t vw[kChunk / kGroupsPV];
#pragma unroll
  for (int k = 0; k < kChunk / kGroupsPV; ++k) {
    const int sl = t0 + gi + k * kGroupsPV;
    vw[k] = sl < p ? reinterpret_cast<const uint32_t*>(vc + (size_t)sl * kHeadDim)[dp]
            : sl == p ? ld_c16(vnew + 2 * dp) | (ld_c16(vnew + 2 * dp + 1) << 16)
                      : 0u;
  }

  // rotated q head and new key (bf16-rounded); the group's first query head
  // appends k and v at slot p
  if (tid < 2 * kHalf) {
    const int j = tid & (kHalf - 1);
    const bool is_k = tid >= kHalf;
    const uint16_t* src = qkv + (is_k ? kr : qr);
    const float cs = a.cos_tab[(size_t)p * kHalf + j];
    const float sn = a.sin_tab[(size_t)p * kHalf + j];
    const float x1 = bf16_to_f32(ld_c16(src + j)), x2 = bf16_to_f32(ld_c16(src + j + kHalf));
    const uint32_t r1 = f32_to_bf16(x1 * cs - x2 * sn);
    const uint32_t r2 = f32_to_bf16(x2 * cs + x1 * sn);
    float* dst = is_k ? knew : qs;
    dst[j] = bf16_to_f32(r1);
    dst[j + kHalf] = bf16_to_f32(r2);
    if (is_k && holds_new && h % S::QPK == 0) {
      uint16_t* kd = a.kcache + (head_base + p) * kHeadDim;
      uint16_t* vd = a.vcache + (head_base + p) * kHeadDim;
      kd[j] = (uint16_t)r1;
      kd[j + kHalf] = (uint16_t)r2;
      vd[j] = (uint16_t)ld_c16(vnew + j);
      vd[j + kHalf] = (uint16_t)ld_c16(vnew + j + kHalf);
    }
  }
  __syncthreads();

  const float scale = 1.0f / 8.0f;  // head_dim ** -0.5 for head_dim 64 (exact)
  float sc = -INFINITY;
  if (tid < n) {
    float dot = 0.0f;
    if (slot == p) {
#pragma unroll
      for (int d = 0; d < kHeadDim; ++d) dot = fmaf(qs[d], knew[d], dot);
    } else {
#pragma unroll
      for (int ch = 0; ch < kHeadDim / 8; ++ch) {
        const uint32_t w[4] = {krow[ch].x, krow[ch].y, krow[ch].z, krow[ch].w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          dot = fmaf(qs[ch * 8 + 2 * q], bf_lo(w[q]), dot);
          dot = fmaf(qs[ch * 8 + 2 * q + 1], bf_hi(w[q]), dot);
        }
      }
    }
    sc = dot * scale;
  }
  float m = group_max<64>(sc);
  if (c.lane == 0) c.sm->red[0][c.wave] = m;
  __syncthreads();
  m = c.sm->red[0][0];
#pragma unroll
  for (int w = 1; w < kPW; ++w) m = fmaxf(m, c.sm->red[0][w]);
  const float e = tid < n ? expf(sc - m) : 0.0f;
  float sum = group_sum<64>(e);
  if (c.lane == 0) c.sm->red[1][c.wave] = sum;
  __syncthreads();
  sum = c.sm->red[1][0];
#pragma unroll
  for (int w = 1; w < kPW; ++w) sum += c.sm->red[1][w];
  pr[tid] = nsplit == 1 ? e / sum : e;  // a single chunk normalises first, as NumPy does
  __syncthreads();

  float o0 = 0.0f, o1 = 0.0f;
#pragma unroll
  for (int k = 0; k < kChunk / kGroupsPV; ++k) {
    const int t = gi + k * kGroupsPV;
    if (t < n) {
      const float pt = pr[t];
      o0 = fmaf(pt, bf_lo(vw[k]), o0);
      o1 = fmaf(pt, bf_hi(vw[k]), o1);
    }
  }
  acc[gi * kHeadDim + 2 * dp] = o0;
  acc[gi * kHeadDim + 2 * dp + 1] = o1;
  __syncthreads();
  float o = 0.0f;
  if (tid < kHeadDim) {
#pragma unroll
    for (int k = 0; k < kGroupsPV; ++k) o += acc[k * kHeadDim + tid];
  }
  uint16_t* out = a.attn + (size_t)h * kHeadDim;
  if (nsplit == 1) {
    if (tid < kHeadDim) st_c16(out + tid, f32_to_bf16(o));
    publish(c, a.headflag + (size_t)h * kFlagStride, ep_a);
    return true;
  }

  // split-KV: publish this chunk's (p @ V, max, sum); the last task of the
  // head (ticket) merges all chunks with log-sum-exp rescaling
  float* mine = a.partial + ((size_t)h * a.max_splits + s) * kPartStride;
  if (tid < kHeadDim) st_cf(mine + tid, o);
  if (tid == 0) {
    st_cf(mine + kHeadDim, m);
    st_cf(mine + kHeadDim + 1, sum);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0)
    c.sm->ticket = (int)__hip_atomic_fetch_add(a.counters + h, 1u, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  if (c.sm->ticket != nsplit - 1) return true;
  if (tid < kHeadDim) {
    const float* base = a.partial + (size_t)h * a.max_splits * kPartStride;
    float mx = -INFINITY;
    for (int j = 0; j < nsplit; ++j) mx = fmaxf(mx, ld_cf(base + (size_t)j * kPartStride + kHeadDim));
    float lsum = 0.0f, r = 0.0f;
    for (int j = 0; j < nsplit; ++j) {
      const float* pj = base + (size_t)j * kPartStride;
      const float f = expf(ld_cf(pj + kHeadDim) - mx);
      lsum = fmaf(ld_cf(pj + kHeadDim + 1), f, lsum);
      r = fmaf(ld_cf(pj + tid), f, r);
    }
    st_c16(out + tid, f32_to_bf16(r / lsum));
  }
  if (tid == 0)
    (void)__hip_atomic_exchange(a.counters + h, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  publish(c, a.headflag + (size_t)h * kFlagStride, ep_a);
  return true;
}

// ---- the step kernel ----
template <class S>
__global__ __launch_bounds__(kPT) void decode_step_kernel(PersistentArgs args) {
  __shared__ PShared sm;
  Ctx c;
  c.a = &args;
  c.sm = &sm;
  c.wg = blockIdx.x;
  c.wave = threadIdx.x >> 6;
  c.lane = threadIdx.x & 63;
  c.gw = c.wg * kPW + c.wave;
  if (threadIdx.x == 0) sm.abort = 0;

  const PersistentArgs& a = args;
  const int L = a.layers;
  const unsigned base = ld_c32(a.progress + (size_t)c.wg * kFlagStride);  // this workgroup's last epoch
  const int token = a.ctrl->token;
  const int p = a.ctrl->position;
  const uint16_t* embed_row =
      token >= 0 ? a.embed + (size_t)min(token, a.vocab - 1) * S::H : nullptr;
  unsigned* my_flag = a.progress + (size_t)c.wg * kFlagStride;

  constexpr int nq = producers(S::q, S::QKV), no = producers(S::o, S::H);
  constexpr int ng = producers(S::g, S::I), nd = producers(S::d, S::H);
  const bool is_q = c.wg < nq, is_o = c.wg < no, is_g = c.wg < ng, is_d = c.wg < nd;
  const int nsplit = p / kChunk + 1;
  const int tasks = S::HQ * nsplit;

  u32x4 pf[kPf];
  float acc, accu;
  if (is_q) prefetch<S::q.lpr, S::q.nj, false>(pf, a.w[0].qkv, S::QKV, S::H, c.gw);
  __syncthreads();

  for (int l = 0; l < L; ++l) {
    const PersistentLayer& lw = a.w[l];
    const unsigned ep = base + 5u * (unsigned)l;
    // ---- Q ----
    if (is_q) {
      const uint16_t* xsrc = (l == 0 && embed_row) ? embed_row : a.h;
      if (l > 0 && !wait_all(c, a.progress, nd, ep)) return;
      stage_x<S::H>(c, xsrc, xsrc == a.h, lw.in_norm, a.eps);
      dot_group<S::q.lpr, S::q.nj, false>(pf, sm.xs, S::H, acc, accu);
      const int row = c.gw * (64 / S::q.lpr) + c.lane / S::q.lpr;
      if (c.lane % S::q.lpr == 0 && row < S::QKV) {
        const uint32_t y = lw.qkv_bias ? f32_to_bf16(round_bf16(acc) + lw.qkv_bias[row])
                                       : f32_to_bf16(acc);
        st_c16(a.qkv + row, y);
      }
      publish(c, my_flag, ep + 1);
    }
    // ---- A ---- (tasks go to the highest workgroups, which own no Q rows)
    for (int t = kPersistentGrid - 1 - c.wg; t < tasks; t += kPersistentGrid) {
      __syncthreads();  // LDS reuse
      if (!attention_task<S>(c, l, t % S::HQ, t / S::HQ, p, ep + 1, ep + 2)) return;
    }
    if (is_o) prefetch<S::o.lpr, S::o.nj, false>(pf, lw.o, S::H, S::AO, c.gw);
    // ---- O ----
    if (is_o) {
      if (!wait_all(c, a.headflag, S::HQ, ep + 2)) return;
      stage_x<S::AO>(c, a.attn, true, nullptr, 0.0f);
      dot_group<S::o.lpr, S::o.nj, false>(pf, sm.xs, S::AO, acc, accu);
      const int row = c.gw * (64 / S::o.lpr) + c.lane / S::o.lpr;
      if (c.lane % S::o.lpr == 0 && row < S::H) {
        const float r = (l == 0 && embed_row) ? bf16_to_f32(embed_row[row])
                                               : bf16_to_f32(ld_c16(a.h + row));
        st_c16(a.h1 + row, f32_to_bf16(round_bf16(acc) + r));
      }
      publish(c, my_flag, ep + 3);
    }
    if (is_g) prefetch<S::g.lpr, S::g.nj, true>(pf, lw.gate_up, S::I, S::H, c.gw);
    // ---- G ----
    if (is_g) {
      if (!wait_all(c, a.progress, no, ep + 3)) return;
      stage_x<S::H>(c, a.h1, true, lw.post_norm, a.eps);
      dot_group<S::g.lpr, S::g.nj, true>(pf, sm.xs, S::H, acc, accu);
      const int row = c.gw * (64 / S::g.lpr) + c.lane / S::g.lpr;
      if (c.lane % S::g.lpr == 0 && row < S::I)
        st_c16(a.act + row, f32_to_bf16(silu_mul(round_bf16(acc), round_bf16(accu))));
      publish(c, my_flag, ep + 4);
    }
    if (is_d) prefetch<S::d.lpr, S::d.nj, false>(pf, lw.down, S::H, S::I, c.gw);
    // ---- D ----
    if (is_d) {
      if (!wait_all(c, a.progress, ng, ep + 4)) return;
      stage_x<S::I>(c, a.act, true, nullptr, 0.0f);
      dot_group<S::d.lpr, S::d.nj, false>(pf, sm.xs, S::I, acc, accu);
      const int row = c.gw * (64 / S::d.lpr) + c.lane / S::d.lpr;
      if (c.lane % S::d.lpr == 0 && row < S::H)
        st_c16(a.h + row, f32_to_bf16(round_bf16(acc) + bf16_to_f32(ld_c16(a.h1 + row))));
      publish(c, my_flag, ep + 5);
    }
    if (l + 1 < L && is_q) prefetch<S::q.lpr, S::q.nj, false>(pf, a.w[l + 1].qkv, S::QKV, S::H, c.gw);
  }
  const unsigned ep_layers = base + 5u * (unsigned)L;
  if (!a.head) {
    if (threadIdx.x == 0) st_c32(my_flag, ep_layers);
    return;
  }

  // ---- H: LM head over all waves, double-buffered row groups ----
  constexpr int HL = S::head_lpr, HNJ = S::head_nj, HRPW = 64 / HL;
  const int groups = (a.vocab + HRPW - 1) / HRPW;
  const int stride = kPersistentGrid * kPW;
  u32x4 wb[kPf];
  int grp = c.gw;
  if (grp < groups) prefetch<HL, HNJ, false>(pf, a.lm_head, a.vocab, S::H, grp);
  if (!wait_all(c, a.progress, nd, ep_layers)) return;
  stage_x<S::H>(c, a.h, true, a.final_norm, a.eps);
  unsigned long long best = 0ull;
  const int sub = c.lane / HL;
  const bool lead = c.lane % HL == 0;
  for (;;) {
    if (grp >= groups) break;
    int nxt = grp + stride;
    if (nxt < groups) prefetch<HL, HNJ, false>(wb, a.lm_head, a.vocab, S::H, nxt);
    dot_group<HL, HNJ, false>(pf, sm.xs, S::H, acc, accu);
    int row = grp * HRPW + sub;
    if (lead && row < a.vocab) {
      a.logits[row] = acc;
      best = umax64(best, argmax_key(acc, (uint32_t)row));
    }
    grp = nxt;
    if (grp >= groups) break;
    nxt = grp + stride;
    if (nxt < groups) prefetch<HL, HNJ, false>(pf, a.lm_head, a.vocab, S::H, nxt);
    dot_group<HL, HNJ, false>(wb, sm.xs, S::H, acc, accu);
    row = grp * HRPW + sub;
    if (lead && row < a.vocab) {
      a.logits[row] = acc;
      best = umax64(best, argmax_key(acc, (uint32_t)row));
    }
    grp = nxt;
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) best = umax64(best, shfl_xor_u64(best, m));
  if (c.lane == 0) sm.keys[c.wave] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned long long k = sm.keys[0];
#pragma unroll
    for (int w = 1; w < kPW; ++w) k = umax64(k, sm.keys[w]);
    st_c64(a.keys + c.wg, k);
  }
  const unsigned ep_head = ep_layers + 1;
  publish(c, my_flag, ep_head);
  if (c.wg != 0) return;

  // ---- argmax over the workgroups' keys; token feedback (generate.py:709-730) ----
  if (!wait_all(c, a.progress, kPersistentGrid, ep_head)) return;
  unsigned long long k = 0ull;
  for (int i = threadIdx.x; i < kPersistentGrid; i += kPT) k = umax64(k, ld_c64(a.keys + i));
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) k = umax64(k, shfl_xor_u64(k, m));
  if (c.lane == 0) sm.keys[c.wave] = k;
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned long long best_key = sm.keys[0];
#pragma unroll
    for (int w = 1; w < kPW; ++w) best_key = umax64(best_key, sm.keys[w]);
    const int32_t index = (int32_t)argmax_key_index(best_key);
    a.result[0] = index;
    StepCtrl* ctrl = a.ctrl;
    if (ctrl->advance) {
      const int slot = ctrl->n_out;
      if (slot >= 0 && slot < a.max_ctx) a.out_tokens[slot] = index;
      ctrl->n_out = slot + 1;
      ctrl->token = index;
      ctrl->position = p + 1;
    }
  }
}

using SmolShape = Shape<576, 1536, 9, 3>;
using QwenShape = Shape<896, 4864, 14, 2>;

template <class S>
bool matches(int hidden, int intermediate, int q_heads, int kv_heads) {
  return hidden == S::H && intermediate == S::I && q_heads == S::HQ && kv_heads == S::HKV;
}

template <class S>
int launch_shape(const PersistentArgs& a, hipStream_t stream) {
  hipLaunchKernelGGL(decode_step_kernel<S>, dim3(kPersistentGrid), dim3(kPT), 0, stream, a);
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? 0 : hip_fail(err, "persistent step launch");
}

template <class S>
int occupancy_ok() {
  int blocks = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, decode_step_kernel<S>, kPT, 0) !=
      hipSuccess)
    return 0;
  return blocks >= 1;
}

}  // namespace

int persistent_shape(int hidden, int intermediate, int q_heads, int kv_heads, bool w8) {
  if (w8) return -1;
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return -1;
  // one resident workgroup per CU is what keeps every wait finite
  if (cus < kPersistentGrid) return -1;
  if (matches<QwenShape>(hidden, intermediate, q_heads, kv_heads))
    return occupancy_ok<QwenShape>() ? 1 : -1;
  if (matches<SmolShape>(hidden, intermediate, q_heads, kv_heads))
    return occupancy_ok<SmolShape>() ? 0 : -1;
  return -1;
}

int launch_persistent_step(int shape, const PersistentArgs& a, hipStream_t stream) {
  if (a.max_splits < (a.max_ctx + kChunk - 1) / kChunk) return fail("persistent step: partials too small");
  switch (shape) {
    case 0: return launch_shape<SmolShape>(a, stream);
    case 1: return launch_shape<QwenShape>(a, stream);
    default: return fail("persistent step: unsupported model shape");
  }
}

}  // namespace hk
