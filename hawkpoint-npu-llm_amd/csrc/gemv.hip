// Batch-1 GEMV for the decode step: y = W @ x with W row-major BF16 or int8.
//
// Covers every projection of the reference's decode step
// (npu_llm/runtime/cpu_backend.py:64-69 `project`, used by `layer` :131-171
// and `logits` :173-181) and the W8 device formula of
// npu_llm/kernels/project_w8bf16.cc:14-38.
//
// Mapping (wave64): `LPR` lanes share one output row; a wave owns a group of
// 64/LPR rows at a time and a 256-thread workgroup 4 waves.  Each lane streams
// NJ 16-byte chunks of its row (8 bf16 or 16 int8 weights per chunk) with
// non-temporal loads; the first group's loads are issued *before* the
// prologue, so the RMSNorm/x staging latency hides under the HBM fetch, and a
// wave that owns several groups loads the next while reducing the current.
// x lives in LDS as packed bf16 pairs (and float32 for the RMSNorm
// prologue); the dot products run on v_dot2_f32_bf16 (int8 weights widened
// to bf16 pairs first).  Partial sums are reduced across the LPR lanes
// with butterfly shuffles.  The LM-head form also keeps a running argmax key
// per workgroup (no atomics); launch_argmax_finalize reduces those keys.
//
// Rounding points follow the reference exactly:
//   EPI_BF16   bf16(acc)                         project()
//   EPI_BIAS   bf16(f32(bf16(acc)) + bias)       cpu_backend.py:140-143
//   EPI_RESID  bf16(f32(bf16(acc)) + f32(res))   cpu_backend.py:145-150, 166-171
//   EPI_F32    acc (no rounding)                 cpu_backend.py:179-181
//   EPI_SWIGLU bf16((g / (1 + exp(-clip(g)))) * u) on bf16 g, u   :154-165
// W8 rows are dequantised after accumulation: acc * scale[row], then as above.
#include "hk_common.h"
#include "hk_internal.h"

namespace hk {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr unsigned kGemvOutside = 0x7ffffff0u;  // a byte offset past every buffer resource

// Stage x (optionally RMS-normalised) into LDS as float32.
// RMSNorm follows cpu_backend.py:71-76: v = f32(bf16 x); mean of v*v in f32;
// inv = 1 / sqrt(mean + eps); out = bf16((v * inv) * gamma).
// With xp, also as packed bf16 pairs (every staged value is bf16-exact).
__device__ __forceinline__ void stage_x(const GemvArgs& a, float* xs, float* red, uint32_t* xp = nullptr) {
  const int tid = threadIdx.x;
  const int K = a.K;
  const uint16_t* x = a.x;
  bool copy = false;
  if (a.x_index != nullptr) {
    int t = *a.x_index;
    if (t >= 0) {
      if (t >= a.vocab_limit) t = a.vocab_limit - 1;
      x = a.x_table + (size_t)t * (size_t)K;
      copy = (a.x_copy != nullptr) && blockIdx.x == 0;
    }
  }
  const uint32_t* x2 = reinterpret_cast<const uint32_t*>(x);
  float ss = 0.0f;
  for (int i = tid; i < K / 2; i += kThreads) {
    const uint32_t w = ldg(x2 + i);
    const float v0 = bf_lo(w), v1 = bf_hi(w);
    xs[2 * i] = v0;
    xs[2 * i + 1] = v1;
    if (xp) xp[i] = w;
    if (copy) reinterpret_cast<uint32_t*>(a.x_copy)[i] = w;
    ss += v0 * v0;
    ss += v1 * v1;
  }
  if (a.pro != PRO_NORM) return;
  ss = group_sum<64>(ss);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  float total = red[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) total += red[w];
  const float mean = total / (float)K;
  const float inv = 1.0f / sqrtf(mean + a.eps);
  const uint32_t* g2 = reinterpret_cast<const uint32_t*>(a.gamma);
  for (int i = tid; i < K / 2; i += kThreads) {
    const uint32_t g = ldg(g2 + i);
    const float n0 = round_bf16((xs[2 * i] * inv) * bf_lo(g)), n1 = round_bf16((xs[2 * i + 1] * inv) * bf_hi(g));
    xs[2 * i] = n0;
    xs[2 * i + 1] = n1;
    if (xp) xp[i] = (__float_as_uint(n0) >> 16) | (__float_as_uint(n1) & 0xffff0000u);
  }
}

// Sixteen int8 weights (one chunk) times x as packed bf16 pairs (xp): each
// weight pair widened exactly to a bf16 pair (i8pair_bf16), then
// v_dot2_f32_bf16 (exact products, float32 sums) -- two VALU instructions per
// weight, and half the LDS bytes of float32 x.
typedef __bf16 gemv_bf16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float dot2_bf16(uint32_t w, uint32_t x, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(gemv_bf16x2, w), __builtin_bit_cast(gemv_bf16x2, x), c,
                                         false);
}
__device__ __forceinline__ void dot_chunk_i8(const u32x4 w, const uint32_t* xp, int c, float& a0, float& a1) {
  const u32x4 xa = *reinterpret_cast<const u32x4*>(xp + 8 * c);
  const u32x4 xb = *reinterpret_cast<const u32x4*>(xp + 8 * c + 4);
  a0 = dot2_bf16(i8pair_bf16(w.x, 0), xa.x, a0);
  a1 = dot2_bf16(i8pair_bf16(w.x, 2), xa.y, a1);
  a0 = dot2_bf16(i8pair_bf16(w.y, 0), xa.z, a0);
  a1 = dot2_bf16(i8pair_bf16(w.y, 2), xa.w, a1);
  a0 = dot2_bf16(i8pair_bf16(w.z, 0), xb.x, a0);
  a1 = dot2_bf16(i8pair_bf16(w.z, 2), xb.y, a1);
  a0 = dot2_bf16(i8pair_bf16(w.w, 0), xb.z, a0);
  a1 = dot2_bf16(i8pair_bf16(w.w, 2), xb.w, a1);
}

// Eight bf16 weights (one chunk) times x as packed bf16 pairs: four v_dot2.
__device__ __forceinline__ void dot_chunk_bf16(const u32x4 w, const uint32_t* xp, int c, float& a0, float& a1) {
  const u32x4 x = *reinterpret_cast<const u32x4*>(xp + 4 * c);
  a0 = dot2_bf16(w.x, x.x, a0);
  a1 = dot2_bf16(w.y, x.y, a1);
  a0 = dot2_bf16(w.z, x.z, a0);
  a1 = dot2_bf16(w.w, x.w, a1);
}

__device__ __forceinline__ float silu_mul(float g, float u) {
  const float clipped = fminf(fmaxf(g, -80.0f), 80.0f);
  const float denom = 1.0f + expf(-clipped);
  return (g / denom) * u;
}

// Reduce one row group's partial sums and apply the epilogue.
template <int LPR, bool W8, bool PAIR>
__device__ __forceinline__ void finish_row(const GemvArgs& a, int row, bool live, int l, float a0,
                                           float a1, float b0, float b1,
                                           unsigned long long& best) {
  float acc = lane_sum<LPR>(a0 + a1);
  float accu = PAIR ? lane_sum<LPR>(b0 + b1) : 0.0f;
  if (!live || l != 0) return;
  if constexpr (W8) {
    acc = acc * ldg(a.scale + row);
    if constexpr (PAIR) accu = accu * ldg(a.scale + row + a.M);
  }
  switch (a.epi) {
    case EPI_BF16:
      stg(a.y + row, (uint16_t)f32_to_bf16(acc));
      break;
    case EPI_BIAS:
      stg(a.y + row, (uint16_t)f32_to_bf16(round_bf16(acc) + ldg(a.bias + row)));
      break;
    case EPI_RESID:
      stg(a.y + row, (uint16_t)f32_to_bf16(round_bf16(acc) + bf16_to_f32(ldg(a.resid + row))));
      break;
    case EPI_F32:
      stg(a.yf + row, acc);
      break;
    case EPI_F32_ARGMAX:
      stg(a.yf + row, acc);
      best = umax64(best, argmax_key(acc, (uint32_t)row));
      break;
    case EPI_SWIGLU:
      stg(a.y + row, (uint16_t)f32_to_bf16(silu_mul(round_bf16(acc), round_bf16(accu))));
      break;
    default:
      break;
  }
}

// Each wave owns row groups (64/LPR rows; paired with the up rows for
// SwiGLU) g = wave_id, wave_id + waves_in_grid, ...; the next group's weights
// are loaded while the current one is reduced, so a wave always has its
// loads in flight.  Rows longer than LPR*NJ chunks take several passes.
// BUF: branch-free buffer loads (always for bf16 rows; for int8 rows only
// where they measured faster, the LM head).
template <int LPR, int NJ, bool W8, bool PAIR, bool BUF = !W8>
__global__ __launch_bounds__(kThreads) void gemv_kernel(GemvArgs a) {
  extern __shared__ float smem[];
  float* xs = smem;
  float* red = smem + a.K;
  uint32_t* xp = reinterpret_cast<uint32_t*>(smem + a.K + 8);  // W8: x as packed bf16 pairs
  __shared__ unsigned long long wave_keys[kWaves];

  constexpr int RPW = 64 / LPR;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int l = lane % LPR;
  const int sub = lane / LPR;
  const int CH = W8 ? (a.K >> 4) : (a.K >> 3);
  const size_t row_bytes = W8 ? (size_t)a.K : (size_t)a.K * 2;
  const size_t pair_off = (size_t)a.M * row_bytes;
  const int groups = (a.M + RPW - 1) / RPW;
  const int stride = gridDim.x * kWaves;
  const bool single_pass = CH <= LPR * NJ;
  const u32x4 zero = {0u, 0u, 0u, 0u};

  u32x4 wa[NJ], wb[NJ];
  u32x4 ua[PAIR ? NJ : 1], ub[PAIR ? NJ : 1];

  // Branch-free loads through a buffer resource: a chunk past the row or a
  // group past the matrix takes an offset past the resource and reads zero.
  // With a branch around each load the compiler waited for all of them
  // (the next group's too) before the first product.  The host keeps the
  // matrix below 2 GiB (32-bit offsets).  (int8 rows keep the branches
  // unless BUF: measured, the branch-free form took their GEMVs 5-25%
  // longer, all but the LM head's.)
  const __amdgpu_buffer_rsrc_t wr = rsrc(a.W, (int)((PAIR ? 2 : 1) * pair_off));
  auto load = [&](int g, int base, u32x4 (&w)[NJ], u32x4 (&u)[PAIR ? NJ : 1]) {
    const int row = g * RPW + sub;
    const bool live = g < groups && row < a.M;
    if constexpr (W8 && !BUF) {
      const char* wrow = static_cast<const char*>(a.W) + (size_t)(live ? row : 0) * row_bytes;
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const int c = base + l + j * LPR;
        const bool ok = live && c < CH;
        w[j] = ok ? load_stream16(wrow + (size_t)c * 16) : zero;
        if constexpr (PAIR) u[j] = ok ? load_stream16(wrow + pair_off + (size_t)c * 16) : zero;
      }
      return;
    }
    const unsigned rofs = (unsigned)((size_t)(live ? row : 0) * row_bytes);
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int c = base + l + j * LPR;
      const unsigned off = live && c < CH ? rofs + (unsigned)c * 16u : kGemvOutside;
      w[j] = __builtin_amdgcn_raw_buffer_load_b128(wr, off, 0, 2);
      if constexpr (PAIR)
        u[j] = __builtin_amdgcn_raw_buffer_load_b128(wr, off == kGemvOutside ? off : off + (unsigned)pair_off, 0, 2);
    }
  };
  // chunks past the row hold zero weights and their x index is clamped, so
  // the products read a finite x and need no branch
  auto dot = [&](int base, const u32x4 (&w)[NJ], const u32x4 (&u)[PAIR ? NJ : 1], float& a0,
                 float& a1, float& b0, float& b1) {
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int c = base + l + j * LPR;
      const int cx = c < CH ? c : 0;
      if constexpr (W8) {
        dot_chunk_i8(w[j], xp, cx, a0, a1);
        if constexpr (PAIR) dot_chunk_i8(u[j], xp, cx, b0, b1);
      } else {
        dot_chunk_bf16(w[j], xp, cx, a0, a1);
        if constexpr (PAIR) dot_chunk_bf16(u[j], xp, cx, b0, b1);
      }
    }
  };

  unsigned long long best = 0ull;
  int g = blockIdx.x * kWaves + wave;
  load(g, 0, wa, ua);
  stage_x(a, xs, red, xp);
  __syncthreads();

  if (single_pass) {
    for (;;) {
      if (g >= groups) break;
      const int gn = g + stride;
      if (gn < groups) load(gn, 0, wb, ub);
      float a0 = 0.f, a1 = 0.f, b0 = 0.f, b1 = 0.f;
      dot(0, wa, ua, a0, a1, b0, b1);
      finish_row<LPR, W8, PAIR>(a, g * RPW + sub, g * RPW + sub < a.M, l, a0, a1, b0, b1, best);
      g = gn;
      if (g >= groups) break;
      const int gn2 = g + stride;
      if (gn2 < groups) load(gn2, 0, wa, ua);
      a0 = a1 = b0 = b1 = 0.f;
      dot(0, wb, ub, a0, a1, b0, b1);
      finish_row<LPR, W8, PAIR>(a, g * RPW + sub, g * RPW + sub < a.M, l, a0, a1, b0, b1, best);
      g = gn2;
    }
  } else {
    bool first = true;
    for (; g < groups; g += stride) {
      float a0 = 0.f, a1 = 0.f, b0 = 0.f, b1 = 0.f;
      for (int base = 0; base < CH; base += LPR * NJ) {
        if (!first) load(g, base, wa, ua);
        first = false;
        dot(base, wa, ua, a0, a1, b0, b1);
      }
      finish_row<LPR, W8, PAIR>(a, g * RPW + sub, g * RPW + sub < a.M, l, a0, a1, b0, b1, best);
    }
  }

  if (a.epi == EPI_F32_ARGMAX) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) best = umax64(best, shfl_xor_u64(best, m));
    if (lane == 0) wave_keys[wave] = best;
    __syncthreads();
    if (tid == 0) {
      unsigned long long k = wave_keys[0];
#pragma unroll
      for (int i = 1; i < kWaves; ++i) k = umax64(k, wave_keys[i]);
      a.keys[blockIdx.x] = k;
    }
  }
}

// bf16 GEMV with x in registers: every lane loads the x chunks that match its
// weight chunks straight from memory (L2-resident), and for RMSNorm each wave
// reduces the sum of squares over the whole x itself, so the kernel needs no
// LDS staging and no workgroup barrier before the first FMA.  Used when each
// wave owns about one row group (all projections but the LM head); measured
// 20-25% faster than the LDS-staged form on the 896- and 4864-wide rows.
template <int LPR, int NJ, bool PAIR>
__global__ __launch_bounds__(kThreads) void gemv_xreg_kernel(GemvArgs a) {
  __shared__ unsigned long long wave_keys[kWaves];
  constexpr int RPW = 64 / LPR;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int l = lane % LPR;
  const int sub = lane / LPR;
  const int K = a.K;
  const int CH = K >> 3;
  const size_t row_bytes = (size_t)K * 2;
  const size_t pair_off = (size_t)a.M * row_bytes;
  const int groups = (a.M + RPW - 1) / RPW;
  const int stride = gridDim.x * kWaves;
  const u32x4 zero = {0u, 0u, 0u, 0u};

  const uint16_t* x = a.x;
  if (a.x_index != nullptr) {
    int t = *a.x_index;
    if (t >= 0) {
      if (t >= a.vocab_limit) t = a.vocab_limit - 1;
      x = a.x_table + (size_t)t * (size_t)K;
      if (a.x_copy != nullptr && blockIdx.x == 0) {
        const uint32_t* src = reinterpret_cast<const uint32_t*>(x);
        for (int i = tid; i < K / 2; i += kThreads) reinterpret_cast<uint32_t*>(a.x_copy)[i] = src[i];
      }
    }
  }

  u32x4 wa[NJ], wb[NJ];
  u32x4 ua[PAIR ? NJ : 1], ub[PAIR ? NJ : 1];
  auto load = [&](int g, u32x4 (&w)[NJ], u32x4 (&u)[PAIR ? NJ : 1]) {
    const int row = g * RPW + sub;
    const bool live = g < groups && row < a.M;
    const char* wrow = static_cast<const char*>(a.W) + (size_t)(live ? row : 0) * row_bytes;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int c = l + j * LPR;
      const bool ok = live && c < CH;
      w[j] = ok ? load_stream16(wrow + (size_t)c * 16) : zero;
      if constexpr (PAIR) u[j] = ok ? load_stream16(wrow + pair_off + (size_t)c * 16) : zero;
    }
  };

  int g = blockIdx.x * kWaves + wave;
  load(g, wa, ua);

  // RMSNorm scale, reduced by each wave over the whole vector (cpu_backend.py:71-76)
  float inv = 1.0f;
  if (a.pro == PRO_NORM) {
    float ss = 0.0f;
    for (int c = lane; c < CH; c += 64) {
      const u32x4 v = load16(x + c * 8);
      const uint32_t words[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float lo = bf_lo(words[q]), hi = bf_hi(words[q]);
        ss += lo * lo;
        ss += hi * hi;
      }
    }
    ss = lane_sum<64>(ss);
    inv = 1.0f / sqrtf(ss / (float)K + a.eps);
  }
  // this lane's x chunks (normalised when asked), kept for every row group
  float xv[NJ][8];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int c = l + j * LPR;
    if (c < CH) {
      const u32x4 v = load16(x + c * 8);
      const uint32_t words[4] = {v.x, v.y, v.z, v.w};
      if (a.pro == PRO_NORM) {
        const u32x4 gm = load16(a.gamma + c * 8);
        const uint32_t gw[4] = {gm.x, gm.y, gm.z, gm.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          xv[j][2 * q] = round_bf16((bf_lo(words[q]) * inv) * bf_lo(gw[q]));
          xv[j][2 * q + 1] = round_bf16((bf_hi(words[q]) * inv) * bf_hi(gw[q]));
        }
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          xv[j][2 * q] = bf_lo(words[q]);
          xv[j][2 * q + 1] = bf_hi(words[q]);
        }
      }
    } else {
#pragma unroll
      for (int q = 0; q < 8; ++q) xv[j][q] = 0.0f;
    }
  }

  auto dot = [&](const u32x4 (&w)[NJ], const u32x4 (&u)[PAIR ? NJ : 1], float& a0, float& a1,
                 float& b0, float& b1) {
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const uint32_t ww[4] = {w[j].x, w[j].y, w[j].z, w[j].w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        a0 = fmaf(bf_lo(ww[q]), xv[j][2 * q], a0);
        a1 = fmaf(bf_hi(ww[q]), xv[j][2 * q + 1], a1);
      }
      if constexpr (PAIR) {
        const uint32_t uu[4] = {u[j].x, u[j].y, u[j].z, u[j].w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          b0 = fmaf(bf_lo(uu[q]), xv[j][2 * q], b0);
          b1 = fmaf(bf_hi(uu[q]), xv[j][2 * q + 1], b1);
        }
      }
    }
  };

  unsigned long long best = 0ull;
  for (;;) {
    if (g >= groups) break;
    const int gn = g + stride;
    if (gn < groups) load(gn, wb, ub);
    float a0 = 0.f, a1 = 0.f, b0 = 0.f, b1 = 0.f;
    dot(wa, ua, a0, a1, b0, b1);
    finish_row<LPR, false, PAIR>(a, g * RPW + sub, g * RPW + sub < a.M, l, a0, a1, b0, b1, best);
    g = gn;
    if (g >= groups) break;
    const int gn2 = g + stride;
    if (gn2 < groups) load(gn2, wa, ua);
    a0 = a1 = b0 = b1 = 0.f;
    dot(wb, ub, a0, a1, b0, b1);
    finish_row<LPR, false, PAIR>(a, g * RPW + sub, g * RPW + sub < a.M, l, a0, a1, b0, b1, best);
    g = gn2;
  }

  if (a.epi == EPI_F32_ARGMAX) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) best = umax64(best, shfl_xor_u64(best, m));
    if (lane == 0) wave_keys[wave] = best;
    __syncthreads();
    if (tid == 0) {
      unsigned long long k = wave_keys[0];
#pragma unroll
      for (int i = 1; i < kWaves; ++i) k = umax64(k, wave_keys[i]);
      a.keys[blockIdx.x] = k;
    }
  }
}

// Register-x GEMV for rows of int8 or bf16 weights, one row group (64 / LPR
// rows) per KS waves: each of the KS waves takes a contiguous slice of the
// row's 16-byte chunks (a split of K inside the workgroup), every lane loads
// the x chunks of its weight chunks straight from memory (L2-resident) as
// packed bf16 pairs, and the products run on v_dot2_f32_bf16 (int8 pairs
// widened exactly to bf16 first).  The KS partial sums of a row meet in LDS
// and the slice-0 wave adds them in slice order and applies the epilogue.
// A workgroup of kWaves waves owns kWaves / KS row groups, one pass, no
// loop.  This gives the short W8 projections (QKV, O: 36 workgroups of the
// LDS-staged form, under one wave per CU) a wave per row group, and the long
// bf16 rows (down_proj, K = 4864) four waves per row.
template <int LPR, int NJ, bool W8, int KS>
__global__ __launch_bounds__(kThreads) void gemv_rx_kernel(GemvArgs a) {
  static_assert(kWaves % KS == 0, "whole row groups per workgroup");
  constexpr int RPW = 64 / LPR, GPW = kWaves / KS, EPC = W8 ? 16 : 8;
  __shared__ float part[kWaves][RPW];
  __shared__ unsigned long long wave_keys[kWaves];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int l = lane % LPR, sub = lane / LPR;
  const int slice = wave % KS, gl = wave / KS;
  const int K = a.K, CH = K / EPC, CHS = (CH + KS - 1) / KS, c0 = slice * CHS, c1 = min(CH, c0 + CHS);
  const int g = blockIdx.x * GPW + gl;
  const int row = g * RPW + sub;
  const bool live = row < a.M;
  const size_t row_bytes = (size_t)K * (W8 ? 1 : 2);

  // weights first (the longest latency); chunks past the slice read zero
  const __amdgpu_buffer_rsrc_t wr = rsrc(a.W, (int)((size_t)a.M * row_bytes));
  const unsigned rofs = (unsigned)((size_t)(live ? row : 0) * row_bytes);
  u32x4 w[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int c = c0 + l + j * LPR;
    w[j] = __builtin_amdgcn_raw_buffer_load_b128(wr, live && c < c1 ? rofs + (unsigned)c * 16u : kGemvOutside, 0, 2);
  }
  const uint16_t* x = a.x;
  if (a.x_index != nullptr) {
    int t = *a.x_index;
    if (t >= 0) {
      if (t >= a.vocab_limit) t = a.vocab_limit - 1;
      x = a.x_table + (size_t)t * (size_t)K;
      if (a.x_copy != nullptr && blockIdx.x == 0) {
        const uint32_t* src = reinterpret_cast<const uint32_t*>(x);
        for (int i = tid; i < K / 2; i += kThreads) reinterpret_cast<uint32_t*>(a.x_copy)[i] = src[i];
      }
    }
  }
  // this lane's x values for each weight chunk as packed bf16 pairs, zero
  // past the slice; for an RMSNorm input also the gains of the same columns
  constexpr int XW = EPC / 2;  // x words per chunk
  uint32_t xp[NJ][XW], gp[NJ][XW];
  const bool norm = a.pro == PRO_NORM;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int c = c0 + l + j * LPR;
    const bool ok = c < c1;
#pragma unroll
    for (int h = 0; h < EPC / 8; ++h) {
      const int e0 = c * EPC + 8 * h;
      const u32x4 v = ok ? load16(x + e0) : u32x4{0u, 0u, 0u, 0u};
      const u32x4 gm = ok && norm ? load16(a.gamma + e0) : u32x4{0u, 0u, 0u, 0u};
      xp[j][4 * h] = v.x, xp[j][4 * h + 1] = v.y, xp[j][4 * h + 2] = v.z, xp[j][4 * h + 3] = v.w;
      gp[j][4 * h] = gm.x, gp[j][4 * h + 1] = gm.y, gp[j][4 * h + 2] = gm.z, gp[j][4 * h + 3] = gm.w;
    }
  }
  if (norm) {
    // RMSNorm (cpu_backend.py:71-76): the LPR lanes of a row hold the slice's
    // values once, so their sum of squares is the slice's; the KS slices of
    // a row group meet in LDS (every wave holds the same x)
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int q = 0; q < XW; ++q) {
        const float lo = bf_lo(xp[j][q]), hi = bf_hi(xp[j][q]);
        ss += lo * lo;
        ss += hi * hi;
      }
    ss = lane_sum<LPR>(ss);
    if constexpr (KS > 1) {
      if (lane == 0) part[wave][0] = ss;
      __syncthreads();
      ss = 0.0f;
#pragma unroll
      for (int k = 0; k < KS; ++k) ss += part[gl * KS + k][0];
      __syncthreads();  // part is reused for the row sums
    }
    const float inv = 1.0f / sqrtf(ss / (float)K + a.eps);
    // bf16((v * inv) * gamma), exact in bf16
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int q = 0; q < XW; ++q) {
        const float n0 = round_bf16((bf_lo(xp[j][q]) * inv) * bf_lo(gp[j][q]));
        const float n1 = round_bf16((bf_hi(xp[j][q]) * inv) * bf_hi(gp[j][q]));
        xp[j][q] = (__float_as_uint(n0) >> 16) | (__float_as_uint(n1) & 0xffff0000u);
      }
  }
  float a0 = 0.f, a1 = 0.f;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const uint32_t ww[4] = {w[j].x, w[j].y, w[j].z, w[j].w};
    if constexpr (W8) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        a0 = dot2_bf16(i8pair_bf16(ww[q], 0), xp[j][2 * q], a0);
        a1 = dot2_bf16(i8pair_bf16(ww[q], 2), xp[j][2 * q + 1], a1);
      }
    } else {
#pragma unroll
      for (int q = 0; q < 4; q += 2) {
        a0 = dot2_bf16(ww[q], xp[j][q], a0);
        a1 = dot2_bf16(ww[q + 1], xp[j][q + 1], a1);
      }
    }
  }
  unsigned long long best = 0ull;
  if constexpr (KS == 1) {
    finish_row<LPR, W8, false>(a, row, live, l, a0, a1, 0.f, 0.f, best);
  } else {
    const float s = lane_sum<LPR>(a0 + a1);
    if (l == 0) part[wave][sub] = s;
    __syncthreads();
    if (slice == 0) {
      float t = 0.0f;
#pragma unroll
      for (int k = 0; k < KS; ++k) t += part[wave + k][sub];
      // finish_row's reduction of (t, 0) over the LPR lanes: lane 0 holds t
      finish_row<LPR, W8, false>(a, row, live, l, l == 0 ? t : 0.0f, 0.0f, 0.f, 0.f, best);
    }
  }
  if (a.epi == EPI_F32_ARGMAX) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) best = umax64(best, shfl_xor_u64(best, m));
    if (lane == 0) wave_keys[wave] = best;
    __syncthreads();
    if (tid == 0) {
      unsigned long long k = wave_keys[0];
#pragma unroll
      for (int i = 1; i < kWaves; ++i) k = umax64(k, wave_keys[i]);
      a.keys[blockIdx.x] = k;
    }
  }
}

}  // namespace

int cu_count() {
  static int count = 0;
  if (count == 0) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
      count = n;
    else
      count = 256;
  }
  return count;
}

namespace {

// Workgroups for a launch: one row group per wave when that fits in four
// workgroups per CU, otherwise four per CU looping over the groups.
int blocks_for(int groups) {
  const int needed = (groups + kWaves - 1) / kWaves;
  int cap = cu_count() * 4;
  if (cap > kMaxPartialKeys) cap = kMaxPartialKeys;
  return needed < cap ? needed : cap;
}

// Workgroups of gemv_kernel<...> that stay resident on one CU with `lds`
// bytes of LDS each (registers limit most forms to three: a grid of four per
// CU would leave a quarter of the workgroups to start after the others and
// run the tail alone).  Cached per form for the last LDS size asked.
template <int LPR, int NJ, bool W8, bool PAIR, bool BUF>
int resident_per_cu(size_t lds) {
  static size_t cached_lds = 0;
  static int cached = 0;
  if (cached == 0 || cached_lds != lds) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, gemv_kernel<LPR, NJ, W8, PAIR, BUF>, kThreads, lds) !=
            hipSuccess ||
        n <= 0)
      n = 1;
    cached = n < 4 ? n : 4;
    cached_lds = lds;
  }
  return cached;
}

template <int LPR, int NJ, bool W8, bool PAIR, bool BUF = !W8>
int launch_cfg(const GemvArgs& a, hipStream_t stream, int* blocks_out) {
  constexpr int RPW = 64 / LPR;
  // x as float32 and a reduction scratch; W8 also x as packed bf16 pairs
  const size_t lds = (size_t)(a.K + 8) * sizeof(float) + (size_t)a.K * 2;
  const int needed = ((a.M + RPW - 1) / RPW + kWaves - 1) / kWaves;
  int cap = cu_count() * resident_per_cu<LPR, NJ, W8, PAIR, BUF>(lds);
  if (cap > kMaxPartialKeys) cap = kMaxPartialKeys;
  const int blocks = needed < cap ? needed : cap;
  if (blocks_out) *blocks_out = blocks;
  hipLaunchKernelGGL((gemv_kernel<LPR, NJ, W8, PAIR, BUF>), dim3(blocks), dim3(kThreads), lds, stream,
                     a);
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? 0 : hip_fail(err, "gemv launch");
}

template <int LPR, bool W8, bool PAIR>
int launch_nj(int nj, const GemvArgs& a, hipStream_t stream, int* blocks_out) {
  if (nj <= 6) return launch_cfg<LPR, 6, W8, PAIR>(a, stream, blocks_out);
  if (nj <= 7) return launch_cfg<LPR, 7, W8, PAIR>(a, stream, blocks_out);
  if (nj <= 8) return launch_cfg<LPR, 8, W8, PAIR>(a, stream, blocks_out);
  if (nj <= 10) return launch_cfg<LPR, 10, W8, PAIR>(a, stream, blocks_out);
  return launch_cfg<LPR, 12, W8, PAIR>(a, stream, blocks_out);
}

// Fewest lanes per row that keep every lane's chunk count at or below 12;
// longer rows use 64 lanes and several passes of 8 chunks.
int pick_lpr(int CH) {
  if ((CH + 7) / 8 <= 12) return 8;
  if ((CH + 15) / 16 <= 12) return 16;
  if ((CH + 31) / 32 <= 12) return 32;
  return 64;
}

template <bool W8, bool PAIR>
int launch_shape(const GemvArgs& a, hipStream_t stream, int* blocks_out) {
  const int CH = W8 ? a.K / 16 : a.K / 8;
  // the int8 LM head (rows of up to 96 chunks) with branch-free loads
  if (W8 && !PAIR && a.epi == EPI_F32_ARGMAX && pick_lpr(CH) == 8) {
    const int nj = (CH + 7) / 8;
    if (nj <= 6) return launch_cfg<8, 6, true, false, true>(a, stream, blocks_out);
    if (nj <= 7) return launch_cfg<8, 7, true, false, true>(a, stream, blocks_out);
    if (nj <= 8) return launch_cfg<8, 8, true, false, true>(a, stream, blocks_out);
    if (nj <= 10) return launch_cfg<8, 10, true, false, true>(a, stream, blocks_out);
    return launch_cfg<8, 12, true, false, true>(a, stream, blocks_out);
  }
  switch (pick_lpr(CH)) {
    case 8: return launch_nj<8, W8, PAIR>((CH + 7) / 8, a, stream, blocks_out);
    case 16: return launch_nj<16, W8, PAIR>((CH + 15) / 16, a, stream, blocks_out);
    case 32: return launch_nj<32, W8, PAIR>((CH + 31) / 32, a, stream, blocks_out);
    default:
      if ((CH + 63) / 64 <= 12) return launch_nj<64, W8, PAIR>((CH + 63) / 64, a, stream, blocks_out);
      return launch_cfg<64, 8, W8, PAIR>(a, stream, blocks_out);
  }
}

// Register-x plan: 32 or 64 lanes per row (whichever pads the row's chunks
// less; 32 for short paired rows), at most kXregMaxNJ chunks per lane (8 when
// paired), and only when every wave owns at most one row group.  Returns
// false when the LDS-staged kernel should run instead.
constexpr int kXregMaxNJ = 12;

struct XregPlan {
  int lpr = 0;
  int nj = 0;
};

bool xreg_plan(const GemvArgs& a, bool w8, XregPlan* plan) {
  if (w8) return false;
  // x and gamma are read in 16-byte chunks here (the LDS form reads 4 bytes)
  const uintptr_t align = reinterpret_cast<uintptr_t>(a.x) | reinterpret_cast<uintptr_t>(a.gamma) |
                          reinterpret_cast<uintptr_t>(a.x_table);
  if (align & 15) return false;
  const bool pair = a.epi == EPI_SWIGLU;
  const int CH = a.K / 8;
  const int nj64 = (CH + 63) / 64, nj32 = (CH + 31) / 32;
  const int max_nj = pair ? 8 : kXregMaxNJ;
  int lpr;
  if (nj32 * 32 < nj64 * 64 || (pair && nj32 * 32 == nj64 * 64 && CH <= 128))
    lpr = nj32 <= max_nj ? 32 : 64;
  else
    lpr = 64;
  const int nj = lpr == 32 ? nj32 : nj64;
  if (nj > max_nj) return false;
  const int rpw = 64 / lpr;
  const int groups = (a.M + rpw - 1) / rpw;
  int cap = cu_count() * 4;
  if (cap > kMaxPartialKeys) cap = kMaxPartialKeys;
  if ((groups + kWaves - 1) / kWaves > cap) return false;
  plan->lpr = lpr;
  plan->nj = nj;
  return true;
}

template <int LPR, int NJ, bool PAIR>
int launch_xreg_cfg(const GemvArgs& a, hipStream_t stream, int* blocks_out) {
  constexpr int RPW = 64 / LPR;
  const int blocks = blocks_for((a.M + RPW - 1) / RPW);
  if (blocks_out) *blocks_out = blocks;
  hipLaunchKernelGGL((gemv_xreg_kernel<LPR, NJ, PAIR>), dim3(blocks), dim3(kThreads), 0, stream, a);
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? 0 : hip_fail(err, "gemv launch");
}

template <int LPR, bool PAIR>
int launch_xreg_nj(int nj, const GemvArgs& a, hipStream_t stream, int* blocks_out) {
  switch (nj) {
    case 1: return launch_xreg_cfg<LPR, 1, PAIR>(a, stream, blocks_out);
    case 2: return launch_xreg_cfg<LPR, 2, PAIR>(a, stream, blocks_out);
    case 3: return launch_xreg_cfg<LPR, 3, PAIR>(a, stream, blocks_out);
    case 4: return launch_xreg_cfg<LPR, 4, PAIR>(a, stream, blocks_out);
    case 5: return launch_xreg_cfg<LPR, 5, PAIR>(a, stream, blocks_out);
    case 6: return launch_xreg_cfg<LPR, 6, PAIR>(a, stream, blocks_out);
    case 7:
    case 8: return launch_xreg_cfg<LPR, 8, PAIR>(a, stream, blocks_out);
    default:
      if constexpr (!PAIR) {
        if (nj <= 10) return launch_xreg_cfg<LPR, 10, PAIR>(a, stream, blocks_out);
        return launch_xreg_cfg<LPR, 12, PAIR>(a, stream, blocks_out);
      }
      return fail("gemv: no register-x configuration for this row length");
  }
}

template <bool PAIR>
int launch_xreg(const XregPlan& p, const GemvArgs& a, hipStream_t stream, int* blocks_out) {
  if (p.lpr == 32) return launch_xreg_nj<32, PAIR>(p.nj, a, stream, blocks_out);
  return launch_xreg_nj<64, PAIR>(p.nj, a, stream, blocks_out);
}

// The register-x split plan (gemv_rx_kernel): int8 rows (split four ways
// past 2048 columns) or bf16 rows longer than 1024 columns (split four
// ways), when a one-pass grid fits four workgroups per CU; false otherwise.
// HK_GEMV_RX=0 turns it off.
struct RxPlan {
  int lpr = 0, nj = 0, ks = 0;
};

bool rx_plan(const GemvArgs& a, bool w8, RxPlan* plan) {
  static const bool off = [] {
    const char* e = getenv("HK_GEMV_RX");
    return e && e[0] == '0';
  }();
  // HK_GEMV_RX_SHAPE=lpr,ks (lpr 32 or 64, ks 1, 2 or 4): one launch shape
  // for every register-x launch, for tuning sweeps
  static const RxPlan forced = [] {
    RxPlan f;
    const char* e = getenv("HK_GEMV_RX_SHAPE");
    int lpr = 0, ks = 0;
    if (e && sscanf(e, "%d,%d", &lpr, &ks) == 2 && (lpr == 32 || lpr == 64) && (ks == 1 || ks == 2 || ks == 4)) {
      f.lpr = lpr;
      f.ks = ks;
    }
    return f;
  }();
  if (off || a.epi == EPI_SWIGLU) return false;
  const uintptr_t align = reinterpret_cast<uintptr_t>(a.x) | reinterpret_cast<uintptr_t>(a.gamma) |
                          reinterpret_cast<uintptr_t>(a.x_table);
  if (align & 15) return false;
  const int CH = a.K / (w8 ? 16 : 8);
  RxPlan p;
  if (w8) {
    p.ks = CH > 128 ? 4 : 1;
    p.lpr = CH <= 32 ? 32 : 64;
  } else {
    if (a.K <= 1024) return false;
    p.ks = 4;
    p.lpr = 64;
  }
  if (forced.lpr) {
    p.lpr = forced.lpr;
    p.ks = forced.ks;
  }
  const int chs = (CH + p.ks - 1) / p.ks;
  p.nj = (chs + p.lpr - 1) / p.lpr;
  if (p.nj > 6) return false;
  const int groups = (a.M + 64 / p.lpr - 1) / (64 / p.lpr);
  const int blocks = (groups + kWaves / p.ks - 1) / (kWaves / p.ks);
  int cap = cu_count() * 4;
  if (cap > kMaxPartialKeys) cap = kMaxPartialKeys;
  if (blocks > cap) return false;
  *plan = p;
  return true;
}

template <int LPR, bool W8, int KS>
int launch_rx_nj(int nj, const GemvArgs& a, hipStream_t stream, int* blocks_out) {
  const int groups = (a.M + 64 / LPR - 1) / (64 / LPR);
  const int blocks = (groups + kWaves / KS - 1) / (kWaves / KS);
  if (blocks_out) *blocks_out = blocks;
  switch (nj) {
    case 1: hipLaunchKernelGGL((gemv_rx_kernel<LPR, 1, W8, KS>), dim3(blocks), dim3(kThreads), 0, stream, a); break;
    case 2: hipLaunchKernelGGL((gemv_rx_kernel<LPR, 2, W8, KS>), dim3(blocks), dim3(kThreads), 0, stream, a); break;
    case 3: hipLaunchKernelGGL((gemv_rx_kernel<LPR, 3, W8, KS>), dim3(blocks), dim3(kThreads), 0, stream, a); break;
    case 4: hipLaunchKernelGGL((gemv_rx_kernel<LPR, 4, W8, KS>), dim3(blocks), dim3(kThreads), 0, stream, a); break;
    default: hipLaunchKernelGGL((gemv_rx_kernel<LPR, 6, W8, KS>), dim3(blocks), dim3(kThreads), 0, stream, a); break;
  }
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? 0 : hip_fail(err, "gemv launch");
}

template <bool W8, int KS>
int launch_rx_ks(const RxPlan& p, const GemvArgs& a, hipStream_t stream, int* blocks_out) {
  if (p.lpr == 32) return launch_rx_nj<32, W8, KS>(p.nj, a, stream, blocks_out);
  return launch_rx_nj<64, W8, KS>(p.nj, a, stream, blocks_out);
}

template <bool W8>
int launch_rx_w(const RxPlan& p, const GemvArgs& a, hipStream_t stream, int* blocks_out) {
  if (p.ks == 4) return launch_rx_ks<W8, 4>(p, a, stream, blocks_out);
  if (p.ks == 2) return launch_rx_ks<W8, 2>(p, a, stream, blocks_out);
  return launch_rx_ks<W8, 1>(p, a, stream, blocks_out);
}

int launch_rx(const RxPlan& p, const GemvArgs& a, bool w8, hipStream_t stream, int* blocks_out) {
  return w8 ? launch_rx_w<true>(p, a, stream, blocks_out) : launch_rx_w<false>(p, a, stream, blocks_out);
}
}  // namespace

int launch_gemv(const GemvArgs& a, bool w8, hipStream_t stream, int* blocks_out) {
  if (a.M <= 0 || a.K <= 0) return fail("gemv: M and K must be positive");
  if (a.K % (w8 ? 16 : 8) != 0)
    return fail(w8 ? "gemv: K must be a multiple of 16 for int8 weights"
                   : "gemv: K must be a multiple of 8 for bf16 weights");
  if (a.K > 16384) return fail("gemv: K above 16384 is not supported");
  if ((a.epi == EPI_SWIGLU ? 2.0 : 1.0) * a.M * a.K * (w8 ? 1 : 2) >= 2147483632.0)
    return fail("gemv: weight matrices of 2 GiB or more are not supported");
  if (a.pro == PRO_NORM && a.gamma == nullptr) return fail("gemv: RMSNorm needs gamma");
  if (w8 && a.scale == nullptr) return fail("gemv: int8 weights need per-row scales");
  const bool pair = a.epi == EPI_SWIGLU;
  if ((a.epi == EPI_F32 || a.epi == EPI_F32_ARGMAX) && a.yf == nullptr)
    return fail("gemv: float32 output missing");
  if (a.epi != EPI_F32 && a.epi != EPI_F32_ARGMAX && a.y == nullptr)
    return fail("gemv: bf16 output missing");
  if (a.epi == EPI_BIAS && a.bias == nullptr) return fail("gemv: bias missing");
  if (a.epi == EPI_RESID && a.resid == nullptr) return fail("gemv: residual missing");
  if (a.epi == EPI_F32_ARGMAX && a.keys == nullptr) return fail("gemv: argmax key buffer missing");
  RxPlan rx;
  if (rx_plan(a, w8, &rx)) return launch_rx(rx, a, w8, stream, blocks_out);
  XregPlan plan;
  if (xreg_plan(a, w8, &plan))
    return pair ? launch_xreg<true>(plan, a, stream, blocks_out)
                : launch_xreg<false>(plan, a, stream, blocks_out);
  if (w8)
    return pair ? launch_shape<true, true>(a, stream, blocks_out)
                : launch_shape<true, false>(a, stream, blocks_out);
  return pair ? launch_shape<false, true>(a, stream, blocks_out)
              : launch_shape<false, false>(a, stream, blocks_out);
}

}  // namespace hk
