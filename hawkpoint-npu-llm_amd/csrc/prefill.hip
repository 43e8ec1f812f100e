// Batched prefill: every prompt token of a chunk goes through a layer at once.
//
// The reference prefills position by position with the decode step
// (npu_llm/runtime/generate.py:1110-1125); the arithmetic per token is the
// same as cpu_backend.py:131-181, so this path keeps every rounding point of
// the decode kernels and only changes how the work is batched:
//   embed_rows         X[i] = E[token_i]
//   rmsnorm_rows       Xn[i] = bf16((v * inv_rms) * gamma)            :71-76
//   gemm (MFMA bf16)   Y = Xn @ W^T with the GEMV epilogues (bias, residual,
//                      SwiGLU on paired gate/up rows), f32 accumulation
//   rope_append        rotated q of every token; K/V appended at slots
//                      start..start+n-1                                 :78-108
//   attention_prefill  causal GQA: token i attends to slots 0..start+i    :110-129
//
// GEMM tiling (wave64, v_mfma_f32_16x16x32_bf16): a 256-thread workgroup owns
// a 64-token x 64-output tile (two weight tiles for SwiGLU pairs); each wave
// owns a 32x32 quarter as 2x2 MFMA blocks.  K advances 32 at a time through
// LDS; A and W tiles arrive with one 16-byte load per thread each.
#include <algorithm>

#include "hk_common.h"
#include "hk_internal.h"

namespace hk {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef short v4s16 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kTM = 64;       // tokens per tile
constexpr int kTN = 64;       // outputs per tile
constexpr int kTK = 32;       // K per step
constexpr int kLdsRow = kTK + 8;  // bf16 per LDS row (padding against bank conflicts)

__device__ __forceinline__ float silu_mul(float g, float u) {
  const float clipped = fminf(fmaxf(g, -80.0f), 80.0f);
  return (g / (1.0f + expf(-clipped))) * u;
}

// W8: int8 weight rows, converted exactly to bf16 as they are loaded; the
// row scale multiplies the finished sum in the epilogue.
template <bool PAIR, bool W8 = false>
__global__ __launch_bounds__(kThreads) void gemm_kernel(PrefillGemmArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t As[kTM][kLdsRow];
  __shared__ __attribute__((aligned(16))) uint16_t Ws[kTN][kLdsRow];
  __shared__ __attribute__((aligned(16))) uint16_t Us[PAIR ? kTN : 1][kLdsRow];

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int m0 = blockIdx.y * kTM;
  const int n0 = blockIdx.x * kTN;
  const int wm = (wave >> 1) * 32;  // wave's token offset in the tile
  const int wn = (wave & 1) * 32;   // wave's output offset in the tile

  // Grouped mode: this workgroup's expert, row count and row offset.
  const uint16_t* Wb = a.W;
  int M = a.M;
  int row_off = 0;
  const bool grouped = a.grp_count != nullptr;
  if (grouped) {
    const int z = blockIdx.z;
    if (z >= *a.n_groups) return;
    M = a.grp_count[z];
    if (m0 >= M) return;
    row_off = a.grp_offset[z];
    Wb = a.W + (size_t)a.grp_expert[z] * (size_t)a.w_stride;
  }

  // one 16-byte piece of each tile per thread: row = tid / 4, k8 = (tid % 4) * 8
  const int lr = tid >> 2;
  const int lk = (tid & 3) * 8;
  const bool a_ok = (m0 + lr) < M;
  const bool w_ok = (n0 + lr) < a.N;
  int arow = a_ok ? m0 + lr : 0;
  if (grouped) arow = a.a_rows ? a.a_rows[row_off + (a_ok ? m0 + lr : 0)] : row_off + arow;
  const uint16_t* a_src = a.A + (size_t)arow * a.lda + lk;
  const size_t w_off = (size_t)(w_ok ? n0 + lr : 0) * a.K + lk;
  const size_t u_off = (size_t)(w_ok ? n0 + lr + a.N : 0) * a.K + lk;
  auto wload = [&](size_t off) -> u32x4 {
    if constexpr (W8)
      return load_stream_i8_bf16(reinterpret_cast<const int8_t*>(Wb) + off);
    else
      return load_stream16(Wb + off);
  };
  const u32x4 zero = {0u, 0u, 0u, 0u};

  f32x4 acc[2][2], accu[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
      accu[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

  const int fr = lane & 15;        // fragment row / column
  const int fk = (lane >> 4) * 8;  // fragment k offset

  for (int k0 = 0; k0 < a.K; k0 += kTK) {
    const u32x4 av = a_ok ? load16(a_src + k0) : zero;
    const u32x4 wv = w_ok ? wload(w_off + k0) : zero;
    u32x4 uv = zero;
    if constexpr (PAIR) uv = w_ok ? wload(u_off + k0) : zero;
    __syncthreads();
    *reinterpret_cast<u32x4*>(&As[lr][lk]) = av;
    *reinterpret_cast<u32x4*>(&Ws[lr][lk]) = wv;
    if constexpr (PAIR) *reinterpret_cast<u32x4*>(&Us[lr][lk]) = uv;
    __syncthreads();
    bf16x8 af[2], bfr[2], ufr[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) af[i] = *reinterpret_cast<const bf16x8*>(&As[wm + i * 16 + fr][fk]);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      bfr[j] = *reinterpret_cast<const bf16x8*>(&Ws[wn + j * 16 + fr][fk]);
      if constexpr (PAIR) ufr[j] = *reinterpret_cast<const bf16x8*>(&Us[wn + j * 16 + fr][fk]);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
        if constexpr (PAIR)
          accu[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], ufr[j], accu[i][j], 0, 0, 0);
      }
  }

  // D layout: lane holds rows 4*(lane/16) + r, column lane % 16 of each block.
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int mt = m0 + wm + i * 16 + (lane >> 4) * 4 + r;
        const int n = n0 + wn + j * 16 + (lane & 15);
        if (mt >= M || n >= a.N) continue;
        const int m = row_off + mt;
        float v = acc[i][j][r], u = accu[i][j][r];
        if constexpr (W8) {
          v *= a.scale[n];
          if constexpr (PAIR) u *= a.scale[a.N + n];
        }
        uint16_t* y = a.Y + (size_t)m * a.ldy + n;
        switch (a.epi) {
          case EPI_BF16:
            *y = (uint16_t)f32_to_bf16(v);
            break;
          case EPI_BIAS:
            *y = (uint16_t)f32_to_bf16(round_bf16(v) + a.bias[n]);
            break;
          case EPI_RESID:
            *y = (uint16_t)f32_to_bf16(round_bf16(v) + bf16_to_f32(a.resid[(size_t)m * a.ldr + n]));
            break;
          case EPI_SWIGLU:
            *y = (uint16_t)f32_to_bf16(silu_mul(round_bf16(v), round_bf16(u)));
            break;
          default:
            break;
        }
      }
}

// X[i] = E[token_i] (bf16 rows), tokens read from device memory.
// Row i of X = the embedding of tokens[i]; with kb_rows (the row count) X is
// k-blocked: element (i, k) at ((k / 8) kb_rows + i) 8 + k % 8.
__global__ __launch_bounds__(kThreads) void embed_rows_kernel(const int32_t* tokens, int vocab,
                                                              const uint16_t* table, int H,
                                                              uint16_t* X, int kb_rows) {
  const int i = blockIdx.x;
  int t = tokens[i];
  t = t < 0 ? 0 : (t >= vocab ? vocab - 1 : t);
  const uint32_t* src = reinterpret_cast<const uint32_t*>(table + (size_t)t * H);
  if (kb_rows) {
    uint32_t* dst = reinterpret_cast<uint32_t*>(X);
    for (int j = threadIdx.x; j < H / 2; j += kThreads)
      dst[((size_t)(j >> 2) * kb_rows + i) * 4 + (j & 3)] = src[j];
    return;
  }
  uint32_t* dst = reinterpret_cast<uint32_t*>(X + (size_t)i * H);
  for (int j = threadIdx.x; j < H / 2; j += kThreads) dst[j] = src[j];
}

// One row per workgroup: out = bf16((v * inv_rms) * gamma).
// RMSNorm of eight bf16 inputs (one 16-byte fragment) with the token's
// inverse rms and eight gains: bf16((x * inv) * gamma), the reference's order.
__device__ __forceinline__ u32x4 norm8(u32x4 x, float inv, u32x4 g) {
  const uint32_t xs[4] = {x.x, x.y, x.z, x.w}, gs[4] = {g.x, g.y, g.z, g.w};
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    o[i] = f32x2_to_bf16x2((bf_lo(xs[i]) * inv) * bf_lo(gs[i]), (bf_hi(xs[i]) * inv) * bf_hi(gs[i]));
  return u32x4{o[0], o[1], o[2], o[3]};
}

__device__ __forceinline__ float sq8(u32x4 x) {
  const uint32_t xs[4] = {x.x, x.y, x.z, x.w};
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    s += bf_lo(xs[i]) * bf_lo(xs[i]);
    s += bf_hi(xs[i]) * bf_hi(xs[i]);
  }
  return s;
}

__global__ __launch_bounds__(kThreads) void rmsnorm_rows_kernel(const uint16_t* X, int ldx,
                                                                const uint16_t* gamma, float eps,
                                                                uint16_t* out, int ldo, int H, int rows) {
  // one wave per row, 16-byte pieces of 8 values (H a multiple of 8): the
  // squares in one pass, then the row again (from the caches) normalised
  const int row = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= rows) return;
  const uint16_t* x = X + (size_t)row * ldx;
  const int chunks = H / 8;
  float ss = 0.0f;
  for (int c = lane; c < chunks; c += 64) ss += sq8(load16(x + 8 * c));
  ss = group_sum<64>(ss);
  const float inv = 1.0f / sqrtf(ss / (float)H + eps);
  uint16_t* o = out + (size_t)row * ldo;
  for (int c = lane; c < chunks; c += 64)
    *reinterpret_cast<u32x4*>(o + 8 * c) = norm8(load16(x + 8 * c), inv, load16(gamma + 8 * c));
}

// Token i at slot p = start + i: rotated q heads to Qr[i], rotated k and raw v
// to the caches at slot p.
__global__ __launch_bounds__(kThreads) void rope_append_kernel(PrefillAttnArgs a) {
  const int i = blockIdx.x;
  const int p = a.start + i;
  const int half = kHeadDim / 2;
  const float* ct = a.cos_tab + (size_t)p * half;
  const float* st = a.sin_tab + (size_t)p * half;
  const uint16_t* row = a.qkv + (size_t)i * a.ld_qkv;
  const int heads = a.q_heads + a.kv_heads;
  for (int e = threadIdx.x; e < heads * half; e += kThreads) {
    const int h = e / half, j = e % half;
    const uint16_t* src = row + (size_t)h * kHeadDim;
    const float x1 = bf16_to_f32(src[j]), x2 = bf16_to_f32(src[j + half]);
    const uint32_t r1 = f32_to_bf16(x1 * ct[j] - x2 * st[j]);
    const uint32_t r2 = f32_to_bf16(x2 * ct[j] + x1 * st[j]);
    uint16_t* dst;
    if (h < a.q_heads) {
      dst = a.qrot + (size_t)i * a.q_heads * kHeadDim + (size_t)h * kHeadDim;
    } else {
      const int g = h - a.q_heads;
      dst = a.kcache + ((size_t)g * a.max_ctx + p) * kHeadDim;
    }
    dst[j] = (uint16_t)r1;
    dst[j + half] = (uint16_t)r2;
  }
  for (int e = threadIdx.x; e < a.kv_heads * kHeadDim; e += kThreads) {
    const int g = e / kHeadDim, d = e % kHeadDim;
    a.vcache[((size_t)g * a.max_ctx + p) * kHeadDim + d] =
        row[(size_t)(a.q_heads + a.kv_heads + g) * kHeadDim + d];
  }
}

// Large-M GEMM (prompt chunks of 128+ tokens): a 256-thread workgroup owns
// 128 tokens x BN outputs (for SwiGLU, BN gate and BN up rows); the waves
// split it 2 x 2, so each owns 64 x BN/2 as 4 x BN/32 MFMA blocks (twice
// that for SwiGLU).  K advances 64 at a time through two LDS buffers: the
// next step's tiles are loaded into registers while this step's MFMAs run,
// then written to the other buffer, so one barrier per step suffices.
constexpr int kBM = 128;
constexpr int kBK = 64;
constexpr int kBRow = kBK + 8;  // bf16 per LDS row (rows 144 B apart: no bank conflicts)

// The epilogue of the large-M GEMMs: the tile's outputs go through LDS (ep:
// BM x (BN + 8) bf16, free once every wave is past the last K step) so that
// they leave as 16-byte stores of 8 outputs of a row, with the residual rows
// read the same way.  Wave tiles: rows wm.., columns wn.. of the tile, MB x
// NB MFMA 16 x 16 blocks (D layout: lane holds rows 4 (lane / 16) + r,
// column lane % 16 of each block).
// DM 32: the blocks are MFMA 32 x 32 ones (lane holds rows 8 (r / 4) +
// 4 (lane / 32) + r % 4, column lane % 32, r = 0..15).
template <int DM> struct DBlock { using T = f32x4; };
template <> struct DBlock<32> { using T = f32x16; };

// The QKV epilogue with RoPE and the KV append (rope_append_kernel's
// arithmetic) for outputs n .. n + 7 of token row m: src holds their
// bf16(sum), partner the bf16(sum) of the RoPE partners n ^ 32 .. (the tiles
// start at multiples of 64 outputs, so a head's 64 rows share a tile); the
// bias is added as in the plain epilogue, then q and k rotate and go to the
// rotated queries and the key cache, v to the value cache, at slot
// rope.start + m.
__device__ __forceinline__ void rope_chunk(const PrefillGemmArgs& a, const uint16_t* src, const uint16_t* partner, int m,
                                           int n) {
  const auto& at = a.rope;
  const int hd = n / kHeadDim, j = n % kHeadDim, p = at.start + m;
  const int np = n ^ (kHeadDim / 2);
  const u32x4 w = *reinterpret_cast<const u32x4*>(src), wp = *reinterpret_cast<const u32x4*>(partner);
  const uint32_t ww[4] = {w.x, w.y, w.z, w.w}, wwp[4] = {wp.x, wp.y, wp.z, wp.w};
  float v[8], vp[8];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    v[2 * q] = bf_lo(ww[q]);
    v[2 * q + 1] = bf_hi(ww[q]);
    vp[2 * q] = bf_lo(wwp[q]);
    vp[2 * q + 1] = bf_hi(wwp[q]);
  }
  if (a.bias) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      v[e] = round_bf16(v[e] + a.bias[n + e]);
      vp[e] = round_bf16(vp[e] + a.bias[np + e]);
    }
  }
  uint32_t o[4];
  uint16_t* dst;
  if (hd < at.q_heads + at.kv_heads) {
    const float* ct = at.cos_tab + (size_t)p * (kHeadDim / 2) + (j & (kHeadDim / 2 - 1));
    const float* st = at.sin_tab + (size_t)p * (kHeadDim / 2) + (j & (kHeadDim / 2 - 1));
    float r[8];
#pragma unroll
    for (int e = 0; e < 8; ++e)  // first half: x1 c - x2 s; second half: x2 c + x1 s (x1 the first-half value)
      r[e] = j < kHeadDim / 2 ? v[e] * ct[e] - vp[e] * st[e] : v[e] * ct[e] + vp[e] * st[e];
#pragma unroll
    for (int q = 0; q < 4; ++q) o[q] = f32x2_to_bf16x2(r[2 * q], r[2 * q + 1]);
    dst = hd < at.q_heads ? at.qrot + (size_t)m * at.q_heads * kHeadDim + (size_t)hd * kHeadDim + j
                          : at.kcache + ((size_t)(hd - at.q_heads) * at.max_ctx + p) * kHeadDim + j;
  } else {
#pragma unroll
    for (int q = 0; q < 4; ++q) o[q] = f32x2_to_bf16x2(v[2 * q], v[2 * q + 1]);
    dst = at.vcache + ((size_t)(hd - at.q_heads - at.kv_heads) * at.max_ctx + p) * kHeadDim + j;
  }
  *reinterpret_cast<u32x4*>(dst) = u32x4{o[0], o[1], o[2], o[3]};
}

template <int BM, int BN, bool PAIR, bool W8, int MB, int NB, int DM = 16>
__device__ __forceinline__ void tile_epilogue(const PrefillGemmArgs& a, const typename DBlock<DM>::T (&acc)[MB][NB],
                                              const typename DBlock<DM>::T (&accu)[PAIR ? MB : 1][PAIR ? NB : 1],
                                              uint16_t* ep, int m0, int n0, int wm, int wn, int tid, int lane) {
  // LDS holds, per output,
  // the bf16 that the epilogue's first rounding gives: the finished value
  // for EPI_BF16 and EPI_SWIGLU, bf16(sum) (exact, the value the bias or the
  // residual is added to) for EPI_BIAS and EPI_RESID.  The rounding points
  // are those of the other GEMM kernels.
  constexpr int ER = BN + 8;  // bf16 per LDS row of the tile
  const int fr = lane & 15;
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int r = 0; r < (DM == 16 ? 4 : 16); ++r) {
        const int ml = DM == 16 ? wm + 16 * i + (lane >> 4) * 4 + r : wm + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        const int nl = DM == 16 ? wn + 16 * j + fr : wn + 32 * j + (lane & 31);
        const int n = min(n0 + nl, a.N - 1);
        float v = acc[i][j][r];
        float u = 0.0f;
        if constexpr (PAIR) u = accu[i][j][r];
        if constexpr (W8) {
          v *= a.scale[n];
          if constexpr (PAIR) u *= a.scale[a.N + n];
        }
        uint32_t y;
        if constexpr (PAIR)
          y = a.epi == EPI_SWIGLU ? f32_to_bf16(silu_mul(round_bf16(v), round_bf16(u))) : f32_to_bf16(v);
        else
          y = f32_to_bf16(v);
        ep[ml * ER + nl] = (uint16_t)y;
      }
  __syncthreads();
  const bool add_bias = a.epi == EPI_BIAS, add_resid = a.epi == EPI_RESID;
  for (int c = tid; c < BM * BN / 8; c += kThreads) {
    const int ml = c / (BN / 8), nl = (c % (BN / 8)) * 8;
    const int m = m0 + ml, n = n0 + nl;
    if (m >= a.M || n >= a.N) continue;
    const uint16_t* src = ep + ml * ER + nl;
    if constexpr (!PAIR) {
      if (a.rope.on) {
        rope_chunk(a, src, ep + ml * ER + (nl ^ (kHeadDim / 2)), m, n);
        continue;
      }
    }
    uint16_t* y = a.Y + (size_t)m * a.ldy + n;
    if (n + 8 > a.N) {  // a ragged last chunk of the row
      for (int e = 0; e < a.N - n; ++e) {
        float f = bf16_to_f32(src[e]);
        if (add_bias) f = round_bf16(f + a.bias[n + e]);
        if (add_resid) f = round_bf16(f + bf16_to_f32(a.resid[(size_t)m * a.ldr + n + e]));
        y[e] = (uint16_t)f32_to_bf16(f);
      }
      continue;
    }
    u32x4 w = *reinterpret_cast<const u32x4*>(src);
    if (add_bias || add_resid) {
      float addend[8];
      if (add_resid) {
        const u32x4 rr = load16(a.resid + (size_t)m * a.ldr + n);
        const uint32_t rw[4] = {rr.x, rr.y, rr.z, rr.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          addend[2 * q] = bf_lo(rw[q]);
          addend[2 * q + 1] = bf_hi(rw[q]);
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) addend[e] = a.bias[n + e];
      }
      const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
      uint32_t o[4];
#pragma unroll
      for (int q = 0; q < 4; ++q)
        o[q] = f32x2_to_bf16x2(bf_lo(ww[q]) + addend[2 * q], bf_hi(ww[q]) + addend[2 * q + 1]);
      w = u32x4{o[0], o[1], o[2], o[3]};
    }
    *reinterpret_cast<u32x4*>(y) = w;
  }
}

// SPLIT (too few tiles to fill the GPU): workgroup (x, y) takes tile x
// (token tiles varying fastest) and the y-th of gridDim.y runs of K steps,
// and stores float32 partial sums to split_ws[y][m][outputs] (SwiGLU: up
// outputs at N + n) for split_reduce_kernel.
template <int BM, int BN, bool PAIR, bool SPLIT, bool W8 = false>
__global__ __launch_bounds__(kThreads) void gemm_big_kernel(PrefillGemmArgs a) {
  constexpr int WR = PAIR ? 2 * BN : BN;  // weight rows per tile
  constexpr int MB = BM / 32;             // 16-row blocks per wave
  constexpr int NB = BN / 32;             // 16-wide output blocks per wave
  constexpr int AL = BM * kBK / 8 / kThreads;  // 16-byte pieces per thread, A tile
  constexpr int WL = WR * kBK / 8 / kThreads;  // and weight tile
  __shared__ __attribute__((aligned(16))) uint16_t As[2][BM][kBRow];
  __shared__ __attribute__((aligned(16))) uint16_t Ws[2][WR][kBRow];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int mt = (a.M + BM - 1) / BM, ntile = (a.N + BN - 1) / BN;
  int m0, n0, kt0 = 0, kt1 = a.K / kBK;
  if constexpr (SPLIT) {
    m0 = (blockIdx.x % mt) * BM;
    n0 = (blockIdx.x / mt) * BN;
    const int per = (kt1 + gridDim.y - 1) / gridDim.y;
    kt0 = blockIdx.y * per;
    kt1 = min(kt1, kt0 + per);
  } else {
    // Workgroups go to the 8 XCDs in turn (workgroup b to XCD b % 8).  Tile
    // order t = (b % 8) * per + b / 8 gives each XCD a contiguous run.  The
    // order walks groups of up to 12 output tiles (4 when there are more)
    // with the output tile fastest, so the tiles an XCD holds at once share a
    // few token tiles and a few weight tiles, which its own L2 keeps.
    const int per = (mt * ntile + 7) / 8;
    const int t = (int)(blockIdx.x % 8) * per + (int)(blockIdx.x / 8);
    if (t >= mt * ntile) return;
    const int GN = ntile <= 12 ? ntile : 4;
    const int grp = t / (GN * mt), gn = min(GN, ntile - grp * GN), in = t - grp * GN * mt;
    m0 = (in / gn) * BM;
    n0 = (grp * GN + in % gn) * BN;
  }
  const int wm = (wave >> 1) * (BM / 2), wn = (wave & 1) * (BN / 2);
  const int fr = lane & 15, fk = (lane >> 4) * 8;
  const u32x4 zero = {0u, 0u, 0u, 0u};

  // piece i of this thread: row tid / 8 + 32 i, k (tid % 8) * 8 of the tile
  const int pr = tid >> 3, pk = (tid & 7) * 8;
  const uint16_t* a_src[AL];
  bool a_ok[AL];
#pragma unroll
  for (int i = 0; i < AL; ++i) {
    const int m = m0 + pr + 32 * i;
    a_ok[i] = m < a.M;
    a_src[i] = a.A + (size_t)(a_ok[i] ? m : 0) * a.lda + pk;
  }
  const void* w_src[WL];  // bf16, or int8 (W8) at the same element offset
  bool w_ok[WL];
#pragma unroll
  for (int i = 0; i < WL; ++i) {
    const int r = pr + 32 * i;  // tile row: gate rows first, then up rows
    const int n = n0 + (PAIR ? r % BN : r);
    w_ok[i] = n < a.N;
    const size_t off = (size_t)((w_ok[i] ? n : 0) + (PAIR && r >= BN ? a.N : 0)) * a.K + pk;
    if constexpr (W8)
      w_src[i] = reinterpret_cast<const int8_t*>(a.W) + off;
    else
      w_src[i] = a.W + off;
  }

  u32x4 av[AL], wv[WL];
  auto load = [&](int k0) {
#pragma unroll
    for (int i = 0; i < AL; ++i) av[i] = a_ok[i] ? load16(a_src[i] + k0) : zero;
#pragma unroll
    for (int i = 0; i < WL; ++i) {
      if constexpr (W8)
        wv[i] = w_ok[i] ? load_stream_i8_bf16(static_cast<const int8_t*>(w_src[i]) + k0) : zero;
      else
        wv[i] = w_ok[i] ? load_stream16(static_cast<const uint16_t*>(w_src[i]) + k0) : zero;
    }
  };
  auto store = [&](int b) {
#pragma unroll
    for (int i = 0; i < AL; ++i) *reinterpret_cast<u32x4*>(&As[b][pr + 32 * i][pk]) = av[i];
#pragma unroll
    for (int i = 0; i < WL; ++i) *reinterpret_cast<u32x4*>(&Ws[b][pr + 32 * i][pk]) = wv[i];
  };

  f32x4 acc[MB][NB], accu[PAIR ? MB : 1][PAIR ? NB : 1];
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
      if constexpr (PAIR) accu[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

  if (kt0 < kt1) {  // always true: split_parts leaves no part empty
    load(kt0 * kBK);
    store(0);
    __syncthreads();
  }
  for (int kt = kt0; kt < kt1; ++kt) {
    const int b = (kt - kt0) & 1;
    if (kt + 1 < kt1) load((kt + 1) * kBK);
#pragma unroll
    for (int ks = 0; ks < kBK; ks += 32) {
      bf16x8 af[MB], bf[NB], uf[PAIR ? NB : 1];
#pragma unroll
      for (int i = 0; i < MB; ++i) af[i] = *reinterpret_cast<const bf16x8*>(&As[b][wm + 16 * i + fr][ks + fk]);
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        bf[j] = *reinterpret_cast<const bf16x8*>(&Ws[b][wn + 16 * j + fr][ks + fk]);
        if constexpr (PAIR) uf[j] = *reinterpret_cast<const bf16x8*>(&Ws[b][BN + wn + 16 * j + fr][ks + fk]);
      }
#pragma unroll
      for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j) {
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bf[j], acc[i][j], 0, 0, 0);
          if constexpr (PAIR)
            accu[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], uf[j], accu[i][j], 0, 0, 0);
        }
    }
    if (kt + 1 < kt1) store(b ^ 1);
    __syncthreads();
  }

  // D layout: lane holds rows 4 (lane / 16) + r, column lane % 16 of each block
  if constexpr (SPLIT) {
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
      for (int j = 0; j < NB; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = m0 + wm + 16 * i + (lane >> 4) * 4 + r;
          const int n = n0 + wn + 16 * j + fr;
          if (m >= a.M || n >= a.N) continue;
          const int outs = PAIR ? 2 * a.N : a.N;
          float* part = a.split_ws + ((size_t)blockIdx.y * a.M + m) * outs;
          part[n] = acc[i][j][r];
          if constexpr (PAIR) part[a.N + n] = accu[i][j][r];
        }
    return;
  }
  static_assert(BM * (BN + 8) <= 2 * BM * kBRow, "the tile fits the A buffers");
  tile_epilogue<BM, BN, PAIR, W8, MB, NB>(a, acc, accu, &As[0][0][0], m0, n0, wm, wn, tid, lane);
}

// Large-M GEMM, bf16 weights, with a ring of NS LDS stages of RK (32 or 64)
// K each filled by buffer -> LDS loads (16 bytes per lane, 1 KiB per
// instruction): the workgroup keeps NS - 1 stages of loads in flight while
// it multiplies one, where gemm_big_kernel's register staging keeps one.
// Tiles, waves and epilogue as gemm_big_kernel (128 tokens x BN outputs,
// 2 x 2 waves).  A stage row is RK bf16 = RK / 8 16-byte pieces; piece c of
// tile row r sits at position c ^ ring_key<RK>(r), so that a fragment read
// (16 rows, one piece) touches distinct banks in every group of 8 lanes
// (128 bytes) and of 16 lanes (256 bytes).  Every load goes through a buffer
// resource: rows past M (tokens) or N (outputs) read zero.  Load i of wave w
// covers A rows RPL (w AI + i) .. and weight rows RPL (w WI + i) .. (RPL =
// 512 / RK rows per load); each wave waits for its own loads of a stage, the
// barrier after that for everyone's.
constexpr int kRK = 32;  // K per ring stage of the SwiGLU pair and of the narrower tiles

// The ring's piece position key of tile row r (only r % 16 matters).  32-deep
// stages (four pieces per 64-byte row): 0 0 1 1 2 2 3 3 1 1 0 0 3 3 2 2, so
// rows r and r + 2 (the same 128-byte bank window) get different keys, and
// so do rows r and r + 4, r + 8, r + 12 (the same 256-byte window).  64-deep
// stages (eight pieces per 128-byte row): (r mod 8) ^ (r / 8 mod 2), so rows
// r .. r + 7 (one row per 128-byte window) get eight keys, and so do the
// eight rows of each parity among 16 (the 256-byte window holds two rows).
__device__ __forceinline__ int ring_swizzle(int r) { return ((r >> 1) & 3) ^ ((r >> 3) & 1); }
template <int RK>
__device__ __forceinline__ int ring_key(int r) {
  static_assert(RK == 32 || RK == 64, "32- or 64-deep stages");
  return RK == 32 ? ring_swizzle(r) : (r & 7) ^ ((r >> 3) & 1);
}

// 16 bytes from LDS, issued as assembly: the caller waits (lgkmcnt) before
// it uses the value, then passes it through lds_ready.  (The VGPR operand
// constraints exist in the device pass only.)
__device__ __forceinline__ bf16x8 lds_read16(const uint16_t* p) {
  bf16x8 v;
#if __HIP_DEVICE_COMPILE__
  const unsigned addr = (unsigned)(uintptr_t)(const __attribute__((address_space(3))) uint16_t*)p;
  asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(addr) : "memory");
#endif
  return v;
}

// n buffer -> LDS loads of 16 bytes per lane: load i of the wave fills the
// 1 KiB at dst + 512 i (elements) from byte offsets off[i] + kb of r.  (A
// device function: in a lambda the LDS address-space cast would be checked
// for the host too.)
template <int n>
__device__ __forceinline__ void ring_loads(__amdgpu_buffer_rsrc_t r, uint16_t* dst, const unsigned* off,
                                           unsigned kb) {
#pragma unroll
  for (int i = 0; i < n; ++i)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)(dst + 512 * i), 16,
                                             off[i] + kb, 0, 0, 0);
}

// A value of lds_read16 as used after the wait that follows the reads: an
// empty statement after that wait, which the uses depend on.
__device__ __forceinline__ void lds_ready(bf16x8& v) {
#if __HIP_DEVICE_COMPILE__
  asm volatile("" : "+v"(v));
#endif
}

template <int BN, bool PAIR, int NS, int RK = kRK>
__global__ __launch_bounds__(kThreads, PAIR && BN == 128 ? 2 : 1) void gemm_ring_kernel(PrefillGemmArgs a) {
  constexpr int BM = kBM;
  constexpr int WR = PAIR ? 2 * BN : BN;  // weight rows per tile
  constexpr int MB = BM / 64, NB = BN / 64;  // MFMA 32 x 32 blocks per wave (64 x BN / 2 outputs)
  constexpr int SA = BM * RK, SW = WR * RK;  // bf16 per stage
  constexpr int RPL = 512 / RK, PPR = RK / 8;  // rows per load, pieces per row
  constexpr int AI = BM / RPL / (kThreads / 64), WI = WR / RPL / (kThreads / 64);
  constexpr int NH = RK / 16;  // 16-deep MFMA steps per stage
  constexpr int PER = AI + WI;  // loads per wave per stage
  static_assert(AI >= 1 && WI >= 1 && NS >= 3 && (NS - 2) * (AI + WI) < 64, "ring shape");
  static_assert(BM * (BN + 8) <= NS * (SA + SW), "the epilogue tile fits the ring");
  __shared__ __attribute__((aligned(16))) uint16_t ring[NS][SA + SW];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int mt = (a.M + BM - 1) / BM, ntile = (a.N + BN - 1) / BN;
  // tile order as gemm_big_kernel (each XCD a contiguous run, grouped so the
  // tiles an XCD holds at once share token and weight tiles)
  const int per = (mt * ntile + 7) / 8;
  const int t = (int)(blockIdx.x % 8) * per + (int)(blockIdx.x / 8);
  if (t >= mt * ntile) return;
  const int GN = ntile <= 12 ? ntile : 4;
  const int grp = t / (GN * mt), gn = min(GN, ntile - grp * GN), in = t - grp * GN * mt;
  const int m0 = (in / gn) * BM;
  const int n0 = (grp * GN + in % gn) * BN;
  const int wm = (wave >> 1) * (BM / 2), wn = (wave & 1) * (BN / 2);
  const int fr = lane & 31;
  const int steps = a.K / RK;

  const __amdgpu_buffer_rsrc_t ra = rsrc(a.A, a.M * a.lda * 2);
  const __amdgpu_buffer_rsrc_t rw = rsrc(a.W, (PAIR ? 2 : 1) * a.N * a.K * 2);
  // this lane's row within an RPL-row load block and the global piece it
  // fetches into its LDS position lane % PPR
  const int lr = lane / PPR, lp = lane % PPR;
  unsigned aoff[AI], woff[WI];
#pragma unroll
  for (int i = 0; i < AI; ++i) {
    const int r = RPL * (wave * AI + i) + lr;  // tile row
    aoff[i] = (unsigned)(((m0 + r) * a.lda + 8 * (lp ^ ring_key<RK>(r))) * 2);
  }
#pragma unroll
  for (int i = 0; i < WI; ++i) {
    const int r = RPL * (wave * WI + i) + lr;  // tile row: gate rows first, then up rows
    const int row = PAIR ? (r < BN ? n0 + r : a.N + n0 + r - BN) : n0 + r;
    woff[i] = (unsigned)((row * a.K + 8 * (lp ^ ring_key<RK>(r))) * 2);
  }
  f32x16 acc[MB][NB], accu[PAIR ? MB : 1][PAIR ? NB : 1];
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        acc[i][j][r] = 0.f;
        if constexpr (PAIR) accu[i][j][r] = 0.f;
      }
#pragma unroll
  for (int st = 0; st < NS - 1; ++st)
    if (st < steps) {
      ring_loads<AI>(ra, &ring[st][512 * wave * AI], aoff, (unsigned)(st * RK * 2));
      ring_loads<WI>(rw, &ring[st][SA + 512 * wave * WI], woff, (unsigned)(st * RK * 2));
    }
  // MFMA 32 x 32 x 16: this lane's fragment piece in each 16-deep step h of
  // the stage (k 16 h + 8 (lane / 32) ..) at its swizzled position in rows of
  // its fragment (row & 15 = lane & 15)
  int pos[NH];
#pragma unroll
  for (int h = 0; h < NH; ++h) pos[h] = ((2 * h + (lane >> 5)) ^ ring_key<RK>(lane & 15)) * 8;
  for (int k = 0; k < steps; ++k) {
    // stage k has landed once at most NS - 2 later stages are in flight
    if (k + NS - 2 < steps)
      __builtin_amdgcn_s_waitcnt(((NS - 2) * PER & 15) | ((((NS - 2) * PER) >> 4) << 14) | (7 << 4) | (15 << 8));
    else
      __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));  // vmcnt(0)
    // A barrier without a fence, and the fragment reads in assembly: the
    // compiler would otherwise wait for every buffer -> LDS load in flight
    // (the later stages' too) before the barrier or before the first read.
    // The waits above and below are the ones these reads need.
    asm volatile("s_barrier" ::: "memory");
    // the buffer of stage k - 1 is free: every wave is past its products
    if (k + NS - 1 < steps) {
      const int st = k + NS - 1;
      ring_loads<AI>(ra, &ring[st % NS][512 * wave * AI], aoff, (unsigned)(st * RK * 2));
      ring_loads<WI>(rw, &ring[st % NS][SA + 512 * wave * WI], woff, (unsigned)(st * RK * 2));
    }
    const uint16_t* as = &ring[k % NS][0];
    const uint16_t* ws = as + SA;
    bf16x8 af[NH][MB], bf[NH][NB], uf[NH][PAIR ? NB : 1];
#pragma unroll
    for (int h = 0; h < NH; ++h) {
#pragma unroll
      for (int i = 0; i < MB; ++i) af[h][i] = lds_read16(as + (wm + 32 * i + fr) * RK + pos[h]);
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        bf[h][j] = lds_read16(ws + (wn + 32 * j + fr) * RK + pos[h]);
        if constexpr (PAIR) uf[h][j] = lds_read16(ws + (BN + wn + 32 * j + fr) * RK + pos[h]);
      }
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    // (the products take the fragments from here on: after the wait)
#pragma unroll
    for (int h = 0; h < NH; ++h) {
#pragma unroll
      for (int i = 0; i < MB; ++i) lds_ready(af[h][i]);
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        lds_ready(bf[h][j]);
        if constexpr (PAIR) lds_ready(uf[h][j]);
      }
    }
#pragma unroll
    for (int h = 0; h < NH; ++h)
#pragma unroll
      for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j) {
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[h][i], bf[h][j], acc[i][j], 0, 0, 0);
          if constexpr (PAIR)
            accu[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[h][i], uf[h][j], accu[i][j], 0, 0, 0);
        }
  }
  __syncthreads();  // the ring becomes the epilogue's tile
  tile_epilogue<BM, BN, PAIR, false, MB, NB, 32>(a, acc, accu, &ring[0][0], m0, n0, wm, wn, tid, lane);
}

// ---- slab GEMM: prompts of at most 64 tokens ----
// One workgroup of 16 waves per slab of 16 outputs (and, for SwiGLU, the
// matching up rows), over all of K: wave w takes K steps w, w + 16, ... (32
// deep each) and the waves' sums are added in LDS in wave order, so there is
// no workspace and no second pass, and every run gives the same result.  A
// wave issues the weight and token loads of two steps before it waits for
// any, and loads the next two while it multiplies (the weights are read once
// from HBM, the token rows come from L2).  Every load goes through a buffer
// resource, and a load that falls outside (a step the wave does not own, a
// token or output row past the end) takes an offset past the resource and
// reads zero: no branch around a load, so the compiler's wait counts stay
// exact and the next batch stays in flight.  With RMSNorm gains the token
// rows are normalised as they arrive: every lane adds the squares of its
// fragments, the waves add theirs in LDS (every step belongs to exactly one
// wave, so the sums cover each row once) and the fragments are scaled in
// registers before their products; K is then at most 32 steps, one batch.
// MFMA 16x16x32: A = 16 tokens x 32 k, B = 32 k x 16 outputs; lane L holds
// token / output L % 16 and k 8 (L / 16) .. + 7 of each operand and, after
// the product, tokens 4 (L / 16) .. + 3 of output L % 16.
constexpr int kSlabBlocks = kSlabMaxTokens / 16;  // 16-token blocks at most
constexpr int kSlabBatch = 2;                     // K steps per wave in flight together
constexpr int kSlabLongWaves = 8;                 // waves of a long-K workgroup
constexpr int kSlabWPre = 20;                     // its weight steps per wave requested at once
constexpr unsigned kSlabOutside = 0x7ffffff0u;    // a byte offset past every resource

// QKV rows of slab s and lane row r (0..15) when the QKV GEMM applies RoPE
// itself: slab s covers rows 8 (s % 4) .. + 7 and 32 + 8 (s % 4) .. + 7 of
// head s / 4, so each RoPE pair (j, j + 32) of a head sits in one workgroup,
// eight lanes apart.
__device__ __forceinline__ int rope_row(int s, int r) {
  return (s >> 2) * kHeadDim + 8 * (s & 3) + (r & 7) + (r >= 8 ? kHeadDim / 2 : 0);
}

// The plain epilogues of a slab GEMM output (m, n): bf16, bias or residual
// (k-blocked outputs and residuals: element (m, n) at ((n / 8) M + m) 8 + n % 8).
__device__ __forceinline__ void slab_store(const PrefillGemmArgs& a, int m, int n, float x) {
  const size_t yo = a.kblock == 2 ? ((size_t)(n >> 3) * a.M + m) * 8 + (n & 7) : (size_t)m * a.ldy + n;
  const size_t ro = a.kblock == 2 ? yo : (size_t)m * a.ldr + n;
  uint16_t* y = a.Y + yo;
  switch (a.epi) {
    case EPI_BF16:
      *y = (uint16_t)f32_to_bf16(x);
      break;
    case EPI_BIAS:
      *y = (uint16_t)f32_to_bf16(round_bf16(x) + a.bias[n]);
      break;
    case EPI_RESID:
      *y = (uint16_t)f32_to_bf16(round_bf16(x) + bf16_to_f32(a.resid[ro]));
      break;
    default:
      break;
  }
}

// The K-split slab's end: each thread sums its outputs over the waves (wave
// order); parts 1.. store them as tagged words in the XCD's L2 and are done;
// part 0 polls those words (loads that miss the CU's L1 and read the L2),
// adds the parts in order, scales (W8) and stores.  A tagged 64-bit word is
// seen whole or not at all, so no flag or fence is needed; a wait gives up
// after slab_spin polls and reports it.
template <bool W8, int KS, int WAVES, int NB>
__device__ void split_epilogue(const PrefillGemmArgs& a, const f32x4 (&red)[WAVES][NB][64], int slab, int part,
                               int mb) {
  constexpr int kLocalPol = 3;  // sc0 | nt: miss L1, read the XCD's L2
  constexpr int E = (NB * 256 + WAVES * 64 - 1) / (WAVES * 64);  // outputs per thread
  const int tid = threadIdx.x;
  const int M = a.M, N = a.N, ns = 16 * slab;
  const __amdgpu_buffer_rsrc_t ws = rsrc(a.slab_ws, ((N + 15) / 16) * KS * kSlabMaxTokens * 16 * 8);
  const unsigned base = (unsigned)slab * KS * kSlabMaxTokens * 16;
  float xv[E];
  int mv[E], nv[E];
  bool ok[E];
#pragma unroll
  for (int i = 0; i < E; ++i) {
    const int f = tid + i * WAVES * 64;
    const int b = f >> 8, l = (f >> 2) & 63, r = f & 3;
    mv[i] = 16 * b + 4 * (l >> 4) + r;
    nv[i] = ns + (l & 15);
    ok[i] = f < mb * 256 && mv[i] < M && nv[i] < N;
    float x = 0.0f;
    if (ok[i]) {
#pragma unroll
      for (int w = 0; w < WAVES; ++w) x += red[w][b][l][r];
    }
    xv[i] = x;
  }
  auto word = [&](int q, int i) { return (base + (unsigned)(q * kSlabMaxTokens + mv[i]) * 16u + (nv[i] & 15)) * 8u; };
  if (part != 0) {
#pragma unroll
    for (int i = 0; i < E; ++i)
      if (ok[i])
        __builtin_amdgcn_raw_buffer_store_b64(u32x2_t{__float_as_uint(xv[i]), a.slab_tag}, ws, word(part, i), 0, 0);
    return;
  }
  float pv[E][KS - 1];
  for (unsigned spins = 1;; ++spins) {
    bool have = true;
#pragma unroll
    for (int i = 0; i < E; ++i)
#pragma unroll
      for (int q = 1; q < KS; ++q) {
        const u32x2_t v = __builtin_bit_cast(
            u32x2_t, __builtin_amdgcn_raw_buffer_load_b64(ws, ok[i] ? word(q, i) : kSlabOutside, 0, kLocalPol));
        pv[i][q - 1] = __uint_as_float(v.x);
        have = have && (!ok[i] || v.y == a.slab_tag);
      }
    if (have) break;
    if (spins > a.slab_spin) {
      __hip_atomic_store(a.slab_error, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
#pragma unroll
  for (int i = 0; i < E; ++i) {
    if (!ok[i]) continue;
    float x = xv[i];
#pragma unroll
    for (int q = 0; q < KS - 1; ++q) x += pv[i][q];
    if constexpr (W8) x *= a.scale[nv[i]];
    slab_store(a, mv[i], nv[i], x);
  }
}

// One batch of a wave's K steps: weight fragments (raw int8 for W8, widened
// just before the product) and the token fragments of every block.
template <bool PAIR, bool W8, int B, int NB>
struct SlabBatch {
  using WRaw = typename std::conditional<W8, u32x2_t, u32x4>::type;
  WRaw w[B], u[PAIR ? B : 1];
  u32x4 x[B][NB];
};

// WAVES 16 for K up to 16 batches of steps; WAVES kSlabLongWaves for longer
// K (non-normalised A): each wave then requests the weights of up to
// kSlabWPre of its steps at once (one HBM latency for all of them) and
// streams the token fragments two steps at a time, double buffered.  NB: the
// prompt's 16-token blocks (a 40-token prompt takes three: a quarter fewer
// token loads, products and LDS sums than the four a 64-token prompt needs).
// TWO (gate/up with more slabs than CUs): a workgroup may take a second slab.
// KS > 1 (slab_ws): K split KS ways over workgroups of one XCD, the parts'
// partial sums added by part 0 in part order (PrefillGemmArgs::slab_ws).
template <bool PAIR, bool NORM, bool W8, int WAVES, int NB = kSlabBlocks, bool TWO = false, int KS = 1>
__global__ __launch_bounds__(WAVES * 64) void gemm_slab_kernel(PrefillGemmArgs a) {
  static_assert(!TWO || (PAIR && NORM), "second slabs for gate/up with the norm");
  static_assert(KS == 1 || (!PAIR && !NORM && !TWO), "the K split is for plain slabs");
  constexpr int kSlabWaves = WAVES;
  constexpr int P = PAIR ? 2 : 1;
  constexpr int EB = W8 ? 1 : 2;  // bytes per weight
  // SwiGLU pairs without the norm keep one step per batch (two batches of
  // two would not fit the registers of 16 waves)
  constexpr int B = PAIR && !NORM ? 1 : kSlabBatch;
  using Batch = SlabBatch<PAIR, W8, B, NB>;
  __shared__ f32x4 red[kSlabWaves][P * NB][64];
  __shared__ float ssq[NORM ? kSlabWaves : 1][kSlabMaxTokens];
  __shared__ float inv_s[kSlabMaxTokens];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  // this workgroup's slab and K part: the KS parts of slab s are workgroups
  // s % 8 + 8 (KS (s / 8) + q), q = 0..KS-1, all on XCD s % 8
  int slab = blockIdx.x, part = 0;
  if constexpr (KS > 1) {
    const int xcd = blockIdx.x % 8, r = blockIdx.x / 8;
    part = r % KS;
    slab = xcd + 8 * (r / KS);
    unsigned xcc;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    if ((xcc & 15u) != (unsigned)xcd) {  // the parts would not share an L2: report, leave
      if (tid == 0) __hip_atomic_store(a.slab_error, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return;
    }
    if (slab * 16 >= a.N) return;
  }
  const int n0 = slab * 16;
  const int M = a.M, N = a.N, K = a.K;
  const int mb = (M + 15) / 16;
  const int fr = lane & 15, fk = (lane >> 4) * 8;
  // this part's K steps (of 32 columns): [st0, st0 + steps)
  const int sp = (K / 32 + KS - 1) / KS, st0 = part * sp;
  const int steps = KS > 1 ? max(0, min(K / 32, st0 + sp) - st0) : K / 32;
  const int mine = steps > wave ? (steps - wave + kSlabWaves - 1) / kSlabWaves : 0;  // this wave's steps
  // byte offsets of this lane's weight row (and up row) and token rows at k
  // = fk; kSlabOutside for a row past the end
  const int wrow = a.rope.on ? rope_row(slab, fr) : n0 + fr;
  // weight piece (8 weights) of row n at k group g: row-major, or in the
  // MFMA-native copy Wn ([N/16][K/8][16] pieces: a fragment's 16 rows are one
  // run); wkm: bytes from column k to column k + 1 along a row
  const bool native = a.Wn != nullptr;
  const unsigned pb = 8u * EB;  // bytes per piece
  auto wpiece = [&](int n) -> unsigned {
    return native ? (unsigned)((((n >> 4) * (K >> 3) + (fk >> 3)) * 16 + (n & 15))) * pb : (unsigned)(n * K + fk) * EB;
  };
  const unsigned wkm = native ? 2u * pb : (unsigned)EB;
  // the copy holds each slab's rows in fragment order (RoPE's permutation too)
  const int nrow = native ? n0 + fr : wrow;
  const unsigned wofs = wrow < N ? wpiece(nrow) : kSlabOutside;
  const unsigned uofs = wrow < N ? wpiece(nrow + N) : kSlabOutside;
  unsigned aofs[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const int t = 16 * b + fr;
    aofs[b] = t >= M ? kSlabOutside
              : a.kblock ? (unsigned)(((fk >> 3) * M + t) * 16) : (unsigned)(t * a.lda + fk) * 2u;
  }
  // bytes from column k to column k + 1 of a token row (k a multiple of 8)
  const unsigned akm = a.kblock ? 2u * (unsigned)M : 2u;
  const __amdgpu_buffer_rsrc_t wr = rsrc(native ? a.Wn : a.W, P * N * K * EB);
  const __amdgpu_buffer_rsrc_t ar = rsrc(a.A, a.kblock ? M * K * 2 : ((M - 1) * a.lda + K) * 2);

  // loads of the batch starting at this wave's step index j0 (nontemporal
  // weights: each is read once)
  auto load = [&](Batch& bt, int j0) {
#pragma unroll
    for (int i = 0; i < B; ++i) {
      const int j = j0 + i;
      const unsigned k0 = (unsigned)(32 * (st0 + wave + kSlabWaves * j));
      const bool live = j < mine;
      const unsigned wo = live ? wofs + k0 * wkm : kSlabOutside;
      const unsigned uo = live ? uofs + k0 * wkm : kSlabOutside;
      if constexpr (W8) {
        bt.w[i] = __builtin_bit_cast(u32x2_t, __builtin_amdgcn_raw_buffer_load_b64(wr, wo, 0, 2));
        if constexpr (PAIR) bt.u[i] = __builtin_bit_cast(u32x2_t, __builtin_amdgcn_raw_buffer_load_b64(wr, uo, 0, 2));
      } else {
        bt.w[i] = __builtin_amdgcn_raw_buffer_load_b128(wr, wo, 0, 2);
        if constexpr (PAIR) bt.u[i] = __builtin_amdgcn_raw_buffer_load_b128(wr, uo, 0, 2);
      }
#pragma unroll
      for (int b = 0; b < NB; ++b)
        bt.x[i][b] = __builtin_amdgcn_raw_buffer_load_b128(ar, live ? aofs[b] + akm * k0 : kSlabOutside, 0, 0);
    }
  };
  auto widen = [&](const typename Batch::WRaw& r) -> bf16x8 {
    if constexpr (W8)
      return __builtin_bit_cast(bf16x8, (u32x4{i8pair_bf16(r.x, 0), i8pair_bf16(r.x, 2), i8pair_bf16(r.y, 0),
                                              i8pair_bf16(r.y, 2)}));
    else
      return __builtin_bit_cast(bf16x8, r);
  };

  f32x4 acc[NB], accu[PAIR ? NB : 1];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    acc[b] = f32x4{0.f, 0.f, 0.f, 0.f};
    if constexpr (PAIR) accu[b] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  auto multiply = [&](const Batch& bt) {
#pragma unroll
    for (int i = 0; i < B; ++i) {
      const bf16x8 w = widen(bt.w[i]);
      const bf16x8 wu = PAIR ? widen(bt.u[i]) : w;
#pragma unroll
      for (int b = 0; b < NB; ++b) {  // blocks past the last token hold zeros
        const bf16x8 xa = __builtin_bit_cast(bf16x8, bt.x[i][b]);
        acc[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa, w, acc[b], 0, 0, 0);
        if constexpr (PAIR) accu[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa, wu, accu[b], 0, 0, 0);
      }
    }
  };

  // SwiGLU with the norm and more slabs than workgroups (gate/up): workgroup
  // b also takes slab s2 = b + gridDim.x when there is one.  Its weights are
  // requested with the first slab's and its products reuse the normalised
  // token fragments, so it costs no second start, token loads or norm; each
  // slab's arithmetic is that of a workgroup of its own.
  const int s2 = blockIdx.x + gridDim.x;
  const bool two = TWO && s2 * 16 < N;  // uniform
  Batch nbt;
  typename Batch::WRaw w2[TWO ? B : 1], u2[TWO ? B : 1];
  if constexpr (NORM) {
    // one batch holds every step of the wave (the host keeps K <= 32 steps)
    Batch& bt = nbt;
    load(bt, 0);
    if constexpr (TWO) {
      const unsigned wofs2 = two ? wpiece(s2 * 16 + fr) : kSlabOutside;
      const unsigned uofs2 = two ? wpiece(s2 * 16 + fr + N) : kSlabOutside;
#pragma unroll
      for (int i = 0; i < B; ++i) {
        const unsigned k0 = (unsigned)(32 * (st0 + wave + kSlabWaves * i));
        const bool live = two && i < mine;
        const unsigned wo = live ? wofs2 + k0 * wkm : kSlabOutside, uo = live ? uofs2 + k0 * wkm : kSlabOutside;
        if constexpr (W8) {
          w2[i] = __builtin_bit_cast(u32x2_t, __builtin_amdgcn_raw_buffer_load_b64(wr, wo, 0, 2));
          u2[i] = __builtin_bit_cast(u32x2_t, __builtin_amdgcn_raw_buffer_load_b64(wr, uo, 0, 2));
        } else {
          w2[i] = __builtin_amdgcn_raw_buffer_load_b128(wr, wo, 0, 2);
          u2[i] = __builtin_amdgcn_raw_buffer_load_b128(wr, uo, 0, 2);
        }
      }
    }
    u32x4 g[B];
    const __amdgpu_buffer_rsrc_t gr = rsrc(a.gamma, K * 2);
#pragma unroll
    for (int i = 0; i < B; ++i)
      g[i] = __builtin_amdgcn_raw_buffer_load_b128(
          gr, i < mine ? (unsigned)(32 * (st0 + wave + kSlabWaves * i) + fk) * 2u : kSlabOutside, 0, 0);
    // squares of this lane's fragments, per token row; the four lanes of a
    // row hold its four 8-wide k groups
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      float sq = 0.0f;
#pragma unroll
      for (int i = 0; i < B; ++i) sq += sq8(bt.x[i][b]);
      sq += __shfl_xor(sq, 16, 64);
      sq += __shfl_xor(sq, 32, 64);
      if (lane < 16) ssq[wave][16 * b + fr] = sq;
    }
    __syncthreads();
    if (tid < kSlabMaxTokens) {
      float ss = 0.0f;
#pragma unroll
      for (int w = 0; w < kSlabWaves; ++w) ss += ssq[w][tid];
      inv_s[tid] = tid < M ? 1.0f / sqrtf(ss / (float)K + a.eps) : 0.0f;
    }
    __syncthreads();
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const float inv = inv_s[16 * b + fr];
#pragma unroll
      for (int i = 0; i < B; ++i) bt.x[i][b] = norm8(bt.x[i][b], inv, g[i]);
    }
    multiply(bt);
  } else if (steps <= kSlabWaves * B) {
    // every step of the wave in one batch
    Batch bt;
    load(bt, 0);
    multiply(bt);
  } else if constexpr (!PAIR && WAVES != kSlabLongWaves) {
    // (long K runs on kSlabLongWaves waves; this form stays correct for any K)
    for (int j = 0; j < mine; j += B) {
      Batch bt;
      load(bt, j);
      multiply(bt);
    }
  } else if constexpr (PAIR) {
    // two batches in flight: the next one loads while this one multiplies
    // (unconditionally: steps past the wave's last read zero and add zero;
    // sched_barrier keeps the next batch's loads ahead of the products)
    Batch b0, b1;
    load(b0, 0);
    for (int j = 0; j < mine; j += 2 * B) {
      load(b1, j + B);
      __builtin_amdgcn_sched_barrier(0);
      multiply(b0);
      load(b0, j + 2 * B);
      __builtin_amdgcn_sched_barrier(0);
      multiply(b1);
    }
  } else {
    // long K: the weights of kSlabWPre steps at once, token fragments two
    // steps at a time in two buffers (sched_barrier keeps the next buffer's
    // loads ahead of this one's products; steps past the wave's last read
    // zero and add zero)
    using WRaw = typename Batch::WRaw;
    for (int g0 = 0; g0 < mine; g0 += kSlabWPre) {
      WRaw wv[kSlabWPre];
#pragma unroll
      for (int i = 0; i < kSlabWPre; ++i) {
        const int j = g0 + i;
        const unsigned k0 = (unsigned)(32 * (st0 + wave + kSlabWaves * j));
        const unsigned wo = j < mine ? wofs + k0 * wkm : kSlabOutside;
        if constexpr (W8)
          wv[i] = __builtin_bit_cast(u32x2_t, __builtin_amdgcn_raw_buffer_load_b64(wr, wo, 0, 2));
        else
          wv[i] = __builtin_amdgcn_raw_buffer_load_b128(wr, wo, 0, 2);
      }
      u32x4 x0[2][NB], x1[2][NB];
      auto load_x = [&](u32x4 (&x)[2][NB], int j0) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const int j = j0 + i;
          const unsigned k0 = (unsigned)(32 * (st0 + wave + kSlabWaves * j));
#pragma unroll
          for (int b = 0; b < NB; ++b)
            x[i][b] = __builtin_amdgcn_raw_buffer_load_b128(ar, j < mine ? aofs[b] + akm * k0 : kSlabOutside, 0, 0);
        }
      };
      auto mul_x = [&](const u32x4 (&x)[2][NB], int i0) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const bf16x8 w = widen(wv[i0 + i]);
#pragma unroll
          for (int b = 0; b < NB; ++b)
            acc[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, x[i][b]), w, acc[b], 0, 0, 0);
        }
      };
      load_x(x0, g0);
      // (the rounds stop at the wave's last step: a round past it would
      // still wait for its loads, which read zero)
#pragma unroll
      for (int i = 0; i < kSlabWPre; i += 4) {
        if (g0 + i >= mine) break;
        load_x(x1, g0 + i + 2);
        __builtin_amdgcn_sched_barrier(0);
        mul_x(x0, i);
        if (i + 4 < kSlabWPre) load_x(x0, g0 + i + 4);
        __builtin_amdgcn_sched_barrier(0);
        mul_x(x1, i + 2);
      }
    }
  }

  for (int pass = 0; pass < 2; ++pass) {
    const int s = pass ? s2 : slab, ns = 16 * s;
    if (pass) {
      if (!two) break;
      __syncthreads();  // the first slab's sums have been read
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        acc[b] = f32x4{0.f, 0.f, 0.f, 0.f};
        if constexpr (PAIR) accu[b] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
      if constexpr (TWO) {
#pragma unroll
        for (int i = 0; i < B; ++i) {
          const bf16x8 w = widen(w2[i]), wu = widen(u2[i]);
#pragma unroll
          for (int b = 0; b < NB; ++b) {
            const bf16x8 xa = __builtin_bit_cast(bf16x8, nbt.x[i][b]);
            acc[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa, w, acc[b], 0, 0, 0);
            accu[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa, wu, accu[b], 0, 0, 0);
          }
        }
      }
    }
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      red[wave][b][lane] = acc[b];
      if constexpr (PAIR) red[wave][NB + b][lane] = accu[b];
    }
    __syncthreads();

    // values f = t, t + 64 WAVES, ... of [mb][64 lanes][4 rows] on thread t,
    // each summed over the waves in wave order, then the epilogue (the
    // rounding points of the other GEMM kernels)
    if constexpr (KS > 1) {
      split_epilogue<W8, KS, WAVES, NB>(a, red, slab, part, mb);
      return;
    }
    for (int f = tid; f < mb * 256; f += kSlabWaves * 64) {
      const int b = f >> 8, l = (f >> 2) & 63, r = f & 3;
      const int m = 16 * b + 4 * (l >> 4) + r, n = a.rope.on ? rope_row(s, l & 15) : ns + (l & 15);
      if (m >= M || n >= N) continue;
      float x = 0.0f, u = 0.0f;
  #pragma unroll
      for (int w = 0; w < kSlabWaves; ++w) {
        x += red[w][b][l][r];
        if constexpr (PAIR) u += red[w][NB + b][l][r];
      }
      if constexpr (W8) {
        x *= a.scale[n];
        if constexpr (PAIR) u *= a.scale[N + n];
      }
      if (a.rope.on) {
        // QKV with RoPE and the KV append (the rope_append_kernel arithmetic):
        // the pair partner of row n is lane l ^ 8 of the same token
        const int lp = l ^ 8, np = rope_row(s, lp & 15);
        float xp = 0.0f;
  #pragma unroll
        for (int w = 0; w < kSlabWaves; ++w) xp += red[w][b][lp][r];
        if constexpr (W8) xp *= a.scale[np];
        const float v = a.bias ? round_bf16(round_bf16(x) + a.bias[n]) : round_bf16(x);
        const float vp = a.bias ? round_bf16(round_bf16(xp) + a.bias[np]) : round_bf16(xp);
        const int hd = n / kHeadDim, j = n % kHeadDim, p = a.rope.start + m;
        const auto& at = a.rope;
        if (hd < at.q_heads + at.kv_heads) {
          const int jj = j & (kHeadDim / 2 - 1);
          const float c = at.cos_tab[(size_t)p * (kHeadDim / 2) + jj], sn = at.sin_tab[(size_t)p * (kHeadDim / 2) + jj];
          // first half: x1 c - x2 s; second half: x2 c + x1 s (x1 the first-half value)
          const uint16_t rot = (uint16_t)(j < kHeadDim / 2 ? f32_to_bf16(v * c - vp * sn) : f32_to_bf16(v * c + vp * sn));
          if (hd < at.q_heads)
            at.qrot[(size_t)m * at.q_heads * kHeadDim + (size_t)hd * kHeadDim + j] = rot;
          else
            at.kcache[((size_t)(hd - at.q_heads) * at.max_ctx + p) * kHeadDim + j] = rot;
        } else {
          at.vcache[((size_t)(hd - at.q_heads - at.kv_heads) * at.max_ctx + p) * kHeadDim + j] = (uint16_t)f32_to_bf16(v);
        }
        continue;
      }
      // (k-blocked outputs and residuals: element (m, n) at ((n / 8) M + m) 8 + n % 8)
      const size_t yo = a.kblock == 2 ? ((size_t)(n >> 3) * M + m) * 8 + (n & 7) : (size_t)m * a.ldy + n;
      const size_t ro = a.kblock == 2 ? yo : (size_t)m * a.ldr + n;
      uint16_t* y = a.Y + yo;
      switch (a.epi) {
        case EPI_BF16:
          *y = (uint16_t)f32_to_bf16(x);
          break;
        case EPI_BIAS:
          *y = (uint16_t)f32_to_bf16(round_bf16(x) + a.bias[n]);
          break;
        case EPI_RESID:
          *y = (uint16_t)f32_to_bf16(round_bf16(x) + bf16_to_f32(a.resid[ro]));
          break;
        case EPI_SWIGLU:
          if constexpr (PAIR) *y = (uint16_t)f32_to_bf16(silu_mul(round_bf16(x), round_bf16(u)));
          break;
        default:
          break;
      }
    }
  }
}

// Sum of the split-K partial sums of output (m, n) in slice order, then the
// epilogue of the GEMM (the same rounding points as gemm_big_kernel's).
__global__ __launch_bounds__(kThreads) void split_reduce_kernel(PrefillGemmArgs a, int parts) {
  const int e = blockIdx.x * kThreads + threadIdx.x;
  if (e >= a.M * a.N) return;
  const int m = e / a.N, n = e % a.N;
  const bool pair = a.epi == EPI_SWIGLU;
  const int outs = pair ? 2 * a.N : a.N;
  float v = 0.0f, u = 0.0f;
  for (int s = 0; s < parts; ++s) {
    const float* part = a.split_ws + ((size_t)s * a.M + m) * outs;
    v += part[n];
    if (pair) u += part[a.N + n];
  }
  if (a.scale) {  // W8: the row scales, on the finished sums
    v *= a.scale[n];
    if (pair) u *= a.scale[a.N + n];
  }
  uint16_t* y = a.Y + (size_t)m * a.ldy + n;
  switch (a.epi) {
    case EPI_BF16:
      *y = (uint16_t)f32_to_bf16(v);
      break;
    case EPI_BIAS:
      *y = (uint16_t)f32_to_bf16(round_bf16(v) + a.bias[n]);
      break;
    case EPI_RESID:
      *y = (uint16_t)f32_to_bf16(round_bf16(v) + bf16_to_f32(a.resid[(size_t)m * a.ldr + n]));
      break;
    case EPI_SWIGLU:
      *y = (uint16_t)f32_to_bf16(silu_mul(round_bf16(v), round_bf16(u)));
      break;
    default:
      break;
  }
}

// Token rows per tile: 64 for prompts that fit one such tile, else kBM.
int split_bm(int M) { return M <= 64 ? 64 : kBM; }

// Tiles of the un-split GEMM (64-wide outputs).
int gemm_tiles(int M, int N) { return ((M + split_bm(M) - 1) / split_bm(M)) * ((N + 63) / 64); }

// K parts of the split path: enough that the tiles times the parts reach
// about kSplitTarget workgroups, every part holding ceil(nk / parts) steps
// or, the last, fewer but at least one.  1 means no split.
int split_parts(int M, int N, int K) {
  const int tiles = gemm_tiles(M, N), nk = K / kBK;
  const int want = std::max(1, std::min(nk, (kSplitTarget + tiles - 1) / tiles));
  const int per = (nk + want - 1) / want;
  return (nk + per - 1) / per;
}

// Causal GQA attention for a block of 64 query tokens (token i at slot
// p = start + i) of one query head, flash-style over the KV cache in blocks
// of 128 slots (slots 0..p of each token; cpu_backend.py:110-129):
//   S^T = K Q^T        v_mfma_f32_16x16x32_bf16: bf16 products are exact, f32 sums
//   online softmax     per token: running max m and sum l, P = exp(S / 8 - m)
//   O^T += V^T P^T     v_mfma_f32_16x16x32_bf16 three times, on P split
//                      into three bf16 terms that together are the float32
//                      P exactly (the reference's NumPy softmax), far below
//                      the cost of float32 MFMAs
// and out = bf16(O / l).  Computing S^T rather than S leaves lane L holding
// P[token L % 16][slots 16 sb + 4 (L / 16) + r], which serves directly as the
// B operand of P @ V once the MFMA's k index is read as the matching slot;
// V^T is staged in LDS so that the A values (4 consecutive slots of one
// dimension) are 8-byte reads.  A workgroup runs ST streams of four waves;
// stream s takes KV blocks s, s + ST, ... with its own K and V tiles, and
// wave w of each stream owns tokens 16 w .. 16 w + 15 of the block.  The
// streams' running (max, sum, O) are folded in stream order at the end, so
// a long query block's serial chain is 1 / ST of its blocks.
constexpr int kFaRows = 64;                 // query tokens per workgroup
constexpr int kFaSlots = 128;               // KV slots per block
// LDS row pitches (bf16): a K row 36 dwords, so the eight 16-byte fragment
// reads of one LDS pass (rows 4 banks apart) cover all 32 banks once; a V
// row 40 dwords, so the four rows of 32 bytes that a pass of transposed
// 8-byte reads touches lie 8 banks apart (at 36 dwords they overlapped in
// pairs of banks, and the V reads took two passes each)
constexpr int kFaKRow = kHeadDim + 8;
constexpr int kFaVRow = kHeadDim + 16;
constexpr int kFaStreams = 2;               // KV streams per workgroup for 128-slot blocks
// exp(s / 8 - m) = exp2(s * log2(e) / 8 - m'): the scores are kept in base-2
// units so that each exponential is one v_exp_f32
constexpr float kFaScale = 0.125f * 1.4426950408889634f;

// The maximum and the sum over lanes L, L ^ 16, L ^ 32, L ^ 48 (a token's
// four lane groups), the same value in each of the four: permlane32_swap of
// two copies leaves lanes L and L ^ 32 in the two results, permlane16_swap
// then lanes L and L ^ 16 (VALU lane swaps, where a shuffle goes through the
// LDS).  The sum is (v_L + v_L^32) + (v_L^16 + v_L^48) in every lane.
__device__ __forceinline__ float quad_max(float v) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  const float m = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(m), __float_as_uint(m), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

__device__ __forceinline__ float quad_sum(float v) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  const float s = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(s), __float_as_uint(s), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// KS: KV slots per block, kFaSlots, or 64 when the whole context fits 64
// slots (a short prompt from slot 0: half the products of a 128-slot block,
// whose second half is masked; the masked slots add exact zeros, so both
// forms give the same result).  With up to 128 VGPRs (four waves per SIMD
// for ST > 1, at least two for ST = 1) the compiler keeps the MFMA sums in
// VGPRs; in AGPRs every score and every rescale of O cost extra moves.
template <int KS, int ST>
__global__ __launch_bounds__(kThreads * ST, ST == 1 ? 2 : 4) void attention_prefill_kernel(PrefillAttnArgs a) {
  constexpr int kSB = KS / 16;  // 16-slot S^T blocks per KV block
  static_assert(KS == 64 || KS == kFaSlots, "64 or kFaSlots slots per block");
  static_assert(kThreads == 256, "a stream is four waves");
  __shared__ __attribute__((aligned(16))) uint16_t Ks[ST][KS][kFaKRow];  // [stream][slot][dim]
  __shared__ __attribute__((aligned(16))) uint16_t Vs[ST][KS][kFaVRow];  // [stream][slot][dim]
  // Tasks (head, query block) ranked longest first (rank r: block
  // nblk - 1 - r / q_heads of head r % q_heads), dealt to the workgroup ids
  // in a snake over runs of `period` ids (the CU count): the ids a CU
  // receives are about `period` apart, so each CU's long and short tasks
  // add up to about the same work.
  const int nblk = (a.n + kFaRows - 1) / kFaRows, tasks = nblk * a.q_heads;
  const int run = (int)blockIdx.x / a.period, pos = (int)blockIdx.x % a.period;
  const int run_len = min(a.period, tasks - run * a.period);
  const int rank = run * a.period + ((run & 1) ? run_len - 1 - pos : pos);
  const int h = rank % a.q_heads;
  const int qb = nblk - 1 - rank / a.q_heads;
  const int g = h / (a.q_heads / a.kv_heads);
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int stream = wave >> 2, sw = wave & 3, stid = tid & (kThreads - 1);
  const int col = lane & 15, quad = lane >> 4;
  const int tok = qb * kFaRows + sw * 16 + col;  // this lane's token
  const bool tok_ok = tok < a.n;
  const int p = a.start + (tok_ok ? tok : 0);
  const int last_slot = a.start + min(qb * kFaRows + kFaRows - 1, a.n - 1);
  const int nkv = last_slot / KS + 1;
  const int iters = (nkv + ST - 1) / ST;  // rounds of ST blocks
  const size_t kv_base = (size_t)g * a.max_ctx;
  const u32x4 zero = {0u, 0u, 0u, 0u};

  // B operand of S^T = K Q^T: Q[tok][32 kk + 8 quad .. + 8]
  bf16x8 qf[2];
  {
    const uint16_t* qrow = a.qrot + (size_t)(tok_ok ? tok : 0) * a.q_heads * kHeadDim + (size_t)h * kHeadDim + quad * 8;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) qf[kk] = __builtin_bit_cast(bf16x8, tok_ok ? load16(qrow + 32 * kk) : zero);
  }

  // tile loads through buffer resources that end at the block's last slot,
  // so later slots (and the blocks past the last of a stream's final round)
  // read as zero with no branch: load i of thread t of a stream takes slot
  // t / 8 + 32 i, dimensions 8 (t % 8) .. + 8, of K and of V (eight lanes per
  // 128-byte row, a wave's load one 1 KiB run; both stay [slot][dim] in LDS,
  // and the P @ V products read V transposed with ds_read_b64_tr_b16)
  const int ls = stid >> 3, ld0 = (stid & 7) * 8;
  const __amdgpu_buffer_rsrc_t kres = rsrc(a.kcache + kv_base * kHeadDim, (last_slot + 1) * kHeadDim * 2);
  const __amdgpu_buffer_rsrc_t vres = rsrc(a.vcache + kv_base * kHeadDim, (last_slot + 1) * kHeadDim * 2);
  constexpr int kLoads = KS / 32;  // loads per thread and matrix
  u32x4 kr[kLoads], vr[kLoads];
  auto load_tile = [&](int kb) {
    // (a block past the last has no slot: its offsets lie past the resources)
    const unsigned off = kb < nkv ? (unsigned)((kb * KS + ls) * kHeadDim + ld0) * 2u : 0x7ffffff0u;
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      kr[i] = __builtin_amdgcn_raw_buffer_load_b128(kres, off, 32 * kHeadDim * 2 * i, 0);
      vr[i] = __builtin_amdgcn_raw_buffer_load_b128(vres, off, 32 * kHeadDim * 2 * i, 0);
    }
  };

  float m_run = -INFINITY, l_run = 0.0f;
  f32x4 o[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) o[db] = f32x4{0.f, 0.f, 0.f, 0.f};
  load_tile(stream);
  for (int it = 0; it < iters; ++it) {
    const int kb = it * ST + stream;
    __syncthreads();  // the previous tiles have been read
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      *reinterpret_cast<u32x4*>(&Ks[stream][ls + 32 * i][ld0]) = kr[i];
      *reinterpret_cast<u32x4*>(&Vs[stream][ls + 32 * i][ld0]) = vr[i];
    }
    __syncthreads();
    if (it + 1 < iters) load_tile(kb + ST);  // in flight during this tile's math
    if (kb >= nkv) continue;  // this stream's final round holds no block (uniform per stream)

    // S^T blocks: lane holds slots s0 + 16 sb + 4 quad + r of token `tok`
    const int s0 = kb * KS;
    f32x4 sv[kSB];
#pragma unroll
    for (int sb = 0; sb < kSB; ++sb) {
      sv[sb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        const bf16x8 kf = *reinterpret_cast<const bf16x8*>(&Ks[stream][16 * sb + col][32 * kk + 8 * quad]);
        sv[sb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf, qf[kk], sv[sb], 0, 0, 0);
      }
    }
    // a block whose slots all precede every token of the workgroup needs no
    // causal mask (uniform: the block's first token and the last slot);
    // masked scores become -inf in place
    const bool full = s0 + KS - 1 <= a.start + qb * kFaRows && qb * kFaRows + kFaRows <= a.n;
    if (!full) {
#pragma unroll
      for (int sb = 0; sb < kSB; ++sb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int slot = s0 + 16 * sb + 4 * quad + r;
          if (!(tok_ok && slot <= p)) sv[sb][r] = -INFINITY;
        }
    }
    // the maximum of the unscaled scores, scaled once: rounding is monotonic,
    // so it is the maximum of the scaled scores
    float mx = -INFINITY;
#pragma unroll
    for (int sb = 0; sb < kSB; ++sb)
#pragma unroll
      for (int r = 0; r < 4; ++r) mx = fmaxf(mx, sv[sb][r]);
    mx = quad_max(mx);
    const float m_new = fmaxf(m_run, mx * kFaScale);
    const float m_use = m_new == -INFINITY ? 0.0f : m_new;  // a token with no live slot yet
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
    float rs = 0.0f;
#pragma unroll
    for (int sb = 0; sb < kSB; ++sb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        // scale and shift in one rounding (a masked -inf gives exp2(-inf) = 0)
        const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[sb][r], kFaScale, -m_use));
        sv[sb][r] = e;
        rs += e;
      }
    l_run = l_run * alpha + quad_sum(rs);
    m_run = m_new;
    // once the running maxima settle, alpha is 1 in every lane and the
    // rescale (exact then) is skipped
    if (__any(alpha != 1.0f)) {
#pragma unroll
      for (int db = 0; db < 4; ++db) o[db] *= alpha;
    }
    // O^T[16 db + 4 quad + r][tok] += sum over the block's slots of V^T P^T,
    // 32 slots per bf16 MFMA: k index 8 quad + e stands for slot
    // 32 t + 16 (e / 4) + 4 quad + e % 4, the 8 P values this lane holds for
    // blocks 2t, 2t + 1.  P (finite, non-negative, at most 1 up to exp2 of
    // a rounding error) goes in as three bf16 terms (split3_bf16), which
    // together are the float32 P exactly; with two (16 significant bits)
    // about one output in 200 rounded to another bf16 value than the float32
    // P @ V.
#pragma unroll
    for (int t = 0; t < kSB / 2; ++t) {
      float pv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) pv[e] = sv[2 * t + (e >> 2)][e & 3];
      u32x4 ph, pm, pl;
      split3_bf16(pv, ph, pm, pl);
      const bf16x8 phi = __builtin_bit_cast(bf16x8, ph);
      const bf16x8 pmid = __builtin_bit_cast(bf16x8, pm);
      const bf16x8 plo = __builtin_bit_cast(bf16x8, pl);
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        // V^T fragment: lane (quad, col) needs dimension 16 db + col of slots
        // 32 t + 4 quad + 0..3 and 32 t + 16 + 4 quad + 0..3.  In each group
        // of 16 lanes the transpose read hands lane i the values 4k + i / 4
        // of the group's lanes' 4-element rows, position i % 4 (k = 0..3), so
        // lane c of the group points at slot base + c / 4, dimensions
        // 16 db + 4 (c % 4) .. + 3.
        const int rs = 32 * t + 4 * quad + (col >> 2), rd = 16 * db + 4 * (col & 3);
        const v4s16 t0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) v4s16*)&Vs[stream][rs][rd]);
        const v4s16 t1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) v4s16*)&Vs[stream][rs + 16][rd]);
        const u32x2_t w0 = __builtin_bit_cast(u32x2_t, t0), w1 = __builtin_bit_cast(u32x2_t, t1);
        const bf16x8 va = __builtin_bit_cast(bf16x8, u32x4{w0.x, w0.y, w1.x, w1.y});
        o[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, plo, o[db], 0, 0, 0);
        o[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pmid, o[db], 0, 0, 0);
        o[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, phi, o[db], 0, 0, 0);
      }
    }
  }
  if constexpr (ST > 1) {
    // streams 1.. leave their (max, sum, O) in LDS (over the tiles, which
    // every stream has finished with), and stream 0 folds them in stream order
    constexpr int kW = 18;  // floats per lane: m, l, O
    static_assert((ST - 1) * 4 * 64 * kW * 4 <= (int)sizeof(Ks), "the exchange fits the K tiles");
    float* xs = reinterpret_cast<float*>(&Ks[0][0][0]);
    __syncthreads();
    if (stream > 0) {
      float* d = xs + (((stream - 1) * 4 + sw) * 64 + lane) * kW;
      d[0] = m_run;
      d[1] = l_run;
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int r = 0; r < 4; ++r) d[2 + 4 * db + r] = o[db][r];
    }
    __syncthreads();
    if (stream > 0) return;
#pragma unroll
    for (int q = 1; q < ST; ++q) {
      const float* d = xs + (((q - 1) * 4 + sw) * 64 + lane) * kW;
      const float mq = d[0];
      const float m_new = fmaxf(m_run, mq);
      const float m_use = m_new == -INFINITY ? 0.0f : m_new;
      const float a0 = __builtin_amdgcn_exp2f(m_run - m_use), a1 = __builtin_amdgcn_exp2f(mq - m_use);
      l_run = l_run * a0 + d[1] * a1;
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int r = 0; r < 4; ++r) o[db][r] = o[db][r] * a0 + d[2 + 4 * db + r] * a1;
      m_run = m_new;
    }
  }
  if (!tok_ok) return;
#pragma unroll
  for (int db = 0; db < 4; ++db) {
    const uint32_t lo = f32_to_bf16(o[db][0] / l_run) | (f32_to_bf16(o[db][1] / l_run) << 16);
    const uint32_t hi = f32_to_bf16(o[db][2] / l_run) | (f32_to_bf16(o[db][3] / l_run) << 16);
    const int d = h * kHeadDim + 16 * db + 4 * quad;  // four dimensions, within one 8-wide block
    const size_t at = a.out_kblock ? ((size_t)(d >> 3) * a.n + tok) * 8 + (d & 7) : (size_t)tok * a.ld_out + d;
    *reinterpret_cast<uint2*>(a.out + at) = make_uint2(lo, hi);
  }
}

}  // namespace

size_t split_ws_need(int M, int N, int K, bool pair) {
  const int parts = split_parts(M, N, K);
  return parts > 1 ? (size_t)parts * M * (pair ? 2 * N : N) : 0;
}

namespace {
// NB: 16-token blocks of the prompt
template <bool PAIR, bool W8, int NB>
void launch_slab_nb(const PrefillGemmArgs& a, hipStream_t stream) {
  const int slabs = (a.N + 15) / 16;
  const dim3 grid(slabs);
  const bool long_k = a.K / 32 > 16 * kSlabBatch;
  if (a.gamma) {
    // gate/up with more slabs than CUs (up to twice as many): one workgroup
    // per CU, some of them taking a second slab
    const int cus = cu_count();
    if (PAIR && slabs > cus && slabs <= 2 * cus)
      hipLaunchKernelGGL((gemm_slab_kernel<PAIR, true, W8, 16, NB, PAIR>), dim3(cus), dim3(16 * 64), 0, stream, a);
    else
      hipLaunchKernelGGL((gemm_slab_kernel<PAIR, true, W8, 16, NB>), grid, dim3(16 * 64), 0, stream, a);
  } else if constexpr (!PAIR) {
    // long K split kSlabParts ways inside an XCD, on 16 waves per part, when
    // every part can be resident at once (part 0 waits for the others)
    const int split_grid = kSlabParts * 8 * ((slabs + 7) / 8);
    if (long_k && a.slab_ws && !a.rope.on && split_grid <= cu_count())
      hipLaunchKernelGGL((gemm_slab_kernel<false, false, W8, 16, NB, false, kSlabParts>), dim3(split_grid),
                         dim3(16 * 64), 0, stream, a);
    else if (long_k)
      hipLaunchKernelGGL((gemm_slab_kernel<false, false, W8, kSlabLongWaves, NB>), grid, dim3(kSlabLongWaves * 64),
                         0, stream, a);
    else
      hipLaunchKernelGGL((gemm_slab_kernel<false, false, W8, 16, NB>), grid, dim3(16 * 64), 0, stream, a);
  } else {
    hipLaunchKernelGGL((gemm_slab_kernel<true, false, W8, 16, NB>), grid, dim3(16 * 64), 0, stream, a);
  }
}

template <bool PAIR, bool W8>
int launch_slab(const PrefillGemmArgs& a, hipStream_t stream) {
  static_assert(kSlabBlocks == 4, "one instantiation per block count");
  switch ((a.M + 15) / 16) {
    case 1:
      launch_slab_nb<PAIR, W8, 1>(a, stream);
      break;
    case 2:
      launch_slab_nb<PAIR, W8, 2>(a, stream);
      break;
    case 3:
      launch_slab_nb<PAIR, W8, 3>(a, stream);
      break;
    default:
      launch_slab_nb<PAIR, W8, 4>(a, stream);
      break;
  }
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? 0 : hip_fail(err, "slab gemm launch");
}

// HK_GEMM_RING=0 runs the long-prompt bf16 GEMMs on gemm_big_kernel
// instead of gemm_ring_kernel (read once).
bool ring_gemm() {
  static const bool on = [] {
    const char* v = std::getenv("HK_GEMM_RING");
    return !(v && v[0] == '0');
  }();
  return on;
}

template <bool W8>
int launch_gemm(const PrefillGemmArgs& a, hipStream_t stream) {
  const bool pair = a.epi == EPI_SWIGLU;
  const bool slab_path = a.grp_count == nullptr && a.M <= kSlabMaxTokens;
  if (a.kblock && !slab_path) return fail("prefill gemm: k-blocked operands need the slab path (M <= 64)");
  if (a.rope.on && !slab_path && (a.grp_count != nullptr || !prefill_rope_fusable(a.M, a.K)))
    return fail("prefill gemm: RoPE needs the slab path (M <= 64) or 128-token tiles with K a multiple of 64");
  if (a.rope.on && (a.N != (a.rope.q_heads + 2 * a.rope.kv_heads) * kHeadDim || a.epi == EPI_SWIGLU))
    return fail("prefill gemm: RoPE needs the QKV projection");
  if (a.slab_ws && (a.gamma || a.rope.on || pair || a.grp_count != nullptr || a.M > kSlabMaxTokens ||
                    a.slab_error == nullptr || a.slab_tag == 0))
    return fail("slab gemm: the K split is for plain slabs, with an error word and a nonzero tag");
  if (a.grp_count == nullptr && a.M <= kSlabMaxTokens) {
    if (a.gamma && a.K > kSlabNormMaxK) return fail("slab gemm: a normalised A operand needs K <= 1024");
    if (a.Wn && a.N % 16) return fail("slab gemm: the MFMA-native copy needs whole 16-row slabs");
    return pair ? launch_slab<true, W8>(a, stream) : launch_slab<false, W8>(a, stream);
  }
  if (a.gamma) return fail("prefill gemm: a normalised A operand needs the slab path (M <= 64)");
  dim3 grid((a.N + kTN - 1) / kTN, (a.M + kTM - 1) / kTM);
  if (a.grp_count != nullptr) {
    if (a.max_groups <= 0 || a.max_rows <= 0 || a.n_groups == nullptr || a.grp_expert == nullptr ||
        a.grp_offset == nullptr)
      return fail("grouped gemm: group description incomplete");
    grid.y = (a.max_rows + kTM - 1) / kTM;
    grid.z = a.max_groups;
  }
  if (a.grp_count == nullptr && a.split_ws != nullptr && !a.rope.on && a.K % kBK == 0 && split_parts(a.M, a.N, a.K) > 1 &&
      split_ws_need(a.M, a.N, a.K, pair) <= a.split_ws_floats) {
    // too few tiles to fill the GPU: K split over ~kSplitTarget workgroups
    const int parts = split_parts(a.M, a.N, a.K);
    const dim3 g(gemm_tiles(a.M, a.N), parts);
    if (split_bm(a.M) == 64) {
      if (pair)
        hipLaunchKernelGGL((gemm_big_kernel<64, 64, true, true, W8>), g, dim3(kThreads), 0, stream, a);
      else
        hipLaunchKernelGGL((gemm_big_kernel<64, 64, false, true, W8>), g, dim3(kThreads), 0, stream, a);
    } else if (pair) {
      hipLaunchKernelGGL((gemm_big_kernel<kBM, 64, true, true, W8>), g, dim3(kThreads), 0, stream, a);
    } else {
      hipLaunchKernelGGL((gemm_big_kernel<kBM, 64, false, true, W8>), g, dim3(kThreads), 0, stream, a);
    }
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return hip_fail(err, "split gemm launch");
    hipLaunchKernelGGL(split_reduce_kernel, dim3((a.M * a.N + kThreads - 1) / kThreads), dim3(kThreads), 0,
                       stream, a, parts);
    err = hipGetLastError();
    return err == hipSuccess ? 0 : hip_fail(err, "split reduce launch");
  }
  if (!W8 && ring_gemm() && a.grp_count == nullptr && a.M >= kBM && a.K % kRK == 0) {
    // the LDS-ring form of the 128-token tiles below (bf16 weights), with
    // the same choice of tile width
    const int mt = (a.M + kBM - 1) / kBM, slots = 2 * cu_count();
    const int rounds64 = (mt * ((a.N + 63) / 64) + slots - 1) / slots;
    const int rounds128 = (mt * ((a.N + 127) / 128) + slots - 1) / slots;
    // when the 128-wide tiles fit one per CU (N = hidden at 4096 tokens),
    // 64-wide tiles on three 64-deep stages (72 KiB of LDS) run two per CU
    // instead, with K a multiple of 64; else the 128-wide tiles take a
    // deeper ring, 9 stages, 144 KiB of LDS
    const bool one_per_cu = !pair && mt * ((a.N + 127) / 128) <= cu_count();
    const bool deep64 = one_per_cu && a.K % 64 == 0;
    const bool wide = !pair && !deep64 && (one_per_cu || rounds64 >= 2 * rounds128);
    const int bn = wide ? 128 : 64;
    // (SwiGLU: 128 gate and 128 up rows per tile, each wave 64 tokens x 64
    // gate + 64 up outputs, three 24 KiB stages; the kernel is held to two
    // waves per SIMD, i.e. two workgroups per CU)
    const int bnt = pair ? 128 : bn;
    const dim3 g(8 * ((mt * ((a.N + bnt - 1) / bnt) + 7) / 8));
    if (pair)
      hipLaunchKernelGGL((gemm_ring_kernel<128, true, 3>), g, dim3(kThreads), 0, stream, a);
    else if (deep64)
      hipLaunchKernelGGL((gemm_ring_kernel<64, false, 3, 64>), g, dim3(kThreads), 0, stream, a);
    else if (one_per_cu)
      hipLaunchKernelGGL((gemm_ring_kernel<128, false, 9>), g, dim3(kThreads), 0, stream, a);
    else if (wide)
      hipLaunchKernelGGL((gemm_ring_kernel<128, false, 5>), g, dim3(kThreads), 0, stream, a);
    else
      hipLaunchKernelGGL((gemm_ring_kernel<64, false, 6>), g, dim3(kThreads), 0, stream, a);
  } else if (a.grp_count == nullptr && a.M >= kBM && a.K % kBK == 0) {
    // 128-token tiles, 64 or 128 outputs wide: two workgroups fit a CU, and
    // the wide tiles (about 1.7 times the work each) are taken when the
    // narrow ones would need at least twice as many rounds of workgroups
    const int mt = (a.M + kBM - 1) / kBM, slots = 2 * cu_count();
    const int rounds64 = (mt * ((a.N + 63) / 64) + slots - 1) / slots;
    const int rounds128 = (mt * ((a.N + 127) / 128) + slots - 1) / slots;
    const bool wide = !pair && rounds64 >= 2 * rounds128;
    const int bn = wide ? 128 : 64;
    const dim3 g(8 * ((mt * ((a.N + bn - 1) / bn) + 7) / 8));
    if (pair)
      hipLaunchKernelGGL((gemm_big_kernel<kBM, 64, true, false, W8>), g, dim3(kThreads), 0, stream, a);
    else if (wide)
      hipLaunchKernelGGL((gemm_big_kernel<kBM, 128, false, false, W8>), g, dim3(kThreads), 0, stream, a);
    else
      hipLaunchKernelGGL((gemm_big_kernel<kBM, 64, false, false, W8>), g, dim3(kThreads), 0, stream, a);
  } else if (pair) {
    hipLaunchKernelGGL((gemm_kernel<true, W8>), grid, dim3(kThreads), 0, stream, a);
  } else {
    hipLaunchKernelGGL((gemm_kernel<false, W8>), grid, dim3(kThreads), 0, stream, a);
  }
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? 0 : hip_fail(err, "prefill gemm launch");
}
}  // namespace

bool prefill_rope_fusable(int M, int K) { return M > kSlabMaxTokens && M >= kBM && K % kBK == 0; }

int launch_prefill_gemm(const PrefillGemmArgs& a, hipStream_t stream) {
  if (a.M <= 0 || a.N <= 0 || a.K <= 0) return fail("prefill gemm: sizes must be positive");
  if (a.K % kTK != 0) return fail("prefill gemm: K must be a multiple of 32");
  if (a.lda % 8 != 0) return fail("prefill gemm: lda must be a multiple of 8");
  if (a.scale && a.grp_count) return fail("prefill gemm: int8 weights in grouped mode are not supported");
  return a.scale ? launch_gemm<true>(a, stream) : launch_gemm<false>(a, stream);
}

int launch_embed_rows(const int32_t* tokens, int n, int vocab, const uint16_t* table, int H,
                      uint16_t* X, hipStream_t stream, int kb_rows) {
  hipLaunchKernelGGL(embed_rows_kernel, dim3(n), dim3(kThreads), 0, stream, tokens, vocab, table, H, X, kb_rows);
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? 0 : hip_fail(err, "embed launch");
}

// The MFMA-native copy of a row-major [R, K] weight matrix (R a multiple of
// 16, K of 8): slab s (16 rows) holds, for each k group c of 8 weights, the
// 16 pieces of its rows in fragment order at (s (K / 8) + c) 16 + r, so a
// slab GEMM fragment load is one run.  Row r of slab s is source row
// 16 s + r, or rope_row(s, r) for a QKV matrix whose GEMM applies RoPE.
template <typename T>
__global__ __launch_bounds__(kThreads) void repack_mfma_kernel(const T* src, T* dst, int R, int K, int rope) {
  const size_t groups = K / 8, pieces = (size_t)R * groups;
  for (size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x; i < pieces; i += (size_t)gridDim.x * kThreads) {
    const int slab = (int)(i / (16 * groups)), r = (int)(i & 15);
    const size_t c = (i / 16) % groups;
    const int row = rope ? rope_row(slab, r) : 16 * slab + r;
    dst[i] = src[(size_t)row * groups + c];
  }
}

int launch_repack_mfma(const void* src, void* dst, int R, int K, int weight_bytes, int rope, hipStream_t stream) {
  if (R % 16 || K % 8 || (weight_bytes != 1 && weight_bytes != 2)) return fail("repack: R % 16, K % 8, 1 or 2 bytes");
  if (rope && R % 64) return fail("repack: a RoPE QKV matrix has whole 64-row heads");
  const size_t pieces = (size_t)R * (K / 8);
  const int blocks = (int)std::min<size_t>((pieces + kThreads - 1) / kThreads, 8192);
  if (weight_bytes == 2)
    hipLaunchKernelGGL(repack_mfma_kernel<u32x4>, dim3(blocks), dim3(kThreads), 0, stream,
                       static_cast<const u32x4*>(src), static_cast<u32x4*>(dst), R, K, rope);
  else
    hipLaunchKernelGGL(repack_mfma_kernel<uint2>, dim3(blocks), dim3(kThreads), 0, stream,
                       static_cast<const uint2*>(src), static_cast<uint2*>(dst), R, K, rope);
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? 0 : hip_fail(err, "repack launch");
}

int launch_rmsnorm_rows(const uint16_t* X, int ldx, const uint16_t* gamma, float eps, uint16_t* out,
                        int ldo, int rows, int H, hipStream_t stream) {
  if (H % 8 || ldx % 8 || ldo % 8) return fail("rmsnorm rows: H and the row strides must be multiples of 8");
  const int per = kThreads / 64;
  hipLaunchKernelGGL(rmsnorm_rows_kernel, dim3((rows + per - 1) / per), dim3(kThreads), 0, stream, X, ldx, gamma,
                     eps, out, ldo, H, rows);
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? 0 : hip_fail(err, "rmsnorm rows launch");
}

int launch_prefill_attention(const PrefillAttnArgs& a, hipStream_t stream) {
  if (a.q_heads % a.kv_heads != 0) return fail("prefill attention: unsupported head grouping");
  if (a.ld_out % 4 != 0) return fail("prefill attention: output rows must be 8-byte aligned");
  if (a.start < 0 || a.start + a.n > a.max_ctx) return fail("prefill attention: slots out of range");
  hipError_t err;
  if (!a.rope_done) {
    hipLaunchKernelGGL(rope_append_kernel, dim3(a.n), dim3(kThreads), 0, stream, a);
    err = hipGetLastError();
    if (err != hipSuccess) return hip_fail(err, "rope append launch");
  }
  PrefillAttnArgs b = a;
  b.period = cu_count();
  const dim3 grid(a.q_heads * ((a.n + kFaRows - 1) / kFaRows));
  if (a.start + a.n <= 64)
    hipLaunchKernelGGL((attention_prefill_kernel<64, 1>), grid, dim3(kThreads), 0, stream, b);
  else
    hipLaunchKernelGGL((attention_prefill_kernel<kFaSlots, kFaStreams>), grid, dim3(kThreads * kFaStreams), 0,
                       stream, b);
  err = hipGetLastError();
  return err == hipSuccess ? 0 : hip_fail(err, "prefill attention launch");
}

}  // namespace hk
