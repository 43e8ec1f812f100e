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
#include "hk_common.h"
#include "hk_internal.h"

namespace hk {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kTM = 64;       // tokens per tile
constexpr int kTN = 64;       // outputs per tile
constexpr int kTK = 32;       // K per step
constexpr int kLdsRow = kTK + 8;  // bf16 per LDS row (padding against bank conflicts)

__device__ __forceinline__ float silu_mul(float g, float u) {
  const float clipped = fminf(fmaxf(g, -80.0f), 80.0f);
  return (g / (1.0f + expf(-clipped))) * u;
}

template <bool PAIR>
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
  const uint16_t* w_src = Wb + (size_t)(w_ok ? n0 + lr : 0) * a.K + lk;
  const uint16_t* u_src = Wb + (size_t)(w_ok ? n0 + lr + a.N : 0) * a.K + lk;
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
    const u32x4 wv = w_ok ? load_stream16(w_src + k0) : zero;
    u32x4 uv = zero;
    if constexpr (PAIR) uv = w_ok ? load_stream16(u_src + k0) : zero;
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
        const float v = acc[i][j][r];
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
            *y = (uint16_t)f32_to_bf16(silu_mul(round_bf16(v), round_bf16(accu[i][j][r])));
            break;
          default:
            break;
        }
      }
}

// X[i] = E[token_i] (bf16 rows), tokens read from device memory.
__global__ __launch_bounds__(kThreads) void embed_rows_kernel(const int32_t* tokens, int vocab,
                                                              const uint16_t* table, int H,
                                                              uint16_t* X) {
  const int i = blockIdx.x;
  int t = tokens[i];
  t = t < 0 ? 0 : (t >= vocab ? vocab - 1 : t);
  const uint32_t* src = reinterpret_cast<const uint32_t*>(table + (size_t)t * H);
  uint32_t* dst = reinterpret_cast<uint32_t*>(X + (size_t)i * H);
  for (int j = threadIdx.x; j < H / 2; j += kThreads) dst[j] = src[j];
}

// One row per workgroup: out = bf16((v * inv_rms) * gamma).
__global__ __launch_bounds__(kThreads) void rmsnorm_rows_kernel(const uint16_t* X, int ldx,
                                                                const uint16_t* gamma, float eps,
                                                                uint16_t* out, int ldo, int H) {
  __shared__ float red[kThreads / 64];
  const int row = blockIdx.x;
  const uint16_t* x = X + (size_t)row * ldx;
  const int tid = threadIdx.x;
  float ss = 0.0f;
  for (int j = tid; j < H; j += kThreads) {
    const float v = bf16_to_f32(x[j]);
    ss += v * v;
  }
  ss = group_sum<64>(ss);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  float total = red[0];
#pragma unroll
  for (int w = 1; w < kThreads / 64; ++w) total += red[w];
  const float inv = 1.0f / sqrtf(total / (float)H + eps);
  uint16_t* o = out + (size_t)row * ldo;
  for (int j = tid; j < H; j += kThreads)
    o[j] = (uint16_t)f32_to_bf16((bf16_to_f32(x[j]) * inv) * bf16_to_f32(gamma[j]));
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

// Causal GQA attention for token i (slot p = start + i) and KV head g, over
// slots 0..p in chunks of 256.  One chunk: P = p / sum, then P @ V (NumPy's
// order).  Several chunks: running max / sum / P@V with log-sum-exp rescaling.
__global__ __launch_bounds__(kThreads) void attention_prefill_kernel(PrefillAttnArgs a) {
  const int g = blockIdx.x;
  const int i = blockIdx.y;
  const int p = a.start + i;
  const int qpk = a.q_heads / a.kv_heads;
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int half = kHeadDim / 2;
  const size_t head_base = (size_t)g * a.max_ctx;

  __shared__ float qs[kMaxQPerKV][kHeadDim];
  __shared__ float sc[kMaxQPerKV][kAttnChunk];
  __shared__ uint32_t vs[kAttnChunk][kHeadDim / 2];
  __shared__ float hmax[kMaxQPerKV], hsum[kMaxQPerKV], hscale[kMaxQPerKV];
  __shared__ float run_m[kMaxQPerKV], run_l[kMaxQPerKV];

  for (int e = tid; e < qpk * kHeadDim; e += kThreads) {
    const int h = e / kHeadDim, d = e % kHeadDim;
    qs[h][d] = bf16_to_f32(a.qrot[(size_t)i * a.q_heads * kHeadDim + (size_t)(g * qpk + h) * kHeadDim + d]);
  }
  if (tid < qpk) {
    run_m[tid] = -INFINITY;
    run_l[tid] = 0.0f;
  }
  const int nchunks = p / kAttnChunk + 1;
  // running P@V: thread owns (head, dim pair) entries e = tid + k * 256
  float o0[4] = {0.f, 0.f, 0.f, 0.f}, o1[4] = {0.f, 0.f, 0.f, 0.f};
  const float scale = 1.0f / 8.0f;
  for (int c = 0; c < nchunks; ++c) {
    const int t0 = c * kAttnChunk;
    const int n = min(kAttnChunk, p + 1 - t0);
    __syncthreads();
    for (int e = tid; e < n * (kHeadDim / 8); e += kThreads) {
      const int t = e / (kHeadDim / 8), cc = e % (kHeadDim / 8);
      const u32x4 w = load16(a.vcache + (head_base + t0 + t) * kHeadDim + cc * 8);
      vs[t][cc * 4 + 0] = w.x;
      vs[t][cc * 4 + 1] = w.y;
      vs[t][cc * 4 + 2] = w.z;
      vs[t][cc * 4 + 3] = w.w;
    }
    for (int e = tid; e < n * qpk; e += kThreads) {
      const int t = e / qpk, h = e % qpk;
      const uint16_t* kr = a.kcache + (head_base + t0 + t) * kHeadDim;
      float dot = 0.0f;
#pragma unroll
      for (int cc = 0; cc < kHeadDim / 8; ++cc) {
        const u32x4 w = load16(kr + cc * 8);
        dot = fmaf(qs[h][cc * 8 + 0], bf_lo(w.x), dot);
        dot = fmaf(qs[h][cc * 8 + 1], bf_hi(w.x), dot);
        dot = fmaf(qs[h][cc * 8 + 2], bf_lo(w.y), dot);
        dot = fmaf(qs[h][cc * 8 + 3], bf_hi(w.y), dot);
        dot = fmaf(qs[h][cc * 8 + 4], bf_lo(w.z), dot);
        dot = fmaf(qs[h][cc * 8 + 5], bf_hi(w.z), dot);
        dot = fmaf(qs[h][cc * 8 + 6], bf_lo(w.w), dot);
        dot = fmaf(qs[h][cc * 8 + 7], bf_hi(w.w), dot);
      }
      sc[h][t] = dot * scale;
    }
    __syncthreads();
    for (int h = wave; h < qpk; h += kThreads / 64) {
      float m = -INFINITY;
      for (int t = lane; t < n; t += 64) m = fmaxf(m, sc[h][t]);
      m = group_max<64>(m);
      float sum = 0.0f;
      for (int t = lane; t < n; t += 64) {
        const float e = expf(sc[h][t] - m);
        sc[h][t] = e;
        sum += e;
      }
      sum = group_sum<64>(sum);
      if (lane == 0) {
        hmax[h] = m;
        hsum[h] = sum;
      }
    }
    __syncthreads();
    if (nchunks == 1) {
      for (int e = tid; e < qpk * n; e += kThreads) {
        const int h = e / n, t = e % n;
        sc[h][t] = sc[h][t] / hsum[h];
      }
    } else if (tid < qpk) {
      // rescale factors for the running sums
      const float mn = fmaxf(run_m[tid], hmax[tid]);
      const float fo = expf(run_m[tid] - mn);  // 0 on the first chunk
      const float fc = expf(hmax[tid] - mn);
      run_l[tid] = fmaf(run_l[tid], fo, hsum[tid] * fc);
      run_m[tid] = mn;
      hscale[tid] = fo;
      hsum[tid] = fc;  // reused: factor for this chunk's p @ V
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int e = tid + k * kThreads;
      if (e >= qpk * half) break;
      const int h = e / half, dp = e % half;
      float c0 = 0.f, c1 = 0.f;
      for (int t = 0; t < n; ++t) {
        const uint32_t v2 = vs[t][dp];
        c0 = fmaf(sc[h][t], bf_lo(v2), c0);
        c1 = fmaf(sc[h][t], bf_hi(v2), c1);
      }
      if (nchunks == 1) {
        o0[k] = c0;
        o1[k] = c1;
      } else {
        o0[k] = fmaf(o0[k], hscale[h], c0 * hsum[h]);
        o1[k] = fmaf(o1[k], hscale[h], c1 * hsum[h]);
      }
    }
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int e = tid + k * kThreads;
    if (e >= qpk * half) break;
    const int h = e / half, dp = e % half;
    float r0 = o0[k], r1 = o1[k];
    if (nchunks > 1) {
      r0 = r0 / run_l[h];
      r1 = r1 / run_l[h];
    }
    uint32_t* out = reinterpret_cast<uint32_t*>(a.out + (size_t)i * a.ld_out +
                                                (size_t)(g * qpk + h) * kHeadDim);
    out[dp] = f32_to_bf16(r0) | (f32_to_bf16(r1) << 16);
  }
}

}  // namespace

int launch_prefill_gemm(const PrefillGemmArgs& a, hipStream_t stream) {
  if (a.M <= 0 || a.N <= 0 || a.K <= 0) return fail("prefill gemm: sizes must be positive");
  if (a.K % kTK != 0) return fail("prefill gemm: K must be a multiple of 32");
  if (a.lda % 8 != 0) return fail("prefill gemm: lda must be a multiple of 8");
  dim3 grid((a.N + kTN - 1) / kTN, (a.M + kTM - 1) / kTM);
  if (a.grp_count != nullptr) {
    if (a.max_groups <= 0 || a.max_rows <= 0 || a.n_groups == nullptr || a.grp_expert == nullptr ||
        a.grp_offset == nullptr)
      return fail("grouped gemm: group description incomplete");
    grid.y = (a.max_rows + kTM - 1) / kTM;
    grid.z = a.max_groups;
  }
  if (a.epi == EPI_SWIGLU)
    hipLaunchKernelGGL(gemm_kernel<true>, grid, dim3(kThreads), 0, stream, a);
  else
    hipLaunchKernelGGL(gemm_kernel<false>, grid, dim3(kThreads), 0, stream, a);
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? 0 : hip_fail(err, "prefill gemm launch");
}

int launch_embed_rows(const int32_t* tokens, int n, int vocab, const uint16_t* table, int H,
                      uint16_t* X, hipStream_t stream) {
  hipLaunchKernelGGL(embed_rows_kernel, dim3(n), dim3(kThreads), 0, stream, tokens, vocab, table, H, X);
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? 0 : hip_fail(err, "embed launch");
}

int launch_rmsnorm_rows(const uint16_t* X, int ldx, const uint16_t* gamma, float eps, uint16_t* out,
                        int ldo, int rows, int H, hipStream_t stream) {
  hipLaunchKernelGGL(rmsnorm_rows_kernel, dim3(rows), dim3(kThreads), 0, stream, X, ldx, gamma, eps,
                     out, ldo, H);
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? 0 : hip_fail(err, "rmsnorm rows launch");
}

int launch_prefill_attention(const PrefillAttnArgs& a, hipStream_t stream) {
  if (a.q_heads % a.kv_heads != 0 || a.q_heads / a.kv_heads > kMaxQPerKV)
    return fail("prefill attention: unsupported head grouping");
  if (a.start < 0 || a.start + a.n > a.max_ctx) return fail("prefill attention: slots out of range");
  hipLaunchKernelGGL(rope_append_kernel, dim3(a.n), dim3(kThreads), 0, stream, a);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return hip_fail(err, "rope append launch");
  hipLaunchKernelGGL(attention_prefill_kernel, dim3(a.kv_heads, a.n), dim3(kThreads), 0, stream, a);
  err = hipGetLastError();
  return err == hipSuccess ? 0 : hip_fail(err, "prefill attention launch");
}

}  // namespace hk
