// Decode-step attention: RoPE on the new q/k heads, in-place KV append at slot
// `position`, and grouped-query softmax attention over slots 0..position.
//
// Follows npu_llm/runtime/cpu_backend.py:78-129:
//   rotate   [x1*c - x2*s, x2*c + x1*s] on the two 32-wide halves, then bf16
//            (cos/sin come from host tables built with the reference's own
//            NumPy expression, so they match bit for bit)
//   append   K[:, p] = bf16(rot k), V[:, p] = v                    :105-108
//   scores   (q . k) * head_dim**-0.5, minus the row max, exp, / sum   :110-125
//   output   bf16(P @ V)                                          :126-129
//
// Work split: one workgroup per (KV head, chunk of 256 slots), so positions
// below 256 use one workgroup per KV head and no merge.  With a single chunk
// the workgroup normalises P = p / sum first and then forms P @ V, as NumPy
// does.  With
// several chunks each workgroup publishes (max, sum, p @ V) for its chunk and
// the last one to finish (a per-head ticket) merges them with log-sum-exp
// rescaling.  The KV cache layout is [kv head][slot][64] BF16 per layer, so
// one slot of one head is a contiguous 128-byte row.
#include "hk_common.h"
#include "hk_internal.h"

namespace hk {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kHalf = kHeadDim / 2;
constexpr int kPartStride = kHeadDim + 2;  // acc[64], max, sum

__device__ __forceinline__ void unpack_row(const uint16_t* src, float (&dst)[kHeadDim]) {
#pragma unroll
  for (int c = 0; c < kHeadDim / 8; ++c) {
    const u32x4 w = load16(src + c * 8);
    dst[c * 8 + 0] = bf_lo(w.x);
    dst[c * 8 + 1] = bf_hi(w.x);
    dst[c * 8 + 2] = bf_lo(w.y);
    dst[c * 8 + 3] = bf_hi(w.y);
    dst[c * 8 + 4] = bf_lo(w.z);
    dst[c * 8 + 5] = bf_hi(w.z);
    dst[c * 8 + 6] = bf_lo(w.w);
    dst[c * 8 + 7] = bf_hi(w.w);
  }
}

__global__ __launch_bounds__(kThreads) void attention_decode_kernel(AttnArgs a) {
  const int g = blockIdx.x;
  const int s = blockIdx.y;
  const int p = *a.position;
  const int t0 = s * kAttnChunk;
  if (t0 > p) return;
  const int t1 = min(t0 + kAttnChunk, p + 1);
  const int n = t1 - t0;
  const int nsplit = p / kAttnChunk + 1;
  const bool holds_new = (s == nsplit - 1);
  const int qpk = a.q_heads / a.kv_heads;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;

  __shared__ float qs[kMaxQPerKV][kHeadDim];
  __shared__ float knew[kHeadDim];
  __shared__ float sc[kMaxQPerKV][kAttnChunk];
  __shared__ float hmax[kMaxQPerKV];
  __shared__ float hsum[kMaxQPerKV];
  __shared__ uint32_t vs[kAttnChunk][kHalf];  // V rows of the chunk, bf16 pairs
  __shared__ unsigned int ticket_s;

  const float* ct = a.cos_tab + (size_t)p * kHalf;
  const float* st = a.sin_tab + (size_t)p * kHalf;
  const size_t head_base = (size_t)g * a.max_ctx;

  // Rotated query heads of this group, rounded to bf16 as the reference does.
  for (int i = tid; i < qpk * kHalf; i += kThreads) {
    const int h = i / kHalf, j = i % kHalf;
    const uint16_t* q = a.qkv + (size_t)(g * qpk + h) * kHeadDim;
    const float x1 = bf16_to_f32(q[j]), x2 = bf16_to_f32(q[j + kHalf]);
    const float c = ct[j], sn = st[j];
    qs[h][j] = round_bf16(x1 * c - x2 * sn);
    qs[h][j + kHalf] = round_bf16(x2 * c + x1 * sn);
  }
  // The new key (rotated) and value of this KV head, appended at slot p by
  // the workgroup whose chunk holds p.
  if (holds_new && tid < kHalf) {
    const uint16_t* k = a.qkv + (size_t)(a.q_heads + g) * kHeadDim;
    const uint16_t* v = a.qkv + (size_t)(a.q_heads + a.kv_heads + g) * kHeadDim;
    const float x1 = bf16_to_f32(k[tid]), x2 = bf16_to_f32(k[tid + kHalf]);
    const float c = ct[tid], sn = st[tid];
    const uint32_t r1 = f32_to_bf16(x1 * c - x2 * sn);
    const uint32_t r2 = f32_to_bf16(x2 * c + x1 * sn);
    knew[tid] = bf16_to_f32(r1);
    knew[tid + kHalf] = bf16_to_f32(r2);
    uint16_t* kd = a.kcache + (head_base + p) * kHeadDim;
    uint16_t* vd = a.vcache + (head_base + p) * kHeadDim;
    kd[tid] = (uint16_t)r1;
    kd[tid + kHalf] = (uint16_t)r2;
    vd[tid] = v[tid];
    vd[tid + kHalf] = v[tid + kHalf];
  }
  // Stage the chunk's cached V rows (16-byte loads); slot p comes from qkv.
  for (int i = tid; i < n * (kHeadDim / 8); i += kThreads) {
    const int t = i / (kHeadDim / 8), c = i % (kHeadDim / 8);
    const int slot = t0 + t;
    const uint16_t* src = (slot == p)
                              ? a.qkv + (size_t)(a.q_heads + a.kv_heads + g) * kHeadDim + c * 8
                              : a.vcache + (head_base + slot) * kHeadDim + c * 8;
    const u32x4 w = load16(src);
    vs[t][c * 4 + 0] = w.x;
    vs[t][c * 4 + 1] = w.y;
    vs[t][c * 4 + 2] = w.z;
    vs[t][c * 4 + 3] = w.w;
  }
  __syncthreads();

  // Scores: one (slot, head) pair per thread.
  const float scale = 1.0f / 8.0f;  // head_dim ** -0.5 for head_dim 64 (exact)
  for (int i = tid; i < n * qpk; i += kThreads) {
    const int t = i / qpk, h = i % qpk;
    const int slot = t0 + t;
    float kv[kHeadDim];
    if (slot == p) {
#pragma unroll
      for (int d = 0; d < kHeadDim; ++d) kv[d] = knew[d];
    } else {
      unpack_row(a.kcache + (head_base + slot) * kHeadDim, kv);
    }
    float dot = 0.0f;
#pragma unroll
    for (int d = 0; d < kHeadDim; ++d) dot = fmaf(qs[h][d], kv[d], dot);
    sc[h][t] = dot * scale;
  }
  __syncthreads();

  // Per-head max and exp-sum over this chunk (one wave per head).
  for (int h = wave; h < qpk; h += kWaves) {
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

  if (nsplit == 1) {
    for (int i = tid; i < qpk * n; i += kThreads) {
      const int h = i / n, t = i % n;
      sc[h][t] = sc[h][t] / hsum[h];
    }
    __syncthreads();
  }

  // Weighted sum of values from the LDS copy of this chunk's V rows:
  // thread = (head, pair of dimensions), loop over the slots.
  float* mine = a.partial + ((size_t)g * a.max_splits + s) * kMaxQPerKV * kPartStride;
  for (int i = tid; i < qpk * kHalf; i += kThreads) {
    const int h = i / kHalf, dp = i % kHalf;
    float o0 = 0.0f, o1 = 0.0f;
#pragma unroll 8
    for (int t = 0; t < n; ++t) {
      const uint32_t v2 = vs[t][dp];
      const float pt = sc[h][t];
      o0 = fmaf(pt, bf_lo(v2), o0);
      o1 = fmaf(pt, bf_hi(v2), o1);
    }
    if (nsplit == 1) {
      const uint32_t packed = f32_to_bf16(o0) | (f32_to_bf16(o1) << 16);
      reinterpret_cast<uint32_t*>(a.out + (size_t)(g * qpk + h) * kHeadDim)[dp] = packed;
    } else {
      mine[h * kPartStride + 2 * dp] = o0;
      mine[h * kPartStride + 2 * dp + 1] = o1;
    }
  }
  if (nsplit == 1) return;

  // Split-KV: publish this chunk's max and sum, the last workgroup merges.
  if (tid < qpk) {
    mine[tid * kPartStride + kHeadDim] = hmax[tid];
    mine[tid * kPartStride + kHeadDim + 1] = hsum[tid];
  }
  __threadfence();
  __syncthreads();
  if (tid == 0) ticket_s = atomicAdd(&a.counters[g], 1u);
  __syncthreads();
  if (ticket_s != (unsigned int)(nsplit - 1)) return;
  __threadfence();
  const float* base = a.partial + (size_t)g * a.max_splits * kMaxQPerKV * kPartStride;
  for (int i = tid; i < qpk * kHeadDim; i += kThreads) {
    const int h = i / kHeadDim, d = i % kHeadDim;
    float m = -INFINITY;
    for (int j = 0; j < nsplit; ++j)
      m = fmaxf(m, base[(size_t)j * kMaxQPerKV * kPartStride + h * kPartStride + kHeadDim]);
    float l = 0.0f, o = 0.0f;
    for (int j = 0; j < nsplit; ++j) {
      const float* pj = base + (size_t)j * kMaxQPerKV * kPartStride + h * kPartStride;
      const float f = expf(pj[kHeadDim] - m);
      l = fmaf(pj[kHeadDim + 1], f, l);
      o = fmaf(pj[d], f, o);
    }
    a.out[(size_t)(g * qpk + h) * kHeadDim + d] = (uint16_t)f32_to_bf16(o / l);
  }
  if (tid == 0) atomicExch(&a.counters[g], 0u);
}

}  // namespace

int launch_attention_decode(const AttnArgs& a, hipStream_t stream) {
  if (a.kv_heads <= 0 || a.q_heads <= 0 || a.q_heads % a.kv_heads != 0)
    return fail("attention: q_heads must be a positive multiple of kv_heads");
  if (a.q_heads / a.kv_heads > kMaxQPerKV) return fail("attention: more than 16 q heads per kv head");
  if (a.max_ctx <= 0 || a.max_ctx > kMaxContext) return fail("attention: context out of range");
  if (a.max_splits < attention_splits(a.max_ctx)) return fail("attention: too few split-KV slots");
  hipLaunchKernelGGL(attention_decode_kernel, dim3(a.kv_heads, a.max_splits), dim3(kThreads), 0,
                     stream, a);
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? 0 : hip_fail(err, "attention launch");
}

}  // namespace hk
