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
// Work split: one workgroup per (query head, chunk of 256 slots), so
// positions below 256 use one workgroup per query head and no merge; the K/V
// rows of a KV head are shared by its query heads through L2.  Thread t of a
// chunk scores slot t; the P @ V sum is split over 8 slot groups of 32 lanes
// (one dimension pair per lane) and the groups are added in LDS.  With a single
// chunk the workgroup normalises P = p / sum first and then forms P @ V, as
// NumPy does.  With several chunks each workgroup publishes (max, sum, p @ V)
// for its chunk and the last one to finish (a per-head ticket) merges them
// with log-sum-exp rescaling.  The KV cache layout is [kv head][slot][64] BF16
// per layer, so one slot of one head is a contiguous 128-byte row.
#include "hk_common.h"
#include "hk_internal.h"

namespace hk {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kHalf = kHeadDim / 2;
constexpr int kPartStride = kHeadDim + 2;  // acc[64], max, sum
constexpr int kGroups = kThreads / kHalf;  // slot groups of the P @ V loop
static_assert(kThreads == kAttnChunk, "one thread per slot of a chunk");
static_assert(kHeadDim == 64, "the merge runs on wave 0 alone");

// One workgroup per (query head, chunk of 256 slots).  Every load whose
// address does not depend on a reduction (the K row of the thread's slot, the
// V words of its slot group, q, the new k/v) is issued before the first
// barrier, so a launch costs about one memory latency plus the reductions.
__global__ __launch_bounds__(kThreads) void attention_decode_kernel(AttnArgs a) {
  const int h = blockIdx.x;
  const int s = blockIdx.y;
  const int p = *a.position;
  const int t0 = s * kAttnChunk;
  if (t0 > p) return;
  const int t1 = min(t0 + kAttnChunk, p + 1);
  const int n = t1 - t0;
  const int nsplit = p / kAttnChunk + 1;
  const bool holds_new = (s == nsplit - 1);
  const int qpk = a.q_heads / a.kv_heads;
  const int g = h / qpk;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;

  __shared__ float qs[kHeadDim];
  __shared__ float knew[kHeadDim];
  __shared__ float pr[kAttnChunk];
  __shared__ float red[2][kWaves];
  __shared__ float acc[kGroups][kHeadDim];

  const size_t head_base = (size_t)g * a.max_ctx;
  const uint16_t* vnew = a.qkv + (size_t)(a.q_heads + a.kv_heads + g) * kHeadDim;

  // K row of this thread's slot (slot p comes from the rotated new key below)
  const int slot = t0 + tid;
  const bool has_slot = tid < n && slot != p;
  u32x4 krow[kHeadDim / 8];
  {
    const uint16_t* src = a.kcache + (head_base + (has_slot ? slot : 0)) * kHeadDim;
#pragma unroll
    for (int c = 0; c < kHeadDim / 8; ++c) krow[c] = has_slot ? load16(src + c * 8) : u32x4{0u, 0u, 0u, 0u};
  }
  // V words for the P @ V loop: thread (group gi, dimension pair dp) takes
  // slots gi, gi + kGroups, ... of the chunk.
  const int dp = tid & (kHalf - 1);
  const int gi = tid / kHalf;
  uint32_t vw[kAttnChunk / kGroups];
#pragma unroll
  for (int k = 0; k < kAttnChunk / kGroups; ++k) {
    const int t = gi + k * kGroups;
    const int sl = t0 + t;
    const uint32_t* src = reinterpret_cast<const uint32_t*>(
        sl == p ? vnew : a.vcache + (head_base + (sl < p ? sl : 0)) * kHeadDim);
    vw[k] = t < n ? src[dp] : 0u;
  }

  // Rotated query head and new key (bf16-rounded as the reference does);
  // the first query head of the group appends k and v at slot p.
  if (tid < 2 * kHalf) {
    const int j = tid & (kHalf - 1);
    const bool is_k = tid >= kHalf;
    const uint16_t* src = is_k ? a.qkv + (size_t)(a.q_heads + g) * kHeadDim
                               : a.qkv + (size_t)h * kHeadDim;
    const float c = a.cos_tab[(size_t)p * kHalf + j];
    const float sn = a.sin_tab[(size_t)p * kHalf + j];
    const float x1 = bf16_to_f32(src[j]), x2 = bf16_to_f32(src[j + kHalf]);
    const uint32_t r1 = f32_to_bf16(x1 * c - x2 * sn);
    const uint32_t r2 = f32_to_bf16(x2 * c + x1 * sn);
    float* dst = is_k ? knew : qs;
    dst[j] = bf16_to_f32(r1);
    dst[j + kHalf] = bf16_to_f32(r2);
    if (is_k && holds_new && h % qpk == 0) {
      uint16_t* kd = a.kcache + (head_base + p) * kHeadDim;
      uint16_t* vd = a.vcache + (head_base + p) * kHeadDim;
      kd[j] = (uint16_t)r1;
      kd[j + kHalf] = (uint16_t)r2;
      vd[j] = vnew[j];
      vd[j + kHalf] = vnew[j + kHalf];
    }
  }
  __syncthreads();

  // score of this thread's slot
  const float scale = 1.0f / 8.0f;  // head_dim ** -0.5 for head_dim 64 (exact)
  float sc = -INFINITY;
  if (tid < n) {
    float dot = 0.0f;
    if (slot == p) {
#pragma unroll
      for (int d = 0; d < kHeadDim; ++d) dot = fmaf(qs[d], knew[d], dot);
    } else {
#pragma unroll
      for (int c = 0; c < kHeadDim / 8; ++c) {
        const uint32_t w[4] = {krow[c].x, krow[c].y, krow[c].z, krow[c].w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          dot = fmaf(qs[c * 8 + 2 * q], bf_lo(w[q]), dot);
          dot = fmaf(qs[c * 8 + 2 * q + 1], bf_hi(w[q]), dot);
        }
      }
    }
    sc = dot * scale;
  }
  // chunk max and exp-sum
  float m = group_max<64>(sc);
  if (lane == 0) red[0][wave] = m;
  __syncthreads();
  m = red[0][0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) m = fmaxf(m, red[0][w]);
  const float e = tid < n ? expf(sc - m) : 0.0f;
  float sum = group_sum<64>(e);
  if (lane == 0) red[1][wave] = sum;
  __syncthreads();
  sum = red[1][0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) sum += red[1][w];
  // a single chunk normalises first (P = e / sum), as the reference does
  if (tid < kAttnChunk) pr[tid] = nsplit == 1 ? e / sum : e;
  __syncthreads();

  float o0 = 0.0f, o1 = 0.0f;
#pragma unroll
  for (int k = 0; k < kAttnChunk / kGroups; ++k) {
    const int t = gi + k * kGroups;
    if (t < n) {
      const float pt = pr[t];
      o0 = fmaf(pt, bf_lo(vw[k]), o0);
      o1 = fmaf(pt, bf_hi(vw[k]), o1);
    }
  }
  acc[gi][2 * dp] = o0;
  acc[gi][2 * dp + 1] = o1;
  __syncthreads();
  if (tid >= kHeadDim) return;
  float o = 0.0f;
#pragma unroll
  for (int k = 0; k < kGroups; ++k) o += acc[k][tid];
  if (nsplit == 1) {
    a.out[(size_t)h * kHeadDim + tid] = (uint16_t)f32_to_bf16(o);
    return;
  }

  // Split-KV: publish (p @ V, max, sum) of this chunk; the last workgroup of
  // this head (ticket) merges all chunks with log-sum-exp rescaling.
  float* mine = a.partial + ((size_t)h * a.max_splits + s) * kPartStride;
  mine[tid] = o;
  if (tid == 0) {
    mine[kHeadDim] = m;
    mine[kHeadDim + 1] = sum;
  }
  __threadfence();
  // only wave 0 (tid < 64) is left here, so a shuffle broadcasts the ticket
  unsigned int ticket = 0;
  if (tid == 0) ticket = atomicAdd(&a.counters[h], 1u);
  ticket = __shfl(ticket, 0, 64);
  if (ticket != (unsigned int)(nsplit - 1)) return;
  __threadfence();
  const float* base = a.partial + (size_t)h * a.max_splits * kPartStride;
  float mx = -INFINITY;
  for (int j = 0; j < nsplit; ++j) mx = fmaxf(mx, base[(size_t)j * kPartStride + kHeadDim]);
  float l = 0.0f, out = 0.0f;
  for (int j = 0; j < nsplit; ++j) {
    const float* pj = base + (size_t)j * kPartStride;
    const float f = expf(pj[kHeadDim] - mx);
    l = fmaf(pj[kHeadDim + 1], f, l);
    out = fmaf(pj[tid], f, out);
  }
  a.out[(size_t)h * kHeadDim + tid] = (uint16_t)f32_to_bf16(out / l);
  if (tid == 0) atomicExch(&a.counters[h], 0u);
}

}  // namespace

int launch_attention_decode(const AttnArgs& a, hipStream_t stream) {
  if (a.kv_heads <= 0 || a.q_heads <= 0 || a.q_heads % a.kv_heads != 0)
    return fail("attention: q_heads must be a positive multiple of kv_heads");
  if (a.q_heads / a.kv_heads > kMaxQPerKV) return fail("attention: more than 16 q heads per kv head");
  if (a.max_ctx <= 0 || a.max_ctx > kMaxContext) return fail("attention: context out of range");
  if (a.max_splits < attention_splits(a.max_ctx)) return fail("attention: too few split-KV slots");
  hipLaunchKernelGGL(attention_decode_kernel, dim3(a.q_heads, a.max_splits), dim3(kThreads), 0,
                     stream, a);
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? 0 : hip_fail(err, "attention launch");
}

}  // namespace hk
