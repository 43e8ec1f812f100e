// Expert-GEMV shims for the reference's MoE offload contracts (GGML
// MUL_MAT_ID and Colibri's coli_cuda_* expert group); hk_experts.h states
// the formulas.
//
// Weights are requantised on the host, as both reference backends do, into
// int8 rows with one float32 scale each, padded to whole 16-byte chunks and
// kept on the device.  A call rounds its float32 activations to bf16 on the
// host (the reference's float_to_bf16 before its upload), copies them in,
// runs the projections and copies float32 results back.
//
// The kernel gives each wave kRows consecutive rows of one projection; every
// lane loads 16 int8 weights per row and the 16 matching bf16 activations per
// chunk, two chunks per 2048-column tile, all before the first FMA.  A row's
// tile sum is scaled, rounded to bf16 and added to the row total in float32
// (backend_xdna.cpp:159-206).  For an expert group, gate row r and up row r
// share a wave (PAIR), which then writes bf16(silu(g) * u) for the down
// projection: the SwiGLU of backend_xdna.cpp:341-342 followed by the bf16
// rounding that the down projection's input load applies (:190-191).
//
// GGML's Q4_K and Q6_K weights stay in their 4.5- and 6.6-bit blocks and are
// dequantised next to the dot product, as the reference's native kernels do
// (npu_llm/kernels/project_q4k_bf16.cc:76-117, project_q6k_bf16.cc:53-99);
// each tile's sum is rounded to bf16 with no further scale.  The dense GGML
// MUL_MAT keeps the W8 path with one scale per (row, 2048-column tile), as
// the reference's dense tiles have (ggml-xdna.cpp:768-832).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <vector>

#include "hk.h"
#include "hk_common.h"
#include "hk_experts.h"
#include "hk_internal.h"

namespace hk {
namespace {

constexpr int kGroupMax = 8;     // experts per call (ggml-xdna.cpp:36, backend_xdna.cpp:24)
constexpr int kTileCols = 2048;  // columns per rounded partial (backend_xdna.cpp:25)
constexpr int kGgmlDimMax = 2048;
constexpr int kChunk = 16;  // int8 weights per 16-byte load; a tile is two chunks per lane
constexpr int kRows = 4;    // rows per wave
constexpr int kWavesPerBlock = 4;
constexpr int kRowsPerBlock = kRows * kWavesPerBlock;

// Device row stride in elements: whole 16-element chunks, zero past the end.
inline int padded(int cols) { return (cols + kChunk - 1) / kChunk * kChunk; }
__device__ __forceinline__ int padded_dev(int cols) { return (cols + kChunk - 1) / kChunk * kChunk; }

struct ExpertArgs {
  const int8_t* q[kGroupMax];    // [out][ld] weights (gate when PAIR), zero past `in`
  const int8_t* q2[kGroupMax];   // [out][ld] up weights (PAIR)
  const float* s[kGroupMax];     // [out] row scales
  const float* s2[kGroupMax];    // [out] up row scales (PAIR)
  const uint16_t* x[kGroupMax];  // [ld] bf16 input, zero past `in`
  float* y[kGroupMax];           // [out] float32 output (not PAIR)
  uint16_t* act[kGroupMax];      // [padded(out)] bf16 silu(g) * u, zero past `out` (PAIR)
  int in, ld, out;
  int s_row, s_tile;  // scale of (row, tile) at s[row * s_row + tile * s_tile]
};

// Sum over 16 columns of int8 weight x bf16 activation (both exact in f32).
__device__ __forceinline__ float dot16(const u32x4& w, const u32x4& x0, const u32x4& x1) {
  float acc = 0.0f;
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const float q = (float)((int)(w[k >> 2] << (24 - 8 * (k & 3))) >> 24);
    const uint32_t xw = (k < 8 ? x0 : x1)[(k & 7) >> 1];
    acc = fmaf(q, (k & 1) ? bf_hi(xw) : bf_lo(xw), acc);
  }
  return acc;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

template <bool PAIR>
__global__ __launch_bounds__(64 * kWavesPerBlock) void expert_w8_kernel(ExpertArgs a) {
  const int slot = blockIdx.y;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int row0 = (blockIdx.x * kWavesPerBlock + wave) * kRows;
  if constexpr (PAIR) {
    // the act padding, which the down projection reads as zero
    if (blockIdx.x == 0 && wave == 0 && a.out + lane < padded_dev(a.out)) a.act[slot][a.out + lane] = 0;
  }
  if (row0 >= a.out) return;  // whole waves
  const int rows = min(kRows, a.out - row0);
  const int8_t* q = a.q[slot] + (size_t)row0 * a.ld;
  const int8_t* q2 = PAIR ? a.q2[slot] + (size_t)row0 * a.ld : nullptr;
  const uint16_t* x = a.x[slot];
  float tg[kRows] = {}, tu[kRows] = {};
  for (int t0 = 0; t0 < a.in; t0 += kTileCols) {
    const int t1 = min(t0 + kTileCols, a.in);
    // Every load is issued: a chunk past the tile reads the tile's first
    // chunk and a row past `rows` the wave's last row, and their products
    // are dropped below.
    u32x4 xv[2][2], w[kRows][2], u[PAIR ? kRows : 1][2];
    bool ok[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int c0 = t0 + (lane + 64 * j) * kChunk;
      ok[j] = c0 < t1;
      const int c = ok[j] ? c0 : t0;
      xv[j][0] = load16(x + c);
      xv[j][1] = load16(x + c + 8);
#pragma unroll
      for (int r = 0; r < kRows; ++r) {
        const size_t ro = (size_t)min(r, rows - 1) * a.ld + c;
        w[r][j] = load_stream16(q + ro);
        if constexpr (PAIR) u[r][j] = load_stream16(q2 + ro);
      }
    }
    auto dot = [&](const u32x4 (&v)[2]) {
      const float p0 = dot16(v[0], xv[0][0], xv[0][1]), p1 = dot16(v[1], xv[1][0], xv[1][1]);
      return (ok[0] ? p0 : 0.0f) + (ok[1] ? p1 : 0.0f);
    };
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
      const float pg = wave_sum(dot(w[r]));
      const int si = (row0 + r) * a.s_row + (t0 / kTileCols) * a.s_tile;
      if (r < rows) tg[r] += round_bf16(pg * a.s[slot][si]);
      if constexpr (PAIR) {
        const float pu = wave_sum(dot(u[r]));
        if (r < rows) tu[r] += round_bf16(pu * a.s2[slot][si]);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < kRows; ++r) {
    if (lane != r || r >= rows) continue;
    if constexpr (PAIR) {
      const float g = tg[r];
      a.act[slot][row0 + r] = (uint16_t)f32_to_bf16((g / (1.0f + expf(-g))) * tu[r]);
    } else {
      a.y[slot][row0 + r] = tg[r];
    }
  }
}

int launch_experts(const ExpertArgs& a, int slots, bool pair, hipStream_t stream) {
  if (slots < 1 || slots > kGroupMax || a.in <= 0 || a.out <= 0 || a.ld != padded(a.in) || a.s_row < 1 ||
      a.s_tile < 0)
    return fail("expert launch: bad shape");
  const dim3 grid((a.out + kRowsPerBlock - 1) / kRowsPerBlock, slots);
  if (pair)
    hipLaunchKernelGGL(expert_w8_kernel<true>, grid, dim3(64 * kWavesPerBlock), 0, stream, a);
  else
    hipLaunchKernelGGL(expert_w8_kernel<false>, grid, dim3(64 * kWavesPerBlock), 0, stream, a);
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? 0 : hip_fail(err, "expert launch");
}

// ---- GGML Q4_K / Q6_K ----

constexpr int kQK = 256;          // weights per GGML super-block
constexpr int kQ4KBytes = 144;    // d, dmin (fp16), 12 scale bytes, 128 quant bytes
constexpr int kQ6KBytes = 210;    // ql[128], qh[64], int8 scales[16], d (fp16)
constexpr int kTileBlocks = kTileCols / kQK;  // 8 blocks per tile: 8 lanes per block

enum SetKind : int { kW8Row = 0, kW8Tile = 1, kQ4K = HK_GGML_Q4_K, kQ6K = HK_GGML_Q6_K };

// Q4_K experts keep GGML's blocks ([out][in / 256][144], rows back to back).
// Q6_K experts are split into planes so that every load is aligned:
// ql [out][in / 2], qh [out][in / 4], scales [out][in / 16], d [out][in / 256].
struct QArgs {
  const uint8_t* w[kGroupMax];   // one expert's weights
  const uint16_t* x[kGroupMax];  // [in] bf16
  float* y[kGroupMax];           // [out]
  int in, out;                   // in a multiple of 256
};

__device__ __forceinline__ float f16_to_f32(uint32_t bits) {
  return (float)__builtin_bit_cast(_Float16, (unsigned short)(bits & 0xffffu));
}

// Quantised weights reach the dot product as bf16 pairs biased by 128: for a
// byte value n (0..63), bf16 0x4300 | n is exactly 128 + n, and
// v_dot2_f32_bf16 multiplies it by a bf16 activation without rounding (8 x 8
// significant bits).  sum (128 + n) x - 128 sum x is the unbiased sum; the
// activations stay in the packed pairs they are loaded as.
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c, false);
}

// Bytes 0, 1 (lo) or 2, 3 (hi) of `m` as a biased bf16 pair: one v_perm_b32
// each, selector bytes 4..7 taking bytes of `m`, 0 taking 0x43.
__device__ __forceinline__ uint32_t biased_lo(uint32_t m) { return __builtin_amdgcn_perm(m, 0x43434343u, 0x00050004u); }
__device__ __forceinline__ uint32_t biased_hi(uint32_t m) { return __builtin_amdgcn_perm(m, 0x43434343u, 0x00070006u); }

// sum over the 4 byte values of `m` times activations x0 (pair for bytes 0,
// 1) and x1 (bytes 2, 3), each value biased by 128.
__device__ __forceinline__ float dot_bytes4(uint32_t m, uint32_t x0, uint32_t x1, float acc) {
  return dot2(biased_hi(m), x1, dot2(biased_lo(m), x0, acc));
}

constexpr uint32_t kOnes = 0x3f803f80u;  // bf16 pair (1, 1)

// Sum of the 8 bf16 values of a 16-byte load.
__device__ __forceinline__ float sum8(const u32x4& v, float acc) {
#pragma unroll
  for (int k = 0; k < 4; ++k) acc = dot2(v[k], kOnes, acc);
  return acc;
}

// One lane's share of a Q4_K block: quant bytes 16 j .. 16 j + 15 of the
// block, i.e. sub-block 2g (low nibbles, columns 64 g + i) and 2g + 1 (high
// nibbles, columns 64 g + 32 + i) for i = 16 (j & 1) .. + 15, g = j / 2.
// xa / xb are those two runs of activations (8 bf16 each in a0/a1, b0/b1)
// and sa / sb their sums:
//   sum_i (d1 q_i - m1) x_i = d1 sum_i q_i x_i - m1 sum_i x_i.
__device__ __forceinline__ float q4k_lane(const u32x4& hdr, const u32x4& qv, int j, const u32x4& a0,
                                          const u32x4& a1, const u32x4& b0, const u32x4& b1, float sa, float sb) {
  const float d = f16_to_f32(hdr[0]), dmin = f16_to_f32(hdr[0] >> 16);
  // 6-bit scale and min of sub-block `idx` (GGML's get_scale_min_k4); scale
  // bytes 0..3 are hdr[1], 4..7 hdr[2], 8..11 hdr[3]
  auto scale_min = [&](int idx, uint32_t& sc, uint32_t& mn) {
    const uint32_t sh = 8 * (idx & 3);
    const uint32_t c0 = hdr[1] >> sh, c4 = hdr[2] >> sh, c8 = hdr[3] >> sh;
    const uint32_t sc_lo = c0 & 63u, mn_lo = c4 & 63u;
    const uint32_t sc_hi = (c8 & 15u) | (((c0 >> 6) & 3u) << 4);
    const uint32_t mn_hi = ((c8 >> 4) & 15u) | (((c4 >> 6) & 3u) << 4);
    sc = idx < 4 ? sc_lo : sc_hi;
    mn = idx < 4 ? mn_lo : mn_hi;
  };
  const int g = j >> 1;
  uint32_t sc1, mn1, sc2, mn2;
  scale_min(2 * g, sc1, mn1);
  scale_min(2 * g + 1, sc2, mn2);
  float pa = 0.0f, pb = 0.0f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    // quant word k holds columns 4k .. 4k + 3 of both runs
    const u32x4& xa = k < 2 ? a0 : a1;
    const u32x4& xb = k < 2 ? b0 : b1;
    const int w = 2 * (k & 1);
    pa = dot_bytes4(qv[k] & 0x0f0f0f0fu, xa[w], xa[w + 1], pa);
    pb = dot_bytes4((qv[k] >> 4) & 0x0f0f0f0fu, xb[w], xb[w + 1], pb);
  }
  const float d1 = d * (float)sc1, m1 = dmin * (float)mn1;
  const float d2 = d * (float)sc2, m2 = dmin * (float)mn2;
  return (d1 * (pa - 128.0f * sa) - m1 * sa) + (d2 * (pb - 128.0f * sb) - m2 * sb);
}

// One lane's share of a Q6_K half-block: l = l0 .. l0 + 7 of the half's 32,
// giving runs of 8 columns at l0 + 32 k (k = 0..3, xr[k], sums sx[k]), each
// under one scale: sum (d sc_k) (q - 32) x = d sc_k (sum q x - 32 sum x).
__device__ __forceinline__ float q6k_lane(uint2 qa, uint2 qb, uint2 qh, uint2 sc8, uint32_t dbits, int is,
                                          const u32x4 (&xr)[4], const float (&sx)[4]) {
  const float d = f16_to_f32(dbits);
  const uint64_t sc = (uint64_t)sc8.x | ((uint64_t)sc8.y << 32);
  float acc = 0.0f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    float p = 0.0f;
#pragma unroll
    for (int wv = 0; wv < 2; ++wv) {  // columns l0 + 4 wv .. + 3 of run k
      const uint32_t a = wv ? qa.y : qa.x, b = wv ? qb.y : qb.x, h = wv ? qh.y : qh.x;
      const uint32_t nib = (k == 0) ? (a & 0x0f0f0f0fu)
                           : (k == 1) ? (b & 0x0f0f0f0fu)
                           : (k == 2) ? ((a >> 4) & 0x0f0f0f0fu)
                                      : ((b >> 4) & 0x0f0f0f0fu);
      const uint32_t q = nib | (((h >> (2 * k)) & 0x03030303u) << 4);
      p = dot_bytes4(q, xr[k][2 * wv], xr[k][2 * wv + 1], p);
    }
    const float ds = d * (float)(int8_t)((sc >> (8 * (is + 2 * k))) & 0xffu);
    acc += ds * (p - 160.0f * sx[k]);  // biased by 128, then the format's 32
  }
  return acc;
}

// Each wave owns kRows rows; per 2048-column tile, lane L works on block
// 8 t + L / 8 of each row, so one tile is one pass of the wave.
template <int FMT>
__global__ __launch_bounds__(64 * kWavesPerBlock) void expert_q_kernel(QArgs a) {
  const int slot = blockIdx.y;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int row0 = (blockIdx.x * kWavesPerBlock + wave) * kRows;
  if (row0 >= a.out) return;  // whole waves
  const int rows = min(kRows, a.out - row0);
  const int nb = a.in / kQK;
  const int j = lane & 7;
  const uint8_t* base = a.w[slot];
  const uint16_t* x = a.x[slot];
  float total[kRows] = {};
  for (int t = 0; t * kTileBlocks < nb; ++t) {
    // Every load is issued: a lane past the last block reads the row's last
    // block and a row past `rows` the wave's last row; their results are
    // dropped (part = 0, no store).
    const int bl0 = t * kTileBlocks + (lane >> 3);
    const bool ok = bl0 < nb;
    const int bl = ok ? bl0 : nb - 1;
    float part[kRows];
    if constexpr (FMT == kQ4K) {
      const int col = bl * kQK + (j >> 1) * 64 + (j & 1) * 16;
      const u32x4 xa0 = load16(x + col), xa1 = load16(x + col + 8);
      const u32x4 xb0 = load16(x + col + 32), xb1 = load16(x + col + 40);
      u32x4 hdr[kRows], qv[kRows];
#pragma unroll
      for (int r = 0; r < kRows; ++r) {
        const uint8_t* blk = base + ((size_t)(row0 + min(r, rows - 1)) * nb + bl) * kQ4KBytes;
        hdr[r] = load_stream16(blk);
        qv[r] = load_stream16(blk + 16 + j * 16);
      }
      const float sa = sum8(xa1, sum8(xa0, 0.0f)), sb = sum8(xb1, sum8(xb0, 0.0f));
#pragma unroll
      for (int r = 0; r < kRows; ++r) {
        const float v = q4k_lane(hdr[r], qv[r], j, xa0, xa1, xb0, xb1, sa, sb);
        part[r] = ok ? v : 0.0f;
      }
    } else {
      const int h = j >> 2, l0 = (j & 3) * 8;
      const int col = bl * kQK + h * 128 + l0;
      u32x4 xr[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) xr[k] = load16(x + col + 32 * k);
      const size_t n = (size_t)a.out;
      const uint8_t* qh_plane = base + n * (a.in / 2);
      const uint8_t* sc_plane = qh_plane + n * (a.in / 4);
      const uint16_t* d_plane = reinterpret_cast<const uint16_t*>(sc_plane + n * (a.in / 16));
      uint2 qa[kRows], qb[kRows], qh[kRows], sc[kRows];
      uint32_t db[kRows];
#pragma unroll
      for (int r = 0; r < kRows; ++r) {
        const size_t row = (size_t)(row0 + min(r, rows - 1));
        const uint8_t* ql = base + row * (a.in / 2) + bl * 128 + h * 64 + l0;
        qa[r] = ldg_u2(ql);
        qb[r] = ldg_u2(ql + 32);
        qh[r] = ldg_u2(qh_plane + row * (a.in / 4) + bl * 64 + h * 32 + l0);
        sc[r] = ldg_u2(sc_plane + row * (a.in / 16) + bl * 16 + h * 8);
        db[r] = (uint32_t)ldg(d_plane + row * nb + bl);
      }
      float sx[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) sx[k] = sum8(xr[k], 0.0f);
#pragma unroll
      for (int r = 0; r < kRows; ++r) {
        const float v = q6k_lane(qa[r], qb[r], qh[r], sc[r], db[r], l0 >> 4, xr, sx);
        part[r] = ok ? v : 0.0f;
      }
    }
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
      const float p = wave_sum(part[r]);
      if (r < rows) total[r] += round_bf16(p);
    }
  }
#pragma unroll
  for (int r = 0; r < kRows; ++r)
    if (lane == r && r < rows) a.y[slot][row0 + r] = total[r];
}

int launch_quant(const QArgs& a, int slots, int kind, hipStream_t stream) {
  if (slots < 1 || slots > kGroupMax || a.in <= 0 || a.in % kQK || a.out <= 0)
    return fail("expert launch: bad shape");
  const dim3 grid((a.out + kRowsPerBlock - 1) / kRowsPerBlock, slots);
  if (kind == kQ4K)
    hipLaunchKernelGGL(expert_q_kernel<kQ4K>, grid, dim3(64 * kWavesPerBlock), 0, stream, a);
  else if (kind == kQ6K)
    hipLaunchKernelGGL(expert_q_kernel<kQ6K>, grid, dim3(64 * kWavesPerBlock), 0, stream, a);
  else
    return fail("expert launch: unknown weight type");
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? 0 : hip_fail(err, "expert launch");
}

// float32 -> bf16 bits, round to nearest even: ggml-xdna.cpp:178-183 and
// backend_xdna.cpp:35-40, which round NaN payloads like any other pattern.
inline uint16_t host_bf16(float v) {
  uint32_t bits;
  std::memcpy(&bits, &v, sizeof bits);
  return (uint16_t)((bits + 0x7fffu + ((bits >> 16) & 1u)) >> 16);
}

// `rows` float32 rows of `cols` values, `src_stride` apart, as bf16 rows of
// padded(cols) values with zeros after the last column.
void pack_inputs(const float* src, int rows, int cols, size_t src_stride, std::vector<uint16_t>& out) {
  const int ld = padded(cols);
  out.assign((size_t)rows * ld, 0);
  for (int r = 0; r < rows; ++r)
    for (int c = 0; c < cols; ++c) out[(size_t)r * ld + c] = host_bf16(src[r * src_stride + c]);
}

// Element (row, col) of a weight tensor in Colibri's upload formats
// (backend_xdna.cpp:122-136): 0 float32, 1 int8 x scale[row], 2 int4 (low
// nibble first, bias 8) x scale[row], 4 int4 x scale[row][col / group].
float weight_at(const void* w, const float* scales, int fmt, int in, int row, int col, int group) {
  const int64_t idx = (int64_t)row * in + col;
  if (fmt == 0) return static_cast<const float*>(w)[idx];
  if (fmt == 1) return static_cast<const int8_t*>(w)[idx] * scales[row];
  const uint8_t byte = static_cast<const uint8_t*>(w)[(int64_t)row * ((in + 1) / 2) + col / 2];
  const int v = ((col & 1) ? (byte >> 4) : (byte & 15)) - 8;
  if (fmt == 4) return v * scales[(int64_t)row * ((in + group - 1) / group) + col / group];
  return v * scales[row];
}

// int8 rows with scale max|w| / 127 (1 for a zero row), round half to even,
// clamped to +-127 (ggml-xdna.cpp:712-731, backend_xdna.cpp:138-157); rows
// are stored padded(in) apart with zeros after the last column.
template <class Get>
void requantise(int in, int out, Get get, std::vector<int8_t>& q, std::vector<float>& s) {
  const int ld = padded(in);
  q.assign((size_t)ld * out, 0);
  s.resize(out);
  std::vector<float> row(in);
  for (int r = 0; r < out; ++r) {
    float peak = 0.0f;
    for (int c = 0; c < in; ++c) {
      row[c] = get(r, c);
      peak = std::max(peak, std::fabs(row[c]));
    }
    const float scale = peak > 0.0f ? peak / 127.0f : 1.0f;
    s[r] = scale;
    for (int c = 0; c < in; ++c)
      q[(size_t)r * ld + c] = (int8_t)std::clamp(std::nearbyint(row[c] / scale), -127.0f, 127.0f);
  }
}

// Device scratch, grown on demand (bytes).
struct Scratch {
  char* buf = nullptr;
  size_t bytes = 0;
  int reserve(size_t n) {
    if (n <= bytes) return 0;
    if (buf) (void)hipFree(buf);
    buf = nullptr;
    bytes = 0;
    const hipError_t err = hipMalloc(&buf, n);
    if (err != hipSuccess) return hip_fail(err, "expert scratch");
    bytes = n;
    return 0;
  }
  void release() {
    if (buf) (void)hipFree(buf);
    buf = nullptr;
    bytes = 0;
  }
};

inline size_t align256(size_t n) { return (n + 255) / 256 * 256; }

}  // namespace
}  // namespace hk

using namespace hk;

// ---- GGML MUL_MAT_ID and MUL_MAT ----

// One GGML weight tensor on the device: n_experts matrices of out x in.
//   kW8Row   int8 [experts][out][ld] + float32 [experts][out]        (MUL_MAT_ID)
//   kW8Tile  int8 [out][ld] + float32 [out][tiles], one matrix        (MUL_MAT)
//   kQ4K     GGML Q4_K blocks, experts `stride` bytes apart           (both)
//   kQ6K     Q6_K planes, experts `stride` bytes apart                (both)
struct hk_ggml_experts {
  int kind = kW8Row;
  int64_t experts = 0, out = 0, in = 0, ld = 0, tiles = 1;
  size_t stride = 0;        // bytes between experts (quantised kinds)
  int8_t* q = nullptr;      // W8 weights
  float* s = nullptr;       // W8 scales
  uint8_t* blocks = nullptr;  // Q4_K / Q6_K weights
  Scratch scratch;          // bf16 inputs [rows][ld], then float32 outputs [n][out]
  const uint16_t* last_x = nullptr;  // the last call's device input and output,
  float* last_y = nullptr;           // for hk_ggml_mul_mat_id_repeat
  int last_slots = 0, last_input_rows = 0;
  std::vector<uint16_t> staging;
  std::mutex mu;
};

namespace {

constexpr int64_t kDenseRowsMax = 32768;  // ggml-xdna.cpp:1738
constexpr int64_t kQuantColsMax = 1 << 20;

// One launch over n slots: slot i uses expert ids[i] and input row 0 or i.
int launch_set(const hk_ggml_experts* set, const int32_t* ids, int n, int input_rows, const uint16_t* dx,
               float* dy, hipStream_t stream = nullptr) {
  if (set->kind == kQ4K || set->kind == kQ6K) {
    QArgs a{};
    a.in = (int)set->in;
    a.out = (int)set->out;
    for (int i = 0; i < n; ++i) {
      a.w[i] = set->blocks + (size_t)ids[i] * set->stride;
      a.x[i] = dx + (size_t)(input_rows == 1 ? 0 : i) * set->ld;
      a.y[i] = dy + (size_t)i * set->out;
    }
    return launch_quant(a, n, set->kind, stream);
  }
  ExpertArgs a{};
  a.in = (int)set->in;
  a.ld = (int)set->ld;
  a.out = (int)set->out;
  a.s_row = set->kind == kW8Tile ? (int)set->tiles : 1;
  a.s_tile = set->kind == kW8Tile ? 1 : 0;
  for (int i = 0; i < n; ++i) {
    a.q[i] = set->q + (size_t)ids[i] * set->out * set->ld;
    a.s[i] = set->s + (size_t)ids[i] * set->out * (set->kind == kW8Tile ? set->tiles : 1);
    a.x[i] = dx + (size_t)(input_rows == 1 ? 0 : i) * set->ld;
    a.y[i] = dy + (size_t)i * set->out;
  }
  return launch_experts(a, n, false, stream);
}

int check_ids(const hk_ggml_experts* set, const int32_t* ids, int64_t n) {
  for (int64_t i = 0; i < n; ++i)
    if (ids[i] < 0 || ids[i] >= set->experts) return fail("expert id out of range");
  return HK_OK;
}

// Input rows to the device, one launch, results back (holds set->mu).
int run_set(hk_ggml_experts* set, const float* input, int input_rows, const int32_t* ids, int n, float* out) {
  const size_t in_bytes = align256((size_t)input_rows * set->ld * 2), out_floats = (size_t)n * set->out;
  if (int rc = set->scratch.reserve(in_bytes + out_floats * sizeof(float))) return rc;
  auto* dx = reinterpret_cast<uint16_t*>(set->scratch.buf);
  auto* dy = reinterpret_cast<float*>(set->scratch.buf + in_bytes);
  pack_inputs(input, input_rows, (int)set->in, set->in, set->staging);
  hipError_t err = hipMemcpy(dx, set->staging.data(), set->staging.size() * 2, hipMemcpyHostToDevice);
  if (err != hipSuccess) return hip_fail(err, "expert input copy");
  if (int rc = launch_set(set, ids, n, input_rows, dx, dy)) return rc;
  set->last_x = dx;
  set->last_y = dy;
  set->last_slots = n;
  set->last_input_rows = input_rows;
  err = hipMemcpy(out, dy, out_floats * sizeof(float), hipMemcpyDeviceToHost);
  return err == hipSuccess ? HK_OK : hip_fail(err, "expert output copy");
}

// Q6_K blocks of one expert ([out][nb][210]) as planes (see QArgs).
void q6k_planes(const uint8_t* src, int64_t out, int64_t in, uint8_t* dst) {
  const int64_t nb = in / kQK;
  uint8_t* ql = dst;
  uint8_t* qh = ql + out * (in / 2);
  uint8_t* sc = qh + out * (in / 4);
  uint8_t* d = sc + out * (in / 16);
  for (int64_t r = 0; r < out; ++r)
    for (int64_t b = 0; b < nb; ++b) {
      const uint8_t* blk = src + (r * nb + b) * kQ6KBytes;
      std::memcpy(ql + r * (in / 2) + b * 128, blk, 128);
      std::memcpy(qh + r * (in / 4) + b * 64, blk + 128, 64);
      std::memcpy(sc + r * (in / 16) + b * 16, blk + 192, 16);
      std::memcpy(d + (r * nb + b) * 2, blk + 208, 2);
    }
}

}  // namespace

extern "C" {

int hk_ggml_experts_supported(int64_t in_dim, int64_t out_dim, int64_t n_experts, int64_t n_ids,
                              int64_t input_rows) {
  return in_dim > 0 && in_dim <= kGgmlDimMax && out_dim > 0 && out_dim <= kGgmlDimMax &&
         n_experts >= kGroupMax && n_ids >= 1 && n_ids <= kGroupMax && (input_rows == 1 || input_rows == n_ids);
}

int hk_ggml_dense_supported(int64_t in_dim, int64_t out_dim, int64_t input_rows) {
  return in_dim > 0 && out_dim > 0 && out_dim <= kDenseRowsMax && input_rows == 1;
}

int hk_ggml_quant_supported(int ggml_type, int64_t in_dim) {
  return (ggml_type == HK_GGML_Q4_K || ggml_type == HK_GGML_Q6_K) && in_dim > 0 && in_dim % kQK == 0 &&
         in_dim <= kQuantColsMax;
}

int hk_ggml_experts_create(const float* weights, int64_t n_experts, int64_t out_dim, int64_t in_dim,
                           hk_ggml_experts** out) {
  if (!weights || !out) return fail("hk_ggml_experts_create: null argument");
  *out = nullptr;
  if (n_experts < 1 || out_dim < 1 || in_dim < 1 || out_dim > kGgmlDimMax || in_dim > kGgmlDimMax)
    return fail("hk_ggml_experts_create: shape outside the MUL_MAT_ID contract");
  auto* set = new hk_ggml_experts;
  set->kind = kW8Row;
  set->experts = n_experts;
  set->out = out_dim;
  set->in = in_dim;
  set->ld = padded((int)in_dim);
  const size_t per_w = (size_t)out_dim * in_dim, per_q = (size_t)out_dim * set->ld;
  hipError_t err = hipMalloc(&set->q, per_q * n_experts);
  if (err == hipSuccess) err = hipMalloc(&set->s, (size_t)out_dim * n_experts * sizeof(float));
  std::vector<int8_t> q;
  std::vector<float> s;
  for (int64_t e = 0; e < n_experts && err == hipSuccess; ++e) {
    const float* w = weights + e * per_w;
    requantise((int)in_dim, (int)out_dim, [&](int r, int c) { return w[(size_t)r * in_dim + c]; }, q, s);
    err = hipMemcpy(set->q + e * per_q, q.data(), per_q, hipMemcpyHostToDevice);
    if (err == hipSuccess)
      err = hipMemcpy(set->s + e * out_dim, s.data(), out_dim * sizeof(float), hipMemcpyHostToDevice);
  }
  if (err != hipSuccess) {
    hk_ggml_experts_destroy(set);
    return hip_fail(err, "hk_ggml_experts_create");
  }
  *out = set;
  return HK_OK;
}

int hk_ggml_dense_create(const float* weights, int64_t out_dim, int64_t in_dim, hk_ggml_experts** out) {
  if (!weights || !out) return fail("hk_ggml_dense_create: null argument");
  *out = nullptr;
  if (!hk_ggml_dense_supported(in_dim, out_dim, 1) || in_dim > kQuantColsMax)
    return fail("hk_ggml_dense_create: shape outside the dense MUL_MAT contract");
  auto* set = new hk_ggml_experts;
  set->kind = kW8Tile;
  set->experts = 1;
  set->out = out_dim;
  set->in = in_dim;
  set->ld = padded((int)in_dim);
  set->tiles = (in_dim + kTileCols - 1) / kTileCols;
  // one scale per (row, tile): max over the tile's columns (ggml-xdna.cpp:800-826)
  std::vector<int8_t> q((size_t)out_dim * set->ld, 0);
  std::vector<float> s((size_t)out_dim * set->tiles);
  for (int64_t r = 0; r < out_dim; ++r) {
    const float* row = weights + r * in_dim;
    for (int64_t t = 0; t < set->tiles; ++t) {
      const int64_t c0 = t * kTileCols, c1 = std::min<int64_t>(c0 + kTileCols, in_dim);
      float peak = 0.0f;
      for (int64_t c = c0; c < c1; ++c) peak = std::max(peak, std::fabs(row[c]));
      const float scale = peak > 0.0f ? peak / 127.0f : 1.0f;
      s[r * set->tiles + t] = scale;
      for (int64_t c = c0; c < c1; ++c)
        q[r * set->ld + c] = (int8_t)std::clamp(std::nearbyint(row[c] / scale), -127.0f, 127.0f);
    }
  }
  hipError_t err = hipMalloc(&set->q, q.size());
  if (err == hipSuccess) err = hipMalloc(&set->s, s.size() * sizeof(float));
  if (err == hipSuccess) err = hipMemcpy(set->q, q.data(), q.size(), hipMemcpyHostToDevice);
  if (err == hipSuccess) err = hipMemcpy(set->s, s.data(), s.size() * sizeof(float), hipMemcpyHostToDevice);
  if (err != hipSuccess) {
    hk_ggml_experts_destroy(set);
    return hip_fail(err, "hk_ggml_dense_create");
  }
  *out = set;
  return HK_OK;
}

int hk_ggml_quant_create(int ggml_type, const void* blocks, int64_t n_experts, int64_t out_dim, int64_t in_dim,
                         hk_ggml_experts** out) {
  if (!blocks || !out) return fail("hk_ggml_quant_create: null argument");
  *out = nullptr;
  if (!hk_ggml_quant_supported(ggml_type, in_dim))
    return fail("hk_ggml_quant_create: type must be Q4_K or Q6_K and in_dim a multiple of 256");
  if (n_experts < 1 || out_dim < 1 || out_dim > kDenseRowsMax)
    return fail("hk_ggml_quant_create: bad expert count or output dimension");
  auto* set = new hk_ggml_experts;
  set->kind = ggml_type;
  set->experts = n_experts;
  set->out = out_dim;
  set->in = in_dim;
  set->ld = in_dim;
  const int64_t nb = in_dim / kQK;
  const size_t src_bytes = (size_t)out_dim * nb * (ggml_type == kQ4K ? kQ4KBytes : kQ6KBytes);
  set->stride = align256(src_bytes);
  hipError_t err = hipMalloc(&set->blocks, set->stride * n_experts);
  std::vector<uint8_t> planes(ggml_type == kQ6K ? src_bytes : 0);
  for (int64_t e = 0; e < n_experts && err == hipSuccess; ++e) {
    const uint8_t* src = static_cast<const uint8_t*>(blocks) + e * src_bytes;
    if (ggml_type == kQ6K) {
      q6k_planes(src, out_dim, in_dim, planes.data());
      src = planes.data();
    }
    err = hipMemcpy(set->blocks + e * set->stride, src, src_bytes, hipMemcpyHostToDevice);
  }
  if (err != hipSuccess) {
    hk_ggml_experts_destroy(set);
    return hip_fail(err, "hk_ggml_quant_create");
  }
  *out = set;
  return HK_OK;
}

int hk_ggml_mul_mat_id(hk_ggml_experts* set, const float* input, int64_t input_rows, const int32_t* ids,
                       int64_t n_ids, float* out) {
  if (!set || !input || !ids || !out) return fail("hk_ggml_mul_mat_id: null argument");
  if (set->kind == kW8Tile) return fail("hk_ggml_mul_mat_id: a dense weight set takes hk_ggml_mul_mat");
  if (set->in > kGgmlDimMax || set->out > kGgmlDimMax)
    return fail("hk_ggml_mul_mat_id: weights wider than the MUL_MAT_ID contract's 2048");
  if (n_ids < 1 || n_ids > kGroupMax || (input_rows != 1 && input_rows != n_ids))
    return fail("hk_ggml_mul_mat_id: ids or input rows outside the MUL_MAT_ID contract");
  if (int rc = check_ids(set, ids, n_ids)) return rc;
  std::lock_guard<std::mutex> lock(set->mu);
  return run_set(set, input, (int)input_rows, ids, (int)n_ids, out);
}

int hk_ggml_mul_mat(hk_ggml_experts* set, const float* input, float* out) {
  if (!set || !input || !out) return fail("hk_ggml_mul_mat: null argument");
  if (set->kind == kW8Row || set->experts != 1)
    return fail("hk_ggml_mul_mat: needs a dense set (hk_ggml_dense_create, or quantised with one matrix)");
  const int32_t id = 0;
  std::lock_guard<std::mutex> lock(set->mu);
  return run_set(set, input, 1, &id, 1, out);
}

int hk_ggml_mul_mat_id_repeat(hk_ggml_experts* set, const int32_t* ids, int64_t launches, float* ms_per_launch) {
  if (!set || !ids || !ms_per_launch || launches < 1) return fail("hk_ggml_mul_mat_id_repeat: bad argument");
  std::lock_guard<std::mutex> lock(set->mu);
  const int n = set->last_slots;
  if (n < 1) return fail("hk_ggml_mul_mat_id_repeat: no earlier call on this set");
  if (int rc = check_ids(set, ids, launches * n)) return rc;
  // The launches are captured into a graph and replayed once untimed, once
  // between two events, so that the host's per-launch cost stays out of the
  // figure.  HK_EAGER=1 launches them directly instead (profilers that
  // cannot follow graph launches).
  const char* eager_env = std::getenv("HK_EAGER");
  const bool eager = eager_env && eager_env[0] == '1';
  hipStream_t stream = nullptr;
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  int rc = HK_OK;
  auto enqueue = [&]() {
    for (int64_t i = 0; i < launches && rc == HK_OK; ++i)
      rc = launch_set(set, ids + i * n, n, set->last_input_rows, set->last_x, set->last_y, stream);
  };
  hipError_t err = hipStreamCreateWithFlags(&stream, hipStreamNonBlocking);
  if (!eager) {
    if (err == hipSuccess) err = hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal);
    if (err == hipSuccess) {
      enqueue();
      err = hipStreamEndCapture(stream, &graph);
    }
    if (err == hipSuccess && rc == HK_OK) err = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    if (err == hipSuccess && rc == HK_OK) err = hipGraphLaunch(exec, stream);
  }
  if (err == hipSuccess && rc == HK_OK) err = hipEventCreate(&e0);
  if (err == hipSuccess && rc == HK_OK) err = hipEventCreate(&e1);
  if (err == hipSuccess && rc == HK_OK) err = hipEventRecord(e0, stream);
  if (err == hipSuccess && rc == HK_OK) {
    if (eager)
      enqueue();
    else
      err = hipGraphLaunch(exec, stream);
  }
  if (err == hipSuccess && rc == HK_OK) err = hipEventRecord(e1, stream);
  if (err == hipSuccess && rc == HK_OK) err = hipEventSynchronize(e1);
  float ms = 0.0f;
  if (err == hipSuccess && rc == HK_OK) err = hipEventElapsedTime(&ms, e0, e1);
  if (stream) (void)hipStreamSynchronize(stream);
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  if (exec) (void)hipGraphExecDestroy(exec);
  if (graph) (void)hipGraphDestroy(graph);
  if (stream) (void)hipStreamDestroy(stream);
  if (rc != HK_OK) return rc;
  if (err != hipSuccess) return hip_fail(err, "hk_ggml_mul_mat_id_repeat");
  *ms_per_launch = ms / (float)launches;
  return HK_OK;
}

void hk_ggml_experts_destroy(hk_ggml_experts* set) {
  if (!set) return;
  if (set->q) (void)hipFree(set->q);
  if (set->s) (void)hipFree(set->s);
  if (set->blocks) (void)hipFree(set->blocks);
  set->scratch.release();
  delete set;
}

}  // extern "C"

// ---- Colibri ----

struct ColiCudaTensor {
  int fmt = 0, input = 0, output = 0, group = 0, device = 0;
  int8_t* q = nullptr;  // [output][padded(input)]
  float* s = nullptr;   // [output]
};

namespace {

struct ColiRuntime {
  std::atomic<bool> up{false};
  Scratch scratch;
  std::vector<uint16_t> staging;
  std::mutex mu;
};

ColiRuntime& coli() {
  static ColiRuntime rt;
  return rt;
}

bool coli_pack(ColiCudaTensor* t, const void* weights, const float* scales) {
  if (!t || !weights || t->input <= 0 || t->output <= 0 || (t->fmt == 4 && t->group <= 0)) return false;
  if (t->fmt < 0 || t->fmt > 4 || t->fmt == 3) return false;
  std::vector<int8_t> q;
  std::vector<float> s;
  requantise(t->input, t->output,
             [&](int r, int c) { return weight_at(weights, scales, t->fmt, t->input, r, c, t->group); }, q, s);
  if (!t->q && hipMalloc(&t->q, q.size()) != hipSuccess) return false;
  if (!t->s && hipMalloc(&t->s, s.size() * sizeof(float)) != hipSuccess) return false;
  return hipMemcpy(t->q, q.data(), q.size(), hipMemcpyHostToDevice) == hipSuccess &&
         hipMemcpy(t->s, s.data(), s.size() * sizeof(float), hipMemcpyHostToDevice) == hipSuccess;
}

// Copies `rows` float32 input rows (back to back) into the scratch as padded
// bf16 rows, reserving `extra_bytes` after them (returned in *rest); returns
// the rows' device address, or null on failure.  Holds coli().mu.
uint16_t* coli_stage_inputs(const float* input, int rows, int cols, size_t extra_bytes, char** rest) {
  ColiRuntime& rt = coli();
  const size_t in_bytes = align256((size_t)rows * padded(cols) * 2);
  if (rt.scratch.reserve(in_bytes + extra_bytes)) return nullptr;
  pack_inputs(input, rows, cols, cols, rt.staging);
  if (hipMemcpy(rt.scratch.buf, rt.staging.data(), rt.staging.size() * 2, hipMemcpyHostToDevice) != hipSuccess)
    return nullptr;
  *rest = rt.scratch.buf + in_bytes;
  return reinterpret_cast<uint16_t*>(rt.scratch.buf);
}

}  // namespace

extern "C" {

int coli_cuda_init(const int* devices, int count) {
  if (count != 1 || !devices || devices[0] != 0) return 0;
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n < 1) return 0;
  coli().up = true;
  return 1;
}

void coli_cuda_shutdown(void) {
  std::lock_guard<std::mutex> lock(coli().mu);
  coli().scratch.release();
  coli().up = false;
}

int coli_cuda_available_device_count(void) {
  int n = 0;
  return hipGetDeviceCount(&n) == hipSuccess && n > 0 ? 1 : 0;
}
int coli_cuda_device_count(void) { return coli().up ? 1 : 0; }
int coli_cuda_device_at(int index) { return index == 0 && coli().up ? 0 : -1; }

int coli_cuda_tensor_upload_g(ColiCudaTensor** out, const void* weights, const float* scales, int fmt,
                              int input, int output, int device, int group) {
  if (!out || device != 0 || !coli().up || !weights || (fmt != 0 && !scales)) return 0;
  auto* t = new ColiCudaTensor;
  t->fmt = fmt;
  t->input = input;
  t->output = output;
  t->group = group;
  if (!coli_pack(t, weights, scales)) {
    coli_cuda_tensor_free(t);
    return 0;
  }
  *out = t;
  return 1;
}

int coli_cuda_tensor_upload(ColiCudaTensor** out, const void* weights, const float* scales, int fmt, int input,
                            int output, int device) {
  return coli_cuda_tensor_upload_g(out, weights, scales, fmt, input, output, device, 0);
}

void coli_cuda_tensor_free(ColiCudaTensor* t) {
  if (!t) return;
  if (t->q) (void)hipFree(t->q);
  if (t->s) (void)hipFree(t->s);
  delete t;
}

int coli_cuda_tensor_device(const ColiCudaTensor* t) { return t ? t->device : -1; }

int coli_cuda_tensor_update(ColiCudaTensor* t, const void* weights, const float* scales) {
  return coli_pack(t, weights, scales) ? 1 : 0;
}

int coli_cuda_expert_group_pinned(ColiCudaTensor* const* gate, ColiCudaTensor* const* up,
                                  ColiCudaTensor* const* down, const int* rows, int count, float* output,
                                  const float* input, int) {
  if (!coli().up || !gate || !up || !down || !rows || !output || !input || count < 1 || count > kGroupMax)
    return 0;
  for (int i = 0; i < count; ++i) {
    if (rows[i] != 1 || !gate[i] || !up[i] || !down[i] || gate[i]->input != up[i]->input ||
        gate[i]->output != up[i]->output || down[i]->input != gate[i]->output ||
        down[i]->output != gate[i]->input)
      return 0;
    // a stage runs only over tensors of one shape (backend_xdna.cpp:164-172)
    if (gate[i]->input != gate[0]->input || gate[i]->output != gate[0]->output) return 0;
  }
  const int in = gate[0]->input, mid = gate[0]->output;
  const int ld_in = padded(in), ld_mid = padded(mid);
  std::lock_guard<std::mutex> lock(coli().mu);
  const size_t act_bytes = align256((size_t)count * ld_mid * 2), ny = (size_t)count * in;
  char* rest = nullptr;
  uint16_t* dx = coli_stage_inputs(input, count, in, act_bytes + ny * sizeof(float), &rest);
  if (!dx) return 0;
  auto* dact = reinterpret_cast<uint16_t*>(rest);
  auto* dy = reinterpret_cast<float*>(rest + act_bytes);
  // gate and up rows in pairs, writing bf16(silu(g) * u)
  ExpertArgs a{};
  a.in = in;
  a.ld = ld_in;
  a.out = mid;
  a.s_row = 1;
  for (int i = 0; i < count; ++i) {
    a.q[i] = gate[i]->q;
    a.s[i] = gate[i]->s;
    a.q2[i] = up[i]->q;
    a.s2[i] = up[i]->s;
    a.x[i] = dx + (size_t)i * ld_in;
    a.act[i] = dact + (size_t)i * ld_mid;
  }
  if (launch_experts(a, count, true, nullptr)) return 0;
  ExpertArgs b{};
  b.in = mid;
  b.ld = ld_mid;
  b.out = in;
  b.s_row = 1;
  for (int i = 0; i < count; ++i) {
    b.q[i] = down[i]->q;
    b.s[i] = down[i]->s;
    b.x[i] = dact + (size_t)i * ld_mid;
    b.y[i] = dy + (size_t)i * in;
  }
  if (launch_experts(b, count, false, nullptr)) return 0;
  return hipMemcpy(output, dy, ny * sizeof(float), hipMemcpyDeviceToHost) == hipSuccess ? 1 : 0;
}

int coli_cuda_expert_group(ColiCudaTensor* const* gate, ColiCudaTensor* const* up, ColiCudaTensor* const* down,
                           const int* rows, int count, float* output, const float* input) {
  return coli_cuda_expert_group_pinned(gate, up, down, rows, count, output, input, 0);
}

int coli_cuda_expert_mlp(ColiCudaTensor* gate, ColiCudaTensor* up, ColiCudaTensor* down, float* output,
                         const float* input, int rows) {
  ColiCudaTensor* g[] = {gate};
  ColiCudaTensor* u[] = {up};
  ColiCudaTensor* d[] = {down};
  int r[] = {rows};
  return coli_cuda_expert_group(g, u, d, r, 1, output, input);
}

int coli_cuda_matmul(ColiCudaTensor** tensor, float* output, const float* input, const void* weights,
                     const float* scales, int fmt, int rows, int input_size, int output_size, int device,
                     int group) {
  if (!tensor || !output || !input || rows != 1) return 0;
  if (!*tensor && !coli_cuda_tensor_upload_g(tensor, weights, scales, fmt, input_size, output_size, device, group))
    return 0;
  ColiCudaTensor* t = *tensor;
  if (!coli().up) return 0;
  std::lock_guard<std::mutex> lock(coli().mu);
  char* rest = nullptr;
  uint16_t* dx = coli_stage_inputs(input, 1, t->input, (size_t)t->output * sizeof(float), &rest);
  if (!dx) return 0;
  auto* dy = reinterpret_cast<float*>(rest);
  ExpertArgs a{};
  a.in = t->input;
  a.ld = padded(t->input);
  a.out = t->output;
  a.s_row = 1;
  a.q[0] = t->q;
  a.s[0] = t->s;
  a.x[0] = dx;
  a.y[0] = dy;
  if (launch_experts(a, 1, false, nullptr)) return 0;
  return hipMemcpy(output, dy, (size_t)t->output * sizeof(float), hipMemcpyDeviceToHost) == hipSuccess ? 1 : 0;
}

}  // extern "C"
