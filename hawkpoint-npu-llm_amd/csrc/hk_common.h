// Device-side helpers shared by every hk kernel (gfx950, wave64).
//
// BF16 values travel as uint16 bit patterns.  The float32 -> bfloat16 cast is
// round-to-nearest-even (NaN stays a quiet NaN), the same rounding the
// reference's CPU runtime gets from ml_dtypes (npu_llm/runtime/cpu_backend.py:7-8)
// and writes out as integer code in npu_llm/kernels/qwen_engine_common.h:35-46.
//
// All hk sources are compiled with -ffp-contract=off, so a*b+c below is two
// rounded operations exactly as NumPy evaluates it; fused multiply-adds are
// written out as fmaf() where the reference's summation order is not fixed
// anyway (dot products).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hk {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

// One v_cvt_pk_bf16_f32 (gfx950), round to nearest even.  Run on the device
// over all 2^32 float32 bit patterns it gives exactly
//   (u + 0x7fff + ((u >> 16) & 1)) >> 16   (u the float's bits)
// for every non-NaN input; a NaN stays a quiet NaN of the same sign.
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}

// Two floats as one packed bf16 pair (lo in bits 0..15), one instruction.
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t f32x2_to_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t{lo, hi}), bf16x2_t));
}

__device__ __forceinline__ float round_bf16(float f) {
  return bf16_to_f32(f32_to_bf16(f));
}

// Low / high bf16 of a packed 32-bit word (element 2i is the low half).
__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Buffer resource over [base, base + bytes): loads through it take a 32-bit
// byte offset, and offsets past `bytes` read zero instead of faulting, so a
// load that may fall outside needs no branch around it.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes, 0x00020000);
}

// Global-memory accesses go through address-space-1 pointers.  Through a
// generic pointer the compiler emits flat instructions, which count in both
// the vector-memory and the LDS counter, so every later LDS access would wait
// for all outstanding global loads and stores.
typedef __attribute__((address_space(1))) const u32x4 global_u32x4;

// (scalar and ext_vector types)
template <typename T>
__device__ __forceinline__ T ldg(const T* p) {
  return *(const __attribute__((address_space(1))) T*)p;
}

template <typename T>
__device__ __forceinline__ void stg(T* p, T v) {
  *(__attribute__((address_space(1))) T*)p = v;
}

// 8 bytes as two 32-bit words (ldg takes scalar types only).
__device__ __forceinline__ uint2 ldg_u2(const void* p) {
  const unsigned long long v = ldg(reinterpret_cast<const unsigned long long*>(p));
  return make_uint2((unsigned int)v, (unsigned int)(v >> 32));
}

// Streaming 16-byte load that does not allocate in the caches: every weight
// byte is read exactly once per decode step.
__device__ __forceinline__ u32x4 load_stream16(const void* p) {
  return __builtin_nontemporal_load((global_u32x4*)p);
}

__device__ __forceinline__ u32x4 load16(const void* p) { return *(global_u32x4*)p; }

// Two int8 weights (bytes lo, lo + 1 of w) as one packed bf16 pair: each
// becomes a float exactly, and integers up to 127 need 7 significant bits,
// so the float's high half is the exact bf16; v_perm_b32 takes both halves.
__device__ __forceinline__ uint32_t i8pair_bf16(uint32_t w, int lo) {
  const float f0 = (float)(int)(int8_t)(w >> (8 * lo));
  const float f1 = (float)(int)(int8_t)(w >> (8 * lo + 8));
  return __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, f1), __builtin_bit_cast(uint32_t, f0), 0x07060302u);
}

// Eight int8 weights (one streaming 8-byte load) as eight bf16 values, in order.
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ u32x4 load_stream_i8_bf16(const void* p) {
  const u32x2_t q = __builtin_nontemporal_load((__attribute__((address_space(1))) const u32x2_t*)p);
  return u32x4{i8pair_bf16(q.x, 0), i8pair_bf16(q.x, 2), i8pair_bf16(q.y, 0), i8pair_bf16(q.y, 2)};
}

// Sum over each group of W adjacent lanes (W = 8, 16, 32 or 64) with DPP row
// moves, a few cycles each against an LDS round trip per ds_bpermute step
// (what __shfl_xor compiles to): swap neighbours (quad_perm 1,0,3,2), swap
// pairs (2,3,0,1), pair quads (row_half_mirror), pair half-rows (row_mirror),
// each step adding lanes that hold equal partial sums, so every lane of a
// group ends with its total.  W = 32 adds the other row with one shuffle;
// W = 64 adds the rows with row_bcast15 / row_bcast31 and hands lane 63's
// total to the whole wave.
template <int CTRL, int ROWS = 0xf>
__device__ __forceinline__ float lane_dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROWS, 0xf, false));
}
template <int W>
__device__ __forceinline__ float lane_sum(float v) {
  static_assert(W == 8 || W == 16 || W == 32 || W == 64, "8, 16, 32 or 64 lanes");
  v += lane_dpp<0xb1>(v);   // quad_perm 1,0,3,2
  v += lane_dpp<0x4e>(v);   // quad_perm 2,3,0,1
  v += lane_dpp<0x141>(v);  // row_half_mirror
  if constexpr (W >= 16) v += lane_dpp<0x140>(v);  // row_mirror
  if constexpr (W == 32) v += __shfl_xor(v, 16, 64);
  if constexpr (W == 64) {
    v += lane_dpp<0x142, 0xa>(v);  // row_bcast15 into rows 1 and 3
    v += lane_dpp<0x143, 0x8>(v);  // row_bcast31 into row 3
    v = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
  }
  return v;
}

// Butterfly sum over groups of `width` adjacent lanes (width a power of two).
template <int width>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int m = width / 2; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

template <int width>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
  for (int m = width / 2; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
  return v;
}

__device__ __forceinline__ uint64_t umax64(uint64_t a, uint64_t b) { return a > b ? a : b; }

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int m) {
  const uint32_t lo = __shfl_xor((uint32_t)v, m, 64);
  const uint32_t hi = __shfl_xor((uint32_t)(v >> 32), m, 64);
  return ((uint64_t)hi << 32) | lo;
}

// Order-preserving 64-bit key for argmax: larger logit wins; on equal logits
// the lower index wins (np.argmax returns the first maximum).  -0.0 is folded
// into +0.0 so the two compare equal, as they do in NumPy.
__device__ __forceinline__ uint64_t argmax_key(float v, uint32_t index) {
  v = v + 0.0f;
  uint32_t u = __float_as_uint(v);
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((uint64_t)u << 32) | (uint64_t)(0xffffffffu - index);
}

__device__ __forceinline__ uint32_t argmax_key_index(uint64_t key) {
  return 0xffffffffu - (uint32_t)(key & 0xffffffffu);
}

// Eight float32 probabilities as three bf16 terms each, packed in pairs as
// the 8-element B operand of a bf16 MFMA (element e in the half e % 2 of
// word e / 2): hi holds each value's top 8 significant bits, mid those of
// the exact remainder, lo those of the remainder after that.  Each
// truncation leaves a remainder that float32 represents exactly, so
// hi + mid + lo is the value itself (24 significant bits; values are
// probabilities in [0, 1], so mid and lo stay normal or tiny enough not
// to matter).  A P @ V product summed over the three terms with bf16 V
// gives float32 P @ V, up to the float32 summation order.
__device__ __forceinline__ void split3_bf16(const float (&p)[8], u32x4& hi, u32x4& mid, u32x4& lo) {
  // the remainders are exact (Sterbenz), and the last one has at most 8
  // significant bits, so its float32 encoding ends in 16 zero bits: every
  // term is the top half of a float32 word, picked in pairs by v_perm_b32
  float r[8], q[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    r[e] = p[e] - __uint_as_float(__float_as_uint(p[e]) & 0xffff0000u);
    q[e] = r[e] - __uint_as_float(__float_as_uint(r[e]) & 0xffff0000u);
  }
  constexpr uint32_t kTops = 0x07060302u;  // bytes 2, 3 of the second operand, then of the first
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    hi[w] = __builtin_amdgcn_perm(__float_as_uint(p[2 * w + 1]), __float_as_uint(p[2 * w]), kTops);
    mid[w] = __builtin_amdgcn_perm(__float_as_uint(r[2 * w + 1]), __float_as_uint(r[2 * w]), kTops);
    lo[w] = __builtin_amdgcn_perm(__float_as_uint(q[2 * w + 1]), __float_as_uint(q[2 * w]), kTops);
  }
}

}  // namespace hk
