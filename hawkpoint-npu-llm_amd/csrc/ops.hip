// Small standalone kernels: RMSNorm, SwiGLU and argmax.
//
// The decode step fuses RMSNorm into the GEMV prologue and SwiGLU into the
// gate/up epilogue (gemv.hip); these separate forms serve the SmolLM-style
// engine output (final-normed hidden state, npu_llm/runtime/engine.py:65-82),
// the argmax of host-supplied logits, and the per-op parity tests.
#include "hk_common.h"
#include "hk_internal.h"

namespace hk {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;

// cpu_backend.py:71-76.
__global__ __launch_bounds__(kThreads) void rmsnorm_kernel(const uint16_t* x,
                                                           const uint16_t* gamma, float eps,
                                                           uint16_t* out, int n) {
  __shared__ float red[kWaves];
  const int tid = threadIdx.x;
  float ss = 0.0f;
  for (int i = tid; i < n; i += kThreads) {
    const float v = bf16_to_f32(x[i]);
    ss += v * v;
  }
  ss = group_sum<64>(ss);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  float total = red[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) total += red[w];
  const float inv = 1.0f / sqrtf(total / (float)n + eps);
  for (int i = tid; i < n; i += kThreads)
    out[i] = (uint16_t)f32_to_bf16((bf16_to_f32(x[i]) * inv) * bf16_to_f32(gamma[i]));
}

// cpu_backend.py:154-165 on a [gate | up] vector of bf16 values.
__global__ __launch_bounds__(kThreads) void swiglu_kernel(const uint16_t* gu, uint16_t* act,
                                                          int inter) {
  const int i = blockIdx.x * kThreads + threadIdx.x;
  if (i >= inter) return;
  const float g = bf16_to_f32(gu[i]);
  const float u = bf16_to_f32(gu[i + inter]);
  const float clipped = fminf(fmaxf(g, -80.0f), 80.0f);
  act[i] = (uint16_t)f32_to_bf16((g / (1.0f + expf(-clipped))) * u);
}

// np.argmax over float32 (generate.py:709-714): first maximum wins.
__global__ __launch_bounds__(kThreads) void argmax_kernel(const float* x, int n, ArgmaxState* am,
                                                          int32_t* out_index) {
  __shared__ unsigned long long keys[kWaves];
  const int tid = threadIdx.x;
  unsigned long long key = 0ull;
  for (int i = blockIdx.x * kThreads + tid; i < n; i += gridDim.x * kThreads)
    key = umax64(key, argmax_key(x[i], (uint32_t)i));
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) key = umax64(key, shfl_xor_u64(key, m));
  if ((tid & 63) == 0) keys[tid >> 6] = key;
  __syncthreads();
  if (tid != 0) return;
  unsigned long long k = keys[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) k = umax64(k, keys[w]);
  atomicMax(&am->key, k);
  __threadfence();
  if (atomicAdd(&am->count, 1u) == gridDim.x - 1) {
    __threadfence();
    *out_index = (int32_t)argmax_key_index(atomicAdd(&am->key, 0ull));
    atomicExch(&am->key, 0ull);
    atomicExch(&am->count, 0u);
  }
}

}  // namespace

int launch_rmsnorm(const uint16_t* x, const uint16_t* gamma, float eps, uint16_t* out, int n,
                   hipStream_t stream) {
  if (n <= 0) return fail("rmsnorm: size must be positive");
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(1), dim3(kThreads), 0, stream, x, gamma, eps, out, n);
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? 0 : hip_fail(err, "rmsnorm launch");
}

int launch_swiglu(const uint16_t* gate_up, uint16_t* act, int inter, hipStream_t stream) {
  if (inter <= 0) return fail("swiglu: size must be positive");
  hipLaunchKernelGGL(swiglu_kernel, dim3((inter + kThreads - 1) / kThreads), dim3(kThreads), 0,
                     stream, gate_up, act, inter);
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? 0 : hip_fail(err, "swiglu launch");
}

int launch_argmax(const float* x, int n, ArgmaxState* am, int32_t* out_index,
                  hipStream_t stream) {
  if (n <= 0) return fail("argmax: size must be positive");
  int blocks = (n + kThreads * 4 - 1) / (kThreads * 4);
  if (blocks > 1024) blocks = 1024;
  hipLaunchKernelGGL(argmax_kernel, dim3(blocks), dim3(kThreads), 0, stream, x, n, am, out_index);
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? 0 : hip_fail(err, "argmax launch");
}

}  // namespace hk
