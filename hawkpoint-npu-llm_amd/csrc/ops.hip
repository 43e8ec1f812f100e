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

// np.argmax over float32 (generate.py:709-714): first maximum wins.  Each
// workgroup writes one partial key; argmax_finalize_kernel reduces them.
__global__ __launch_bounds__(kThreads) void argmax_partial_kernel(const float* x, int n,
                                                                  unsigned long long* keys) {
  __shared__ unsigned long long wk[kWaves];
  const int tid = threadIdx.x;
  unsigned long long key = 0ull;
  for (int i = blockIdx.x * kThreads + tid; i < n; i += gridDim.x * kThreads)
    key = umax64(key, argmax_key(x[i], (uint32_t)i));
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) key = umax64(key, shfl_xor_u64(key, m));
  if ((tid & 63) == 0) wk[tid >> 6] = key;
  __syncthreads();
  if (tid == 0) {
    unsigned long long k = wk[0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) k = umax64(k, wk[w]);
    keys[blockIdx.x] = k;
  }
}

constexpr int kFinalThreads = 1024;

__global__ __launch_bounds__(kFinalThreads) void argmax_finalize_kernel(
    const unsigned long long* keys, int n, StepCtrl* ctrl, int32_t* out_tokens, int out_cap,
    int32_t* token_out) {
  __shared__ unsigned long long wk[kFinalThreads / 64];
  const int tid = threadIdx.x;
  unsigned long long key = 0ull;
  for (int i = tid; i < n; i += kFinalThreads) key = umax64(key, keys[i]);
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) key = umax64(key, shfl_xor_u64(key, m));
  if ((tid & 63) == 0) wk[tid >> 6] = key;
  __syncthreads();
  if (tid != 0) return;
  unsigned long long k = wk[0];
  for (int w = 1; w < kFinalThreads / 64; ++w) k = umax64(k, wk[w]);
  const int32_t index = (int32_t)argmax_key_index(k);
  if (token_out) *token_out = index;
  if (ctrl != nullptr && ctrl->advance) {
    const int slot = ctrl->n_out;
    if (out_tokens && slot >= 0 && slot < out_cap) out_tokens[slot] = index;
    ctrl->n_out = slot + 1;
    ctrl->token = index;
    ctrl->position = ctrl->position + 1;
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

int launch_argmax(const float* x, int n, unsigned long long* keys, int32_t* out_index,
                  hipStream_t stream) {
  if (n <= 0) return fail("argmax: size must be positive");
  int blocks = (n + kThreads * 4 - 1) / (kThreads * 4);
  if (blocks > 1024) blocks = 1024;
  hipLaunchKernelGGL(argmax_partial_kernel, dim3(blocks), dim3(kThreads), 0, stream, x, n, keys);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return hip_fail(err, "argmax launch");
  return launch_argmax_finalize(keys, blocks, nullptr, nullptr, 0, out_index, stream);
}

int launch_argmax_finalize(const unsigned long long* keys, int n, StepCtrl* ctrl,
                           int32_t* out_tokens, int out_cap, int32_t* token_out,
                           hipStream_t stream) {
  if (n <= 0 || n > kMaxPartialKeys) return fail("argmax: bad partial key count");
  hipLaunchKernelGGL(argmax_finalize_kernel, dim3(1), dim3(kFinalThreads), 0, stream, keys, n,
                     ctrl, out_tokens, out_cap, token_out);
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? 0 : hip_fail(err, "argmax finalize launch");
}

}  // namespace hk
