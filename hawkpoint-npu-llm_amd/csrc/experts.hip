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
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
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
  const u32x4 zero = {0u, 0u, 0u, 0u};
  float tg[kRows] = {}, tu[kRows] = {};
  for (int t0 = 0; t0 < a.in; t0 += kTileCols) {
    const int t1 = min(t0 + kTileCols, a.in);
    u32x4 xv[2][2], w[kRows][2], u[PAIR ? kRows : 1][2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int c = t0 + (lane + 64 * j) * kChunk;
      const bool ok = c < t1;
      xv[j][0] = ok ? load16(x + c) : zero;
      xv[j][1] = ok ? load16(x + c + 8) : zero;
#pragma unroll
      for (int r = 0; r < kRows; ++r) {
        const bool live = ok && r < rows;
        w[r][j] = live ? load_stream16(q + (size_t)r * a.ld + c) : zero;
        if constexpr (PAIR) u[r][j] = live ? load_stream16(q2 + (size_t)r * a.ld + c) : zero;
      }
    }
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
      const float pg = wave_sum(dot16(w[r][0], xv[0][0], xv[0][1]) + dot16(w[r][1], xv[1][0], xv[1][1]));
      if (r < rows) tg[r] += round_bf16(pg * a.s[slot][row0 + r]);
      if constexpr (PAIR) {
        const float pu = wave_sum(dot16(u[r][0], xv[0][0], xv[0][1]) + dot16(u[r][1], xv[1][0], xv[1][1]));
        if (r < rows) tu[r] += round_bf16(pu * a.s2[slot][row0 + r]);
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
  if (slots < 1 || slots > kGroupMax || a.in <= 0 || a.out <= 0 || a.ld != padded(a.in))
    return fail("expert launch: bad shape");
  const dim3 grid((a.out + kRowsPerBlock - 1) / kRowsPerBlock, slots);
  if (pair)
    hipLaunchKernelGGL(expert_w8_kernel<true>, grid, dim3(64 * kWavesPerBlock), 0, stream, a);
  else
    hipLaunchKernelGGL(expert_w8_kernel<false>, grid, dim3(64 * kWavesPerBlock), 0, stream, a);
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

// ---- GGML MUL_MAT_ID ----

struct hk_ggml_experts {
  int64_t experts, out, in, ld;
  int8_t* q = nullptr;  // [experts][out][ld]
  float* s = nullptr;   // [experts][out]
  Scratch scratch;      // bf16 inputs [rows][ld], then float32 outputs [n][out]
  const uint16_t* last_x = nullptr;  // the last call's device input and output,
  float* last_y = nullptr;           // for hk_ggml_mul_mat_id_repeat
  int last_slots = 0, last_input_rows = 0;
  std::vector<uint16_t> staging;
  std::mutex mu;
};

namespace {

// Slot i of a MUL_MAT_ID launch: expert ids[i], input row 0 or i.
void ggml_slots(const hk_ggml_experts* set, ExpertArgs& a, const int32_t* ids, int n_ids, int input_rows,
                const uint16_t* dx, float* dy) {
  a.in = (int)set->in;
  a.ld = (int)set->ld;
  a.out = (int)set->out;
  for (int i = 0; i < n_ids; ++i) {
    a.q[i] = set->q + (size_t)ids[i] * set->out * set->ld;
    a.s[i] = set->s + (size_t)ids[i] * set->out;
    a.x[i] = dx + (size_t)(input_rows == 1 ? 0 : i) * set->ld;
    a.y[i] = dy + (size_t)i * set->out;
  }
}

int ggml_check_ids(const hk_ggml_experts* set, const int32_t* ids, int64_t n) {
  for (int64_t i = 0; i < n; ++i)
    if (ids[i] < 0 || ids[i] >= set->experts) return fail("expert id out of range");
  return HK_OK;
}

}  // namespace

extern "C" {

int hk_ggml_experts_supported(int64_t in_dim, int64_t out_dim, int64_t n_experts, int64_t n_ids,
                              int64_t input_rows) {
  return in_dim > 0 && in_dim <= kGgmlDimMax && out_dim > 0 && out_dim <= kGgmlDimMax &&
         n_experts >= kGroupMax && n_ids >= 1 && n_ids <= kGroupMax && (input_rows == 1 || input_rows == n_ids);
}

int hk_ggml_experts_create(const float* weights, int64_t n_experts, int64_t out_dim, int64_t in_dim,
                           hk_ggml_experts** out) {
  if (!weights || !out) return fail("hk_ggml_experts_create: null argument");
  *out = nullptr;
  if (n_experts < 1 || out_dim < 1 || in_dim < 1 || out_dim > kGgmlDimMax || in_dim > kGgmlDimMax)
    return fail("hk_ggml_experts_create: shape outside the MUL_MAT_ID contract");
  auto* set = new hk_ggml_experts;
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

int hk_ggml_mul_mat_id(hk_ggml_experts* set, const float* input, int64_t input_rows, const int32_t* ids,
                       int64_t n_ids, float* out) {
  if (!set || !input || !ids || !out) return fail("hk_ggml_mul_mat_id: null argument");
  if (n_ids < 1 || n_ids > kGroupMax || (input_rows != 1 && input_rows != n_ids))
    return fail("hk_ggml_mul_mat_id: ids or input rows outside the MUL_MAT_ID contract");
  if (int rc = ggml_check_ids(set, ids, n_ids)) return rc;
  std::lock_guard<std::mutex> lock(set->mu);
  const size_t in_bytes = align256((size_t)input_rows * set->ld * 2), out_floats = (size_t)n_ids * set->out;
  if (int rc = set->scratch.reserve(in_bytes + out_floats * sizeof(float))) return rc;
  auto* dx = reinterpret_cast<uint16_t*>(set->scratch.buf);
  auto* dy = reinterpret_cast<float*>(set->scratch.buf + in_bytes);
  pack_inputs(input, (int)input_rows, (int)set->in, set->in, set->staging);
  hipError_t err = hipMemcpy(dx, set->staging.data(), set->staging.size() * 2, hipMemcpyHostToDevice);
  if (err != hipSuccess) return hip_fail(err, "hk_ggml_mul_mat_id input");
  ExpertArgs a{};
  ggml_slots(set, a, ids, (int)n_ids, (int)input_rows, dx, dy);
  if (int rc = launch_experts(a, (int)n_ids, false, nullptr)) return rc;
  set->last_x = dx;
  set->last_y = dy;
  set->last_slots = (int)n_ids;
  set->last_input_rows = (int)input_rows;
  err = hipMemcpy(out, dy, out_floats * sizeof(float), hipMemcpyDeviceToHost);
  return err == hipSuccess ? HK_OK : hip_fail(err, "hk_ggml_mul_mat_id output");
}

int hk_ggml_mul_mat_id_repeat(hk_ggml_experts* set, const int32_t* ids, int64_t launches, float* ms_per_launch) {
  if (!set || !ids || !ms_per_launch || launches < 1) return fail("hk_ggml_mul_mat_id_repeat: bad argument");
  std::lock_guard<std::mutex> lock(set->mu);
  const int n = set->last_slots;
  if (n < 1) return fail("hk_ggml_mul_mat_id_repeat: no earlier call on this set");
  if (int rc = ggml_check_ids(set, ids, launches * n)) return rc;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  hipError_t err = hipEventCreate(&e0);
  if (err == hipSuccess) err = hipEventCreate(&e1);
  if (err == hipSuccess) err = hipEventRecord(e0, nullptr);
  int rc = HK_OK;
  for (int64_t i = 0; i < launches && err == hipSuccess && rc == HK_OK; ++i) {
    ExpertArgs a{};
    ggml_slots(set, a, ids + i * n, n, set->last_input_rows, set->last_x, set->last_y);
    rc = launch_experts(a, n, false, nullptr);
  }
  if (err == hipSuccess && rc == HK_OK) err = hipEventRecord(e1, nullptr);
  if (err == hipSuccess && rc == HK_OK) err = hipEventSynchronize(e1);
  float ms = 0.0f;
  if (err == hipSuccess && rc == HK_OK) err = hipEventElapsedTime(&ms, e0, e1);
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  if (rc != HK_OK) return rc;
  if (err != hipSuccess) return hip_fail(err, "hk_ggml_mul_mat_id_repeat");
  *ms_per_launch = ms / (float)launches;
  return HK_OK;
}

void hk_ggml_experts_destroy(hk_ggml_experts* set) {
  if (!set) return;
  if (set->q) (void)hipFree(set->q);
  if (set->s) (void)hipFree(set->s);
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
  a.q[0] = t->q;
  a.s[0] = t->s;
  a.x[0] = dx;
  a.y[0] = dy;
  if (launch_experts(a, 1, false, nullptr)) return 0;
  return hipMemcpy(output, dy, (size_t)t->output * sizeof(float), hipMemcpyDeviceToHost) == hipSuccess ? 1 : 0;
}

}  // extern "C"
