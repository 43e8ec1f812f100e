// Whole decode step in one persistent launch (bf16 weights).
//
// The step of npu_llm/runtime/cpu_backend.py:131-181 is a chain of small
// dependent GEMVs (QKV, O, gate/up, down per layer, then the LM head).  As
// separate kernels each one pays a launch and a full HBM latency before its
// first byte arrives, so at batch 1 they run at 1-3 TB/s.  Here one
// workgroup per CU stays resident for the whole step and hands results
// from phase to phase through memory:
//
//   Q  qkv = bf16(W_qkv @ rmsnorm(h) [+ bias])           cpu_backend.py:134-143
//   A  RoPE, KV append at slot p, GQA attention          :95-129
//   O  h1 = bf16(bf16(W_o @ attn) + h)                   :144-150
//   G  act = bf16(silu(bf16(W_g @ n)) * bf16(W_u @ n)), n = rmsnorm(h1)  :151-165
//   D  h = bf16(bf16(W_d @ act) + h1)                    :166-171
//   H  logits = W_lm @ rmsnorm(h) (f32), argmax           :173-181
//
// * Activations travel as tagged 32-bit words, (tag << 16) | bf16, where the
//   tag names the phase instance that wrote them.  A consumer polls the words
//   it needs until every one carries the expected tag; a single 32-bit store
//   is seen whole or not at all, so no separate flag (and no wait for store
//   completion before one) is needed.  Tags come from an epoch that only
//   grows: base + phase index, base = the epoch the previous launch ended on,
//   so buffers are never cleared between steps.  Tags are 1..65535, so
//   zeroed memory never matches.
// * In a GEMV phase, waves 6 and 7 of each workgroup are the stagers: they
//   split the input vector's 16-byte chunks between them, poll them and
//   write them to one of two LDS buffers (plus the raw values the residual
//   add needs).  For an RMSNorm input they also stage gamma and their partial
//   sums of squares, and all eight waves normalise the buffer in place after
//   the hand-off barrier (a few values per thread instead of a serial pass
//   on the stagers).  Their only other global loads are weight prefetches aimed
//   outside the buffer, which return zero without a memory access, and they
//   store nothing, so their polls return at the bare memory latency: a wave's
//   loads complete in order, and on gfx9 its stores count in the same
//   counter.  Two pollers matter for the 4864-word down input: one wave
//   waiting on 19 chunks per lane per round sees its hand-off about 1 us
//   later than two waves on 10 each.  Waves 0-5 own at most one row group
//   each and hold its weights in registers, loaded one or two phases ahead
//   (O and gate/up right after attention, down and the next layer's QKV
//   right after O), so weight streaming overlaps attention and the waits.  The LM
//   head streams rows on all eight waves with a double buffer.
// * Cross-workgroup data is written and read with device-coherent (sc1)
//   accesses: the eight XCDs have separate L2 caches, and sc1 accesses bypass
//   their incoherent state without whole-cache write-back or invalidate fences.
//   Hand-offs between workgroups of one XCD may instead use its shared L2
//   (kLocal): plain stores, sc0|nt loads.
// * Two kernels share this protocol (tags, epochs, flags), so launches may
//   alternate.  decode_step_kernel (above) spreads every phase over all 256
//   workgroups.  decode_step_xa_kernel splits the step by XCD: the attention
//   block on XCD 0, with its QKV -> attention -> O hand-offs inside that
//   XCD's L2, and the MLP with down_proj fused in as split-K partials on the
//   other seven.  Its long form moves the attention tasks to the MLP
//   workgroups for contexts whose tasks outnumber XCD 0's.  The engine
//   picks the kernel and form per launch from the position.
// * Every wait is bounded: after spin_limit polls, or once another workgroup
//   has flagged an error, the workgroup records the error and leaves; all
//   later waits then end at once, so the launch always drains.  The host
//   reports the error and clears the tags and flags.
//
// Rounding points are those of the separate kernels (gemv.hip, attention.hip).
#include <type_traits>

#include "hk_common.h"
#include "hk_internal.h"

namespace hk {

// ---- phase stamps (built in only with -DHK_PHASE_STAMPS: lib/libhk_phases.so) ----
// Thread 0 of each workgroup (or the thread named) writes the 100 MHz
// real-time clock at fixed points of each of the first kStampLayers layers
// of the XCD-split step; hk_phase_stamps copies the tables to the host.
// Slots of hk_stamp_phase (per workgroup and layer):
//   0 Q input staged and normalised     1 QKV rows stored
//   2 attention task done               3 O input staged
//   4 O rows published                  5 h1 staged and normalised (MLP)
//   6 gate/up + down partial + barrier  7 workgroup partial stored
//   8 XCD reduction done                9 h reduction done (XCD 0)
//  10 QKV dot products done            11 O dot products done
//  12 gate/up dot products done        13 down partial done
// and of hk_stamp_attn (attention task): 0 start, 1 q/k/v polled, 2 scores,
// 3 softmax, 4 merge barrier, 5 single-chunk store, 6 merged store,
// 7 partial published.
constexpr int kStampLayers = 32, kStampSlots = 16, kStampAttn = 8;
#ifdef HK_PHASE_STAMPS
__device__ unsigned long long hk_stamp_phase[kPersistentGrid][kStampLayers][kStampSlots];
__device__ unsigned long long hk_stamp_attn[kPersistentGrid][kStampLayers][kStampAttn];
#define HK_STAMP_BY(tid, l, k)                                                                       \
  do {                                                                                               \
    if (threadIdx.x == (tid) && (l) < kStampLayers)                                                  \
      hk_stamp_phase[blockIdx.x][l][k] = __builtin_amdgcn_s_memrealtime();                           \
  } while (0)
#define HK_STAMP_ATTN(l, k)                                                                          \
  do {                                                                                               \
    if (threadIdx.x == 0 && (l) < kStampLayers)                                                      \
      hk_stamp_attn[blockIdx.x][l][k] = __builtin_amdgcn_s_memrealtime();                            \
  } while (0)
#else
#define HK_STAMP_BY(tid, l, k) \
  do {                         \
  } while (0)
#define HK_STAMP_ATTN(l, k) \
  do {                      \
  } while (0)
#endif
#define HK_STAMP(l, k) HK_STAMP_BY(0, l, k)

namespace {

constexpr int kPT = kPersistentThreads;  // threads per workgroup (one workgroup per CU)
constexpr int kPW = kPT / 64;             // waves per workgroup
constexpr int kPf = 28;                   // 16-byte weight chunks a lane holds across a wait
constexpr int kXMax = 5120;               // floats per LDS staging buffer
constexpr int kHMax = 1024;               // raw residual values kept in LDS
constexpr int kSW = 2;                    // stager waves: waves kCW .. kPW - 1
constexpr int kCW = kPW - kSW;            // compute waves
constexpr int kChunk = kPersistentChunk;  // attention slots per task
constexpr int kHalf = kHeadDim / 2;
constexpr int kGroupsPV = kPT / kHalf;    // slot groups of the P @ V loop
constexpr int kSlotsPV = kChunk / kGroupsPV;  // consecutive slots per group
constexpr int kPartStride = kHeadDim + 2;
constexpr int kSc1 = 16;                  // buffer-load cache policy: device scope (sc1)
// Cache policy of hand-offs inside one XCD: loads with sc0|nt miss the CU's
// L1 and read the XCD's shared L2, which every CU of the XCD writes through
// to; stores use the default policy (0) and stay in that L2.  Data stored
// with sc1 (written through to memory for other XCDs) is read with sc1 even
// inside the XCD: an sc0|nt load can keep hitting a stale L2 copy of it.
constexpr int kLocal = 3;
// MI355X: 8 XCDs of 32 CUs; workgroup i of a one-per-CU launch runs on XCD
// i % 8 (the XCD split checks this against the XCC_ID register).
constexpr int kXcds = 8;
constexpr int kXcdWg = kPersistentGrid / kXcds;
static_assert(2 * kChunk == kPT, "two threads per attention slot");

// ---- device-coherent accesses ----
__device__ __forceinline__ void st_c32(unsigned* p, unsigned v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned ld_c32(const unsigned* p) {
  return __hip_atomic_load(const_cast<unsigned*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_c64(unsigned long long* p, unsigned long long v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned long long ld_c64(const unsigned long long* p) {
  return __hip_atomic_load(const_cast<unsigned long long*>(p), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}


__device__ __forceinline__ bool reached(unsigned v, unsigned target) {
  return (int)(v - target) >= 0;
}

// Tag of epoch e: 1..65535 (never 0, the value of cleared memory).
__device__ __forceinline__ unsigned tag_of(unsigned e) { return e % 65535u + 1u; }

__device__ __forceinline__ uint32_t tagged(uint32_t bf16, unsigned tag) { return (tag << 16) | bf16; }

// Partial-sum words: (tag << 32) | float bits; the tag (epoch % (2^32 - 1) + 1)
// is never 0, the value of cleared memory.  An aligned 8-byte store is seen
// whole or not at all.
__device__ __forceinline__ unsigned ptag_of(unsigned e) { return e % 0xffffffffu + 1u; }
__device__ __forceinline__ unsigned long long pword(float v, unsigned t) {
  return ((unsigned long long)t << 32) | __float_as_uint(v);
}
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
template <int POL = kSc1>
__device__ __forceinline__ unsigned long long ld_p64(__amdgpu_buffer_rsrc_t r, unsigned off) {
  return __builtin_bit_cast(unsigned long long, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, POL));
}

// ---- cross-lane sums with DPP ----
// Within a 16-lane row DPP moves take a few cycles, against an LDS round trip
// for ds_bpermute (what __shfl_xor compiles to).  Steps: swap neighbours
// (quad_perm 1,0,3,2), swap pairs (2,3,0,1), then pair quads (half-row mirror)
// and halves (row mirror); each step adds lanes holding equal partial sums,
// so every lane of the group ends with the same total.  Across rows,
// row_bcast15 adds row 0 to row 1 and row 2 to row 3, row_bcast31 then adds
// rows 0 + 1 to row 3, and v_readlane hands lane 63's total to the whole wave
// (the same value in every lane).  Checked on the device against shuffle
// butterflies: equal groups, equal maxima, sums within float rounding.
template <int CTRL, int ROWS = 0xf>
__device__ __forceinline__ float dpp_mov(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROWS, 0xf, false));
}
template <int CTRL>
__device__ __forceinline__ float dpp_plus(float v) {
  return v + dpp_mov<CTRL>(v);
}
__device__ __forceinline__ float lane63(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// sum over each group of 8 lanes, in all 8
__device__ __forceinline__ float group_sum8(float v) {
  v = dpp_plus<0xb1>(v);   // quad_perm 1,0,3,2
  v = dpp_plus<0x4e>(v);   // quad_perm 2,3,0,1
  return dpp_plus<0x141>(v);  // row_half_mirror
}

template <int W>
__device__ __forceinline__ float wave_sum(float v) {
  static_assert(W == 16 || W == 64, "a row or the whole wave");
  v = dpp_plus<0xb1>(v);   // quad_perm 1,0,3,2
  v = dpp_plus<0x4e>(v);   // quad_perm 2,3,0,1
  v = dpp_plus<0x141>(v);  // row_half_mirror
  v = dpp_plus<0x140>(v);  // row_mirror
  if constexpr (W == 64) {
    v = v + dpp_mov<0x142, 0xa>(v);  // row_bcast15 into rows 1 and 3
    v = v + dpp_mov<0x143, 0x8>(v);  // row_bcast31 into row 3
    v = lane63(v);
  }
  return v;
}

__device__ __forceinline__ float wave_max64(float v) {
  v = fmaxf(v, dpp_mov<0xb1>(v));
  v = fmaxf(v, dpp_mov<0x4e>(v));
  v = fmaxf(v, dpp_mov<0x141>(v));
  v = fmaxf(v, dpp_mov<0x140>(v));
  v = fmaxf(v, dpp_mov<0x142, 0xa>(v));
  v = fmaxf(v, dpp_mov<0x143, 0x8>(v));
  return lane63(v);
}

// ---- phase shapes ----
struct PhaseCfg {
  int lpr, nj;
};

// Lanes per row (64, 32, 16 or 8) so that a wave owns at most one row group of
// the phase at `waves` waves in the grid, with the group's 16-byte chunks
// (`eb` bytes per weight) fitting in `budget` prefetch registers.
constexpr PhaseCfg pick_cfg(int M, int K, bool pair, int waves, int budget, int max_lpr = 64, int eb = 2) {
  for (int lpr = max_lpr; lpr >= 8; lpr /= 2) {
    const int rpw = 64 / lpr;
    const int groups = (M + rpw - 1) / rpw;
    const int nj = (K * eb / 16 + lpr - 1) / lpr;
    if (groups <= waves && nj * (pair ? 2 : 1) <= budget) return {lpr, nj};
  }
  return {0, 0};
}

// producers of a phase: workgroups whose compute waves own row groups
constexpr int producers(PhaseCfg c, int M, int waves_per_wg = kCW) {
  return ((M + 64 / c.lpr - 1) / (64 / c.lpr) + waves_per_wg - 1) / waves_per_wg;
}

// W8: the four layer projections are int8 with a float32 scale per output
// row (16 weights per 16-byte chunk); the LM head stays bf16.
template <int H_, int I_, int HQ_, int HKV_, bool W8_ = false>
struct Shape {
  static constexpr int H = H_, I = I_, HQ = HQ_, HKV = HKV_;
  static constexpr bool W8 = W8_;
  static constexpr int EB = W8 ? 1 : 2;  // bytes per layer weight
  static constexpr int QPK = HQ / HKV;
  static constexpr int QKV = (HQ + 2 * HKV) * kHeadDim;
  static constexpr int AO = HQ * kHeadDim;
  static constexpr int kWaves = kPersistentGrid * kCW;
  static constexpr PhaseCfg q = pick_cfg(QKV, H, false, kWaves, 4, 64, EB);
  static constexpr PhaseCfg o = pick_cfg(H, AO, false, kWaves, 4, 64, EB);
  static constexpr PhaseCfg d = pick_cfg(H, I, false, kWaves, 12, 64, EB);
  static constexpr PhaseCfg g = pick_cfg(I, H, true, kWaves, kPf - o.nj - d.nj, 64, EB);
  // register slots: O and gate/up are requested together after attention;
  // down, and the next layer's QKV in the O slots, once O has been computed
  static constexpr int off_o = 0, off_g = o.nj, off_d = o.nj + 2 * g.nj, off_q = 0;
  static constexpr int head_lpr = 16;
  static constexpr int head_nj = (H / 8 + head_lpr - 1) / head_lpr;
  static constexpr int nq = producers(q, QKV), no = producers(o, H);
  static constexpr int ng = producers(g, I), nd = producers(d, H);
  static_assert(q.lpr && o.lpr && g.lpr && d.lpr, "no register plan for this shape");
  static_assert(head_nj <= kPf / 2, "LM head rows too long for the double buffer");
  static_assert(q.nj <= o.nj && off_d + d.nj <= kPf, "register slots overlap");
  static_assert(H <= kXMax && I <= kXMax && AO <= kXMax && H <= kHMax, "x staging too small");
  static_assert((I / 4 + 63) / 64 <= 32 && (H / 4 + 63) / 64 <= 32 && (AO / 4 + 63) / 64 <= 32,
                "stager chunk mask is 32 bits");
  static_assert(H % 8 == 0 && I % 8 == 0 && AO % 8 == 0, "rows are read in 16-byte chunks");
  static_assert(!W8 || (H % 16 == 0 && I % 16 == 0 && AO % 16 == 0), "int8 rows are read in 16-byte chunks");
  // residual rows are fetched by workgroups that have just seen the whole
  // source vector: O rows by Q producers, down rows by gate/up producers
  // the stager of an O-row workgroup saw all of h (Q phase), of a down-row
  // workgroup all of h1 (gate/up phase); each such workgroup also takes part
  // in every phase between the write of its raw residual copy and its use
  static_assert(no <= nq && nd <= ng && no <= ng && nd <= nq && nd <= no,
                "residual copies need nested producer sets");
  // XCD split (decode_step_xa_kernel): the attention block runs on the
  // kXcdWg workgroups of XCD 0 (QKV rows in slots 0.., O rows after them),
  // the MLP on the other XCDs (gate/up pairs in slots 0.., down rows after).
  // On XCD 0 all kPW waves of a workgroup take QKV and O rows (the stagers
  // are idle during those dot products), so the rows fit on the lowest
  // workgroups and the attention tasks go to workgroups without rows, whose
  // K/V loads then go out at the start of the layer; O uses no more
  // workgroups than QKV (their stagers keep h for the residual)
  static constexpr int kAW = kXcdWg * kPW, kMW = (kPersistentGrid - kXcdWg) * kCW;
  // (8 lanes per row: QKV on as few workgroups as the register budget allows)
  static constexpr PhaseCfg xq = pick_cfg(QKV, H, false, kAW, kPf / 2, 8, EB);
  static constexpr int xnq = producers(xq, QKV, kPW);
  static constexpr PhaseCfg xo = pick_cfg(H, AO, false, xnq * kPW, kPf / 2, 64, EB);
  // (at most 16 lanes per row: the fused down takes four rows per wave)
  static constexpr PhaseCfg xg = pick_cfg(I, H, true, kMW, kPf / 2, 16, EB);
  static constexpr int xno = producers(xo, H, kPW), xng = producers(xg, I);
  // down is fused into the gate/up waves: a wave's four act values times
  // their down_x group, xdc output chunks (8 outputs each, 16 for W8) over
  // the 64 lanes (xkd each, four 16-byte slots per chunk); each workgroup of
  // an XCD then adds up xsl of the H outputs over the XCD's workgroups
  static constexpr int xdo = 16 / EB, xdc = H / xdo;
  static constexpr int xkd = (xdc + 63) / 64;
  static constexpr int xsl = (H + kXcdWg - 1) / kXcdWg;
  // XCD 0 adds the XCD partials on the stager waves of its workgroups
  // without QKV/O rows (no weight prefetch queues ahead of their polls):
  // slices of xhs outputs, xhn of them
  static constexpr int xhs = 32, xhn = (H + xhs - 1) / xhs;
  // bf16: QKV and O two rows per lane (prefetch_r2), still eight rows per
  // wave, xq2 / xo2 chunks per row and lane
  static constexpr int xq2 = (H / 8 + 15) / 16, xo2 = (AO / 8 + 15) / 16;
  static constexpr bool xr2 = !W8 && xq.lpr == 8 && xo.lpr == 8 && 2 * (xq2 + xo2) <= kPf;
  // O rows take their residual from the Q stagers' copy of h
  static constexpr bool xa = xq.lpr && xo.lpr && xg.lpr == 16 && xq.nj + xo.nj <= kPf &&
                             xnq + HQ <= kXcdWg && xhn <= (kXcdWg - xnq) * kSW &&
                             2 * xg.nj + 4 * xkd <= kPf && xno <= xnq && xsl <= 64 && H <= kHMax &&
                             (!W8 || (2 * (xq.nj + xo.nj) <= kPf && 4 * xg.nj + 8 * xkd <= kPf)) &&
                             I % 4 == 0 && xnq <= kXcdWg && xng <= kPersistentGrid - kXcdWg;
};

struct PShared {
  // layer table: read from LDS, since a global read of it would make the
  // wave wait for all its outstanding loads and stores first
  PersistentLayer layers[kPersistentMaxLayers];
  // staged GEMV inputs as bf16 (alternating buffers); attention scratch in xs[0].
  // Every staged x is bf16-exact (activations, or RMSNorm output rounded to
  // bf16), so a 16-byte LDS read carries 8 of them.
  alignas(16) uint16_t xs[2][kXMax];
  alignas(16) float raw_h[kHMax];   // layer input h before RMSNorm: residual of the O rows
  alignas(16) float raw_h1[kHMax];  // h1 before RMSNorm: residual of the down rows
  float red[2][kPW];
  unsigned long long keys[kPW];
  uint32_t out_val[kCW * 16];  // a phase's tagged outputs, gathered for one store
  unsigned out_count;          // compute-wave arrivals (7 per gathered phase)
  unsigned out_stored;         // out_count value once the gathered store is issued
  alignas(16) uint16_t gs[kHMax];  // RMSNorm gamma of the staged input
  float ssp[kSW];                  // stagers' partial sums of squares of the staged input
  int abort;
  int ticket;
};

struct Ctx {
  const PersistentArgs* a;
  PShared* sm;
  int wg, wave, lane;
  int gw;  // compute-wave index wg * kCW + wave (wave < kCW)
};

constexpr unsigned kOutsideWord = 0x7ffffff0u;  // byte offset beyond every resource (reads zero)

// Record an abandoned launch (first failing wait) for the host.
__device__ __forceinline__ bool give_up(const PersistentArgs& a) {
  st_c32(a.error, 1u);
  return false;
}

// Poll one tagged word until it carries `tag`; false when the launch is abandoned.
// The word is p, also reachable as byte `off` of the buffer `r` (used by the
// XCD-local policy, whose loads go through a buffer resource).
template <int POL>
__device__ bool poll_word(const PersistentArgs& a, const uint32_t* p, unsigned tag, uint32_t& out,
                          __amdgpu_buffer_rsrc_t r, unsigned off) {
  for (unsigned spins = 1;; ++spins) {
    uint32_t w;
    if constexpr (POL == kSc1)
      w = ld_c32(p);
    else
      w = __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, POL);
    if ((w >> 16) == tag) {
      out = w;
      return true;
    }
    if (spins > a.spin_limit || ((spins & 63u) == 0u && ld_c32(a.error) != 0u)) return give_up(a);
    __builtin_amdgcn_s_sleep(1);
  }
}

// Poll the N tagged words at byte offsets off[i] of the buffer r together
// (one round trip per poll round) until each carries `tag`; an offset of
// kOutside marks a word this thread does not wait for (it reads zero).  False
// when the launch is abandoned.
template <int N, int POL>
__device__ bool poll_words(const PersistentArgs& a, __amdgpu_buffer_rsrc_t r, const unsigned (&off)[N],
                           unsigned tag, uint32_t (&w)[N]) {
  bool any = false;
#pragma unroll
  for (int i = 0; i < N; ++i) any = any || off[i] != kOutsideWord;
  if (!any) return true;
  for (unsigned spins = 1;; ++spins) {
#pragma unroll
    for (int i = 0; i < N; ++i) w[i] = __builtin_amdgcn_raw_buffer_load_b32(r, off[i], 0, POL);
    bool have = true;
#pragma unroll
    for (int i = 0; i < N; ++i) have = have && (off[i] == kOutsideWord || (w[i] >> 16) == tag);
    if (have) return true;
    if (spins > a.spin_limit || ((spins & 63u) == 0u && ld_c32(a.error) != 0u)) return give_up(a);
    __builtin_amdgcn_s_sleep(1);
  }
}

// Wave 0 waits until flags[i * kFlagStride] has reached `target` for i < n;
// the other waves wait at the workgroup barrier.  False when abandoned.
__device__ bool wait_all(Ctx& c, const unsigned* flags, int n, unsigned target) {
  if (c.wave == 0) {
    int abort = 0;
    for (unsigned spins = 1;; ++spins) {
      bool ok = true;
      for (int i = c.lane; i < n; i += 64) ok = ok && reached(ld_c32(flags + (size_t)i * kFlagStride), target);
      if (__all(ok)) break;
      if (spins > c.a->spin_limit || ((spins & 63u) == 0u && ld_c32(c.a->error) != 0u)) {
        abort = 1;
        if (c.lane == 0) give_up(*c.a);
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    if (c.lane == 0) c.sm->abort = abort;
  }
  __syncthreads();
  return c.sm->abort == 0;
}

// Publish this workgroup's epoch once every thread's stores have completed.
__device__ __forceinline__ void publish(Ctx& c, unsigned* flag, unsigned epoch) {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) st_c32(flag, epoch);
}

// s_waitcnt vmcnt(N), other counters untouched (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Stagers: poll the K tagged words at src until all carry `tag` (stager
// wave s of kSW takes the 16-byte chunks s*64 + lane + 64*kSW*j, keeping up to
// kBatch of them in flight at once) and write them to xs as bf16, the raw
// values to `raw` when RAW.  For an RMSNorm input (NORM) they also write gamma
// to gs and their partial sums of squares to ssp; normalise_staged finishes
// the job on all waves.  False when abandoned.
constexpr int kBatch = 10;

template <int K, bool NORM, bool RAW, int POL = kSc1>
__device__ bool stage_wave(Ctx& c, const uint32_t* src, unsigned tag, const uint16_t* gamma,
                           uint16_t* xs, float* raw) {
  const PersistentArgs& a = *c.a;
  constexpr int CH = K / 4;  // 16-byte chunks of four tagged words
  constexpr int STRIDE = 64 * kSW;
  constexpr int PER = (CH + STRIDE - 1) / STRIDE;
  constexpr int GPER = NORM ? PER : 1;
  static_assert(!NORM || K <= kHMax, "gamma staging too small");
  const int lane = c.lane, sw = c.wave - kCW;
  const int first = sw * 64 + lane;  // this lane's chunk j is first + STRIDE * j
  // gamma is constant: fetch it before polling so its latency overlaps the wait
  uint2 gv[GPER];
  if constexpr (NORM) {
#pragma unroll
    for (int j = 0; j < GPER; ++j) {
      const int ch = first + STRIDE * j;
      gv[j] = ch < CH ? ldg_u2(gamma + ch * 4) : make_uint2(0u, 0u);
    }
  }
  float ss = 0.0f;
  bool ok = true;
  constexpr int B = PER < kBatch ? PER : kBatch;
#pragma unroll
  for (int j0 = 0; j0 < PER; j0 += kBatch) {
    unsigned pending = 0;
#pragma unroll
    for (int j = 0; j < B; ++j)
      if (j0 + j < PER && first + STRIDE * (j0 + j) < CH) pending |= 1u << j;
    u32x4 v[B];
    for (unsigned spins = 1;; ++spins) {
#pragma unroll
      for (int j = 0; j < B; ++j)
        if ((pending >> j) & 1u)
          v[j] = __builtin_amdgcn_raw_buffer_load_b128(rsrc(src, K * 4), first * 16,
                                                       (j0 + j) * STRIDE * 16, POL);
#pragma unroll
      for (int j = 0; j < B; ++j)
        if (((pending >> j) & 1u) && (v[j].x >> 16) == tag && (v[j].y >> 16) == tag &&
            (v[j].z >> 16) == tag && (v[j].w >> 16) == tag)
          pending &= ~(1u << j);
      if (!__any(pending != 0u)) break;
      if (spins > a.spin_limit || ((spins & 63u) == 0u && ld_c32(a.error) != 0u)) {
        ok = give_up(a);
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    if (!ok) break;
#pragma unroll
    for (int j = 0; j < B; ++j) {
      const int ch = first + STRIDE * (j0 + j);
      if (j0 + j < PER && ch < CH) {
        if constexpr (NORM || RAW) {
          const float f[4] = {bf_lo(v[j].x), bf_lo(v[j].y), bf_lo(v[j].z), bf_lo(v[j].w)};
#pragma unroll
          for (int q = 0; q < 4; ++q) ss += f[q] * f[q];
          if constexpr (RAW) *reinterpret_cast<float4*>(raw + ch * 4) = make_float4(f[0], f[1], f[2], f[3]);
        }
        if constexpr (NORM) *reinterpret_cast<uint2*>(c.sm->gs + ch * 4) = gv[j0 + j < GPER ? j0 + j : 0];
        *reinterpret_cast<uint2*>(xs + ch * 4) =
            make_uint2((v[j].x & 0xffffu) | (v[j].y << 16), (v[j].z & 0xffffu) | (v[j].w << 16));
      }
    }
  }
  if constexpr (NORM) {
    ss = wave_sum<64>(ss);
    if (lane == 0) c.sm->ssp[sw] = ss;
  }
  // every load of this wave has returned by now; saying so leaves the
  // compiler nothing to wait for on this path after the hand-off barrier
  wait_vm<0>();
  return ok;
}

// Stagers for the layer-0 input: plain bf16 written before the launch (the
// embedding row or a preloaded hidden state), staged like an RMSNorm input.
template <int K>
__device__ void stage_wave_plain(Ctx& c, const uint16_t* src, const uint16_t* gamma, uint16_t* xs,
                                 float* raw) {
  constexpr int CH = K / 4;
  const int sw = c.wave - kCW;
  float ss = 0.0f;
  for (int ch = sw * 64 + c.lane; ch < CH; ch += 64 * kSW) {
    const uint2 w = ldg_u2(src + ch * 4);
    const float f[4] = {bf_lo(w.x), bf_hi(w.x), bf_lo(w.y), bf_hi(w.y)};
#pragma unroll
    for (int q = 0; q < 4; ++q) ss += f[q] * f[q];
    *reinterpret_cast<float4*>(raw + ch * 4) = make_float4(f[0], f[1], f[2], f[3]);
    *reinterpret_cast<uint2*>(c.sm->gs + ch * 4) = ldg_u2(gamma + ch * 4);
    *reinterpret_cast<uint2*>(xs + ch * 4) = w;
  }
  ss = wave_sum<64>(ss);
  if (c.lane == 0) c.sm->ssp[sw] = ss;
}

// RMSNorm of the staged input in place (cpu_backend.py:71-76), on all waves
// after the hand-off barrier: bf16((x * inv) * gamma) with
// inv = 1 / sqrt(mean(x^2) + eps); the partial sums are added in a fixed
// order, so every thread uses the same factor.  Ends with a barrier.
template <int K>
__device__ __forceinline__ void normalise_staged(Ctx& c, uint16_t* xs, float eps) {
  float total = 0.0f;
#pragma unroll
  for (int i = 0; i < kSW; ++i) total += c.sm->ssp[i];
  const float inv = 1.0f / sqrtf(total / (float)K + eps);
  uint32_t* xw = reinterpret_cast<uint32_t*>(xs);
  const uint32_t* gw = reinterpret_cast<const uint32_t*>(c.sm->gs);
  for (int i = threadIdx.x; i < K / 2; i += kPT) {
    const uint32_t x = xw[i], g = gw[i];
    const uint32_t n0 = f32_to_bf16((bf_lo(x) * inv) * bf_lo(g));
    const uint32_t n1 = f32_to_bf16((bf_hi(x) * inv) * bf_hi(g));
    xw[i] = n0 | (n1 << 16);
  }
  __syncthreads();
}

// Issue the loads of this wave's row group (rows group*RPW + sub) of W [M, K]
// (plus the paired rows M.. for gate/up) into pf[OFF ...].  The loads are
// unconditional buffer loads -- a row outside [0, M), a chunk past the row
// or a workgroup that is not `live` reads zero through an offset past the
// resource -- so every compute wave issues the same memory instructions in
// every phase and the compiler can wait for exactly the loads it needs.
constexpr unsigned kOutside = 0x7ffffff0u;  // byte offset beyond every resource
constexpr int kNT = 2;                      // buffer-load cache policy: non-temporal
// The LM head's weights load with the default policy, the layers' with nt:
// measured, that keeps part of the 272 MB head in the Infinity Cache from
// one step to the next (304.0 against 307.4 us per Qwen2.5-0.5B step; layer
// weights with the default policy too: 323.8 us)
constexpr int kHeadPol = 0;

template <int LPR, int NJ, bool PAIR, int OFF, int EB = 2, int POL = kNT, int UOFF = OFF + NJ>
__device__ __forceinline__ void prefetch(u32x4 (&pf)[kPf], const void* W, int M, int K,
                                         int group, bool live_wg) {
  constexpr int RPW = 64 / LPR;
  const int lane = threadIdx.x & 63;
  const int l = lane % LPR, sub = lane / LPR;
  const int row = group * RPW + sub;
  const bool live = live_wg && row < M;
  const __amdgpu_buffer_rsrc_t r = rsrc(W, (PAIR ? 2 : 1) * M * K * EB);
  // one VGPR per lane: the chunk stride and the gate/up distance go in the
  // scalar offset.  Chunks past the row end read the next row (ignored by
  // dot_group) or, past the matrix, zero.
  const unsigned voff = live ? (unsigned)row * (unsigned)K * (unsigned)EB + (unsigned)l * 16u : kOutside;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    pf[OFF + j] = __builtin_amdgcn_raw_buffer_load_b128(r, voff, j * LPR * 16, POL);
    if constexpr (PAIR)
      pf[UOFF + j] = __builtin_amdgcn_raw_buffer_load_b128(r, voff, M * K * EB + j * LPR * 16, POL);
  }
}

// Per-row float32 scale of a W8 phase, for the row prefetch() gives this lane
// (1.0 for a row outside the matrix or a lane that takes no row).
template <int LPR>
__device__ __forceinline__ float row_scale(const float* scale, int M, int group, bool live_wg) {
  const int row = group * (64 / LPR) + (threadIdx.x & 63) / LPR;
  const unsigned off = live_wg && row < M ? (unsigned)row * 4u : kOutside;
  const float s = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsrc(scale, M * 4), off, 0, 0));
  return off == kOutside ? 1.0f : s;
}

// Eight bf16 products of a weight chunk and an x chunk, into two float32
// accumulators.  v_dot2_f32_bf16 multiplies the packed halves (bf16 x bf16
// is exact in float32) and adds both products to the accumulator: one VALU
// instruction per two weights and no unpacking, where separate FMAs take
// two shifts/masks and two FMAs -- the dot products are VALU-bound on the
// critical path of every phase.
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float dot2(uint32_t w, uint32_t x, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w), __builtin_bit_cast(bf16x2, x), c,
                                         false);
}
__device__ __forceinline__ void fma8(const u32x4 w, const u32x4 x, float& a0, float& a1) {
  a0 = dot2(w.x, x.x, a0);
  a1 = dot2(w.y, x.y, a1);
  a0 = dot2(w.z, x.z, a0);
  a1 = dot2(w.w, x.w, a1);
}

// Two rows per lane (bf16): lanes 16 s .. 16 s + 15 of a wave take rows
// 2 s and 2 s + 1 of its group of eight (`group`), chunks l + 16 j of both
// rows (l = lane % 16), row 2 s in slots OFF + j and row 2 s + 1 in
// OFF + NJ + j.  Both rows multiply the same x chunks, so a wave reads half
// the x bytes from LDS that eight lanes per row read: when all eight waves of
// a workgroup start a phase together, the LDS read bandwidth (128 bytes per
// clock) is what the last wave waits for.
template <int NJ, int OFF, int POL = kNT>
__device__ __forceinline__ void prefetch_r2(u32x4 (&pf)[kPf], const void* W, int M, int K, int group,
                                            bool live_wg) {
  const int lane = threadIdx.x & 63;
  const int l = lane & 15, row = group * 8 + 2 * (lane >> 4);
  const __amdgpu_buffer_rsrc_t r = rsrc(W, M * K * 2);
  const unsigned va = live_wg && row < M ? (unsigned)row * (unsigned)K * 2u + (unsigned)l * 16u : kOutside;
  const unsigned vb = live_wg && row + 1 < M ? (unsigned)(row + 1) * (unsigned)K * 2u + (unsigned)l * 16u : kOutside;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    pf[OFF + j] = __builtin_amdgcn_raw_buffer_load_b128(r, va, j * 256, POL);
    pf[OFF + NJ + j] = __builtin_amdgcn_raw_buffer_load_b128(r, vb, j * 256, POL);
  }
}


// the row's LPR lanes ends with the sums.  All x chunks are read from LDS
// first (a chunk past the row reads inside the staging buffer and is zeroed
// by a select, not a branch), so the reads overlap instead of each paying
// the LDS latency in turn.
// Sixteen int8 weights (a 16-byte chunk) times sixteen bf16 x values: exact
// bf16 pairs (i8pair_bf16), then v_dot2 as for bf16 weights; the row scale is
// applied to the finished sum.
__device__ __forceinline__ void fma16_i8(const u32x4 w, const u32x4 x0, const u32x4 x1, float& a0, float& a1) {
  a0 = dot2(i8pair_bf16(w.x, 0), x0.x, a0);
  a1 = dot2(i8pair_bf16(w.x, 2), x0.y, a1);
  a0 = dot2(i8pair_bf16(w.y, 0), x0.z, a0);
  a1 = dot2(i8pair_bf16(w.y, 2), x0.w, a1);
  a0 = dot2(i8pair_bf16(w.z, 0), x1.x, a0);
  a1 = dot2(i8pair_bf16(w.z, 2), x1.y, a1);
  a0 = dot2(i8pair_bf16(w.w, 0), x1.z, a0);
  a1 = dot2(i8pair_bf16(w.w, 2), x1.w, a1);
}

// W8 rows widened ahead of their dot products: the N raw 16-byte int8 chunks
// in slots OFF + N .. OFF + 2N - 1 become 2N chunks of bf16 pairs in slots
// OFF .. OFF + 2N - 1 (raw chunk i: its weights 0..7 in slot OFF + 2i, 8..15
// in OFF + 2i + 1).  A wave does this while it waits for the phase's input,
// so the dot products then cost what bf16 rows cost.
template <int OFF, int N>
__device__ __forceinline__ void widen_w8(u32x4 (&pf)[kPf]) {
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const u32x4 w = pf[OFF + N + i];
    pf[OFF + 2 * i] = u32x4{i8pair_bf16(w.x, 0), i8pair_bf16(w.x, 2), i8pair_bf16(w.y, 0), i8pair_bf16(w.y, 2)};
    pf[OFF + 2 * i + 1] = u32x4{i8pair_bf16(w.z, 0), i8pair_bf16(w.z, 2), i8pair_bf16(w.w, 0), i8pair_bf16(w.w, 2)};
  }
}

// A W8 row group loaded from its bf16 copy (PersistentLayer::qkv_wide) straight
// into the layout widen_w8 produces: the NJ raw chunks of lane l (16 weights
// at columns 16 (l + LPR j)) become slots OFF + 2j and OFF + 2j + 1.
template <int LPR, int NJ, int OFF>
__device__ __forceinline__ void prefetch_wide(u32x4 (&pf)[kPf], const uint16_t* Wb, int M, int K, int group,
                                              bool live_wg) {
  const int lane = threadIdx.x & 63;
  const int l = lane % LPR, row = group * (64 / LPR) + lane / LPR;
  const bool live = live_wg && row < M;
  const __amdgpu_buffer_rsrc_t r = rsrc(Wb, M * K * 2);
  const unsigned voff = live ? (unsigned)row * (unsigned)K * 2u + (unsigned)l * 32u : kOutside;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    pf[OFF + 2 * j] = __builtin_amdgcn_raw_buffer_load_b128(r, voff, j * LPR * 32, kNT);
    pf[OFF + 2 * j + 1] = __builtin_amdgcn_raw_buffer_load_b128(r, voff, j * LPR * 32 + 16, kNT);
  }
}

// EB 1 with WIDE: the rows' int8 chunks were widened by widen_w8 (chunk j in
// slots OFF + 2j, OFF + 2j + 1; with PAIR the up rows' from OFF + 2 NJ).
template <int LPR, int NJ, bool PAIR, int OFF, int EB = 2, bool WIDE = false>
__device__ __forceinline__ void dot_group(const u32x4 (&pf)[kPf], const uint16_t* xs, int K,
                                          float& acc, float& accu) {
  if constexpr (EB == 1) {
    // chunk j of this lane: columns 16 (l + j LPR) .. + 15
    static_assert((64 + (NJ - 1) * LPR) * 16 <= kXMax, "x reads stay inside the staging buffer");
    const int l = (threadIdx.x & 63) % LPR;
    const int CH = K / 16;
    u32x4 xv[NJ][2];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      xv[j][0] = *reinterpret_cast<const u32x4*>(xs + (l + j * LPR) * 16);
      xv[j][1] = *reinterpret_cast<const u32x4*>(xs + (l + j * LPR) * 16 + 8);
    }
    const u32x4 zero = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      xv[j][0] = l + j * LPR < CH ? xv[j][0] : zero;
      xv[j][1] = l + j * LPR < CH ? xv[j][1] : zero;
    }
    float a0 = 0.f, a1 = 0.f, b0 = 0.f, b1 = 0.f;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      if constexpr (WIDE) {
        fma8(pf[OFF + 2 * j], xv[j][0], a0, a1);
        fma8(pf[OFF + 2 * j + 1], xv[j][1], a0, a1);
        if constexpr (PAIR) {
          fma8(pf[OFF + 2 * NJ + 2 * j], xv[j][0], b0, b1);
          fma8(pf[OFF + 2 * NJ + 2 * j + 1], xv[j][1], b0, b1);
        }
      } else {
        fma16_i8(pf[OFF + j], xv[j][0], xv[j][1], a0, a1);
        if constexpr (PAIR) fma16_i8(pf[OFF + NJ + j], xv[j][0], xv[j][1], b0, b1);
      }
    }
    if constexpr (LPR == 16 || LPR == 64) {
      acc = wave_sum<LPR>(a0 + a1);
      accu = PAIR ? wave_sum<LPR>(b0 + b1) : 0.0f;
    } else if constexpr (LPR == 8) {
      acc = group_sum8(a0 + a1);
      accu = PAIR ? group_sum8(b0 + b1) : 0.0f;
    } else {
      acc = group_sum<LPR>(a0 + a1);
      accu = PAIR ? group_sum<LPR>(b0 + b1) : 0.0f;
    }
    return;
  }
  static_assert((64 + (NJ - 1) * LPR) * 8 <= kXMax, "x reads stay inside the staging buffer");
  const int l = (threadIdx.x & 63) % LPR;
  const int CH = K / 8;
  u32x4 xv[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) xv[j] = *reinterpret_cast<const u32x4*>(xs + (l + j * LPR) * 8);
  const u32x4 zero = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int j = 0; j < NJ; ++j) xv[j] = l + j * LPR < CH ? xv[j] : zero;
  float a0 = 0.f, a1 = 0.f, b0 = 0.f, b1 = 0.f;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    fma8(pf[OFF + j], xv[j], a0, a1);
    if constexpr (PAIR) fma8(pf[OFF + NJ + j], xv[j], b0, b1);
  }
  if constexpr (LPR == 16 || LPR == 64) {
    acc = wave_sum<LPR>(a0 + a1);
    accu = PAIR ? wave_sum<LPR>(b0 + b1) : 0.0f;
  } else if constexpr (LPR == 8) {
    acc = group_sum8(a0 + a1);
    accu = PAIR ? group_sum8(b0 + b1) : 0.0f;
  } else {
    acc = group_sum<LPR>(a0 + a1);
    accu = PAIR ? group_sum<LPR>(b0 + b1) : 0.0f;
  }
}

// The sums of a prefetch_r2 group: ya for row 2 s, yb for row 2 s + 1, in
// all 16 lanes of the pair.  Chunks past the row are zeroed through x.
template <int NJ, int OFF>
__device__ __forceinline__ void dot_r2(const u32x4 (&pf)[kPf], const uint16_t* xs, int K, float& ya, float& yb) {
  static_assert((16 * NJ) * 8 <= kXMax, "x reads stay inside the staging buffer");
  const int l = threadIdx.x & 15;
  const int CH = K / 8;
  u32x4 xv[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) xv[j] = *reinterpret_cast<const u32x4*>(xs + (l + 16 * j) * 8);
  const u32x4 zero = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int j = 0; j < NJ; ++j) xv[j] = l + 16 * j < CH ? xv[j] : zero;
  float a0 = 0.f, a1 = 0.f, b0 = 0.f, b1 = 0.f;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    fma8(pf[OFF + j], xv[j], a0, a1);
    fma8(pf[OFF + NJ + j], xv[j], b0, b1);
  }
  ya = wave_sum<16>(a0 + a1);
  yb = wave_sum<16>(b0 + b1);
}

__device__ __forceinline__ float silu_mul(float g, float u) {
  const float clipped = fminf(fmaxf(g, -80.0f), 80.0f);
  const float denom = 1.0f + expf(-clipped);
  return (g / denom) * u;
}

// ---- split-KV merge ----
// Fold `count` published chunks (chunk j's (P @ V, max, sum) words at
// j * kPartStride of prs, tagged ptag) into the running (mx, lsum, r) of
// output word `lane` (threads 0..63 of one wave), chunks in order.  Each
// round trip loads a batch of MB chunks: lane k chunk j0 + k's (max, sum)
// pair in one 16-byte load, every lane its own output word of each chunk;
// readlane hands the pairs to the whole wave.  No completion wait or
// ticket: each word carries the epoch.  Returns false if the wait gave up.
template <int PPOL, int MB>
__device__ bool fold_partials(const PersistentArgs& a, __amdgpu_buffer_rsrc_t prs, int count, unsigned ptag,
                              int lane, float& mx, float& lsum, float& r) {
  static_assert(MB <= 64, "one (max, sum) pair per lane");
  auto fold = [&](float mj, float sj, float oj) {
    const float nm = fmaxf(mx, mj);
    const float keep = __builtin_amdgcn_exp2f(mx - nm), f = __builtin_amdgcn_exp2f(mj - nm);
    lsum = fmaf(sj, f, lsum * keep);
    r = fmaf(oj, f, r * keep);
    mx = nm;
  };
  for (int j0 = 0; j0 < count; j0 += MB) {
    unsigned long long ow[MB];
    u32x4 ms;
    for (unsigned spins = 1;; ++spins) {
      const int jm = j0 + lane;
      ms = __builtin_amdgcn_raw_buffer_load_b128(
          prs, lane < MB && jm < count ? (unsigned)(jm * kPartStride + kHeadDim) * 8u : kOutside, 0, PPOL);
      bool have = lane >= MB || jm >= count || (ms.y == ptag && ms.w == ptag);
#pragma unroll
      for (int k = 0; k < MB; ++k) {
        const int j = j0 + k;
        ow[k] = ld_p64<PPOL>(prs, j < count ? (unsigned)(j * kPartStride + lane) * 8u : kOutside);
        have = have && (j >= count || (unsigned)(ow[k] >> 32) == ptag);
      }
      if (__all(have)) break;
      if (spins > a.spin_limit || ((spins & 63u) == 0u && ld_c32(a.error) != 0u)) return give_up(a);
      __builtin_amdgcn_s_sleep(1);
    }
#pragma unroll
    for (int k = 0; k < MB; ++k)
      if (j0 + k < count)
        fold(__uint_as_float((unsigned)__builtin_amdgcn_readlane((int)ms.x, k)),
             __uint_as_float((unsigned)__builtin_amdgcn_readlane((int)ms.z, k)), __uint_as_float((unsigned)ow[k]));
  }
  return true;
}

// ---- attention task: query head h, slots [s * kChunk, ...] of layer l ----
// POL: cache policy of the q/k/v polls and the output store (kSc1 across
// the device, kLocal when producers and consumers share an XCD).
// ptag tags the split-KV partial words (ptag_of of the attention epoch); the
// merging task loads MB chunks' words per round trip (a register budget).
// PPOL: cache policy of those partial words, kLocal when every chunk of the
// head runs on the merging task's XCD.
template <class S, int POL = kSc1, int MB = 8, int PPOL = POL>
__device__ bool attention_task(Ctx& c, int l, int h, int s, int p, unsigned tag_q,
                               unsigned tag_a, unsigned ptag) {
  const PersistentArgs& a = *c.a;
  const int g = h / S::QPK;
  const int t0 = s * kChunk;
  const int n = min(kChunk, p + 1 - t0);
  const int nsplit = p / kChunk + 1;
  const bool holds_new = (s == nsplit - 1);
  const int tid = threadIdx.x;
  uint16_t* qs = c.sm->xs[0];           // [64] rotated q, bf16
  uint16_t* knew = qs + kHeadDim;       // [64] rotated new key, bf16
  float* pr = reinterpret_cast<float*>(knew + kHeadDim);  // [kChunk]
  float* acc = pr + kChunk;             // [kGroupsPV][64]
  const size_t head_base = ((size_t)l * S::HKV + g) * a.max_ctx;
  // this head's cache rows [0, p): slots p and beyond read as zero
  const __amdgpu_buffer_rsrc_t kc = rsrc(a.kcache + head_base * kHeadDim, p * kHeadDim * 2);
  const __amdgpu_buffer_rsrc_t vc = rsrc(a.vcache + head_base * kHeadDim, p * kHeadDim * 2);

  HK_STAMP_ATTN(l, 0);
  // Cached K half-row of this thread's slot (two threads per slot, one per
  // 32 dimensions) and V words of its slot group (rows written by earlier
  // launches) go out before the new q/k/v are polled.
  const int si = tid >> 1, half = tid & 1;
  const int slot = t0 + si;
  u32x4 krow[kHeadDim / 16];
#pragma unroll
  for (int ch = 0; ch < kHeadDim / 16; ++ch)
    krow[ch] = __builtin_amdgcn_raw_buffer_load_b128(kc, slot * kHeadDim * 2 + half * kHeadDim,
                                                     ch * 16, 0);
  // P @ V: thread (gi, dp) takes dimensions 2dp, 2dp+1 of the kSlotsPV
  // consecutive slots gi * kSlotsPV ..; slots past p read zero
  const int dp = tid & (kHalf - 1);
  const int gi = tid / kHalf;
  uint32_t vw[kSlotsPV];
  const int voff = (t0 + gi * kSlotsPV) * kHeadDim * 2 + dp * 4;
#pragma unroll
  for (int k = 0; k < kSlotsPV; ++k)
    vw[k] = __builtin_amdgcn_raw_buffer_load_b32(vc, voff, k * kHeadDim * 2, 0);

  const int qr = h * kHeadDim, kr = (S::HQ + g) * kHeadDim, vr = (S::HQ + S::HKV + g) * kHeadDim;
  const __amdgpu_buffer_rsrc_t tqr = rsrc(a.tqkv, S::QKV * 4);
  // The words this thread waits for, polled together: [0, 1] its halves of
  // q or of the new key (threads 0..63, for RoPE), [2, 3] the new value (the
  // key threads of the group's first query head append k and v at slot p),
  // [4, 5] the slot-p value word of its P @ V group
  const int j = tid & (kHalf - 1);
  const bool rope = tid < 2 * kHalf;
  const bool is_k = tid >= kHalf;
  const bool appends = rope && is_k && holds_new && h % S::QPK == 0;
  const int kp = p - t0 - gi * kSlotsPV;  // slot p's index within this thread's P @ V group
  const bool pv_new = kp >= 0 && kp < kSlotsPV;
  const int src_row = is_k ? kr : qr;
  unsigned off[6];
  off[0] = rope ? (unsigned)(src_row + j) * 4u : kOutsideWord;
  off[1] = rope ? (unsigned)(src_row + j + kHalf) * 4u : kOutsideWord;
  off[2] = appends ? (unsigned)(vr + j) * 4u : kOutsideWord;
  off[3] = appends ? (unsigned)(vr + j + kHalf) * 4u : kOutsideWord;
  off[4] = pv_new ? (unsigned)(vr + 2 * dp) * 4u : kOutsideWord;
  off[5] = pv_new ? (unsigned)(vr + 2 * dp + 1) * 4u : kOutsideWord;
  float cs = 0.0f, sn = 0.0f;  // RoPE of position p (constant tables: fetched ahead of the poll)
  if (rope) {
    cs = ldg(a.cos_tab + (size_t)p * kHalf + j);
    sn = ldg(a.sin_tab + (size_t)p * kHalf + j);
  }
  uint32_t w[6];
  bool ok = poll_words<6, POL>(a, tqr, off, tag_q, w);
  if (pv_new) {
    const uint32_t word = (w[4] & 0xffffu) | (w[5] << 16);
#pragma unroll
    for (int k = 0; k < kSlotsPV; ++k)
      if (k == kp) vw[k] = word;
  }
  // rotated q head and new key (bf16-rounded); the group's first query head
  // appends k and v at slot p
  if (rope && ok) {
    const float x1 = bf_lo(w[0]), x2 = bf_lo(w[1]);
    const uint32_t r1 = f32_to_bf16(x1 * cs - x2 * sn);
    const uint32_t r2 = f32_to_bf16(x2 * cs + x1 * sn);
    uint16_t* dst = is_k ? knew : qs;
    dst[j] = (uint16_t)r1;
    dst[j + kHalf] = (uint16_t)r2;
    if (appends) {
      uint16_t* kd = a.kcache + (head_base + p) * kHeadDim;
      uint16_t* vd = a.vcache + (head_base + p) * kHeadDim;
      stg(kd + j, (uint16_t)r1);
      stg(kd + j + kHalf, (uint16_t)r2);
      stg(vd + j, (uint16_t)w[2]);
      stg(vd + j + kHalf, (uint16_t)w[3]);
    }
  }
  if (__syncthreads_or(!ok)) return false;
  HK_STAMP_ATTN(l, 1);

  // scores in base 2: head_dim ** -0.5 (1/8 for head_dim 64) times log2(e),
  // so every exponential below is one v_exp_f32 (2^x); the split-KV maxima
  // are kept in the same base
  const float scale = 0.125f * 1.44269504088896341f;
  // A wave whose 32 slots all lie past the chunk's n live ones (short
  // contexts) would compute zero scores' exponentials and a zero P @ V; it
  // only publishes an empty (max, sum) pair, which leaves the LDS to the live
  // waves, and the merge below reads the live slot groups only.
  const bool wave_live = c.wave * 2 * kSlotsPV < n;
  float mw = -INFINITY, sw = 0.0f;
  if (wave_live) {
  float dot;
  {
    // q and k are bf16: v_dot2 on packed pairs, exact products, float sums
    const u32x4* qh = reinterpret_cast<const u32x4*>(qs + half * kHalf);
    if (slot == p) {  // the new key, packed like a cached row
      const u32x4* kh = reinterpret_cast<const u32x4*>(knew + half * kHalf);
#pragma unroll
      for (int ch = 0; ch < kHeadDim / 16; ++ch) krow[ch] = kh[ch];
    }
    float d0 = 0.0f, d1 = 0.0f;
#pragma unroll
    for (int ch = 0; ch < kHeadDim / 16; ++ch) {
      const u32x4 q = qh[ch];
      d0 = dot2(krow[ch].x, q.x, d0);
      d1 = dot2(krow[ch].y, q.y, d1);
      d0 = dot2(krow[ch].z, q.z, d0);
      d1 = dot2(krow[ch].w, q.w, d1);
    }
    dot = d0 + d1;
  }
  dot = dpp_plus<0xb1>(dot);  // the two halves of the slot (neighbouring lanes)
  HK_STAMP_ATTN(l, 2);
  const bool live = si < n;
  const float sc = live ? dot * scale : -INFINITY;
  // Softmax and P @ V per wave, flash-style: a wave's 32 slots are exactly
  // those of its two P @ V groups (gi = 2 wave, 2 wave + 1), so its max,
  // exponentials, sum and partial P @ V need no workgroup barrier; one
  // barrier then merges the eight waves by log-sum-exp.  (A wave without
  // live slots has max -inf and contributes exp(-inf) = 0; every chunk has a
  // live slot, so the merged max is finite.)
  mw = wave_max64(sc);
  const float e = live ? __builtin_amdgcn_exp2f(sc - mw) : 0.0f;
  sw = wave_sum<64>(half == 0 ? e : 0.0f);  // each slot once
  if (half == 0) pr[si] = e;
  // the P @ V reads below take probabilities written by other lanes of this
  // wave only; a wave's LDS accesses complete in order
  __builtin_amdgcn_wave_barrier();
  HK_STAMP_ATTN(l, 3);

  // probabilities of slots past the chunk's live ones are zero, and so are
  // their value words, so the loop needs no bounds test; the four 16-byte
  // LDS reads go out together
  float o0 = 0.0f, o1 = 0.0f;
  {
    const float4* pr4 = reinterpret_cast<const float4*>(pr + gi * kSlotsPV);
    float4 pq[kSlotsPV / 4];
#pragma unroll
    for (int q = 0; q < kSlotsPV / 4; ++q) pq[q] = pr4[q];
#pragma unroll
    for (int q = 0; q < kSlotsPV / 4; ++q) {
      const float pt[4] = {pq[q].x, pq[q].y, pq[q].z, pq[q].w};
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        o0 = fmaf(pt[r], bf_lo(vw[4 * q + r]), o0);
        o1 = fmaf(pt[r], bf_hi(vw[4 * q + r]), o1);
      }
    }
  }
  acc[gi * kHeadDim + 2 * dp] = o0;
  acc[gi * kHeadDim + 2 * dp + 1] = o1;
  }
  if (c.lane == 0) {
    c.sm->red[0][c.wave] = mw;
    c.sm->red[1][c.wave] = sw;
  }
  __syncthreads();
  HK_STAMP_ATTN(l, 4);
  float m = c.sm->red[0][0];
#pragma unroll
  for (int w = 1; w < kPW; ++w) m = fmaxf(m, c.sm->red[0][w]);
  float fw[kPW], sum = 0.0f;
#pragma unroll
  for (int w = 0; w < kPW; ++w) {
    fw[w] = __builtin_amdgcn_exp2f(c.sm->red[0][w] - m);
    sum = fmaf(c.sm->red[1][w], fw[w], sum);
  }
  constexpr int kGroupsPerWave = 64 / kHalf;
  float o = 0.0f;
  if (tid < kHeadDim) {
    // every group's word is read at once (no branch between the reads, so
    // they overlap); groups past the live slots hold stale values and are
    // replaced by zero before the product
    float av[kGroupsPV];
#pragma unroll
    for (int k = 0; k < kGroupsPV; ++k) av[k] = acc[k * kHeadDim + tid];
#pragma unroll
    for (int k = 0; k < kGroupsPV; ++k) o = fmaf(k * kSlotsPV < n ? av[k] : 0.0f, fw[k / kGroupsPerWave], o);
  }
  if (nsplit == 1) o *= __builtin_amdgcn_rcpf(sum);  // a single chunk normalises here
  uint32_t* out = a.tattn + (size_t)h * kHeadDim;
  // the head's output words; XCD-local stores go through a buffer resource
  auto store_out = [&](uint32_t v) {
    if constexpr (POL == kSc1)
      st_c32(out + tid, v);
    else
      __builtin_amdgcn_raw_buffer_store_b32(v, rsrc(a.tattn, S::AO * 4), (h * kHeadDim + tid) * 4, 0, 0);
  };
  if (nsplit == 1) {
    if (tid < kHeadDim) store_out(tagged(f32_to_bf16(o), tag_a));
    HK_STAMP_ATTN(l, 5);
    return true;
  }

  // split-KV: every chunk but the last publishes its (P @ V, max, sum) as
  // tagged 64-bit words and is done; the task of the last chunk (which holds
  // slot p and has the fewest live slots) polls them and merges by
  // log-sum-exp, chunks in order.
  const __amdgpu_buffer_rsrc_t prs =
      rsrc(a.partial + (size_t)h * a.max_splits * kPartStride, a.max_splits * kPartStride * 8);
  HK_STAMP_ATTN(l, 7);
  if (s != nsplit - 1) {
    if (tid < kPartStride) {
      const float v = tid < kHeadDim ? o : tid == kHeadDim ? m : sum;
      __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, pword(v, ptag)), prs,
                                            (s * kPartStride + tid) * 8, 0, PPOL == kSc1 ? kSc1 : 0);
    }
    return true;
  }
  // (ok is true here: the q/k/v polls succeeded)
  if (tid < kHeadDim) {
    // one pass over the chunks in order with a running maximum (each chunk
    // has live slots, so its maximum is finite), this task's own chunk last
    float mx = -INFINITY, lsum = 0.0f, r = 0.0f;
    ok = fold_partials<PPOL, MB>(a, prs, nsplit - 1, ptag, tid, mx, lsum, r);
    const float nm = fmaxf(mx, m);
    const float keep = __builtin_amdgcn_exp2f(mx - nm), f = __builtin_amdgcn_exp2f(m - nm);
    lsum = fmaf(sum, f, lsum * keep);
    r = fmaf(o, f, r * keep);
    if (ok) store_out(tagged(f32_to_bf16(r / lsum), tag_a));
    HK_STAMP_ATTN(l, 6);
  }
  return !__syncthreads_or(!ok);
}

// Publish one GEMV phase's outputs.  Each compute wave parks its rows'
// tagged words in LDS; the last of the kCW to arrive stores the workgroup's
// rows (contiguous: kCW * RPW of them from `first`) with one instruction, so a
// cache line of outputs has a few writers instead of one per wave -- that is
// what makes it visible to the pollers quickly.  Every compute wave issues
// exactly one global store here (the others to their pad word), which keeps
// the compiler's wait counts exact.
// With `then_load`, every wave of a producer workgroup then waits until the
// gathered store has been issued before it goes on to issue weight loads:
// the CU's memory pipeline is in order, so the store must not queue behind
// tens of kilobytes of prefetch.
template <int RPW, int POL = kSc1, int NW = kCW>
__device__ __forceinline__ void publish_rows(Ctx& c, bool producer, uint32_t word, bool row_lead,
                                             __amdgpu_buffer_rsrc_t tagged_buf, unsigned first,
                                             int valid_rows, unsigned pad, bool then_load, int row_in_wave = -1) {
  static_assert(NW * RPW <= kCW * 16, "gather buffer too small");
  // word offsets into the tagged-activation buffer (a buffer store with a
  // 32-bit offset holds fewer registers than a 64-bit address)
  unsigned dst = pad;
  uint32_t v = 0;
  unsigned old = 0;
  if (producer) {
    const int sub = row_in_wave >= 0 ? row_in_wave : c.lane / (64 / RPW);
    if (row_lead) c.sm->out_val[c.wave * RPW + sub] = word;
    if (c.lane == 0) old = atomicAdd(&c.sm->out_count, 1u);
    old = __builtin_amdgcn_readlane(old, 0);
    if (old % NW == NW - 1 && c.lane < NW * RPW && c.lane < valid_rows) {
      v = c.sm->out_val[c.lane];
      dst = first + c.lane;
    }
  }
  // device-coherent (sc1) like st_c32, or XCD-local (the default policy)
  __builtin_amdgcn_raw_buffer_store_b32(v, tagged_buf, dst * 4u, 0, POL == kSc1 ? kSc1 : 0);
  if (!producer) return;
  const unsigned done = old - old % NW + NW;
  if (old % NW == NW - 1) {
    if (c.lane == 0) __hip_atomic_store(&c.sm->out_stored, done, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  } else if (then_load) {
    // the last wave is at most a few hundred cycles behind; the bound only
    // guards against an unforeseen schedule (ordering is a performance matter)
    for (unsigned spins = 0; spins < (1u << 16); ++spins) {
      if (__hip_atomic_load(&c.sm->out_stored, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) == done) break;
      __builtin_amdgcn_s_sleep(0);
    }
  }
}

// LM head over all eight waves, double-buffered row groups, then the argmax
// over the workgroups' keys on workgroup 0 (shared by both step kernels).
// `buf` is the free LDS staging buffer, `ep_layers` the epoch of the last
// layer's down phase.
template <class S>
__device__ __forceinline__ void lm_head_phase(Ctx& c, u32x4 (&pf)[kPf], int buf, unsigned ep_layers,
                                              unsigned* my_flag, int p) {
  const PersistentArgs& a = *c.a;
  PShared& sm = *c.sm;
  const bool stager = c.wave >= kCW;
  float acc, accu;
  auto handoff = [&](bool ok) -> bool {
    if (stager && c.lane == 0 && !ok) sm.abort = 1;
    __syncthreads();
    return sm.abort == 0;
  };
  // ---- H: LM head over all eight waves.  Wave w of the grid takes row
  // groups w, w + stride, ...; the register slots hold a ring of D row groups
  // (D - 1 of them in flight while one is multiplied), and the compute waves
  // request the first D - 1 before they wait for the final h.  Every wave
  // runs the same number of groups (a multiple of D); past-the-end groups
  // read zero and store to the pad ----
  constexpr int HL = S::head_lpr, HNJ = S::head_nj, HRPW = 64 / HL;
  constexpr int D = kPf / HNJ >= 4 ? 4 : kPf / HNJ;
  static_assert(D >= 2, "LM head rows too long for two row groups in flight");
  const int groups = (a.vocab + HRPW - 1) / HRPW;
  const int stride = kPersistentGrid * kPW;
  const int iters = (groups + stride - 1) / stride;
  float* const lpad = a.logits + a.vocab + c.wg * kPW + c.wave;
  const int grp0 = c.wg * kPW + c.wave;
  auto head_load = [&](auto slot, int k) {  // row group k of this wave into ring slot `slot`
    prefetch<HL, HNJ, false, decltype(slot)::value * HNJ, 2, kHeadPol>(pf, a.lm_head, a.vocab, S::H,
                                                                        grp0 + k * stride, true);
  };
  auto first_loads = [&]() {
    head_load(std::integral_constant<int, 0>{}, 0);
    if constexpr (D > 2) head_load(std::integral_constant<int, 1>{}, 1);
    if constexpr (D > 3) head_load(std::integral_constant<int, 2>{}, 2);
  };
  if (!stager) first_loads();
  {
    bool ok = true;
    if (stager) ok = stage_wave<S::H, true, false>(c, a.th, tag_of(ep_layers), a.final_norm, sm.xs[buf], nullptr);
    if (!handoff(ok)) return;
    normalise_staged<S::H>(c, sm.xs[buf], a.eps);
  }
  if (stager) first_loads();
  const uint16_t* xh = sm.xs[buf];
  unsigned long long best = 0ull;
  const int sub = c.lane / HL;
  auto finish = [&](int k) {
    const int row = (grp0 + k * stride) * HRPW + sub;
    const bool valid = row < a.vocab;
    stg(valid ? a.logits + row : lpad, acc);
    best = umax64(best, valid ? argmax_key(acc, (uint32_t)row) : 0ull);
  };
  // step d of a round: request group k + D - 1 into the slot group k - 1
  // left, then multiply group k (slot d)
  auto ring_step = [&](auto d, int k) {
    constexpr int DD = decltype(d)::value;
    head_load(std::integral_constant<int, (DD + D - 1) % D>{}, k + D - 1);
    dot_group<HL, HNJ, false, DD * HNJ>(pf, xh, S::H, acc, accu);
    finish(k);
  };
  for (int k = 0; k < iters; k += D) {
    ring_step(std::integral_constant<int, 0>{}, k);
    ring_step(std::integral_constant<int, 1>{}, k + 1);
    if constexpr (D > 2) ring_step(std::integral_constant<int, 2>{}, k + 2);
    if constexpr (D > 3) ring_step(std::integral_constant<int, 3>{}, k + 3);
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) best = umax64(best, shfl_xor_u64(best, m));
  if (c.lane == 0) sm.keys[c.wave] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned long long k = sm.keys[0];
#pragma unroll
    for (int w = 1; w < kPW; ++w) k = umax64(k, sm.keys[w]);
    st_c64(a.keys + c.wg, k);
  }
  const unsigned ep_head = ep_layers + 1;
  publish(c, my_flag, ep_head);
  if (c.wg != 0) return;

  // ---- argmax over the workgroups' keys; token feedback (generate.py:709-730) ----
  if (!wait_all(c, a.progress, kPersistentGrid, ep_head)) return;
  unsigned long long k = 0ull;
  for (int i = threadIdx.x; i < kPersistentGrid; i += kPT) k = umax64(k, ld_c64(a.keys + i));
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) k = umax64(k, shfl_xor_u64(k, m));
  if (c.lane == 0) sm.keys[c.wave] = k;
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned long long best_key = sm.keys[0];
#pragma unroll
    for (int w = 1; w < kPW; ++w) best_key = umax64(best_key, sm.keys[w]);
    const int32_t index = (int32_t)argmax_key_index(best_key);
    a.result[0] = index;
    StepCtrl* ctrl = a.ctrl;
    if (ctrl->advance) {
      const int slot = ctrl->n_out;
      if (slot >= 0 && slot < a.max_ctx) a.out_tokens[slot] = index;
      ctrl->n_out = slot + 1;
      ctrl->token = index;
      ctrl->position = p + 1;
    }
  }
}

// The QKV bias as a buffer: a model without one gets an empty range, so the
// loads read zero instead of dereferencing a null base.
template <class S>
__device__ __forceinline__ __amdgpu_buffer_rsrc_t bias_rsrc(const float* bias) {
  return rsrc(bias, bias ? S::QKV * 4 : 0);
}

// ---- the step kernel ----
template <class S>
__global__ __launch_bounds__(kPT) void decode_step_kernel(PersistentArgs args) {
  __shared__ PShared sm;
  Ctx c;
  c.a = &args;
  c.sm = &sm;
  c.wg = blockIdx.x;
  c.wave = threadIdx.x >> 6;
  c.lane = threadIdx.x & 63;
  c.gw = c.wg * kCW + c.wave;
  const bool stager = c.wave >= kCW;
  if (threadIdx.x == 0) {
    sm.abort = 0;
    sm.out_count = 0;
    sm.out_stored = 0;
  }

  const PersistentArgs& a = args;
  const int L = a.layers;
  static_assert(sizeof(PersistentLayer) % 8 == 0, "layer table is copied in 8-byte words");
  {
    constexpr int kWords = sizeof(PersistentLayer) / 8;
    const unsigned long long* src = reinterpret_cast<const unsigned long long*>(a.w);
    unsigned long long* dst = reinterpret_cast<unsigned long long*>(sm.layers);
    for (int i = threadIdx.x; i < L * kWords; i += kPT) dst[i] = ldg(src + i);
  }
  __syncthreads();
  unsigned* my_flag = a.progress + (size_t)c.wg * kFlagStride;
  const unsigned base = ld_c32(my_flag);  // the epoch this workgroup ended the last launch on
  const int token = ldg(&a.ctrl->token);
  const int p = ldg(&a.ctrl->position);
  // layer 0 reads the embedding row, or the hidden state the host preloaded
  const uint16_t* x0 = token >= 0 ? a.embed + (size_t)min(token, a.vocab - 1) * S::H : a.h;
  const bool is_q = c.wg < S::nq, is_o = c.wg < S::no, is_g = c.wg < S::ng, is_d = c.wg < S::nd;
  const int tasks = S::HQ * (p / kChunk + 1);

  // Row of this lane in each GEMV phase.  Every compute wave stores once per
  // phase: a row it does not own (or a phase its workgroup sits out) goes to
  // the wave's own pad word, so all compute waves issue the same stores.
  // publish targets as word offsets in the one tagged-activation allocation
  // (h, h1, qkv, attn, act, then one pad word per wave)
  const unsigned o_h = 0, o_h1 = (unsigned)(a.th1 - a.th), o_qkv = (unsigned)(a.tqkv - a.th);
  const unsigned o_act = (unsigned)(a.tact - a.th), o_pad = (unsigned)(a.pad - a.th);
  const __amdgpu_buffer_rsrc_t tbuf = rsrc(a.th, (int)(o_pad + kPersistentGrid * kPW) * 4);
  const unsigned pad = o_pad + c.wg * kPW + c.wave;
  const int row_q = c.gw * (64 / S::q.lpr) + c.lane / S::q.lpr;
  const int row_o = c.gw * (64 / S::o.lpr) + c.lane / S::o.lpr;
  const int row_d = c.gw * (64 / S::d.lpr) + c.lane / S::d.lpr;
  // first row of this workgroup in each phase and how many of its rows exist
  constexpr int RQ = 64 / S::q.lpr, RO = 64 / S::o.lpr, RG = 64 / S::g.lpr, RD = 64 / S::d.lpr;
  const int fq = c.wg * kCW * RQ, fo = c.wg * kCW * RO, fg = c.wg * kCW * RG, fd = c.wg * kCW * RD;
  const int nvq = S::QKV - fq, nvo = S::H - fo, nvg = S::I - fg, nvd = S::H - fd;
  const bool lq = c.lane % S::q.lpr == 0, lo = c.lane % S::o.lpr == 0;
  const bool lg = c.lane % S::g.lpr == 0, ld = c.lane % S::d.lpr == 0;
  const unsigned dst_h = is_d && row_d < S::H ? (unsigned)row_d * 2u : kOutside;  // byte offset in h
  const int res_o = min(row_o, S::H - 1), res_d = min(row_d, S::H - 1);
  const unsigned bias_off = is_q && !stager && row_q < S::QKV ? (unsigned)row_q * 4u : kOutside;
  // Every wave issues every weight prefetch (the stager's, like those of
  // workgroups that sit a phase out, read zero from outside the resource):
  // a prefetch skipped on one path would keep the registers' previous values
  // live around the whole layer loop.
  const bool pq = is_q && !stager, po = is_o && !stager, pg = is_g && !stager, pd = is_d && !stager;

  u32x4 pf[kPf];
  float acc, accu, bias_q = 0.0f;
  // W8 row scales of this lane's rows (QKV, O, gate, up, down)
  float sq = 1.0f, so = 1.0f, sg = 1.0f, su = 1.0f, sd = 1.0f;
  int buf = 0;  // LDS staging buffer of the next GEMV phase
  // (a W8 scale is requested ahead of its rows: loads complete in order, so
  // the wait for a scale issued later would also wait for later prefetches)
  if constexpr (S::W8) sq = row_scale<S::q.lpr>(sm.layers[0].qkv_scale, S::QKV, c.gw, pq);
  prefetch<S::q.lpr, S::q.nj, false, S::off_q, S::EB>(pf, sm.layers[0].qkv, S::QKV, S::H, c.gw, pq);
  bias_q = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                         bias_rsrc<S>(sm.layers[0].qkv_bias), bias_off, 0, 0));

  // The stager fills xs[buf]; the barrier hands it to the compute waves.
  // Returns false (in every wave) when the launch is abandoned.
  auto handoff = [&](bool ok) -> bool {
    if (stager && c.lane == 0 && !ok) sm.abort = 1;
    __syncthreads();
    return sm.abort == 0;
  };

  for (int l = 0; l < L; ++l) {
    const PersistentLayer& lw = sm.layers[l];
    const unsigned ep = base + 5u * (unsigned)l;  // epoch of the previous layer's down phase
    // ---- Q ----
    if (is_q) {
      bool ok = true;
      if (stager) {
        if (l == 0)
          stage_wave_plain<S::H>(c, x0, lw.in_norm, sm.xs[buf], sm.raw_h);
        else
          ok = stage_wave<S::H, true, true>(c, a.th, tag_of(ep), lw.in_norm, sm.xs[buf], sm.raw_h);
      }
      if (!handoff(ok)) return;
      normalise_staged<S::H>(c, sm.xs[buf], a.eps);
    }
    if (!stager) {
      dot_group<S::q.lpr, S::q.nj, false, S::off_q, S::EB>(pf, sm.xs[buf], S::H, acc, accu);
      if constexpr (S::W8) acc *= sq;
      const uint32_t y = lw.qkv_bias ? f32_to_bf16(round_bf16(acc) + bias_q) : f32_to_bf16(acc);
      publish_rows<RQ>(c, is_q, tagged(y, tag_of(ep + 1)), lq, tbuf, o_qkv + fq, nvq, pad, true);
    }
    if (is_q) buf ^= 1;
    // ---- A ---- (tasks go to the highest workgroups, which own no Q rows;
    // the O and gate/up weights are requested after it, so that registers
    // are not held across attention)
    for (int t = kPersistentGrid - 1 - c.wg; t < tasks; t += kPersistentGrid) {
      __syncthreads();  // LDS reuse
      if (!attention_task<S>(c, l, t % S::HQ, t / S::HQ, p, tag_of(ep + 1), tag_of(ep + 2), ptag_of(ep + 2)))
        return;
    }
    if constexpr (S::W8) {
      so = row_scale<S::o.lpr>(lw.o_scale, S::H, c.gw, po);
      sg = row_scale<S::g.lpr>(lw.gate_up_scale, S::I, c.gw, pg);
      su = row_scale<S::g.lpr>(lw.gate_up_scale + S::I, S::I, c.gw, pg);
    }
    prefetch<S::o.lpr, S::o.nj, false, S::off_o, S::EB>(pf, lw.o, S::H, S::AO, c.gw, po);
    prefetch<S::g.lpr, S::g.nj, true, S::off_g, S::EB>(pf, lw.gate_up, S::I, S::H, c.gw, pg);
    // ---- O ----
    if (is_o) {
      bool ok = true;
      if (stager) ok = stage_wave<S::AO, false, false>(c, a.tattn, tag_of(ep + 2), nullptr, sm.xs[buf], nullptr);
      if (!handoff(ok)) return;
    }
    if (!stager) {
      dot_group<S::o.lpr, S::o.nj, false, S::off_o, S::EB>(pf, sm.xs[buf], S::AO, acc, accu);
      if constexpr (S::W8) acc *= so;
      publish_rows<RO>(c, is_o, tagged(f32_to_bf16(round_bf16(acc) + sm.raw_h[res_o]), tag_of(ep + 3)),
                       lo, tbuf, o_h1 + fo, nvo, pad, true);
    }
    // down and the next layer's QKV go out here rather than after gate/up:
    // issued there, they would queue in this CU's memory pipeline ahead of the
    // stagers' polls for the down input, the largest one of the layer
    {
      const bool more = l + 1 < L;
      const PersistentLayer& nx = sm.layers[more ? l + 1 : l];
      if constexpr (S::W8) {
        sd = row_scale<S::d.lpr>(lw.down_scale, S::H, c.gw, pd);
        sq = row_scale<S::q.lpr>(nx.qkv_scale, S::QKV, c.gw, pq && more);
      }
      prefetch<S::d.lpr, S::d.nj, false, S::off_d, S::EB>(pf, lw.down, S::H, S::I, c.gw, pd);
      prefetch<S::q.lpr, S::q.nj, false, S::off_q, S::EB>(pf, nx.qkv, S::QKV, S::H, c.gw, pq && more);
      bias_q = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                             bias_rsrc<S>(nx.qkv_bias), bias_off, 0, 0));
    }
    if (is_o) buf ^= 1;
    // ---- G ----
    if (is_g) {
      bool ok = true;
      if (stager) ok = stage_wave<S::H, true, true>(c, a.th1, tag_of(ep + 3), lw.post_norm, sm.xs[buf], sm.raw_h1);
      if (!handoff(ok)) return;
      normalise_staged<S::H>(c, sm.xs[buf], a.eps);
    }
    if (!stager) {
      dot_group<S::g.lpr, S::g.nj, true, S::off_g, S::EB>(pf, sm.xs[buf], S::H, acc, accu);
      if constexpr (S::W8) {
        acc *= sg;
        accu *= su;
      }
      publish_rows<RG>(c, is_g, tagged(f32_to_bf16(silu_mul(round_bf16(acc), round_bf16(accu))), tag_of(ep + 4)),
                       lg, tbuf, o_act + fg, nvg, pad, false);
    }
    if (is_g) buf ^= 1;
    // ---- D ----
    if (is_d) {
      bool ok = true;
      if (stager) ok = stage_wave<S::I, false, false>(c, a.tact, tag_of(ep + 4), nullptr, sm.xs[buf], nullptr);
      if (!handoff(ok)) return;
    }
    if (!stager) {
      dot_group<S::d.lpr, S::d.nj, false, S::off_d, S::EB>(pf, sm.xs[buf], S::I, acc, accu);
      if constexpr (S::W8) acc *= sd;
      const uint32_t y = f32_to_bf16(round_bf16(acc) + sm.raw_h1[res_d]);
      publish_rows<RD>(c, is_d, tagged(y, tag_of(ep + 5)), ld, tbuf, o_h + fd, nvd, pad, false);
      // plain copy: the final hidden for hk_engine_final_hidden
      __builtin_amdgcn_raw_buffer_store_b16((uint16_t)y, rsrc(a.h, S::H * 2), dst_h, 0, 0);
    }
    if (is_d) buf ^= 1;
  }
  const unsigned ep_layers = base + 5u * (unsigned)L;
  if (!a.head) {
    if (threadIdx.x == 0) st_c32(my_flag, ep_layers);
    return;
  }

  lm_head_phase<S>(c, pf, buf, ep_layers, my_flag, p);
}

// ---- the XCD split's fused down projection ----
struct XShared : PShared {
  alignas(16) float wsum[kCW][kHMax];  // the compute waves' partial down products
};


// down_x rows of this wave's row group (four intermediate rows): chunk
// c = lane + 64 k of the group's xdc output chunks goes to slots
// OFF + 4k .. OFF + 4k + 3 (chunks past xdc and dead groups read zero).
template <class S, int OFF>
__device__ __forceinline__ void prefetch_down_x(u32x4 (&pf)[kPf], const uint16_t* dx, int group, bool live) {
  constexpr int CC = S::xdc;
  const __amdgpu_buffer_rsrc_t r = rsrc(dx, S::I * S::H * S::EB);
  const int lane = threadIdx.x & 63;
  const bool ok = live && group < S::I / 4;
#pragma unroll
  for (int k = 0; k < S::xkd; ++k) {
    const int cc = lane + 64 * k;
    const unsigned voff = ok && cc < CC ? (unsigned)(group * CC + cc) * 64u : kOutside;
#pragma unroll
    for (int q = 0; q < 4; ++q) pf[OFF + 4 * k + q] = __builtin_amdgcn_raw_buffer_load_b128(r, voff, q * 16, kNT);
  }
}

// This wave's partial down product: act (bf16 bits; lanes 16 s .. 16 s + 15
// hold row s of the group) times the group's down_x chunks, written to ws[H].
// For W8 (unscaled int8 down rows; the row scale is applied to the finished
// sum in reduce_h) a chunk holds 16 outputs: slot q outputs 4q .. 4q + 3,
// each as the four rows' int8 weights.
template <class S, int OFF, bool WIDE = false>
__device__ __forceinline__ void down_partial(const u32x4 (&pf)[kPf], uint32_t act, float* ws) {
  constexpr int CC = S::xdc;
  const int lane = threadIdx.x & 63;
  const uint32_t a0 = __builtin_amdgcn_readlane(act, 0), a1 = __builtin_amdgcn_readlane(act, 16);
  const uint32_t a2 = __builtin_amdgcn_readlane(act, 32), a3 = __builtin_amdgcn_readlane(act, 48);
  const uint32_t A01 = (a0 & 0xffffu) | (a1 << 16), A23 = (a2 & 0xffffu) | (a3 << 16);
  if constexpr (S::W8 && WIDE) {
    // widened chunks (widen_w8): slot q of chunk k holds outputs 2q, 2q + 1
    // of its 16, the four rows' bf16 weights each, as for bf16 rows
#pragma unroll
    for (int k = 0; k < S::xkd; ++k) {
      const int cc = lane + 64 * k;
      float o[16];
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const u32x4 w = pf[OFF + 8 * k + q];
        o[2 * q] = dot2(w.x, A01, dot2(w.y, A23, 0.0f));
        o[2 * q + 1] = dot2(w.z, A01, dot2(w.w, A23, 0.0f));
      }
      if (cc < CC) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          reinterpret_cast<float4*>(ws + 16 * cc)[q] = make_float4(o[4 * q], o[4 * q + 1], o[4 * q + 2], o[4 * q + 3]);
      }
    }
    return;
  }
  if constexpr (S::W8) {
#pragma unroll
    for (int k = 0; k < S::xkd; ++k) {
      const int cc = lane + 64 * k;
      float o[16];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const u32x4 w = pf[OFF + 4 * k + q];
        o[4 * q] = dot2(i8pair_bf16(w.x, 0), A01, dot2(i8pair_bf16(w.x, 2), A23, 0.0f));
        o[4 * q + 1] = dot2(i8pair_bf16(w.y, 0), A01, dot2(i8pair_bf16(w.y, 2), A23, 0.0f));
        o[4 * q + 2] = dot2(i8pair_bf16(w.z, 0), A01, dot2(i8pair_bf16(w.z, 2), A23, 0.0f));
        o[4 * q + 3] = dot2(i8pair_bf16(w.w, 0), A01, dot2(i8pair_bf16(w.w, 2), A23, 0.0f));
      }
      if (cc < CC) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          reinterpret_cast<float4*>(ws + 16 * cc)[q] = make_float4(o[4 * q], o[4 * q + 1], o[4 * q + 2], o[4 * q + 3]);
      }
    }
    return;
  }
#pragma unroll
  for (int k = 0; k < S::xkd; ++k) {
    const int cc = lane + 64 * k;
    float o[8];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const u32x4 w = pf[OFF + 4 * k + q];  // outputs 2q, 2q + 1 of the chunk, rows 0..3 each
      o[2 * q] = dot2(w.x, A01, dot2(w.y, A23, 0.0f));
      o[2 * q + 1] = dot2(w.z, A01, dot2(w.w, A23, 0.0f));
    }
    if (cc < CC) {
      reinterpret_cast<float4*>(ws + 8 * cc)[0] = make_float4(o[0], o[1], o[2], o[3]);
      reinterpret_cast<float4*>(ws + 8 * cc)[1] = make_float4(o[4], o[5], o[6], o[7]);
    }
  }
}

// Stager wave 0 of MLP workgroup jx of XCD xcd: outputs xsl * jx + lane of
// the XCD's down product, the sum over its nprod producing workgroups (local
// index j, in order) of their partials (tag pt), stored to xpart across the
// device.  False (in every lane) when the launch is abandoned.
template <class S>
__device__ bool reduce_xcd(Ctx& c, int xcd, int jx, int nprod, unsigned pt) {
  const PersistentArgs& a = *c.a;
  const int e = S::xsl * jx + c.lane;
  const bool live = c.lane < S::xsl && e < S::H;
  const __amdgpu_buffer_rsrc_t r = rsrc(a.wpart, kPersistentGrid * S::H * 8);
  unsigned long long v[kXcdWg];
  bool ok = true;
  for (unsigned spins = 1;; ++spins) {
    bool have = true;
#pragma unroll
    for (int j = 0; j < kXcdWg; ++j) {
      const unsigned off = live && j < nprod ? (unsigned)(((kXcds * j + xcd) * S::H + e) * 8) : kOutside;
      v[j] = __builtin_bit_cast(unsigned long long, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, kLocal));
    }
#pragma unroll
    for (int j = 0; j < kXcdWg; ++j) have = have && (!live || j >= nprod || (unsigned)(v[j] >> 32) == pt);
    if (__all(have)) break;
    if (spins > a.spin_limit || ((spins & 63u) == 0u && ld_c32(a.error) != 0u)) {
      ok = give_up(a);
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  if (ok && live) {
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < kXcdWg; ++j)
      if (j < nprod) sum += __uint_as_float((unsigned)v[j]);
    const unsigned long long w = ((unsigned long long)pt << 32) | __float_as_uint(sum);
    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, w), rsrc(a.xpart, kXcds * S::H * 8),
                                          (xcd * S::H + e) * 8, 0, kSc1);
  }
  return __all(ok);
}

// A stager wave of XCD 0: outputs xhs * slice + lane of the layer
// output h = bf16(bf16(sum over XCDs 1..7 of their partials) + h1), the
// down_proj epilogue of the undivided step.  Stored three ways: tagged in
// `local` with the default policy (the next layer's QKV stagers on XCD 0
// poll it there), tagged in h across the device (the LM head polls it), and
// as plain bf16.
template <class S>
__device__ bool reduce_h(Ctx& c, int slice, unsigned pt, unsigned tag_h1, unsigned tag_h, uint32_t* local,
                         const float* dscale) {
  const PersistentArgs& a = *c.a;
  const int e = S::xhs * slice + c.lane;
  const bool live = c.lane < S::xhs && e < S::H;
  // W8: the down row scale of output e, for the finished sum
  float sd = 1.0f;
  if constexpr (S::W8)
    sd = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                       rsrc(dscale, S::H * 4), live ? (unsigned)e * 4u : kOutside, 0, 0));
  const __amdgpu_buffer_rsrc_t r = rsrc(a.xpart, kXcds * S::H * 8);
  const __amdgpu_buffer_rsrc_t rh1 = rsrc(a.th1, S::H * 4);
  unsigned long long v[kXcds - 1];
  uint32_t h1 = 0;
  bool ok = true;
  for (unsigned spins = 1;; ++spins) {
#pragma unroll
    for (int x = 1; x < kXcds; ++x)
      v[x - 1] = __builtin_bit_cast(unsigned long long, __builtin_amdgcn_raw_buffer_load_b64(
                                                          r, live ? (unsigned)((x * S::H + e) * 8) : kOutside, 0, kSc1));
    h1 = __builtin_amdgcn_raw_buffer_load_b32(rh1, live ? (unsigned)e * 4u : kOutside, 0, kSc1);
    bool have = !live || (h1 >> 16) == tag_h1;
#pragma unroll
    for (int x = 0; x < kXcds - 1; ++x) have = have && (!live || (unsigned)(v[x] >> 32) == pt);
    if (__all(have)) break;
    if (spins > a.spin_limit || ((spins & 63u) == 0u && ld_c32(a.error) != 0u)) {
      ok = give_up(a);
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  if (ok && live) {
    float sum = 0.0f;
#pragma unroll
    for (int x = 0; x < kXcds - 1; ++x) sum += __uint_as_float((unsigned)v[x]);
    if constexpr (S::W8) sum *= sd;
    const uint32_t y = f32_to_bf16(round_bf16(sum) + bf_lo(h1));
    __builtin_amdgcn_raw_buffer_store_b32(tagged(y, tag_h), rsrc(local, S::H * 4), e * 4, 0, 0);
    __builtin_amdgcn_raw_buffer_store_b32(tagged(y, tag_h), rsrc(a.th, S::H * 4), e * 4, 0, kSc1);
    __builtin_amdgcn_raw_buffer_store_b16((uint16_t)y, rsrc(a.h, S::H * 2), e * 2, 0, 0);
  }
  return __all(ok);
}

// ---- the step kernel, split by XCD ----
// The attention block (input RMSNorm, QKV, attention, O + residual) runs on
// the 32 workgroups of XCD 0 and the MLP (post-attention RMSNorm, gate/up +
// SwiGLU, down as partial sums) on the 224 workgroups of the other XCDs;
// XCD 0 adds the partials and the residual.  The
// QKV -> attention and attention -> O hand-offs then stay inside one L2
// (kLocal policy, ~0.5 us against ~1.3 us across XCDs), and each side
// streams its next layer's weights while the other side computes, so no
// prefetch queues ahead of a poll.  down_proj is fused into the gate/up
// workgroups (split-K over the intermediate rows, reduced per workgroup, per
// XCD and finally on XCD 0), so act never crosses XCDs; the act buffer holds
// XCD 0's local copy of h instead.  Epochs, tags and flags are those of
// decode_step_kernel: launches of the two kernels may alternate.  Data the
// XCD-local stores leave in XCD 0's L2 is written back at the end of the
// launch, before another kernel can read it from another XCD.
// LONG: the long-context form.  A layer's attention tasks (heads x 256-slot
// chunks) then outnumber XCD 0's row-free workgroups, so they run on the MLP
// workgroups (one task each up to 224 tasks), which sit idle during the
// attention block anyway; the QKV -> attention and attention -> O hand-offs
// then cross XCDs (sc1), the rest is unchanged.
template <class S, bool LONG>
__global__ __launch_bounds__(kPT) void decode_step_xa_kernel(PersistentArgs args) {
  __shared__ XShared sm;
  Ctx c;
  c.a = &args;
  c.sm = &sm;
  c.wg = blockIdx.x;
  c.wave = threadIdx.x >> 6;
  c.lane = threadIdx.x & 63;
  const bool stager = c.wave >= kCW;
  if (threadIdx.x == 0) {
    sm.abort = 0;
    sm.out_count = 0;
    sm.out_stored = 0;
  }
  const PersistentArgs& a = args;
  const int L = a.layers;
  // the epoch, token and position go out with the layer table's loads, so
  // their latencies overlap
  unsigned* my_flag = a.progress + (size_t)c.wg * kFlagStride;
  const unsigned base = ld_c32(my_flag);
  const int token = ldg(&a.ctrl->token);
  const int p = ldg(&a.ctrl->position);
  {
    constexpr int kWords = sizeof(PersistentLayer) / 8;
    const unsigned long long* src = reinterpret_cast<const unsigned long long*>(a.w);
    unsigned long long* dst = reinterpret_cast<unsigned long long*>(sm.layers);
    for (int i = threadIdx.x; i < L * kWords; i += kPT) dst[i] = ldg(src + i);
  }
  __syncthreads();
  // the XCD-local hand-offs are only coherent if the workgroups that share
  // them share an L2: leave (the launch is abandoned) if this workgroup is
  // not on the XCD the split assumes
  unsigned xcc;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
  if ((xcc & 15u) != (unsigned)(c.wg % kXcds)) {
    if (threadIdx.x == 0) give_up(a);
    return;
  }
  const uint16_t* x0 = token >= 0 ? a.embed + (size_t)min(token, a.vocab - 1) * S::H : a.h;
  const bool attn = c.wg % kXcds == 0;
  // rank of the workgroup within its side, and its compute waves' indices
  const int rank = attn ? c.wg / kXcds : (c.wg / kXcds) * (kXcds - 1) + c.wg % kXcds - 1;
  // row-group index of this wave: all kPW waves on XCD 0, the kCW compute
  // waves on the MLP side (a stager's index there is never live)
  c.gw = rank * (attn ? kPW : kCW) + c.wave;

  const unsigned o_h1 = (unsigned)(a.th1 - a.th), o_qkv = (unsigned)(a.tqkv - a.th);
  const unsigned o_pad = (unsigned)(a.pad - a.th);
  const __amdgpu_buffer_rsrc_t tbuf = rsrc(a.th, (int)(o_pad + kPersistentGrid * kPW) * 4);
  const unsigned pad = o_pad + c.wg * kPW + c.wave;
  u32x4 pf[kPf];
  float acc, accu;
  int buf = 0;
  auto handoff = [&](bool ok) -> bool {
    if (stager && c.lane == 0 && !ok) sm.abort = 1;
    __syncthreads();
    return sm.abort == 0;
  };

  if (attn) {
    constexpr PhaseCfg Q = S::xq, O = S::xo;
    // register slots: Q rows from 0, O rows after them; W8 rows are loaded
    // into the upper half of twice their slots and widened there (widen_w8);
    // bf16 rows two per lane (R2: prefetch_r2, dot_r2)
    constexpr bool R2 = S::xr2;
    constexpr int WQ = S::W8 ? 2 : 1;
    constexpr int RQ = 64 / Q.lpr, RO = 64 / O.lpr, OFF_O = R2 ? 2 * S::xq2 : WQ * Q.nj;
    constexpr int LQ = S::W8 ? Q.nj : 0, LO = OFF_O + (S::W8 ? O.nj : 0);  // where the loads land
    static_assert(!R2 || (RQ == 8 && RO == 8), "two rows per lane keep eight rows per wave");
    const bool is_q = rank < S::xnq, is_o = rank < S::xno;
    // R2: lanes 0 and 1 of each 16-lane pair hold its two rows' outputs
    const int sub2 = 2 * (c.lane >> 4) + (c.lane & 1);
    const int row_q = R2 ? c.gw * 8 + sub2 : c.gw * RQ + c.lane / Q.lpr;
    const int row_o = R2 ? c.gw * 8 + sub2 : c.gw * RO + c.lane / O.lpr;
    const int fo = rank * kPW * RO;
    const bool lq = R2 ? (c.lane & 15) < 2 : c.lane % Q.lpr == 0;
    const bool lo = R2 ? (c.lane & 15) < 2 : c.lane % O.lpr == 0;
    const int sub_q = R2 ? sub2 : -1;
    // W8: the stager waves load their rows from the bf16 copies, already in
    // the widened layout (they poll before their rows could be widened; the
    // compute waves widen theirs while they wait)
    auto prefetch_q = [&](const PersistentLayer& w, bool live) {
      if constexpr (R2)
        prefetch_r2<S::xq2, 0>(pf, w.qkv, S::QKV, S::H, c.gw, live);
      else if constexpr (S::W8) {
        if (stager)
          prefetch_wide<Q.lpr, Q.nj, 0>(pf, w.qkv_wide, S::QKV, S::H, c.gw, live);
        else
          prefetch<Q.lpr, Q.nj, false, LQ, S::EB>(pf, w.qkv, S::QKV, S::H, c.gw, live);
      } else
        prefetch<Q.lpr, Q.nj, false, LQ, S::EB>(pf, w.qkv, S::QKV, S::H, c.gw, live);
    };
    auto prefetch_o = [&](const PersistentLayer& w, bool live) {
      if constexpr (R2)
        prefetch_r2<S::xo2, OFF_O>(pf, w.o, S::H, S::AO, c.gw, live);
      else if constexpr (S::W8) {
        if (stager)
          prefetch_wide<O.lpr, O.nj, OFF_O>(pf, w.o_wide, S::H, S::AO, c.gw, live);
        else
          prefetch<O.lpr, O.nj, false, LO, S::EB>(pf, w.o, S::H, S::AO, c.gw, live);
      } else
        prefetch<O.lpr, O.nj, false, LO, S::EB>(pf, w.o, S::H, S::AO, c.gw, live);
    };
    const int res_o = min(row_o, S::H - 1);
    const unsigned bias_off = is_q && row_q < S::QKV ? (unsigned)row_q * 4u : kOutside;
    const bool pq = is_q, po = is_o;
    const int tasks = S::HQ * (p / kChunk + 1);
    const int hslice = rank >= S::xnq ? (rank - S::xnq) * kSW + (c.wave - kCW) : S::xhn;
    // W8 row scales, requested ahead of their rows (loads complete in order)
    float sq = 1.0f, so = 1.0f;
    if constexpr (S::W8) {
      sq = row_scale<Q.lpr>(sm.layers[0].qkv_scale, S::QKV, c.gw, pq);
      so = row_scale<O.lpr>(sm.layers[0].o_scale, S::H, c.gw, po);
    }
    prefetch_q(sm.layers[0], pq);
    prefetch_o(sm.layers[0], po);
    float bias_q = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                 bias_rsrc<S>(sm.layers[0].qkv_bias), bias_off, 0, 0));
    for (int l = 0; l < L; ++l) {
      const PersistentLayer& lw = sm.layers[l];
      const unsigned ep = base + 5u * (unsigned)l;
      const bool more = l + 1 < L;
      const PersistentLayer& nx = sm.layers[more ? l + 1 : l];
      // ---- Q: h from the MLP side (across XCDs) ----
      if (is_q) {
        bool ok = true;
        if constexpr (S::W8) {  // before the wait: the loads have had the MLP phase to land
          if (!stager) {
            widen_w8<0, Q.nj>(pf);
            if (is_o) widen_w8<OFF_O, O.nj>(pf);
          }
        }
        if (stager) {
          if (l == 0)
            stage_wave_plain<S::H>(c, x0, lw.in_norm, sm.xs[buf], sm.raw_h);
          else  // h from XCD 0's own reducers (reduce_h), in its L2
            ok = stage_wave<S::H, true, true, kLocal>(c, a.tact, tag_of(ep), lw.in_norm, sm.xs[buf], sm.raw_h);
        }
        if (!handoff(ok)) return;
        normalise_staged<S::H>(c, sm.xs[buf], a.eps);
        HK_STAMP(l, 0);
      }
      {  // all eight waves; the rows go straight to XCD 0's L2 (only the
         // attention tasks there poll them): each row's first lane stores it,
         // the other lanes the wave's pad word, one store per wave
        if constexpr (R2) {
          float ya, yb;
          dot_r2<S::xq2, 0>(pf, sm.xs[buf], S::H, ya, yb);
          acc = (c.lane & 1) ? yb : ya;
        } else {
          dot_group<Q.lpr, Q.nj, false, 0, S::EB, S::W8>(pf, sm.xs[buf], S::H, acc, accu);
        }
        if constexpr (S::W8) acc *= sq;
        HK_STAMP(l, 10);
        const uint32_t y = lw.qkv_bias ? f32_to_bf16(round_bf16(acc) + bias_q) : f32_to_bf16(acc);
        if constexpr (LONG) {  // to the MLP workgroups: gathered, one writer per workgroup
          publish_rows<RQ, kSc1, kPW>(c, is_q, tagged(y, tag_of(ep + 1)), lq, tbuf, o_qkv + rank * kPW * RQ,
                                      S::QKV - rank * kPW * RQ, pad, true, sub_q);
          HK_STAMP(l, 1);
        } else {
          const unsigned dst = is_q && lq && row_q < S::QKV ? o_qkv + (unsigned)row_q : pad;
          __builtin_amdgcn_raw_buffer_store_b32(tagged(y, tag_of(ep + 1)), tbuf, dst * 4u, 0, 0);
          HK_STAMP(l, 1);
        }
      }
      if (is_q) buf ^= 1;
      // ---- A: tasks on the highest ranks, which hold no QKV or O rows ----
      for (int t = kXcdWg - 1 - rank; !LONG && t < tasks; t += kXcdWg) {
        __syncthreads();  // LDS reuse
        if (!attention_task<S, kLocal, 4>(c, l, t % S::HQ, t / S::HQ, p, tag_of(ep + 1), tag_of(ep + 2),
                                          ptag_of(ep + 2)))
          return;
        HK_STAMP(l, 2);
      }
      // ---- O: h1 to the MLP side ----
      if (is_o) {
        bool ok = true;
        if (stager)
          ok = stage_wave<S::AO, false, false, LONG ? kSc1 : kLocal>(c, a.tattn, tag_of(ep + 2), nullptr,
                                                                     sm.xs[buf], nullptr);
        if (!handoff(ok)) return;
        HK_STAMP(l, 3);
      }
      {  // all eight waves
        // the residual goes out before the dot products' LDS reads, so its
        // latency overlaps them
        const float res_h = sm.raw_h[res_o];
        asm volatile("" ::: "memory");
        if constexpr (R2) {
          float ya, yb;
          dot_r2<S::xo2, OFF_O>(pf, sm.xs[buf], S::AO, ya, yb);
          acc = (c.lane & 1) ? yb : ya;
        } else {
          dot_group<O.lpr, O.nj, false, OFF_O, S::EB, S::W8>(pf, sm.xs[buf], S::AO, acc, accu);
        }
        if constexpr (S::W8) acc *= so;
        HK_STAMP(l, 11);
        publish_rows<RO, kSc1, kPW>(c, is_o, tagged(f32_to_bf16(round_bf16(acc) + res_h), tag_of(ep + 3)),
                                    lo, tbuf, o_h1 + fo, S::H - fo, pad, true, sub_q);
        HK_STAMP(l, 4);
      }
      if (is_o) buf ^= 1;
      // the next layer's QKV and O rows go out once this layer's attention
      // block is done, while the MLP side computes: issued earlier, they
      // would queue in this CU's memory pipeline ahead of the attention
      // task's K/V loads and the O stagers' polls
      if constexpr (S::W8) {
        sq = row_scale<Q.lpr>(nx.qkv_scale, S::QKV, c.gw, pq && more);
        so = row_scale<O.lpr>(nx.o_scale, S::H, c.gw, po && more);
      }
      prefetch_q(nx, pq && more);
      bias_q = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                             bias_rsrc<S>(nx.qkv_bias), bias_off, 0, 0));
      prefetch_o(nx, po && more);
      // ---- h = h1 + down(act) from the MLP XCDs' partials, on the stager
      // waves of the workgroups without rows (an abandoned wait ends every
      // later wait of the launch through the error word) ----
      if (stager && hslice < S::xhn &&
          !reduce_h<S>(c, hslice, ptag_of(ep + 4), tag_of(ep + 3), tag_of(ep + 5), a.tact, lw.down_scale) &&
          c.lane == 0)
        sm.abort = 1;
      if (hslice < S::xhn) HK_STAMP_BY(kCW * 64, l, 9);
    }
  } else {
    constexpr PhaseCfg G = S::xg;
    // slots: gate rows from 0, up rows, then the down chunks; W8 rows and
    // chunks are loaded into the upper half of twice their slots and widened
    constexpr int WG = S::W8 ? 2 : 1;
    constexpr int OFF_U = WG * G.nj, OFF_D = 2 * WG * G.nj;
    constexpr int LG = S::W8 ? G.nj : 0, LU = OFF_U + LG, LD = OFF_D + (S::W8 ? 4 * S::xkd : 0);
    const int xcd = c.wg % kXcds, jx = c.wg / kXcds;  // this XCD, and the index within it
    const bool is_g = rank < S::xng;
    const bool pg = is_g && !stager;
    // workgroups of this XCD with gate/up rows: local index j, rank 7 j + xcd - 1
    int nprod = 0;
    for (int j = 0; j < kXcdWg; ++j) nprod += (kXcds - 1) * j + xcd - 1 < S::xng ? 1 : 0;
    const int tasks_l = S::HQ * (p / kChunk + 1);
    float sg = 1.0f, su = 1.0f;  // W8 row scales of this lane's gate and up rows
    auto scales_g = [&](const PersistentLayer& w, bool live) {
      if constexpr (S::W8) {
        sg = row_scale<G.lpr>(w.gate_up_scale, S::I, c.gw, live);
        su = row_scale<G.lpr>(w.gate_up_scale + S::I, S::I, c.gw, live);
      }
    };
    scales_g(sm.layers[0], pg);
    prefetch<G.lpr, G.nj, true, LG, S::EB, kNT, LU>(pf, sm.layers[0].gate_up, S::I, S::H, c.gw, pg);
    prefetch_down_x<S, LD>(pf, sm.layers[0].down_x, c.gw, pg);
    for (int l = 0; l < L; ++l) {
      const PersistentLayer& lw = sm.layers[l];
      const unsigned ep = base + 5u * (unsigned)l;
      const bool more = l + 1 < L;
      const PersistentLayer& nx = sm.layers[more ? l + 1 : l];
      const unsigned pt = ptag_of(ep + 4);
      if constexpr (LONG) {
        // ---- attention tasks (q/k/v from XCD 0, outputs back to it); the
        // next layer's MLP weights go out after them, not ahead of their
        // K/V loads and polls ----
        // Task t runs on rank t, i.e. on XCD t % 7 + 1: when the query heads
        // are a multiple of 7, every chunk of head h (tasks h + HQ s) runs on
        // XCD h % 7 + 1 beside the head's merging task, and the split-KV
        // partials stay in that XCD's L2
        constexpr int kPartPol = S::HQ % (kXcds - 1) == 0 ? kLocal : kSc1;
        for (int t = rank; t < tasks_l; t += kPersistentGrid - kXcdWg) {
          __syncthreads();  // LDS reuse
          if (!attention_task<S, kSc1, 16, kPartPol>(c, l, t % S::HQ, t / S::HQ, p, tag_of(ep + 1),
                                                     tag_of(ep + 2), ptag_of(ep + 2)))
            return;
        }
        if (l > 0) {
          scales_g(lw, pg);
          prefetch<G.lpr, G.nj, true, LG, S::EB, kNT, LU>(pf, lw.gate_up, S::I, S::H, c.gw, pg);
          prefetch_down_x<S, LD>(pf, lw.down_x, c.gw, pg);
        }
      }
      // ---- gate/up + SwiGLU on h1 from XCD 0, then this wave's rows of down ----
      if (is_g) {
        bool ok = true;
        if constexpr (S::W8) {  // before the wait, as on XCD 0
          if (pg) {
            widen_w8<0, G.nj>(pf);
            widen_w8<OFF_U, G.nj>(pf);
            widen_w8<OFF_D, 4 * S::xkd>(pf);
          }
        }
        if (stager) ok = stage_wave<S::H, true, false>(c, a.th1, tag_of(ep + 3), lw.post_norm, sm.xs[buf], nullptr);
        if (!handoff(ok)) return;
        normalise_staged<S::H>(c, sm.xs[buf], a.eps);
        HK_STAMP(l, 5);
        if (!stager) {
          dot_group<G.lpr, G.nj, true, 0, S::EB, S::W8>(pf, sm.xs[buf], S::H, acc, accu);
          HK_STAMP(l, 12);
          if constexpr (S::W8) {
            acc *= sg;
            accu *= su;
          }
          down_partial<S, OFF_D, S::W8>(pf, f32_to_bf16(silu_mul(round_bf16(acc), round_bf16(accu))), sm.wsum[c.wave]);
          HK_STAMP(l, 13);
        }
        __syncthreads();
        HK_STAMP(l, 6);
        // the workgroup's partial: thread t adds outputs 2t, 2t + 1 over the
        // compute waves, in order
        if (threadIdx.x < S::H / 2) {
          const int t = threadIdx.x;
          float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
          for (int w = 0; w < kCW; ++w) {
            s0 += sm.wsum[w][2 * t];
            s1 += sm.wsum[w][2 * t + 1];
          }
          const u32x4 words = {__float_as_uint(s0), pt, __float_as_uint(s1), pt};
          __builtin_amdgcn_raw_buffer_store_b128(words, rsrc(a.wpart, kPersistentGrid * S::H * 8),
                                                 (c.wg * S::H + 2 * t) * 8, 0, 0);
        }
        HK_STAMP(l, 7);
        buf ^= 1;
      }
      // ---- this workgroup's outputs of the XCD's sum (stager wave 0); the
      // barrier keeps the next weight loads behind its polls ----
      {
        bool ok = true;
        if (c.wave == kCW) ok = reduce_xcd<S>(c, xcd, jx, nprod, pt);
        if (!handoff(ok)) return;
        HK_STAMP(l, 8);
      }
      if constexpr (!LONG) {
        scales_g(nx, pg && more);
        prefetch<G.lpr, G.nj, true, LG, S::EB, kNT, LU>(pf, nx.gate_up, S::I, S::H, c.gw, pg && more);
        prefetch_down_x<S, LD>(pf, nx.down_x, c.gw, pg && more);
      }
    }
  }
  const unsigned ep_layers = base + 5u * (unsigned)L;
  if (!a.head) {
    if (threadIdx.x == 0) st_c32(my_flag, ep_layers);
    return;
  }
  lm_head_phase<S>(c, pf, buf, ep_layers, my_flag, p);
}

using SmolShape = Shape<576, 1536, 9, 3>;
using QwenShape = Shape<896, 4864, 14, 2>;
using SmolShapeW8 = Shape<576, 1536, 9, 3, true>;
using QwenShapeW8 = Shape<896, 4864, 14, 2, true>;

template <class S>
bool matches(int hidden, int intermediate, int q_heads, int kv_heads) {
  return hidden == S::H && intermediate == S::I && q_heads == S::HQ && kv_heads == S::HKV;
}

template <class S>
int launch_shape(const PersistentArgs& a, hipStream_t stream, int form) {
  if (form != kStepUndivided) {
    if constexpr (S::xa) {
      if (form == kStepSplitLong)
        hipLaunchKernelGGL((decode_step_xa_kernel<S, true>), dim3(kPersistentGrid), dim3(kPT), 0, stream, a);
      else
        hipLaunchKernelGGL((decode_step_xa_kernel<S, false>), dim3(kPersistentGrid), dim3(kPT), 0, stream, a);
    } else
      return fail("persistent step: no XCD split for this model shape");
  } else {
    hipLaunchKernelGGL(decode_step_kernel<S>, dim3(kPersistentGrid), dim3(kPT), 0, stream, a);
  }
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? 0 : hip_fail(err, "persistent step launch");
}

template <class K>
int occupancy_of(K kernel) {
  int blocks = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, kernel, kPT, 0) != hipSuccess) return 0;
  return blocks >= 1;
}

template <class S>
int occupancy_ok() {
  return occupancy_of(decode_step_kernel<S>);
}

// XCC_ID of every workgroup of a kPersistentGrid-workgroup launch.
__global__ void xcc_probe_kernel(unsigned* out) {
  unsigned xcc;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
  if (threadIdx.x == 0) out[blockIdx.x] = xcc & 15u;
}

// 1 when workgroup i of a launch runs on XCD i % kXcds; else 0, with the
// reason in hk_last_error().
int xcd_layout_ok(hipStream_t stream) {
  unsigned* d = nullptr;
  if (hipMalloc(&d, kPersistentGrid * sizeof(unsigned)) != hipSuccess) {
    set_error("XCD split: hipMalloc failed");
    return 0;
  }
  unsigned h[kPersistentGrid] = {};
  (void)hipGetLastError();  // an earlier call's error is not this launch's
  hipLaunchKernelGGL(xcc_probe_kernel, dim3(kPersistentGrid), dim3(64), 0, stream, d);
  hipError_t err = hipGetLastError();
  if (err == hipSuccess) err = hipMemcpyAsync(h, d, sizeof(h), hipMemcpyDeviceToHost, stream);
  if (err == hipSuccess) err = hipStreamSynchronize(stream);
  (void)hipFree(d);
  if (err != hipSuccess) {
    set_error(std::string("XCD split: layout probe failed: ") + hipGetErrorString(err));
    return 0;
  }
  for (int i = 0; i < kPersistentGrid; ++i)
    if (h[i] != (unsigned)(i % kXcds)) {
      set_error("XCD split: workgroup " + std::to_string(i) + " ran on XCD " + std::to_string(h[i]) +
                ", not " + std::to_string(i % kXcds));
      return 0;
    }
  return 1;
}

template <class S>
int xcd_split_ok(hipStream_t stream) {
  if constexpr (S::xa) {
    if (!occupancy_of(decode_step_xa_kernel<S, false>) || !occupancy_of(decode_step_xa_kernel<S, true>)) {
      set_error("XCD split: the split step kernel cannot keep one workgroup per CU");
      return 0;
    }
    return xcd_layout_ok(stream);
  } else {
    set_error("XCD split: no register plan for this model shape");
    return 0;
  }
}

}  // namespace

int persistent_shape(int hidden, int intermediate, int q_heads, int kv_heads, bool w8) {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return -1;
  // one resident workgroup per CU is what keeps every wait finite
  if (cus < kPersistentGrid) return -1;
  if (matches<QwenShape>(hidden, intermediate, q_heads, kv_heads))
    return w8 ? (occupancy_ok<QwenShapeW8>() ? 3 : -1) : (occupancy_ok<QwenShape>() ? 1 : -1);
  if (matches<SmolShape>(hidden, intermediate, q_heads, kv_heads))
    return w8 ? (occupancy_ok<SmolShapeW8>() ? 2 : -1) : (occupancy_ok<SmolShape>() ? 0 : -1);
  return -1;
}

int persistent_xcd_split(int shape, hipStream_t stream) {
  switch (shape) {
    case 0: return xcd_split_ok<SmolShape>(stream);
    case 1: return xcd_split_ok<QwenShape>(stream);
    case 2: return xcd_split_ok<SmolShapeW8>(stream);
    case 3: return xcd_split_ok<QwenShapeW8>(stream);
    default:
      set_error("XCD split: no persistent step for this model shape");
      return 0;
  }
}

// The short form runs up to 1.5 tasks per XCD-0 workgroup on average: measured
// at 42 tasks (position 700) it is 6% faster than the long form, at 56 tasks
// (position 960) level with it.
int persistent_split_tasks_max(bool long_form) { return long_form ? kPersistentGrid - kXcdWg : kXcdWg + kXcdWg / 2; }

namespace {
// down_x[((g * (H / R) + c) * R + e) * 4 + j] = down[(R c + e) * I + 4 g + j]
// with R outputs per 16-byte chunk group: 8 for bf16, 16 for int8
template <class T, int R>
__global__ void regroup_down_kernel(const T* __restrict__ down, T* __restrict__ dx, int H, int I) {
  const size_t n = (size_t)H * I;
  for (size_t o = (size_t)blockIdx.x * blockDim.x + threadIdx.x; o < n; o += (size_t)gridDim.x * blockDim.x) {
    const int j = (int)(o & 3);
    const int e = (int)((o >> 2) % R);
    const size_t gc = o / (4 * R);  // g * (H / R) + c
    const int c = (int)(gc % (size_t)(H / R));
    const int g = (int)(gc / (size_t)(H / R));
    dx[o] = down[(size_t)(R * c + e) * I + 4 * g + j];
  }
}
}  // namespace

__global__ void widen_i8_kernel(const int8_t* __restrict__ src, uint16_t* __restrict__ dst, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    dst[i] = (uint16_t)(__float_as_uint((float)src[i]) >> 16);  // |q| <= 127: exact in bf16
}

int launch_widen_i8(const void* src, void* dst, size_t n, hipStream_t stream) {
  hipLaunchKernelGGL(widen_i8_kernel, dim3(1024), dim3(256), 0, stream, static_cast<const int8_t*>(src),
                     static_cast<uint16_t*>(dst), n);
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? 0 : hip_fail(err, "widen_i8 launch");
}

int launch_regroup_down(const void* down, void* down_x, int H, int I, bool w8, hipStream_t stream) {
  if (!down || !down_x || H <= 0 || I <= 0 || H % (w8 ? 16 : 8) != 0 || I % 4 != 0)
    return fail("regroup_down: bad arguments");
  if (w8)
    hipLaunchKernelGGL((regroup_down_kernel<int8_t, 16>), dim3(1024), dim3(256), 0, stream,
                       static_cast<const int8_t*>(down), static_cast<int8_t*>(down_x), H, I);
  else
    hipLaunchKernelGGL((regroup_down_kernel<uint16_t, 8>), dim3(1024), dim3(256), 0, stream,
                       static_cast<const uint16_t*>(down), static_cast<uint16_t*>(down_x), H, I);
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? 0 : hip_fail(err, "regroup_down launch");
}

int launch_persistent_step(int shape, const PersistentArgs& a, hipStream_t stream, int form) {
  if (a.layers <= 0 || a.layers > kPersistentMaxLayers) return fail("persistent step: layer count out of range");
  if (a.max_splits < (a.max_ctx + kChunk - 1) / kChunk) return fail("persistent step: partials too small");
  switch (shape) {
    case 0: return launch_shape<SmolShape>(a, stream, form);
    case 1: return launch_shape<QwenShape>(a, stream, form);
    case 2: return launch_shape<SmolShapeW8>(a, stream, form);
    case 3: return launch_shape<QwenShapeW8>(a, stream, form);
    default: return fail("persistent step: unsupported model shape");
  }
}

}  // namespace hk

#ifdef HK_PHASE_STAMPS
// The phase stamps (see hk_stamp_phase): `phase` gets [256][32][16] and
// `attn` [256][32][8] 64-bit clock values (either may be null), from the last
// launch that wrote each one; with `clear` both tables are zeroed afterwards
// (synchronously), so the next copy shows only later launches.  Only in the
// library built with -DHK_PHASE_STAMPS; call it with no launch in flight.
extern "C" int hk_phase_stamps(void* phase, void* attn, int clear) {
  if (hipDeviceSynchronize() != hipSuccess) return hk::fail("hk_phase_stamps: device synchronise failed");
  if (phase && hipMemcpyFromSymbol(phase, HIP_SYMBOL(hk::hk_stamp_phase), sizeof(hk::hk_stamp_phase)) != hipSuccess)
    return hk::fail("hk_phase_stamps: copy failed");
  if (attn && hipMemcpyFromSymbol(attn, HIP_SYMBOL(hk::hk_stamp_attn), sizeof(hk::hk_stamp_attn)) != hipSuccess)
    return hk::fail("hk_phase_stamps: copy failed");
  if (clear) {
    void *ph = nullptr, *at = nullptr;
    if (hipGetSymbolAddress(&ph, HIP_SYMBOL(hk::hk_stamp_phase)) != hipSuccess ||
        hipGetSymbolAddress(&at, HIP_SYMBOL(hk::hk_stamp_attn)) != hipSuccess ||
        hipMemset(ph, 0, sizeof(hk::hk_stamp_phase)) != hipSuccess ||
        hipMemset(at, 0, sizeof(hk::hk_stamp_attn)) != hipSuccess || hipDeviceSynchronize() != hipSuccess)
      return hk::fail("hk_phase_stamps: clear failed");
  }
  return 0;
}
#endif
