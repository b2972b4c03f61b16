// One decode step of up to 8 independent sequences over a paged KV cache, as ONE persistent
// kernel on MI355X (gfx950): the batched paged decode that the reference describes
// (persistent batched decode over a PagePool with in-kernel page tables,
// knowledge/program.md:214-216, 244-250), each sequence with the semantics of the decode step
// (kernels/multi_sm_decode.py:77-357: embedding, per layer RMSNorm -> q/k/v -> RoPE -> GQA
// attention over the cached rows and the current position's un-rounded K/V -> O -> residual ->
// RMSNorm -> SwiGLU -> down -> residual; final RMSNorm, tied logits, argmax).
//
// Grid: one workgroup per compute unit, all resident (checked with the occupancy API before
// the launch).  A workgroup is 7 worker waves and one loader wave (two waves per SIMD).
//
// Phases, each ended by a grid barrier except QKV: the embedding rows, then per layer
//   QKV   workgroups own groups of 8 packed q/k/v rows: raw projections -> qkv (tagged words,
//         which the attention items poll: no barrier)
//   ATT   workgroups own (sequence, head) items: RoPE, K/V row of the current position to the
//         cache, attention over the cached rows (bf16) and the current K/V (f32) -> att
//   O     groups of 8 O rows: h += O att (each workgroup keeps its residual elements in LDS)
//   GU    groups of 8 packed gate/up rows (4 pairs): silu(gate) * up -> act
//   DN    groups of 8 down rows: h += W_down act
// then the final RMSNorm, the tied logits (groups of 8 vocabulary rows) with a per-row argmax
// key (64-bit atomic max), and a last barrier after which workgroup 0 publishes the tokens.
//
// Projections run on the matrix cores (v_mfma_f32_16x16x32_bf16): MFMA rows 0-7 are the hi
// parts bf16(x) of the 8 sequences' f32 inputs and rows 8-15 the lo parts bf16(x - hi), the 16
// MFMA columns are two groups of 8 weight rows, so one MFMA per 32-wide K step covers every
// sequence at about 2^-17 relative input precision (the f32 activations of model.py); output
// (sequence m, row n) is D[m][n] + D[m + 8][n].  The 7 worker waves split K, and their partial
// tiles are summed in a fixed order through LDS.  Every projection input is written once, by
// its producer, as hi/lo planes in packed order, so a consumer lane loads its 16-byte MFMA
// fragment directly.  RMSNorm (model.py:94-98) is folded: whoever updates a residual element
// writes h * scale (the scale of the norm that reads it next) as those planes, and the sum of
// h^2 over its group of 8 elements; the consumer sums the d / 8 partials of a row in a fixed
// order and multiplies its projection outputs by 1 / sqrt(mean + eps).
//
// Weights: the loader wave streams each workgroup's rows of every phase, in phase order, by
// DMA (global_load_lds) into a ring of LDS slots (2-3 jobs ahead), laid out per (group of 8
// rows, 64-wide K block) as 1 KB blocks with the 16-byte chunks of row r XOR-swizzled by r, so
// that the MFMA operand reads of 16 rows hit distinct banks.
//
// Exchange: the vectors live in the workspace, one buffer per (layer, vector), each written
// once per step with agent-scope (sc1) stores that go through to memory.  A buffer is read only
// after the barrier that follows its writes, and nothing reads it earlier in the step, so no L2
// holds a stale line of it (the L2s start every kernel invalidated): readers use ordinary cached
// 16-byte loads, and each XCD fetches a vector from memory once.  The exception is qkv: its
// words carry the step's epoch in their upper half and are polled with agent-scope loads.  A
// barrier is a flag word per
// workgroup set to the step's epoch after the workgroup's stores have completed
// (s_waitcnt vmcnt(0)), polled by one wave of every workgroup with agent-scope loads.  Epochs
// run 1..0xFFFFFFFE (the last one is kept in the workspace); every flag is rewritten each step,
// so no flag ever holds the current epoch before its workgroup has arrived.  Status bits and
// argmax keys alternate between two slots by epoch parity; workgroup 0 clears the other slot
// after publishing.  Every wait is bounded: a timeout sets status bit 0 and the step runs to
// its end (wrong results, reported).  One step may be in flight per workspace.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <mutex>
#include <vector>

#include "batched.h"
#include "internal.h"

namespace mbd {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kDh = 64;
constexpr int kPage = 16;
constexpr int kRows = 8;                    // sequences per step (MFMA rows: 8 hi + 8 lo)
constexpr int kWorkers = 7;                 // worker waves; wave kWorkers is the loader (2 waves per SIMD)
constexpr int kThreads = 64 * (kWorkers + 1);
constexpr int kStepsD = 5;                  // 32-wide K steps per worker wave over d: d <= 1120
constexpr int kStepsF = 13;                 // ... over d_ff: d_ff <= 2912
constexpr int kBlocks = 8;                  // 64-position attention blocks (waves take blocks w, w + 7)
constexpr int kEpi = 384;                   // epilogue threads (a multiple of 128: a thread keeps its sequence)
constexpr int kTilesD = 2;                  // 16-column tiles (two groups of 8 rows) per job over d
constexpr int kTilesF = 1;                  // ... over d_ff (the down projection)
constexpr int kMaxTiles = kTilesD;
constexpr int kMaxGroups = 2 * kMaxTiles;
static_assert(kEpi % 128 == 0 && 128 * kTilesD <= kEpi && kEpi <= 64 * kWorkers,
              "O and down epilogues: at most one element per thread");
constexpr int kMaxGrid = 1024;
constexpr int kMaxCtx = 64 * kBlocks;
constexpr int kLdsTotal = 160 * 1024;
constexpr uint32_t kStTimeout = 1u, kStBadToken = 2u, kStBadPos = 4u;
constexpr uint32_t kSpinLimit = 1u << 21;      // grid-barrier poll rounds (~1 s)
// Replicas of every barrier flag: workgroup w polls replica w % kFlagReps, so the pollers of a
// barrier spread over kFlagReps regions instead of meeting on one.
#ifndef MBD_FLAG_REPS
#define MBD_FLAG_REPS 8
#endif
constexpr int kFlagReps = MBD_FLAG_REPS;
#ifndef MBD_BAR_SLEEP
#define MBD_BAR_SLEEP 1
#endif
// s_sleep units between the two rounds of an attention item's q/k/v poll kept in flight (0: one round)
#ifndef MBD_QKV_STAGGER
#define MBD_QKV_STAGGER 16
#endif
// s_sleep units between the polls of an LDS counter (0: spin)
#ifndef MBD_LDS_SLEEP
#define MBD_LDS_SLEEP 1
#endif
// Wave priority (s_setprio) of the loader wave; the worker waves keep 0
#ifndef MBD_LOADER_PRIO
#define MBD_LOADER_PRIO 1
#endif
constexpr int kLoaderPrio = MBD_LOADER_PRIO;
// The tied logits' weight rows: streamed by the worker waves straight into registers (1), or by
// the loader through the LDS ring (0)
#ifndef MBD_LOGITS_REG
#define MBD_LOGITS_REG 1
#endif
constexpr bool kLogitsReg = MBD_LOGITS_REG != 0;
// the worker wave that polls an attention item's q, k and v; it requests its block of cached K/V
// rows only afterwards (a wave's loads complete in order: polls issued behind ~40 K/V loads wait
// for them), while the other waves request theirs at once
constexpr int kQkvPoller = kWorkers - 1;
constexpr uint32_t kLdsSpinLimit = 1u << 23;   // LDS-counter spins
// control words (uint32 offsets in the control block)
constexpr int kCtlEpoch = 0, kCtlStatus = 16;   // status slot k at kCtlStatus + 16 k

struct Args {
  int d, ff, H, KV, L, V, ctx, nqkv, M;
  int64_t layer_elems, off_ln2, off_qkv, off_o, off_gu, off_dn;
  const uint16_t* emb;
  const uint16_t* outp;
  const uint16_t* w;
  const uint16_t* lnf;
  const float* rope;
  const int32_t* tokens;
  const int32_t* pos;
  const int32_t* pages;
  int max_pages, pool_pages;
  uint16_t* kv;
  float* logits;
  int32_t* out;
  uint32_t* ctrl;
  uint64_t* keys;   // [2][kRows]
  uint32_t* flags;  // [5 L + 2][kMaxGrid] (barrier 1 + 5 l, after QKV, is no longer used)
  // exchange vectors, one block per layer (each written once per step):
  //   h after O [kRows][d], h after down [kRows][d] (residual stream, packed input order),
  //   qkv [kRows][nqkv] (raw projections, packed row order), att [kRows][d] (packed input
  //   order of O), act [kRows][ff] (packed input order of down)
  float* x;
  int64_t x_layer;
  int slot_bytes, nslots, tchunk;
};

// ---------------------------------------------------------------- profiling build (-DMBD_TRACE)
// Lane 0 of worker wave 0 of every workgroup stamps s_memrealtime (100 MHz) at phase
// boundaries: slot 8 p + k of layer kTraceLayer's phase p (0 QKV .. 4 DN): k = 0 phase start,
// 1 inputs ready, 2 weights landed, 3 summed, 4 outputs stored, 5 barrier passed, 6 own flag set
// (after the workgroup's stores completed); slot 40 + 5 l + p:
// barrier p of layer l passed; slot 168: logits done; 169: final barrier.  Attention of layer
// kTraceLayer (first item): slot 9 q/k/v polled, 7 the item's position (a value), 15 wave 1's
// scores, 160 + w wave w's block done, 10 the waves met, 11 output stored.  The loader stamps slot
// 176 + p when the weights of layer kTraceLayer's phase p are issued and 184 + p when they landed.
constexpr int kTraceLayer = 10;
#ifdef MBD_TRACE
constexpr int kTraceSlots = 192;
__device__ uint64_t mbd_trace_buf[kMaxGrid * kTraceSlots];
#define MBD_T(cond, slot)                                                                       \
  do {                                                                                          \
    if ((cond) && (threadIdx.x & 63) == 0)                                                      \
      mbd_trace_buf[blockIdx.x * kTraceSlots + (slot)] = __builtin_amdgcn_s_memrealtime();      \
  } while (0)
#define MBD_V(cond, slot, v)                                                                    \
  do {                                                                                          \
    if ((cond) && (threadIdx.x & 63) == 0) mbd_trace_buf[blockIdx.x * kTraceSlots + (slot)] = (v); \
  } while (0)
#else
#define MBD_T(cond, slot) \
  do {                    \
  } while (0)
#define MBD_V(cond, slot, v) \
  do {                       \
  } while (0)
#endif

// ---------------------------------------------------------------- small helpers
__device__ __forceinline__ float bf2f(uint16_t b) { return __uint_as_float(uint32_t(b) << 16); }
__device__ __forceinline__ uint16_t f2bf(float f) {   // round to nearest even
  const uint32_t u = __float_as_uint(f);
  return uint16_t((u + (((u >> 16) & 1u) + 0x7fffu)) >> 16);
}

// Packed row layout of the weights: in blocks of 512 inputs (the last one S = 8m long),
// input b*512 + k*m + l sits at position b*512 + 8*l + k.
__device__ __forceinline__ int perm_pos(int i, int K) {
  const int b = i >> 9, r = i & 511;
  const int S = min(512, K - (b << 9));
  const int m = S >> 3;
  const int k = r / m, l = r - k * m;
  return (b << 9) + 8 * l + k;
}

// A value the compiler cannot see through: per-lane address arithmetic derived from it stays
// inside the phase that uses it instead of being hoisted out of the layer loop (where it would
// hold registers across every phase).
__device__ __forceinline__ int opaque(int v) {
  asm volatile("" : "+v"(v));
  return v;
}

__device__ __forceinline__ void split(int total, int parts, int idx, int& lo, int& hi) {
  lo = int((int64_t(total) * idx) / parts);
  hi = int((int64_t(total) * (idx + 1)) / parts);
}

// Exchange block of layer l (block l + 1; block 0 holds the embedding rows as "layer -1"):
//   qkv      u64 [kRows][nqkv]        raw q/k/v projections, packed row order, as tagged words
//                                     (f32 bits | epoch << 32): the attention items poll them
//   att      bf16 [2][kRows][ld(d)]   attention output as hi/lo planes, packed input order of O
//   act      bf16 [2][kRows][ld(ff)]  SwiGLU output as hi/lo planes, packed input order of down
//   hop, hdp bf16 [2][kRows][ld(d)]   the residual stream after O times ln2 and after down times
//                                     the next ln1 (or the final norm), hi/lo planes, packed order
//   sso, ssd f32 [kRows][d / 8]       sums of squares of those residuals over each group of 8
// (the f32 residual stream itself stays in the LDS of the workgroup that owns its elements).
// Plane rows are K + 8 elements apart: with rows a multiple of 128 bytes apart, the 8 sequences'
// fragments an MFMA operand load touches sit at the same offset on one memory channel.
__host__ __device__ __forceinline__ int plane_ld(int K) { return K + 8; }
__device__ __forceinline__ float* x_blk(const Args& a, int l) { return a.x + int64_t(l + 1) * a.x_layer; }
__device__ __forceinline__ uint64_t* x_qkv(const Args& a, int l) { return reinterpret_cast<uint64_t*>(x_blk(a, l)); }
__device__ __forceinline__ uint16_t* x_att(const Args& a, int l) {
  return reinterpret_cast<uint16_t*>(x_blk(a, l) + int64_t(kRows) * 2 * a.nqkv);
}
__device__ __forceinline__ uint16_t* x_act(const Args& a, int l) {
  return reinterpret_cast<uint16_t*>(x_blk(a, l) + int64_t(kRows) * (2 * a.nqkv + plane_ld(a.d)));
}
__device__ __forceinline__ uint16_t* x_hop(const Args& a, int l) {
  return reinterpret_cast<uint16_t*>(x_blk(a, l) + int64_t(kRows) * (2 * a.nqkv + plane_ld(a.d) + plane_ld(a.ff)));
}
__device__ __forceinline__ uint16_t* x_hdp(const Args& a, int l) { return x_hop(a, l) + 2 * kRows * plane_ld(a.d); }
__device__ __forceinline__ float* x_sso(const Args& a, int l) {
  return x_blk(a, l) + int64_t(kRows) * (2 * a.nqkv + 3 * plane_ld(a.d) + plane_ld(a.ff));
}
__device__ __forceinline__ float* x_ssd(const Args& a, int l) { return x_sso(a, l) + a.d; }
// floats of one exchange block
__host__ __device__ __forceinline__ int64_t x_block_floats(int d, int nqkv, int ff) {
  return int64_t(kRows) * (3 * plane_ld(d) + 2 * nqkv + plane_ld(ff)) + 2 * d;
}

__device__ __forceinline__ uint32_t ld_u32(const uint32_t* p) {
  return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld_u64(const uint64_t* p) {
  return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_u32(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_u64(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_u16(uint16_t* p, uint16_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// x as hi = bf16(x) at p and lo = bf16(x - hi) at p + plane
__device__ __forceinline__ void st_split(uint16_t* p, int64_t plane, float x) {
  const uint16_t h = f2bf(x);
  st_u16(p, h);
  st_u16(p + plane, f2bf(x - bf2f(h)));
}
__device__ __forceinline__ float ld_f(const float* p) {
  return __uint_as_float(ld_u32(reinterpret_cast<const uint32_t*>(p)));
}
__device__ __forceinline__ void st_f(float* p, float v) { st_u32(reinterpret_cast<uint32_t*>(p), __float_as_uint(v)); }

__device__ __forceinline__ constexpr int vmcnt_imm(int k) {
  return (k & 0xF) | ((k >> 4) << 14) | (7 << 4) | (0xF << 8);
}
// Wait until at most n of this wave's vector memory instructions are outstanding (n rounded
// down to an encodable bucket: waiting longer is always correct).
__device__ __forceinline__ void wait_vm_atmost(int n) {
  if (n >= 48) __builtin_amdgcn_s_waitcnt(vmcnt_imm(48));
  else if (n >= 32) __builtin_amdgcn_s_waitcnt(vmcnt_imm(32));
  else if (n >= 24) __builtin_amdgcn_s_waitcnt(vmcnt_imm(24));
  else if (n >= 16) __builtin_amdgcn_s_waitcnt(vmcnt_imm(16));
  else if (n >= 12) __builtin_amdgcn_s_waitcnt(vmcnt_imm(12));
  else if (n >= 8) __builtin_amdgcn_s_waitcnt(vmcnt_imm(8));
  else if (n >= 4) __builtin_amdgcn_s_waitcnt(vmcnt_imm(4));
  else if (n >= 2) __builtin_amdgcn_s_waitcnt(vmcnt_imm(2));
  else if (n >= 1) __builtin_amdgcn_s_waitcnt(vmcnt_imm(1));
  else __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
}

// Wave64 reductions with DPP row shifts and row broadcasts; result read from lane 63.
template <int CTRL, int ROWMASK>
__device__ __forceinline__ float dpp(float v, float fill) {
  return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(fill), __float_as_int(v), CTRL, ROWMASK, 0xf, false));
}
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp<0x111, 0xf>(v, 0.f);
  v += dpp<0x112, 0xf>(v, 0.f);
  v += dpp<0x114, 0xf>(v, 0.f);
  v += dpp<0x118, 0xf>(v, 0.f);
  v += dpp<0x142, 0xa>(v, 0.f);
  v += dpp<0x143, 0xc>(v, 0.f);
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
// The sum over each group of 8 consecutive lanes, in every lane of the group: the butterfly
// (lane ^ 1, ^ 2, ^ 4) with DPP quad permutes and the half-row mirror instead of LDS permutes
// (after the two quad steps the lanes of a quad hold the same value, so the mirror adds the
// other quad's sum exactly as lane ^ 4 would)
__device__ __forceinline__ float sum8_lanes(float v) {
  v += dpp<0xB1, 0xf>(v, 0.f);    // quad_perm [1, 0, 3, 2]: lane ^ 1
  v += dpp<0x4E, 0xf>(v, 0.f);    // quad_perm [2, 3, 0, 1]: lane ^ 2
  v += dpp<0x141, 0xf>(v, 0.f);   // row_half_mirror: the other quad of the 8
  return v;
}
// v of this lane plus v of lane ^ 32 (gfx950's row-swapping permute; no LDS traffic)
__device__ __forceinline__ float add_halves(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp<0x111, 0xf>(v, -INFINITY));
  v = fmaxf(v, dpp<0x112, 0xf>(v, -INFINITY));
  v = fmaxf(v, dpp<0x114, 0xf>(v, -INFINITY));
  v = fmaxf(v, dpp<0x118, 0xf>(v, -INFINITY));
  v = fmaxf(v, dpp<0x142, 0xa>(v, -INFINITY));
  v = fmaxf(v, dpp<0x143, 0xc>(v, -INFINITY));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

__device__ __forceinline__ uint64_t argmax_key(float v, int idx) {   // larger key wins; ties: lower idx
  uint32_t b = __float_as_uint(v);
  b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return (uint64_t(b) << 32) | uint64_t(0xffffffffu - uint32_t(idx));
}

// ---------------------------------------------------------------- waits
struct Sync {
  int* landed;     // LDS: jobs whose weights have landed (set by the loader)
  int* consumed;   // LDS: worker waves done with a job's slot (8 per job)
  int* wbar;       // LDS: worker-wave barrier counter
  uint32_t* status;
  int wph;
};

__device__ __forceinline__ int lds_ld(int* c) { return __hip_atomic_load(c, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP); }
// Spin on an LDS counter until it reaches target; gives up (and reports) after kLdsSpinLimit
// spins or once another wave has reported a timeout.
__device__ __forceinline__ void lds_wait(int* c, int target, uint32_t* status) {
  uint32_t spins = 0;
  while (lds_ld(c) < target) {
    if constexpr (MBD_LDS_SLEEP > 0) __builtin_amdgcn_s_sleep(MBD_LDS_SLEEP);
    if ((++spins & 1023u) == 0) {
      if (ld_u32(status) & kStTimeout) return;
      if (spins > kLdsSpinLimit) {
        atomicOr(status, kStTimeout);
        return;
      }
    }
  }
}
__device__ __forceinline__ void lds_bump(int* c, int lane) {
  __builtin_amdgcn_s_waitcnt(0xc07f);   // this wave's LDS accesses done
  if (lane == 0) __hip_atomic_fetch_add(c, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void lds_set(int* c, int v, int lane) {
  __builtin_amdgcn_s_waitcnt(0xc07f);
  if (lane == 0) __hip_atomic_store(c, v, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
}
// barrier of the 8 worker waves
__device__ __forceinline__ void wsync(Sync& sy, int lane) {
  sy.wph += kWorkers;
  lds_bump(sy.wbar, lane);
  lds_wait(sy.wbar, sy.wph, sy.status);
}

// Grid barrier b, in two halves.  arrive: every worker wave's global stores complete, then
// wave 0 sets this workgroup's flag to the epoch.  wait: wave 0 polls every workgroup's flag,
// the other waves wait for it.
__device__ __forceinline__ void grid_arrive(const Args& a, Sync& sy, int b, uint32_t epoch, int wv, int lane) {
  __builtin_amdgcn_s_waitcnt(0);
  wsync(sy, lane);
  if (wv == 0 && lane < kFlagReps) st_u32(a.flags + (int64_t(b) * kFlagReps + lane) * kMaxGrid + blockIdx.x, epoch);
  MBD_T(wv == 0 && b >= 1 + 5 * kTraceLayer && b < 6 + 5 * kTraceLayer, 8 * (b - 1 - 5 * kTraceLayer) + 6);
}
// Four consecutive flags with one agent-scope 16-byte load (each 4-byte flag is read whole).
__device__ __forceinline__ uint4 ld_flags4(const uint32_t* p) {
  uint4 v;
  asm volatile("global_load_dwordx4 %0, %1, off sc1\n\ts_waitcnt vmcnt(0)" : "=v"(v) : "v"(p) : "memory");
  return v;
}
__device__ __forceinline__ void grid_wait(const Args& a, Sync& sy, int b, uint32_t epoch, int wv, int lane,
                                          int poller = 0) {
  if (wv == poller) {
    const uint32_t* f = a.flags + (int64_t(b) * kFlagReps + blockIdx.x % kFlagReps) * kMaxGrid;
    const int G = gridDim.x, nk = (G + 255) / 256;
    uint32_t pend = 0;   // bit k: flags 256 k + 4 lane .. + 3 not all seen yet
    for (int k = 0; k < nk; ++k)
      if (256 * k + 4 * lane < G) pend |= 1u << k;
    uint32_t spins = 0;
    while (true) {
      // a lane reads its four flags of each group not seen yet (one load per round for up to
      // 256 workgroups); flags past the grid count as seen
      for (int k = 0; k < nk; ++k)
        if ((pend >> k) & 1u) {
          const int i = 256 * k + 4 * lane;
          const uint4 v = ld_flags4(f + i);
          if ((v.x == epoch || i >= G) && (v.y == epoch || i + 1 >= G) && (v.z == epoch || i + 2 >= G) &&
              (v.w == epoch || i + 3 >= G))
            pend &= ~(1u << k);
        }
      if (__all(pend == 0)) break;
      if constexpr (MBD_BAR_SLEEP > 0) __builtin_amdgcn_s_sleep(MBD_BAR_SLEEP);
      if ((++spins & 255u) == 0 && (ld_u32(sy.status) & kStTimeout)) break;
      if (spins > kSpinLimit) {
        if (lane == 0) atomicOr(sy.status, kStTimeout);
        break;
      }
    }
  }
  wsync(sy, lane);
}
__device__ __forceinline__ void grid_sync(const Args& a, Sync& sy, int b, uint32_t epoch, int wv, int lane) {
  grid_arrive(a, sy, b, epoch, wv, lane);
  grid_wait(a, sy, b, epoch, wv, lane);
}
// The f32s of N tagged words per lane (f32 bits | epoch << 32) once their tags are the step's
// epoch: every lane of the wave polls its words with agent-scope loads (a stale copy in an L2 is
// not read), bounded like the grid barrier.
template <int N>
__device__ __forceinline__ void poll_words(const uint64_t* const (&p)[N], uint32_t epoch, uint32_t* status,
                                           float (&out)[N]) {
  uint64_t w[N];
#pragma unroll
  for (int i = 0; i < N; ++i) w[i] = ld_u64(p[i]);
#if MBD_QKV_STAGGER > 0
  // a second round in flight, issued about half a memory round trip after the first
  uint64_t w2[N];
  __builtin_amdgcn_s_sleep(MBD_QKV_STAGGER);
#pragma unroll
  for (int i = 0; i < N; ++i) w2[i] = ld_u64(p[i]);
#endif
  uint32_t spins = 0;
  while (true) {
    bool ok = true;
#pragma unroll
    for (int i = 0; i < N; ++i) ok = ok && uint32_t(w[i] >> 32) == epoch;
    if (__all(ok)) break;
#if MBD_QKV_STAGGER > 0
#pragma unroll
    for (int i = 0; i < N; ++i)
      if (uint32_t(w[i] >> 32) != epoch) w[i] = ld_u64(p[i]);
    ok = true;
#pragma unroll
    for (int i = 0; i < N; ++i) ok = ok && uint32_t(w2[i] >> 32) == epoch;
    if (__all(ok)) {
#pragma unroll
      for (int i = 0; i < N; ++i) w[i] = w2[i];
      break;
    }
#pragma unroll
    for (int i = 0; i < N; ++i)
      if (uint32_t(w2[i] >> 32) != epoch) w2[i] = ld_u64(p[i]);
#else
    if constexpr (MBD_BAR_SLEEP > 0) __builtin_amdgcn_s_sleep(MBD_BAR_SLEEP);
#pragma unroll
    for (int i = 0; i < N; ++i)
      if (uint32_t(w[i] >> 32) != epoch) w[i] = ld_u64(p[i]);
#endif
    if ((++spins & 255u) == 0 && (ld_u32(status) & kStTimeout)) break;
    if (spins > kSpinLimit) {
      if ((threadIdx.x & 63) == 0) atomicOr(status, kStTimeout);
      break;
    }
  }
#pragma unroll
  for (int i = 0; i < N; ++i) out[i] = __uint_as_float(uint32_t(w[i]));
}

// ---------------------------------------------------------------- jobs (weight rows of a phase)
struct Job {
  const uint16_t* base;   // row 0 of the matrix
  int K, g0, ng;          // groups g0 .. g0 + ng - 1 of 8 rows, K inputs each
};

// Workgroups that run the QKV phase: the upper half of the grid when that keeps every job within
// its tiles, so that the first half, where the attention items sit (items deal from workgroup
// 0), has no QKV job and requests its items' cached K/V rows as soon as the layer starts.
__host__ __device__ __forceinline__ int qkv_wgs(int groups, int G) {
  const int h = G / 2;
  return (h > 0 && (groups + h - 1) / h <= 2 * kTilesD) ? h : G;
}

// Layer phase ph (0 QKV, 1 O, 2 GU, 3 DN) of layer l for workgroup wg.
__device__ __forceinline__ Job layer_job(const Args& a, int l, int ph, int wg, int G) {
  const uint16_t* wl = a.w + int64_t(l) * a.layer_elems;
  Job j;
  int rows;
  if (ph == 0) {
    j.base = wl + a.off_qkv; j.K = a.d; rows = a.nqkv;
  } else if (ph == 1) {
    j.base = wl + a.off_o; j.K = a.d; rows = a.d;
  } else if (ph == 2) {
    j.base = wl + a.off_gu; j.K = a.d; rows = 2 * a.ff;
  } else {
    j.base = wl + a.off_dn; j.K = a.ff; rows = a.d;
  }
  int g1;
  const int nq = qkv_wgs(rows / 8, G);
  if (ph == 0 && wg < G - nq) {   // QKV runs on the last nq workgroups only
    j.g0 = 0;
    j.ng = 0;
    return j;
  }
  if (ph == 0) split(rows / 8, nq, wg - (G - nq), j.g0, g1);
  else split(rows / 8, G, wg, j.g0, g1);
  j.ng = g1 - j.g0;
  return j;
}

// Loader wave: the DMA of every job of this workgroup, in the workers' order.
__device__ __forceinline__ void loader(const Args& a, Sync& sy, uint8_t* slots, int lane) {
  const int G = gridDim.x, wg = blockIdx.x;
  int j = 0;
#ifdef MBD_TRACE
  int tj[4] = {-1, -1, -1, -1};   // job indices of the traced layer's phases
  auto landed = [&](int v) {
    lds_set(sy.landed, v, lane);
    for (int q = 0; q < 4; ++q)
      if (tj[q] >= 0 && tj[q] < v) {
        MBD_T(true, 184 + q);
        tj[q] = -1;
      }
  };
#else
  auto landed = [&](int v) { lds_set(sy.landed, v, lane); };
#endif
  auto load = [&](const Job& jb, int tag) {
    const int slot = j % a.nslots;
    if (j >= a.nslots && lds_ld(sy.consumed) < kWorkers * (j - a.nslots + 1)) {
      // the slot is still being read: let the workers have everything that is in flight
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
      landed(j);
      lds_wait(sy.consumed, kWorkers * (j - a.nslots + 1), sy.status);
    }
#ifdef MBD_TRACE
    if (tag >= 4 * kTraceLayer && tag < 4 * kTraceLayer + 4) {
      tj[tag - 4 * kTraceLayer] = j;
      MBD_T(true, 176 + tag - 4 * kTraceLayer);
    }
#endif
    uint8_t* dst = slots + int64_t(slot) * a.slot_bytes;
    const int kp = jb.K / 64, nblk = jb.ng * kp;
    const int r = lane >> 3, cp = lane & 7, c = cp ^ r;
    for (int t = 0; t < nblk; ++t) {
      const int gi = t / kp, p = t - gi * kp;
      const uint16_t* src = jb.base + (int64_t(8 * (jb.g0 + gi) + r) * jb.K + 64 * p + 8 * c);
      __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)(dst + 1024 * t), 16, 0, 0);
    }
    if (j > 0) {   // everything before this job has landed once at most nblk are outstanding
      wait_vm_atmost(nblk);
      landed(j);
    }
    ++j;
  };
  for (int l = 0; l < a.L; ++l)
    for (int ph = 0; ph < 4; ++ph) {
      const Job jb = layer_job(a, l, ph, wg, G);
      if (jb.ng > 0) load(jb, 4 * l + ph);
    }
  if constexpr (!kLogitsReg) {
    int t0, t1;
    split(a.V / 8, G, wg, t0, t1);
    for (int c = t0; c < t1; c += a.tchunk) load(Job{a.outp, a.d, c, min(a.tchunk, t1 - c)}, -1);
  }
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
  landed(j);
}

// ---------------------------------------------------------------- MFMA input operand
// The lane's A fragments for its K steps s0 .. s0 + ns - 1: lane L holds sequence m = L & 7 at
// inputs 32 s + 8 (L >> 4) .. + 7, as the hi part (L & 15 < 8) or the lo part (otherwise).
template <int NS>
struct AOp {
  uint4 f[NS];
};

// The A fragments from an exchange vector held as hi/lo bf16 planes [2][kRows][ld]: one 16-byte
// load per K step (lanes 8..15 of each row of 16 read the lo plane).
template <int NS>
__device__ __forceinline__ void load_parts(const uint16_t* src, int ld, int s0, int ns, int lane, AOp<NS>& A) {
  const int m = lane & 7, q = lane >> 4;
  const uint16_t* base = src + ((lane & 15) >= 8 ? int64_t(kRows) * ld : 0) + int64_t(m) * ld + 8 * q;
#pragma unroll
  for (int i = 0; i < NS; ++i) {
    const int s = s0 + min(i, max(ns - 1, 0));
    A.f[i] = *reinterpret_cast<const uint4*>(base + 32 * s);
  }
}

// 1 / sqrt(mean(x^2) + eps) of every sequence's row from the producers' sums of squares over
// groups of 8 elements (ss[kRows][K / 8], summed in a fixed order), into inv[kRows] (LDS).
// One wave: lane L sums row L >> 3's groups 4 nl (L & 7) .. + 4 nl - 1, then the 8 lanes of a row
// combine.
__device__ __forceinline__ void row_inv(const float* ss, int K, float* inv, int lane) {
  const int r = lane >> 3, c = lane & 7, ng = K / 8, nl = ng / 32;   // float4s per lane (K % 256 == 0)
  const float4* src = reinterpret_cast<const float4*>(ss + r * ng) + c * nl;
  float4 u[kStepsD];   // every load first (K <= 1120: at most 4)
#pragma unroll
  for (int k = 0; k < kStepsD; ++k) u[k] = src[min(k, nl - 1)];
  float v = 0.f;
#pragma unroll
  for (int k = 0; k < kStepsD; ++k)
    if (k < nl) v += ((u[k].x + u[k].y) + (u[k].z + u[k].w));
  v = sum8_lanes(v);
  if (c == 0) inv[r] = 1.f / sqrtf(v / float(K) + 1e-5f);
}

// ---------------------------------------------------------------- one job on the matrix cores
// Partial tiles of this wave's K steps; returns the number of tiles.
template <int NS, int MAXT>
__device__ __forceinline__ int job_mfma(const Job& jb, const uint8_t* slot, const AOp<NS>& A, int s0, int ns, int lane,
                                        f32x4 (&acc)[MAXT]) {
  const int tiles = (jb.ng + 1) >> 1, kp = jb.K / 64;
  const int n = lane & 15, r = n & 7, q = lane >> 4;
  // every weight fragment first (clamped: a column past the job's groups reads its last group,
  // and its outputs are never used), then the MFMAs
  uint4 bq[NS][MAXT];
#pragma unroll
  for (int i = 0; i < NS; ++i) {
    const int s = s0 + min(i, ns - 1);
    const int cp = ((((s & 1) << 2) | q) ^ r);
#pragma unroll
    for (int t = 0; t < MAXT; ++t) {
      const int gi = min(2 * t + (n >> 3), jb.ng - 1);
      bq[i][t] = *reinterpret_cast<const uint4*>(slot + (gi * kp + (s >> 1)) * 1024 + r * 128 + cp * 16);
    }
  }
#pragma unroll
  for (int t = 0; t < MAXT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < NS; ++i) {
    if (i < ns) {
      const bf16x8 av = __builtin_bit_cast(bf16x8, A.f[i]);
#pragma unroll
      for (int t = 0; t < MAXT; ++t)
        if (t < tiles) acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, __builtin_bit_cast(bf16x8, bq[i][t]), acc[t], 0, 0, 0);
    }
  }
  return tiles;
}

// Sum of the worker waves' partial tiles (written over the job's slot): output (sequence m,
// column n of tile t) = sum_w D_w[m][n] + sum_w D_w[m + 8][n].
__device__ __forceinline__ float tile_out(const f32x4* red, int tiles, int t, int m, int n) {
  const int l_hi = n + 16 * (m >> 2), l_lo = n + 16 * (2 + (m >> 2)), e = m & 3;
  float hi = 0.f, lo = 0.f;
#pragma unroll
  for (int w = 0; w < kWorkers; ++w) {
    hi += red[(w * tiles + t) * 64 + l_hi][e];
    lo += red[(w * tiles + t) * 64 + l_lo][e];
  }
  return hi + lo;
}

// Runs job jb (slot index j of the ring) and leaves the summed tiles in the slot; the caller
// reads them with tile_out and then releases the slot with lds_bump(consumed).
template <int NS, int MAXT = kTilesD>
__device__ __forceinline__ const f32x4* run_job(const Args& a, const Job& jb, int j, uint8_t* slots, const AOp<NS>& A,
                                                int s0, int ns, Sync& sy, int wv, int lane, int& tiles,
                                                int tslot = -1) {
  lds_wait(sy.landed, j + 1, sy.status);
  MBD_T(tslot >= 0 && wv == 0, tslot);
  uint8_t* slot = slots + int64_t(j % a.nslots) * a.slot_bytes;
  f32x4 acc[MAXT];
  tiles = job_mfma<NS, MAXT>(jb, slot, A, s0, ns, lane, acc);
  wsync(sy, lane);   // every wave has read its weights from the slot
  f32x4* red = reinterpret_cast<f32x4*>(slot);
#pragma unroll
  for (int t = 0; t < MAXT; ++t)
    if (t < tiles) red[(wv * tiles + t) * 64 + lane] = acc[t];
  wsync(sy, lane);
  return red;
}

// ---------------------------------------------------------------- attention of one (sequence, head)
constexpr int kMaxItems = 2;   // (sequence, head) items per workgroup

// What an item needs that is the same in every layer, set up once per step.
struct Item {
  int m, h, p;          // sequence, query head, position (validated)
  int prow;             // cache row of position p
  int row[kMaxCtx];     // cache rows of positions 0 .. p-1 (0 past them)
  float cs[kDh];        // RoPE at p: cos (32) then sin (32)
};
struct AttLds {
  float q[kDh], k[kDh], v[kDh];
  float p[kBlocks][64];
  float o[kBlocks][kDh];
  float ml[kBlocks][2];
  Item it[kMaxItems];
  int nitems;
};

// Cache row of sequence m at position j through its page table (entries outside the pool: 0,
// status bit 2).
__device__ __forceinline__ int64_t cache_row(const Args& a, int m, int j, uint32_t* status) {
  int pg = a.pages[int64_t(m) * a.max_pages + j / kPage];
  if (pg < 0 || pg >= a.pool_pages) {
    atomicOr(status, kStBadPos);
    pg = 0;
  }
  return int64_t(pg) * kPage + j % kPage;
}

// This workgroup's items: (sequence, head) pairs dealt so that the query heads sharing a K/V
// head sit on one XCD (workgroup i runs on XCD i mod 8 when workgroups are dealt round-robin).
__device__ __forceinline__ void att_setup(const Args& a, AttLds& S, Sync& sy, int wv, int lane) {
  const int tid = wv * 64 + lane, G = gridDim.x;
  const int gs = a.H / a.KV, nq = a.M * a.KV;
  const int ni = 8 * gs * ((nq + 7) / 8);
  int n = 0;
  for (int i = blockIdx.x; i < ni && n < kMaxItems; i += G) {
    const int x8 = i & 7, y = i >> 3, r = y % gs, u = y / gs;
    const int q = 8 * u + x8;
    if (q >= nq) continue;
    const int m = q / a.KV, g = q % a.KV;
    Item& it = S.it[n++];
    int p = a.pos[m];
    if (p < 0 || p >= a.ctx || p / kPage >= a.max_pages) {
      if (tid == 0) atomicOr(sy.status, kStBadPos);
      p = 0;
    }
    if (tid == 0) {
      it.m = m;
      it.h = g * gs + r;
      it.p = p;
      it.prow = int(cache_row(a, m, p, sy.status));
    }
    for (int j = tid; j < kMaxCtx; j += 64 * kWorkers) it.row[j] = j < p ? int(cache_row(a, m, j, sy.status)) : 0;
    if (tid < kDh) it.cs[tid] = a.rope[int64_t(p) * kDh + tid];
  }
  if (tid == 0) S.nitems = n;
}

// One 64-position block's cached K rows (lane = position) and V values (lane: dims 2 (lane & 31),
// +1 of positions 32 (lane >> 5) .. + 31).
struct AttPre {
  uint4 ku[kDh / 8];
  uint32_t vv[32];
};
__device__ __forceinline__ void att_load(const Args& a, int l, const Item& it, int b, int lane, AttPre& P) {
  const int pool = a.pool_pages * kPage, g = it.h / (a.H / a.KV);
  const uint16_t* kc = a.kv + int64_t(l) * 2 * a.KV * pool * kDh + int64_t(g) * pool * kDh;
  const uint16_t* vc = kc + int64_t(a.KV) * pool * kDh;
  const int j0 = 64 * b, dp = lane & 31, half = lane >> 5;
  // every row index first (LDS, 16-byte reads), then every global load
  int4 rv[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) rv[k] = *reinterpret_cast<const int4*>(&it.row[j0 + 32 * half + 4 * k]);
  const int rk = it.row[j0 + lane];
  const uint4* kr = reinterpret_cast<const uint4*>(kc + int64_t(rk) * kDh);
#pragma unroll
  for (int e8 = 0; e8 < kDh / 8; ++e8) P.ku[e8] = kr[e8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const int r4[4] = {rv[k].x, rv[k].y, rv[k].z, rv[k].w};
#pragma unroll
    for (int u = 0; u < 4; ++u)
      P.vv[4 * k + u] = *reinterpret_cast<const uint32_t*>(vc + int64_t(r4[u]) * kDh + 2 * dp);
  }
}

// The attention of item it in layer l (model.py:100-107 / multi_sm_decode.py:182-221).  Block wv
// comes in P when `pre` (loaded before the barrier), later blocks are loaded here.
__device__ __forceinline__ void att_compute(const Args& a, int l, const Item& it, AttPre& P, bool pre, AttLds& S,
                                            Sync& sy, uint32_t epoch, int wv, int lane) {
  const int tid = wv * 64 + lane;
  const int gs = a.H / a.KV, h = it.h, g = h / gs, m = it.m, p = it.p;
  const int pool = a.pool_pages * kPage;
  uint16_t* kc = a.kv + int64_t(l) * 2 * a.KV * pool * kDh + int64_t(g) * pool * kDh;
  uint16_t* vc = kc + int64_t(a.KV) * pool * kDh;
  if (!pre && wv != kQkvPoller && 64 * wv <= p) att_load(a, l, it, wv, lane, P);
  if (wv == kQkvPoller) {   // the item's q, k and v (posted by the QKV phase: no barrier)
    const uint64_t* row = x_qkv(a, l) + int64_t(m) * a.nqkv + lane;
    const uint64_t* const src[3] = {row + h * kDh, row + (a.H + g) * kDh, row + (a.H + a.KV + g) * kDh};
    float v[3];
    poll_words<3>(src, epoch, sy.status, v);
    // RoPE (model.py:110-117) in this wave: packed pair (2i, 2i+1) = dims (i, i + 32); lanes 0-31
    // rotate q's pair i = lane, lanes 32-63 k's pair i = lane - 32
    const int i = lane & 31;
    const float qa = __shfl(v[0], 2 * i), qb = __shfl(v[0], 2 * i + 1);
    const float ka = __shfl(v[1], 2 * i), kb = __shfl(v[1], 2 * i + 1);
    const float x0 = lane < 32 ? qa : ka, x1 = lane < 32 ? qb : kb;
    const float c = it.cs[i], sn = it.cs[kDh / 2 + i];
    const float r0 = x0 * c - x1 * sn, r1 = x0 * sn + x1 * c;
    float* dst = lane < 32 ? S.q : S.k;
    dst[i] = r0;
    dst[i + kDh / 2] = r1;
    S.v[lane] = v[2];
    if (h % gs == 0) {   // the current position's K/V row, bf16 (model.py:212-215)
      const int64_t crow = it.prow * kDh;
      if (lane >= 32) {
        kc[crow + i] = f2bf(r0);
        kc[crow + i + kDh / 2] = f2bf(r1);
      }
      vc[crow + lane] = f2bf(v[2]);
    }
    if (64 * wv <= p) att_load(a, l, it, wv, lane, P);   // this wave's block, after the poll
  }
  wsync(sy, lane);
  MBD_T(wv == 0 && l == kTraceLayer, 9);
  MBD_V(wv == 0 && l == kTraceLayer, 7, uint64_t(p));
  const int dp = lane & 31, half = lane >> 5;
  for (int b = wv; b < kBlocks; b += kWorkers) {
    const int j0 = 64 * b, j = j0 + lane;
    float mx = -INFINITY, ls = 0.f;
    if (j0 <= p) {
      if (b != wv) att_load(a, l, it, b, lane, P);
      float4 qv[kDh / 4];   // q in registers (broadcast LDS reads, issued together)
#pragma unroll
      for (int k = 0; k < kDh / 4; ++k) qv[k] = reinterpret_cast<const float4*>(S.q)[k];
      // the current position's score (its f32 K) as one wave sum, by the wave whose block holds it
      // (a sequential loop in its lane waited for an LDS round trip per pair of products)
      const float scur = p < j0 + 64 ? wave_sum(S.q[lane] * S.k[lane]) * 0.125f : 0.f;
      float sc = -INFINITY;
      if (j < p) {
        float a0 = 0.f, a1 = 0.f;
#pragma unroll
        for (int e8 = 0; e8 < kDh / 8; ++e8) {
          const uint32_t wd[4] = {P.ku[e8].x, P.ku[e8].y, P.ku[e8].z, P.ku[e8].w};
          const float qq[8] = {qv[2 * e8].x, qv[2 * e8].y, qv[2 * e8].z, qv[2 * e8].w,
                               qv[2 * e8 + 1].x, qv[2 * e8 + 1].y, qv[2 * e8 + 1].z, qv[2 * e8 + 1].w};
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            a0 += qq[2 * u] * __uint_as_float(wd[u] << 16);
            a1 += qq[2 * u + 1] * __uint_as_float(wd[u] & 0xffff0000u);
          }
        }
        sc = (a0 + a1) * 0.125f;
      } else if (j == p) {
        sc = scur;
      }
      mx = wave_max(sc);
      MBD_T(wv == 1 && b == wv && l == kTraceLayer, 15);
      const float e = (sc == -INFINITY) ? 0.f : expf(sc - mx);
      ls = wave_sum(e);
      S.p[b][lane] = e;
      __builtin_amdgcn_wave_barrier();
      const float vc0 = S.v[2 * dp], vc1 = S.v[2 * dp + 1];
      float pw[32];   // the half block's weights (LDS, 16-byte reads issued together)
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const float4 t = reinterpret_cast<const float4*>(&S.p[b][32 * half])[k];
        pw[4 * k] = t.x;
        pw[4 * k + 1] = t.y;
        pw[4 * k + 2] = t.z;
        pw[4 * k + 3] = t.w;
      }
      float o0[2] = {0.f, 0.f}, o1[2] = {0.f, 0.f};
      if (j0 + 63 < p) {   // every position of the block is cached
#pragma unroll
        for (int jj = 0; jj < 32; ++jj) {
          o0[jj & 1] += pw[jj] * __uint_as_float(P.vv[jj] << 16);
          o1[jj & 1] += pw[jj] * __uint_as_float(P.vv[jj] & 0xffff0000u);
        }
      } else {
        // slots jj < lim hold cached positions; the others (their rows are not this sequence's)
        // count as 0, and position p's f32 V is added after them with its weight
        const int lim = p - j0 - 32 * half;
#pragma unroll
        for (int jj = 0; jj < 32; ++jj) {
          const uint32_t vj = jj < lim ? P.vv[jj] : 0u;
          o0[jj & 1] += pw[jj] * __uint_as_float(vj << 16);
          o1[jj & 1] += pw[jj] * __uint_as_float(vj & 0xffff0000u);
        }
        const float ep = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e), p - j0));
        if (half == ((p - j0) >> 5)) {
          o0[0] += ep * vc0;
          o1[0] += ep * vc1;
        }
      }
      float a0 = o0[0] + o0[1], a1 = o1[0] + o1[1];
      a0 = add_halves(a0);   // the two halves of the block
      a1 = add_halves(a1);
      if (half == 0) {
        S.o[b][2 * dp] = a0;
        S.o[b][2 * dp + 1] = a1;
      }
    } else {
      S.o[b][lane] = 0.f;
    }
    if (lane == 0) {
      S.ml[b][0] = mx;
      S.ml[b][1] = ls;
    }
    MBD_T(b == wv && l == kTraceLayer, 160 + wv);
  }
  wsync(sy, lane);
  MBD_T(wv == 0 && l == kTraceLayer, 10);
  if (wv == 0) {   // merge of the blocks: softmax over all positions (lane b < 8: block b's weight)
    float ob[kBlocks], lb[kBlocks];   // every LDS read first (blocks past p hold zeros)
#pragma unroll
    for (int b = 0; b < kBlocks; ++b) {
      ob[b] = S.o[b][lane];
      lb[b] = S.ml[b][1];
    }
    const float mb = lane < kBlocks ? S.ml[lane][0] : -INFINITY;
    const float M = wave_max(mb);
    const float fb = mb == -INFINITY ? 0.f : expf(mb - M);
    // blocks past p (max -inf) have weight 0 and hold zeros: adding their 0 changes no sum
    float num = 0.f, den = 0.f;
#pragma unroll
    for (int b = 0; b < kBlocks; ++b) {
      const float f = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(fb), b));
      num += f * ob[b];
      den += f * lb[b];
    }
    st_split(x_att(a, l) + int64_t(m) * plane_ld(a.d) + perm_pos(h * kDh + lane, a.d), int64_t(kRows) * plane_ld(a.d),
             num / den);
    MBD_T(l == kTraceLayer, 11);
  }
  wsync(sy, lane);   // the LDS state is reused by the next item
}

// The B fragments of vocabulary groups c .. c + 3 (two 16-column tiles) for one worker wave's K
// steps s0 .. s0 + ns - 1, straight from the tied embedding rows (lane: row 8 g + (lane & 7) of
// group g = c + 2 t + ((lane & 15) >> 3), inputs 32 s + 8 (lane >> 4) .. + 7); groups past t1
// re-read the last one (the loads stay unconditional) and are never stored.
__device__ __forceinline__ void logit_frags(const Args& a, int c, int t1, int s0, int ns, int lane,
                                            uint4 (&b)[kStepsD][2]) {
  const int r = lane & 7, gq = (lane & 15) >> 3, q = lane >> 4;
#pragma unroll
  for (int i = 0; i < kStepsD; ++i) {
    const int st = s0 + min(i, ns - 1);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int g = min(c + 2 * t + gq, t1 - 1);
      b[i][t] = *reinterpret_cast<const uint4*>(a.outp + int64_t(8 * g + r) * a.d + 32 * st + 8 * q);
    }
  }
}

// ---------------------------------------------------------------- the step
// Epilogue of a phase that updates the residual stream (O, down, and the embedding): element e
// of sequence m becomes h1 (kept by the caller in its workgroup's LDS), h1 * scale goes to the
// hi/lo planes the next projection reads, and the 8 lanes of a group add up h1^2 for the next
// RMSNorm.  All 64 lanes of the wave call it (the sums use lane shuffles); act says whether this
// lane has an element.
__device__ __forceinline__ void put_residual(const Args& a, bool act, int m, int grp, int e, float h1,
                                             uint16_t* planes, float* ss, float scale, int n) {
  const int64_t o = int64_t(m) * plane_ld(a.d) + perm_pos(e, a.d);
  if (act) st_split(planes + o, int64_t(kRows) * plane_ld(a.d), h1 * scale);
  float v = act ? h1 * h1 : 0.f;
  v = sum8_lanes(v);
  if (act && (n & 7) == 0) st_f(ss + m * (a.d / 8) + grp, v);
}

__global__ __launch_bounds__(kThreads) void batch_step_kernel(Args a) {
  extern __shared__ __align__(16) uint8_t slots[];
  __shared__ int s_landed, s_consumed, s_wbar;
  __shared__ float s_inv[kRows];
  __shared__ float s_h[2 * kTilesD][kRows][8];   // the residual stream of this workgroup's groups
  __shared__ unsigned long long s_key[kRows];
  __shared__ AttLds s_att;
  const int lane_ = threadIdx.x & 63, wv_ = threadIdx.x >> 6;
  const int lane = lane_, wv = wv_;
  const int wg = blockIdx.x, G = gridDim.x;
  if (threadIdx.x == 0) {
    s_landed = 0;
    s_consumed = 0;
    s_wbar = 0;
  }
  if (threadIdx.x < kRows) s_key[threadIdx.x] = 0;
  __syncthreads();   // the only all-wave barrier: the loader never waits with the workers
  const uint32_t prev = ld_u32(a.ctrl + kCtlEpoch);
  const uint32_t epoch = prev % 0xFFFFFFFEu + 1u;
  const int slot_par = int(epoch & 1u);
  Sync sy{&s_landed, &s_consumed, &s_wbar, a.ctrl + kCtlStatus + 16 * slot_par, 0};
  if (wv == kWorkers) {
    // the loader wave issues ahead of the worker waves on its SIMD (measured: 0.792 -> 0.786 ms
    // per step; the workers raised instead: 0.1-0.3 % slower)
    if constexpr (kLoaderPrio > 0) __builtin_amdgcn_s_setprio(kLoaderPrio);
    loader(a, sy, slots, lane);
    return;
  }
  const int M = a.M;
  const int G8 = a.d / 8;
  int j = 0;   // this workgroup's job counter (the loader's order)
  att_setup(a, s_att, sy, wv, lane);
  // ---- the embedding rows as layer -1's residual stream, by the owners of the residual groups
  {
    int g0, g1;
    split(G8, G, wg, g0, g1);
    const int i = wv * 64 + lane;   // (group, sequence, element) = (i >> 6, (i >> 3) & 7, i & 7)
    if (i < 64 * (g1 - g0)) {       // whole waves (64 lanes per group)
      const int m = (i >> 3) & 7, k = i & 7, grp = g0 + (i >> 6), e = 8 * grp + k;
      int t = a.tokens[min(m, M - 1)];
      if (t < 0 || t >= a.V) {
        if (m < M && k == 0) atomicOr(sy.status, kStBadToken);
        t = 0;
      }
      const float h = bf2f(a.emb[int64_t(t) * a.d + e]);
      s_h[i >> 6][m][k] = h;
      put_residual(a, m < M, m, grp, e, h, x_hdp(a, -1), x_ssd(a, -1), bf2f(a.w[e]), k);
    }
    grid_sync(a, sy, 0, epoch, wv, lane);
  }
  AttPre pre;   // the first item's block of K/V rows, requested while the item's q/k/v are polled
  AOp<kStepsD> A;
  int s0, s1;
  for (int l = 0; l < a.L; ++l) {
    const uint16_t* wl = a.w + int64_t(l) * a.layer_elems;
    const int bl = 1 + 5 * l;   // barrier index of this layer's QKV phase
    // ---- QKV: raw projections of RMSNorm(h) (ln1), 1/rms applied to the outputs
    {
      MBD_T(wv_ == 0 && l == kTraceLayer, 0);
      const Job jb = layer_job(a, l, 0, wg, G);
      if (jb.ng > 0) {
        const int lane = opaque(lane_), wv = opaque(wv_);
        split(a.d / 32, kWorkers, wv, s0, s1);
        load_parts(x_hdp(a, l - 1), plane_ld(a.d), s0, s1 - s0, lane, A);
        if (wv == 0) row_inv(x_ssd(a, l - 1), a.d, s_inv, lane);
        MBD_T(wv == 0 && l == kTraceLayer, 1);
        int tiles;
        const f32x4* red = run_job(a, jb, j, slots, A, s0, s1 - s0, sy, wv, lane, tiles,
                                   l == kTraceLayer ? 2 : -1);
        MBD_T(wv == 0 && l == kTraceLayer, 3);
        for (int i = wv * 64 + lane; i < 128 * tiles && wv * 64 + lane < kEpi; i += kEpi) {
          const int t = i >> 7, m = (i >> 4) & 7, n = i & 15;
          if (2 * t + (n >> 3) < jb.ng && m < M) {
            const float y = tile_out(red, tiles, t, m, n) * s_inv[m];
            const int row = 8 * (jb.g0 + 2 * t + (n >> 3)) + (n & 7);
            st_u64(x_qkv(a, l) + int64_t(m) * a.nqkv + row, (uint64_t(epoch) << 32) | __float_as_uint(y));
          }
        }
        MBD_T(wv == 0 && l == kTraceLayer, 4);
        lds_bump(sy.consumed, lane);
        ++j;
      }
      // no barrier: the attention items poll their q, k and v words; the other waves request
      // their first K/V block meanwhile
      if (s_att.nitems > 0 && wv != kQkvPoller && 64 * wv <= s_att.it[0].p) att_load(a, l, s_att.it[0], wv, lane, pre);
      MBD_T(wv_ == 0, 40 + 5 * l + 0);
      MBD_T(wv_ == 0 && l == kTraceLayer, 5);
    }
    // ---- ATT: items (sequence, head) dealt so that the heads sharing a K/V head sit on one XCD
    {
      MBD_T(wv_ == 0 && l == kTraceLayer, 8);
      for (int n = 0; n < s_att.nitems; ++n) {
        const int lane = opaque(lane_), wv = opaque(wv_);
        att_compute(a, l, s_att.it[n], pre, n == 0, s_att, sy, epoch, wv, lane);
      }
      MBD_T(wv_ == 0 && l == kTraceLayer, 12);
      grid_sync(a, sy, bl + 1, epoch, wv, lane);
      MBD_T(wv_ == 0, 40 + 5 * l + 1);
      MBD_T(wv_ == 0 && l == kTraceLayer, 13);
    }
    // ---- O: h += O att
    {
      MBD_T(wv_ == 0 && l == kTraceLayer, 16);
      const Job jb = layer_job(a, l, 1, wg, G);
      if (jb.ng > 0) {
        const int lane = opaque(lane_), wv = opaque(wv_);
        split(a.d / 32, kWorkers, wv, s0, s1);
        load_parts(x_att(a, l), plane_ld(a.d), s0, s1 - s0, lane, A);
        // the next norm's scale of this thread's epilogue element (one per thread: 2 tiles at most)
        const int i0 = wv * 64 + lane, gi0 = 2 * (i0 >> 7) + ((i0 & 15) >> 3);
        const float sc = bf2f(wl[a.off_ln2 + 8 * (jb.g0 + min(gi0, jb.ng - 1)) + (i0 & 7)]);
        MBD_T(wv == 0 && l == kTraceLayer, 17);
        int tiles;
        const f32x4* red = run_job(a, jb, j, slots, A, s0, s1 - s0, sy, wv, lane, tiles,
                                   l == kTraceLayer ? 18 : -1);
        MBD_T(wv == 0 && l == kTraceLayer, 19);
        for (int i = wv * 64 + lane; i < 128 * tiles && wv * 64 + lane < kEpi; i += kEpi) {
          const int t = i >> 7, m = (i >> 4) & 7, n = i & 15, gi = 2 * t + (n >> 3);
          const bool act = gi < jb.ng && m < M;
          const int grp = jb.g0 + min(gi, jb.ng - 1), e = 8 * grp + (n & 7);
          float h1 = 0.f;
          if (act) {
            h1 = s_h[gi][m][n & 7] + tile_out(red, tiles, t, m, n);
            s_h[gi][m][n & 7] = h1;
          }
          put_residual(a, act, m, grp, e, h1, x_hop(a, l), x_sso(a, l), sc, n);
        }
        MBD_T(wv == 0 && l == kTraceLayer, 20);
        lds_bump(sy.consumed, lane);
        ++j;
      }
      grid_sync(a, sy, bl + 2, epoch, wv, lane);
      MBD_T(wv_ == 0, 40 + 5 * l + 2);
      MBD_T(wv_ == 0 && l == kTraceLayer, 21);
    }
    // ---- GU: act = silu(gate) * up of RMSNorm(h) (ln2)
    {
      MBD_T(wv_ == 0 && l == kTraceLayer, 24);
      const Job jb = layer_job(a, l, 2, wg, G);
      if (jb.ng > 0) {
        const int lane = opaque(lane_), wv = opaque(wv_);
        split(a.d / 32, kWorkers, wv, s0, s1);
        load_parts(x_hop(a, l), plane_ld(a.d), s0, s1 - s0, lane, A);
        if (wv == 0) row_inv(x_sso(a, l), a.d, s_inv, lane);
        MBD_T(wv == 0 && l == kTraceLayer, 25);
        int tiles;
        const f32x4* red = run_job(a, jb, j, slots, A, s0, s1 - s0, sy, wv, lane, tiles,
                                   l == kTraceLayer ? 26 : -1);
        MBD_T(wv == 0 && l == kTraceLayer, 27);
        for (int i = wv * 64 + lane; i < 64 * tiles && wv * 64 + lane < kEpi; i += kEpi) {
          const int t = i >> 6, m = (i >> 3) & 7, n = 2 * (i & 7);
          if (2 * t + (n >> 3) < jb.ng && m < M) {
            const float gt = tile_out(red, tiles, t, m, n) * s_inv[m], up = tile_out(red, tiles, t, m, n + 1) * s_inv[m];
            const int f = (8 * (jb.g0 + 2 * t + (n >> 3)) + (n & 7)) >> 1;
            st_split(x_act(a, l) + int64_t(m) * plane_ld(a.ff) + perm_pos(f, a.ff), int64_t(kRows) * plane_ld(a.ff),
                     (gt * (1.f / (1.f + expf(-gt)))) * up);
          }
        }
        MBD_T(wv == 0 && l == kTraceLayer, 28);
        lds_bump(sy.consumed, lane);
        ++j;
      }
      grid_sync(a, sy, bl + 3, epoch, wv, lane);
      MBD_T(wv_ == 0, 40 + 5 * l + 3);
      MBD_T(wv_ == 0 && l == kTraceLayer, 29);
    }
    // ---- DN: h += W_down act
    {
      MBD_T(wv_ == 0 && l == kTraceLayer, 32);
      const Job jb = layer_job(a, l, 3, wg, G);
      if (jb.ng > 0) {
        const int lane = opaque(lane_), wv = opaque(wv_);
        split(a.ff / 32, kWorkers, wv, s0, s1);
        AOp<kStepsF> Af;
        load_parts(x_act(a, l), plane_ld(a.ff), s0, s1 - s0, lane, Af);
        // the next RMSNorm's scale (the next layer's ln1, or the final norm) of this thread's
        // epilogue element (one per thread: 1 tile)
        const uint16_t* nsc = l + 1 < a.L ? wl + a.layer_elems : a.lnf;
        const int i0 = wv * 64 + lane, gi0 = (i0 & 15) >> 3;
        const float sc = bf2f(nsc[8 * (jb.g0 + min(gi0, jb.ng - 1)) + (i0 & 7)]);
        MBD_T(wv == 0 && l == kTraceLayer, 33);
        int tiles;
        const f32x4* red = run_job<kStepsF, kTilesF>(a, jb, j, slots, Af, s0, s1 - s0, sy, wv, lane, tiles,
                                                     l == kTraceLayer ? 34 : -1);
        MBD_T(wv == 0 && l == kTraceLayer, 35);
        for (int i = wv * 64 + lane; i < 128 * tiles && wv * 64 + lane < kEpi; i += kEpi) {
          const int t = i >> 7, m = (i >> 4) & 7, n = i & 15, gi = 2 * t + (n >> 3);
          const bool act = gi < jb.ng && m < M;
          const int grp = jb.g0 + min(gi, jb.ng - 1), e = 8 * grp + (n & 7);
          float h1 = 0.f;
          if (act) {
            h1 = s_h[gi][m][n & 7] + tile_out(red, tiles, t, m, n);
            s_h[gi][m][n & 7] = h1;
          }
          put_residual(a, act, m, grp, e, h1, x_hdp(a, l), x_ssd(a, l), sc, n);
        }
        MBD_T(wv == 0 && l == kTraceLayer, 36);
        lds_bump(sy.consumed, lane);
        ++j;
      }
      if (kLogitsReg && l + 1 == a.L) break;   // the last barrier follows the loop
      grid_sync(a, sy, bl + 4, epoch, wv, lane);
      MBD_T(wv_ == 0, 40 + 5 * l + 4);
      MBD_T(wv_ == 0 && l == kTraceLayer, 37);
    }
  }
  // ---- final RMSNorm, tied logits and the argmax keys
  int t0, t1;
  split(a.V / 8, G, wg, t0, t1);
  uint4 lfirst[kStepsD][2];   // the first logits chunk's B fragments
  if constexpr (kLogitsReg) {
    // the last layer's down barrier: every wave but the polling one requests its first chunk
    // of logit rows before waiting
    const int bl = 5 * a.L;
    grid_arrive(a, sy, bl, epoch, wv_, lane_);
    split(a.d / 32, kWorkers, wv_, s0, s1);
    if (wv_ != 0 && t1 > t0) logit_frags(a, t0, t1, s0, s1 - s0, lane_, lfirst);
    grid_wait(a, sy, bl, epoch, wv_, lane_);
    MBD_T(wv_ == 0, 40 + 5 * (a.L - 1) + 4);
  }
  if (t1 > t0) {
    const int lane = opaque(lane_), wv = opaque(wv_);
    split(a.d / 32, kWorkers, wv, s0, s1);
    load_parts(x_hdp(a, a.L - 1), plane_ld(a.d), s0, s1 - s0, lane, A);
    if (wv == 0) row_inv(x_ssd(a, a.L - 1), a.d, s_inv, lane);
    const int m = ((wv * 64 + lane) >> 4) & 7;   // the same sequence for every output of this thread
    uint64_t best = 0;
    if constexpr (kLogitsReg) {
      // chunks of 4 groups (two 16-column tiles), each worker wave streaming the B fragments of
      // its K steps into registers one chunk ahead (the first chunk requested before the last
      // barrier by every wave but the polling one).  The partial tiles meet in slot 0 of the
      // ring, which no DMA writes any more (every layer job has been consumed).
      const int ns = s1 - s0;
      f32x4* red = reinterpret_cast<f32x4*>(slots);
      auto load_b = [&](int c, uint4 (&b)[kStepsD][2]) { logit_frags(a, c, t1, s0, ns, lane, b); };
      auto take = [&](const uint4 (&b)[kStepsD][2], int c) {
        f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
        for (int i = 0; i < kStepsD; ++i)
          if (i < ns) {
            const bf16x8 av = __builtin_bit_cast(bf16x8, A.f[i]);
#pragma unroll
            for (int t = 0; t < 2; ++t)
              acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, __builtin_bit_cast(bf16x8, b[i][t]), acc[t], 0, 0, 0);
          }
        wsync(sy, lane);   // every wave has read the previous chunk's tiles
#pragma unroll
        for (int t = 0; t < 2; ++t) red[(wv * 2 + t) * 64 + lane] = acc[t];
        wsync(sy, lane);
        const int ng = min(4, t1 - c);
        for (int i = wv * 64 + lane; i < 256 && wv * 64 + lane < kEpi; i += kEpi) {
          const int t = i >> 7, n = i & 15;
          if (2 * t + (n >> 3) < ng && m < M) {
            const float y = tile_out(red, 2, t, m, n) * s_inv[m];
            const int v = 8 * (c + 2 * t + (n >> 3)) + (n & 7);
            a.logits[int64_t(m) * a.V + v] = y;
            const uint64_t key = argmax_key(y, v);
            best = key > best ? key : best;
          }
        }
      };
      uint4 (&ba)[kStepsD][2] = lfirst;
      uint4 bb[kStepsD][2];
      if (wv == 0) load_b(t0, ba);
      for (int c = t0; c < t1; c += 8) {
        load_b(c + 4, bb);
        take(ba, c);
        if (c + 4 >= t1) break;
        load_b(c + 8, ba);
        take(bb, c + 4);
      }
    }
    for (int c = t0; !kLogitsReg && c < t1; c += a.tchunk) {
      const Job jb{a.outp, a.d, c, min(a.tchunk, t1 - c)};
      int tiles;
      const f32x4* red = run_job(a, jb, j, slots, A, s0, s1 - s0, sy, wv, lane, tiles);
      for (int i = wv * 64 + lane; i < 128 * tiles && wv * 64 + lane < kEpi; i += kEpi) {
        const int t = i >> 7, n = i & 15;
        if (2 * t + (n >> 3) < jb.ng && m < M) {
          const float y = tile_out(red, tiles, t, m, n) * s_inv[m];
          const int v = 8 * (jb.g0 + 2 * t + (n >> 3)) + (n & 7);
          a.logits[int64_t(m) * a.V + v] = y;
          const uint64_t key = argmax_key(y, v);
          best = key > best ? key : best;
        }
      }
      lds_bump(sy.consumed, lane);
      ++j;
    }
    MBD_T(wv == 0, 168);
    if (m < M && best) atomicMax(&s_key[m], (unsigned long long)best);
    wsync(sy, lane);
    if (wv == 0 && lane < M) atomicMax(reinterpret_cast<unsigned long long*>(a.keys + kRows * slot_par + lane),
                                       (unsigned long long)s_key[lane]);
  }
  // ---- last barrier; workgroup 0 publishes the tokens and clears the other parity's slots
  grid_arrive(a, sy, 5 * a.L + 1, epoch, wv, lane);
  if (wg == 0) grid_wait(a, sy, 5 * a.L + 1, epoch, wv, lane);
  MBD_T(wv == 0, 169);
  if (wg == 0 && wv == 0) {
    if (lane < M) {
      const uint64_t k = ld_u64(a.keys + kRows * slot_par + lane);
      a.out[2 * lane] = int32_t(0xffffffffu - uint32_t(k & 0xffffffffu));
      a.out[2 * lane + 1] = int32_t(ld_u32(sy.status));
    }
    if (lane < kRows) st_u64(a.keys + kRows * (slot_par ^ 1) + lane, 0);
    if (lane == 0) {
      st_u32(a.ctrl + kCtlStatus + 16 * (slot_par ^ 1), 0);
      st_u32(a.ctrl + kCtlEpoch, epoch);
    }
  }
}

// ---------------------------------------------------------------- host side
struct Plan {
  bool ok = false;
  int G = 0, slot_bytes = 0, nslots = 0, tchunk = 0;
  size_t lds = 0;
};

struct Region {
  int64_t ctrl, keys, flags, x, x_layer, bytes;
};

static int64_t al256(int64_t x) { return (x + 255) & ~int64_t(255); }

static Region region(const msd_config* c) {
  const int nqkv = (c->n_heads + 2 * c->n_kv_heads) * kDh;
  Region R;
  int64_t o = 0;
  R.ctrl = o;  o += 256;
  R.keys = o;  o += 256;
  R.flags = o; o += al256(int64_t(5 * c->n_layers + 2) * kFlagReps * kMaxGrid * 4);
  R.x_layer = al256(x_block_floats(c->d_model, nqkv, c->d_ff) * 4) / 4;   // floats
  R.x = o;     o += R.x_layer * 4 * (c->n_layers + 1);
  R.bytes = o;
  return R;
}

static bool shape_ok(const msd_config* c) {
  if (!c || c->d_head != kDh || c->n_heads <= 0 || c->n_kv_heads <= 0 || c->n_layers <= 0) return false;
  if (c->n_heads * kDh != c->d_model || c->n_heads % c->n_kv_heads) return false;
  if (c->d_model % 256 || c->d_ff % 64 || c->vocab_size % 8 || c->vocab_size <= 0) return false;
  if (c->d_model < 32 * kWorkers || c->d_ff < 32 * kWorkers) return false;
  if ((c->d_model / 32 + kWorkers - 1) / kWorkers > kStepsD) return false;
  if ((c->d_ff / 32 + kWorkers - 1) / kWorkers > kStepsF) return false;
  if (c->context_len <= 0 || c->context_len > kMaxCtx) return false;
  return true;
}

static size_t static_lds() {
  return sizeof(AttLds) + 3 * sizeof(int) + sizeof(float) * kWorkers * kRows + 8 * kRows + 64;
}

// Slot size and ring depth for a grid of G workgroups.
static Plan make_plan(const msd_config* c, int G) {
  Plan p;
  const int d = c->d_model, ff = c->d_ff, nqkv = (c->n_heads + 2 * c->n_kv_heads) * kDh;
  auto groups_per_wg = [&](int rows) { return (rows / 8 + G - 1) / G; };
  const int nqw = qkv_wgs(nqkv / 8, G);
  const int gq = (nqkv / 8 + nqw - 1) / nqw, go = groups_per_wg(d), ggu = groups_per_wg(2 * ff), gdn = groups_per_wg(d);
  if (std::max(std::max(gq, go), ggu) > 2 * kTilesD || gdn > 2 * kTilesF) return p;
  {   // (sequence, head) item slots per workgroup (att_setup deals 8 gs ceil(M KV / 8) slots)
    const int gs = c->n_heads / c->n_kv_heads, ni = 8 * gs * ((kRows * c->n_kv_heads + 7) / 8);
    if ((ni + G - 1) / G > kMaxItems) return p;
  }
  int64_t job = std::max(std::max(int64_t(gq) * 16 * d, int64_t(go) * 16 * d),
                         std::max(int64_t(ggu) * 16 * d, int64_t(gdn) * 16 * ff));
  const int max_tiles = (std::max(std::max(gq, go), std::max(ggu, gdn)) + 1) / 2;
  int64_t S = std::max(job, int64_t(kWorkers) * std::max(max_tiles, 1) * 1024);
  // logits chunks: as many groups as a slot holds (at most kMaxGroups), and the summed tiles fit
  int tchunk = int(std::min<int64_t>(kMaxGroups, S / (16 * int64_t(d))));
  if (tchunk < 1) return p;
  S = std::max(S, int64_t(kWorkers) * ((tchunk + 1) / 2) * 1024);
  S = (S + 1023) & ~int64_t(1023);
  const int64_t avail = kLdsTotal - int64_t(static_lds());
  const int ns = int(std::min<int64_t>(3, avail / S));
  if (ns < 2) return p;
  p.ok = true;
  p.G = G;
  p.slot_bytes = int(S);
  p.nslots = ns;
  p.tchunk = tchunk;
  p.lds = size_t(ns) * size_t(S);
  return p;
}

struct Cached {
  int dev;
  msd_config cfg;
  Plan plan;
};

static bool same_cfg(const msd_config& a, const msd_config& b) {
  return a.vocab_size == b.vocab_size && a.d_model == b.d_model && a.n_heads == b.n_heads &&
         a.n_kv_heads == b.n_kv_heads && a.n_layers == b.n_layers && a.d_head == b.d_head && a.d_ff == b.d_ff &&
         a.context_len == b.context_len;
}

// The plan for this device: grid = compute units, provided every workgroup is resident
// (occupancy API) at the plan's LDS size; not ok otherwise.
static Plan device_plan(const msd_config* c, hipError_t& err) {
  static std::mutex mu;
  static std::vector<Cached> cache;
  err = hipSuccess;
  int dev = 0;
  if ((err = hipGetDevice(&dev)) != hipSuccess) return Plan{};
  std::lock_guard<std::mutex> lk(mu);
  for (const Cached& e : cache)
    if (e.dev == dev && same_cfg(e.cfg, *c)) return e.plan;
  int cus = 0;
  if ((err = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev)) != hipSuccess) return Plan{};
  Plan p = cus >= 8 && cus <= kMaxGrid ? make_plan(c, cus) : Plan{};
  if (p.ok) {
    const void* fn = reinterpret_cast<const void*>(&batch_step_kernel);
    if ((err = msdc::ensure_dynamic_lds(fn, p.lds)) != hipSuccess) return Plan{};
    int per_cu = 0;
    if ((err = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kThreads, p.lds)) != hipSuccess)
      return Plan{};
    if (per_cu * cus < p.G) p.ok = false;
  }
  cache.push_back({dev, *c, p});
  return p;
}

#ifdef MBD_TRACE
}  // namespace mbd
extern "C" int32_t mbd_trace_copy(void* host) {
  return hipMemcpyFromSymbol(host, HIP_SYMBOL(mbd::mbd_trace_buf), sizeof(mbd::mbd_trace_buf)) == hipSuccess ? 0 : -1;
}
namespace mbd {
#endif

int64_t region_bytes(const msd_config* cfg) { return shape_ok(cfg) ? region(cfg).bytes : 0; }

int32_t try_step(const StepArgs& s) {
  const msd_config* c = s.cfg;
  if (!shape_ok(c) || s.batch <= 0 || s.batch > kRows) return 1;
  hipError_t err;
  const Plan p = device_plan(c, err);
  if (err != hipSuccess) return MSD_E_HIP;
  if (!p.ok) return 1;
  const Region R = region(c);
  char* base = static_cast<char*>(s.region);
  const int d = c->d_model, ff = c->d_ff, nqkv = (c->n_heads + 2 * c->n_kv_heads) * kDh;
  Args a;
  a.d = d;
  a.ff = ff;
  a.H = c->n_heads;
  a.KV = c->n_kv_heads;
  a.L = c->n_layers;
  a.V = c->vocab_size;
  a.ctx = c->context_len;
  a.nqkv = nqkv;
  a.M = s.batch;
  a.off_ln2 = d;
  a.off_qkv = 2 * int64_t(d);
  a.off_o = a.off_qkv + int64_t(nqkv) * d;
  a.off_gu = a.off_o + int64_t(d) * d;
  a.off_dn = a.off_gu + 2 * int64_t(ff) * d;
  a.layer_elems = a.off_dn + int64_t(d) * ff;
  a.emb = s.emb;
  a.outp = s.outp;
  a.w = s.w;
  a.lnf = s.lnf;
  a.rope = s.rope;
  a.tokens = s.tokens;
  a.pos = s.positions;
  a.pages = s.pages;
  a.max_pages = s.max_pages;
  a.pool_pages = s.pool_pages;
  a.kv = s.kv;
  a.logits = s.logits;
  a.out = s.out;
  a.ctrl = reinterpret_cast<uint32_t*>(base + R.ctrl);
  a.keys = reinterpret_cast<uint64_t*>(base + R.keys);
  a.flags = reinterpret_cast<uint32_t*>(base + R.flags);
  a.x = reinterpret_cast<float*>(base + R.x);
  a.x_layer = R.x_layer;
  a.slot_bytes = p.slot_bytes;
  a.nslots = p.nslots;
  a.tchunk = p.tchunk;
  hipLaunchKernelGGL(batch_step_kernel, dim3(p.G), dim3(kThreads), p.lds, s.stream, a);
  return hipGetLastError() == hipSuccess ? MSD_OK : MSD_E_HIP;
}

}  // namespace mbd
