// Fused whole-model decode step for gfx950 (MI355X): one persistent launch per token.
//
// Reference path replaced (zahlmann/transformer): kernels/multi_sm_decode.py:35-357
// (_multi_sm_decode) behind multi_sm_decode_nlayer (:369-432).  The maths follows
// model.py:94-191; the decode-step semantics (f32 residual stream, K/V written to the
// cache as bf16 at `pos`, the current position attending with its un-rounded K/V,
// argmax resolving ties to the lowest index) follow kernels/multi_sm_decode.py.
//
// Execution model
//   * grid = one workgroup per compute unit (256 on MI355X), 9 wave64s per workgroup;
//     every workgroup is resident for the whole step (one per CU, launched on an otherwise
//     idle device), so workgroups may wait on each other.
//   * two kinds of workgroups:
//       - row workgroups (all but the last H * nsplit) own fixed output rows of every
//         projection and of the tied logits.  A loader wave streams this workgroup's layer
//         rows by DMA (global_load_lds) into an LDS ring one layer ahead; 8 worker waves, all
//         alike, keep the residual stream h in registers, take the RMSNorms, the dot
//         products of their rows from LDS, store the outputs and gather an eighth of the
//         next input vector each; at the end they stream the logit rows straight into
//         registers;
//       - attention workgroups (one per query head and context split of 512 positions)
//         hold their KV head's cached rows in LDS (bf16, streamed in by their loader wave
//         during the previous layer); 8 attention waves poll the head's q, take the scores
//         of a block of positions on the matrix cores and P.V on the vector units, poll the
//         new k, v and merge the blocks by log-sum-exp.
//   * weights are bf16 in an (out, in) row layout: every output element is one contiguous
//     dot product; a lane reads 16 bytes (8 bf16) per 512-element block from LDS, widens
//     them to f32 and the wave reduces with DPP.  All activation arithmetic is f32.
//   * cross-workgroup exchange uses tagged 64-bit words: (f32 value | 32-bit epoch tag),
//     written with device-scope atomic stores and polled with device-scope atomic loads.
//     A word carries its own validity, so no separate flag, fence or barrier is needed;
//     each (layer, exchange) has its own buffer so tags only need to differ per step.
//     Weight and KV streaming goes through the LDS-DMA path, whose returns do not queue
//     ahead of the polls the way loads into registers do.
//   * per layer and row workgroup: QKV rows (+RoPE, KV write) -> attention (attention
//     workgroups) -> O rows (+residual) -> gate/up rows (+SwiGLU) -> down rows
//     (+residual); then final RMSNorm, vocabulary rows of the tied embedding, argmax via
//     a 64-bit atomic max of (ordered value, inverted index) and a last-arriver counter.
//   * every cross-workgroup wait is bounded: a workgroup that exceeds the spin bound sets
//     the status word and stops waiting; the others see the status and stop as well, so a
//     broken step still drains the grid.  Waits between the waves of one workgroup use
//     LDS counters (the loader wave never meets a workgroup barrier).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <mutex>
#include <vector>

#include "../../include/msdecode.h"
#include "internal.h"

namespace msd {

// Optional phase timestamps for profiling builds (-DMSD_TRACE): lane 0 of a wave records
// s_memrealtime (100 MHz) at phase boundaries of every layer into
// msd_trace_buffer[layer][workgroup][slot] (the tail after the last layer is recorded as layer
// n_layers), and per-wave stamps of layer MSD_TRACE_LAYER into msd_trace_waves.  Compiled out
// otherwise.
#ifdef MSD_TRACE
#ifndef MSD_TRACE_LAYER
#define MSD_TRACE_LAYER 10
#endif
constexpr int kTraceLayers = 64, kTraceWgs = 512, kTraceSlots = 32;
__device__ uint64_t msd_trace_buffer[kTraceLayers * kTraceWgs * kTraceSlots];
#define MSD_TRACE_POINT(cond, layer, slot)                                                              \
  do {                                                                                                  \
    if ((cond) && (layer) < kTraceLayers && blockIdx.x < kTraceWgs && (threadIdx.x & 63) == 0)          \
      msd_trace_buffer[((layer) * kTraceWgs + blockIdx.x) * kTraceSlots + (slot)] =                     \
          __builtin_amdgcn_s_memrealtime();                                                             \
  } while (0)
__device__ uint64_t msd_trace_waves[4096 * 16 * 8];
#define MSD_TRACE_WAVE(layer, slot)                                                         \
  do {                                                                                    \
    if ((layer) == MSD_TRACE_LAYER && (threadIdx.x & 63) == 0)                            \
      msd_trace_waves[(blockIdx.x * 16 + (threadIdx.x >> 6)) * 8 + (slot)] =              \
          __builtin_amdgcn_s_memrealtime();                                               \
  } while (0)
#else
#define MSD_TRACE_POINT(cond, layer, slot) \
  do {                                     \
  } while (0)
#define MSD_TRACE_WAVE(layer, slot) \
  do {                              \
  } while (0)
#endif

constexpr int kDh = 64;          // head dimension (fixed)
constexpr int kPart = 66;        // per (head, split): m, l, o[64]
constexpr int kAttCap = 512;     // cached positions an attention workgroup holds in LDS
constexpr int kMaxCtx = 2048;    // context: at most 4 splits of kAttCap positions per head
constexpr int kKRowB = 160;      // LDS bytes per cached K row: 128 + 32 padding.  The score tiles
                                 // read 16 bytes of 16 consecutive rows per lane group: with a
                                 // 144-byte pitch that took twice the LDS cycles (a probe of the
                                 // pattern under SQ_LDS_BANK_CONFLICT), with 160 none extra
constexpr int kKSlots = kKRowB / 16;   // 16-byte DMA slots per K row (those past 8 repeat the 8th)
constexpr int kVRowB = 128;      // LDS bytes per cached V row
constexpr uint32_t kSpinLimit = 1u << 20;

#ifndef MSD_ROW_WAVES
#define MSD_ROW_WAVES 8
#endif
constexpr int kWavesR = MSD_ROW_WAVES;   // worker waves of a row workgroup (the rest of 0..7 exit)
constexpr int kWavesA = 8;       // attention waves of an attention workgroup
constexpr int kLoader = kWavesR > 8 ? kWavesR : 8;   // wave index of the loader (both kinds)
constexpr int kThreadsWG = (kLoader + 1) * 64;
constexpr int kMbox = 8;         // outputs per compute wave and phase
#ifndef MSD_REPLICAS
#define MSD_REPLICAS 4
#endif
constexpr int kRep = MSD_REPLICAS;   // replicas of every vector all row workgroups gather
static_assert((kRep % kWavesA == 0 || kRep < kWavesA) && kRep <= 64, "attention waves store whole sets of replicas");
// 1 KB DMA instructions a loader keeps in flight.  Fewer bytes in flight across the device
// shorten the round trip of the exchange polls; the layer weights and KV rows need only a
// few per CU to stay a layer ahead.
#ifndef MSD_DMA_LAYER
#define MSD_DMA_LAYER 8
#endif
#ifndef MSD_DMA_KV
#define MSD_DMA_KV 16
#endif
#ifndef MSD_DMA_FIRST
#define MSD_DMA_FIRST 32
#endif
constexpr int kDmaLayer = MSD_DMA_LAYER, kDmaKV = MSD_DMA_KV;
// the first layer's rows load before any exchange traffic: a wider window
constexpr int kDmaFirst = MSD_DMA_FIRST;

constexpr uint32_t kStatusTimeout = 1u;
constexpr uint32_t kStatusBadToken = 2u;
// next_token[1] between the start of a step and its last arrival
constexpr uint32_t kStatusUnfinished = 0x80000000u;

__host__ __device__ inline int cdiv(int a, int b) { return (a + b - 1) / b; }
__host__ __device__ inline int64_t align64(int64_t v) { return (v + 63) & ~int64_t(63); }

// ---------------------------------------------------------------- layout
struct Layout {
  // packed weights, per layer (bf16 elements)
  int64_t off_ln1, off_ln2, off_qkv, off_o, off_gu, off_dn, layer_elems;
  // exchange words per layer (uint64): x_qkv once, then kRep replicas (stride x_rep) of
  // [attention partials | hd1 | act | hd2]
  int64_t x_qkv, x_att, x_hd1, x_act, x_hd2, x_rep, x_layer;
  int64_t ctrl_bytes;
};

__host__ __device__ inline int att_cap(int ctx) { return ctx < kAttCap ? ctx : kAttCap; }
__host__ __device__ inline int att_splits(int ctx) { return cdiv(ctx, att_cap(ctx)); }
// Attention words per replica: with one split, the normalised head outputs (H * 64); with
// several, every (head, split)'s (max, sum, unnormalised output) for the row workgroups to merge.
__host__ __device__ inline int64_t att_words(int H, int ctx) {
  const int ns = att_splits(ctx);
  return ns == 1 ? int64_t(H) * kDh : int64_t(H) * ns * kPart;
}

__host__ __device__ inline Layout make_layout(int d, int H, int KV, int ff, int ctx) {
  Layout t;
  const int64_t nqkv = int64_t(H + 2 * KV) * kDh;
  t.off_ln1 = 0;
  t.off_ln2 = d;
  t.off_qkv = 2 * int64_t(d);
  t.off_o = t.off_qkv + nqkv * d;
  t.off_gu = t.off_o + int64_t(d) * d;
  t.off_dn = t.off_gu + 2 * int64_t(ff) * d;
  t.layer_elems = t.off_dn + int64_t(d) * ff;
  t.x_qkv = 0;
  t.x_att = align64(nqkv);
  t.x_hd1 = t.x_att + align64(att_words(H, ctx));
  t.x_act = t.x_hd1 + align64(d);
  t.x_hd2 = t.x_act + align64(ff);
  // replicas at a stride that is not a multiple of 4 KB spread the reads over channels
  const int64_t rep_words = t.x_hd2 + align64(d) - t.x_att;
  t.x_rep = ((rep_words + 511) & ~int64_t(511)) + 32;
  t.x_layer = t.x_att + kRep * t.x_rep;
  t.ctrl_bytes = 256;
  return t;
}

struct Args {
  const uint16_t* emb;
  const uint16_t* outp;   // tied output projection: token_emb rows in the kernel row layout
  const uint16_t* w;
  const uint16_t* lnf;
  const float* rope;
  uint16_t* kv;
  float* logits;
  int32_t* next_token;   // [2 * nsteps]: per step (argmax, status)
  const int32_t* token_dev;
  uint32_t* ctrl;   // [0] status, [1] arrival counter, [2..3] argmax key (u64), [16..47] token words
  uint64_t* xw;     // exchange words, n_layers * x_layer
  int token, pos;   // input token and position of step 0 (step s runs at pos + s)
  uint32_t epoch;   // tag of step 0 (step s tags its words epoch + s)
  int nsteps;       // greedy steps of this launch; step s + 1 feeds step s's argmax
  int64_t logits_stride;   // floats between the logits of consecutive steps (0: one buffer)
  int H, KV, L, ff, V, ctx;
  int nsplit, cap, NA, GR;   // attention splits, positions per split, attention / row workgroups
  // row workgroups: LDS ring regions (bytes) of the QKV, O, gate/up and down rows, the
  // ring size
  int ring_q, ring_o, ring_g, ring_d, ring_bytes;
  int keep;   // layers whose rows are read with the caching policy (the rest stream)
  Layout lay;
};

// ---------------------------------------------------------------- helpers
__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float bf2f(uint16_t b) { return __uint_as_float(uint32_t(b) << 16); }
__device__ __forceinline__ uint16_t f2bf(float f) {  // round to nearest even
  uint32_t u = __float_as_uint(f);
  return uint16_t((u + (((u >> 16) & 1u) + 0x7fffu)) >> 16);
}

// Wave64 reductions with DPP (no LDS traffic): rows of 16 lanes are scanned with
// row_shr 1/2/4/8, then row_bcast 15/31 carry the row totals into lane 63, which is read
// back as a wave-uniform value.  The addition order is fixed, so every call is
// deterministic.
__device__ __forceinline__ float dpp_f(float v, int ctrl) {
  switch (ctrl) {   // the control word must be a compile-time constant
    case 0x111: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x111, 0xf, 0xf, true));
    case 0x112: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x112, 0xf, 0xf, true));
    case 0x114: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x114, 0xf, 0xf, true));
    case 0x118: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x118, 0xf, 0xf, true));
    case 0x142: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x142, 0xa, 0xf, true));
    default: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x143, 0xc, 0xf, true));
  }
}
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_f(v, 0x111);
  v += dpp_f(v, 0x112);
  v += dpp_f(v, 0x114);
  v += dpp_f(v, 0x118);
  v += dpp_f(v, 0x142);
  v += dpp_f(v, 0x143);
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
// max over the wave; -inf fills lanes without a DPP source
__device__ __forceinline__ float dppm_f(float v, int ctrl) {
  const int ninf = __float_as_int(-INFINITY);
  switch (ctrl) {
    case 0x111: return __int_as_float(__builtin_amdgcn_update_dpp(ninf, __float_as_int(v), 0x111, 0xf, 0xf, false));
    case 0x112: return __int_as_float(__builtin_amdgcn_update_dpp(ninf, __float_as_int(v), 0x112, 0xf, 0xf, false));
    case 0x114: return __int_as_float(__builtin_amdgcn_update_dpp(ninf, __float_as_int(v), 0x114, 0xf, 0xf, false));
    case 0x118: return __int_as_float(__builtin_amdgcn_update_dpp(ninf, __float_as_int(v), 0x118, 0xf, 0xf, false));
    case 0x142: return __int_as_float(__builtin_amdgcn_update_dpp(ninf, __float_as_int(v), 0x142, 0xa, 0xf, false));
    default: return __int_as_float(__builtin_amdgcn_update_dpp(ninf, __float_as_int(v), 0x143, 0xc, 0xf, false));
  }
}
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dppm_f(v, 0x111));
  v = fmaxf(v, dppm_f(v, 0x112));
  v = fmaxf(v, dppm_f(v, 0x114));
  v = fmaxf(v, dppm_f(v, 0x118));
  v = fmaxf(v, dppm_f(v, 0x142));
  v = fmaxf(v, dppm_f(v, 0x143));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// N independent wave sums taken one DPP step at a time across all N values (the chains
// interleave); same addition order as wave_sum.
template <int N>
__device__ __forceinline__ void wave_sum_n(float (&v)[N]) {
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] += dpp_f(v[i], 0x111);
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] += dpp_f(v[i], 0x112);
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] += dpp_f(v[i], 0x114);
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] += dpp_f(v[i], 0x118);
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] += dpp_f(v[i], 0x142);
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] += dpp_f(v[i], 0x143);
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v[i]), 63));
}

__device__ __forceinline__ void st_tag(uint64_t* p, float v, uint32_t tag) {
  __hip_atomic_store(p, (uint64_t(tag) << 32) | __float_as_uint(v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld_tag(const uint64_t* p) {
  return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Stores to the step outputs (token, status): written by workgroup 0 at the start of a step
// and by the last arriver at its end, on different XCDs, so they go through to memory in the
// order the step imposes instead of waiting in two L2 caches whose write-back order is free.
__device__ __forceinline__ void put_out(int32_t* p, int32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ld_status(uint32_t* ctrl) {
  return __hip_atomic_load(ctrl, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Wave priority (s_setprio) of the row workgroups' worker waves; the loader waves keep 0
#ifndef MSD_WORKER_PRIO
#define MSD_WORKER_PRIO 1
#endif
constexpr int kWorkerPrio = MSD_WORKER_PRIO;

// s_sleep units between poll rounds (measured on this kernel: none is fastest, 316.8 vs 318.6 us
// per token with 2; every round already waits for its loads)
#ifndef MSD_ROUND_SLEEP
#define MSD_ROUND_SLEEP 0
#endif
// One step of a bounded spin: after kSpinLimit rounds, or when another workgroup has
// reported a timeout in the status word, the wave stops waiting and `bad` is set.
__device__ __forceinline__ void spin_step(uint32_t& spins, uint32_t* ctrl, int lane, bool& bad) {
  if constexpr (MSD_ROUND_SLEEP > 0) __builtin_amdgcn_s_sleep(MSD_ROUND_SLEEP);
  ++spins;
  if ((spins & 255u) == 0 && (ld_status(ctrl) & kStatusTimeout)) bad = true;
  if (spins > kSpinLimit) {
    if (lane == 0) atomicOr(ctrl, kStatusTimeout);
    bad = true;
  }
}

// Polling of tagged words.  Lane j of wave w (of nw waves sharing a vector) handles slots
// k < NK, word xidx(k, w, j): 64-word blocks are dealt round-robin to the waves.  Each
// round re-loads only the words whose tag is not yet current and waits for them; a
// single round is in flight, so the polls of one CU never queue many loads ahead of its
// latency-critical stores.
template <int NW>
__device__ __forceinline__ int xidx(int k, int w, int lane) { return 64 * (NW * k + w) + lane; }

template <int NW, int NK>
__device__ __forceinline__ bool repoll(uint64_t (&wd)[NK], const uint64_t* src, int n, uint32_t tag, int w, int lane) {
  bool ok = true;
#pragma unroll
  for (int k = 0; k < NK; ++k) {
    if (uint32_t(wd[k] >> 32) != tag) {
      ok = false;
      wd[k] = ld_tag(src + xidx<NW>(k, w, lane));
    }
  }
  return ok;
}

// The first round waits kFirstPoll s_sleep units (~0.4 us): the remote outputs cannot land
// sooner, and an early round over words still being written costs a full round trip
// (measured: 9% per token).
#ifndef MSD_FIRST_POLL
#define MSD_FIRST_POLL 16
#endif
constexpr int kFirstPoll = MSD_FIRST_POLL;
// Barrier after each phase's output stores, so that no wave's polls of the next vector enter
// the memory pipeline ahead of another wave's stores.
#ifndef MSD_STORE_BAR
#define MSD_STORE_BAR 1
#endif
constexpr bool kStoreBar = MSD_STORE_BAR != 0;
// s_sleep units between the polls of an LDS counter (0: spin; measured fastest)
#ifndef MSD_LDS_SLEEP
#define MSD_LDS_SLEEP 0
#endif
// The attention partials take the attention workgroups' gather and compute (a few us)
// before they can land, so that gather starts polling later.
#ifndef MSD_ATT_FIRST_POLL
#define MSD_ATT_FIRST_POLL 16
#endif
constexpr int kAttFirstPoll = MSD_ATT_FIRST_POLL;

template <int NW, int NK, int SLEEP = 0, int FIRST = kFirstPoll>
__device__ __forceinline__ void poll_words(const uint64_t* src, int n, uint32_t tag, float (&v)[NK],
                                           uint32_t* ctrl, int w, int lane, bool& bad) {
  uint64_t wd[NK];
  if constexpr (FIRST > 0) __builtin_amdgcn_s_sleep(FIRST > 127 ? 127 : FIRST);
  if constexpr (FIRST > 127) __builtin_amdgcn_s_sleep(FIRST - 127 > 127 ? 127 : FIRST - 127);
#pragma unroll
  for (int k = 0; k < NK; ++k) {
    const int i = xidx<NW>(k, w, lane);
    wd[k] = (i < n) ? ld_tag(src + i) : (uint64_t(tag) << 32);
  }
  uint32_t spins = 0;
  while (!bad && !__all(repoll<NW, NK>(wd, src, n, tag, w, lane))) {
    if constexpr (SLEEP > 0) __builtin_amdgcn_s_sleep(SLEEP);   // fewer polls during long waits
    spin_step(spins, ctrl, lane, bad);
  }
#pragma unroll
  for (int k = 0; k < NK; ++k) v[k] = __uint_as_float(uint32_t(wd[k]));
}

// LDS position of element e of a K-long vector in the lane-major order of the row dot
// products: in block b of 512 (the last block holds S = 8m elements, m lanes), element
// 512b + q m + l sits in lane l's 32 bytes at 512b + 8l, so lane l reads its 8 inputs of a block
// as two 16-byte pieces (the order of the kernel row layout's packed weights).  Lanes with bit 3
// set keep their two halves swapped (q at 8l + (q ^ 4)) and read the upper one first: the first
// read of lanes 0-7 then covers the even 16-byte bank groups and that of lanes 8-15 the odd ones.
// Measured with a probe of ds_read_b128 patterns (SQ_LDS_BANK_CONFLICT): reading 32-byte lane
// segments half by half takes twice the LDS cycles without the swap, none extra with it.
template <int K>
__device__ __forceinline__ int lane_major(int e) {
  const int b = e >> 9, r = e & 511;
  constexpr int mt = (K % 512) / 8;   // lanes of a short last block
  const int m = (mt > 0 && b == K / 512) ? mt : 64;
  const int q = m == 64 ? (r >> 6) : r / m;
  const int l = r - q * m;
  return (b << 9) + 8 * l + (q ^ (((l >> 3) & 1) << 2));
}

// Gather n tagged words src[0..n) into dst (LDS floats), NW waves sharing the words; with
// K > 0 the words land in the lane-major order of a K-long vector.
template <int NW, int NK, int SLEEP = 0, int FIRST = kFirstPoll, int K = 0>
__device__ __forceinline__ void gather_x(const uint64_t* src, int n, float* dst, uint32_t tag, uint32_t* ctrl,
                                         int w, int lane, bool& bad) {
  float v[NK];
  poll_words<NW, NK, SLEEP, FIRST>(src, n, tag, v, ctrl, w, lane, bad);
#pragma unroll
  for (int k = 0; k < NK; ++k) {
    const int i = xidx<NW>(k, w, lane);
    if (i < n) dst[K > 0 ? lane_major<K>(i) : i] = v[k];
  }
}

// Store R outputs of a wave (values y, word indices ix; the first nv are valid) to the
// exchange block X: one store instruction per output, lane r writing replica r (lane 0
// only when not replicated).
template <int R>
__device__ __forceinline__ void store_out(uint64_t* X, const float (&y)[R], const int (&ix)[R], int nv,
                                          bool replicated, int64_t x_rep, uint32_t tag, int lane) {
  const int nl = replicated ? kRep : 1;
#pragma unroll
  for (int j = 0; j < R; ++j)
    if (j < nv && lane < nl) st_tag(X + ix[j] + lane * x_rep, y[j], tag);
}

// LDS counters between the waves of one workgroup.
__device__ __forceinline__ int lds_ld(int* ctr) {
  return __hip_atomic_load(ctr, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP);
}
// Bounded like the cross-workgroup waits: every 1024 spins the wave checks the status word
// and gives up once a timeout has been reported; after kLdsSpinLimit spins it reports one.
constexpr uint32_t kLdsSpinLimit = 1u << 22;
__device__ __forceinline__ void lds_wait(int* ctr, int target, uint32_t* gctrl) {
  uint32_t spins = 0;
  while (lds_ld(ctr) < target) {
    if constexpr (MSD_LDS_SLEEP > 0) __builtin_amdgcn_s_sleep(MSD_LDS_SLEEP);
    if ((++spins & 1023u) == 0) {
      if (ld_status(gctrl) & kStatusTimeout) return;
      if (spins > kLdsSpinLimit) {
        atomicOr(gctrl, kStatusTimeout);
        return;
      }
    }
  }
}
// Bump after this wave's LDS writes are done (lgkmcnt(0)).
__device__ __forceinline__ void lds_bump(int* ctr, int lane) {
  __builtin_amdgcn_s_waitcnt(0xc07f);
  if (lane == 0) __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void lds_set(int* ctr, int v, int lane) {
  __builtin_amdgcn_s_waitcnt(0xc07f);
  if (lane == 0) __hip_atomic_store(ctr, v, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
}
// Barrier of n waves on an LDS counter; `phase` counts calls.
__device__ __forceinline__ void wsync(int* ctr, int& phase, int n, int lane, uint32_t* gctrl) {
  phase += n;
  lds_bump(ctr, lane);
  lds_wait(ctr, phase, gctrl);
}

// ---------------------------------------------------------------- LDS-DMA streaming
// global_load_lds_dwordx4: lane i copies 16 bytes from its global address to
// lds_base + 16 * i.  A loader keeps at most W instructions in flight.
__device__ __forceinline__ constexpr int vmcnt_imm(int k) {
  return (k & 0xF) | ((k >> 4) << 14) | (7 << 4) | (0xF << 8);
}
// Cache policy of the weight DMA.  The device's last-level cache (256 MB on MI355X) keeps
// whatever is read with the default policy; the whole model does not fit, so the rows of the
// first `keep` layers (as many as fit in kKeepBytes, leaving room for the KV cache) are read
// with the default policy and stay cached from one step to the next, and every other weight
// row is read non-temporal (nt) so that it streams past without evicting them.
#ifndef MSD_DMA_AUX
#define MSD_DMA_AUX 2
#endif
constexpr int kAuxKeep = 0;
#ifndef MSD_KEEP_MB
#define MSD_KEEP_MB 230
#endif
constexpr int64_t kKeepBytes = int64_t(MSD_KEEP_MB) << 20;
template <int W, int AUX = 0>
struct Dma {
  int inflight = 0;
  __device__ __forceinline__ void issue(const void* src, uint8_t* lds_base) {
    __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)lds_base, 16, 0, AUX);
    if (++inflight == W) {
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(W - 1));
      inflight = W - 1;
    }
  }
  __device__ __forceinline__ void drain() {
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    inflight = 0;
  }
};

// Copy `bytes` (a multiple of 16) from src to lds: instruction t covers bytes
// [1024 t, 1024 t + 1024); lanes past the end re-read the last 16 bytes into the
// padding that rounds every region up to 1 KB.
template <int W, int AUX>
__device__ __forceinline__ void dma_copy(Dma<W, AUX>& d, const uint8_t* src, uint8_t* lds, int64_t bytes, int lane) {
  for (int64_t t = 0; t * 1024 < bytes; ++t) {
    int64_t o = t * 1024 + 16 * lane;
    if (o > bytes - 16) o = bytes - 16;
    d.issue(src + o, lds + t * 1024);
  }
}

// ---------------------------------------------------------------- row dot products
// Row layout: a row of K bf16 values is cut into blocks of 512 (the last block may be
// shorter: S = 8*m values, m lanes); in block b, lane l holds the 16 bytes at packed
// offset 512*b + 8*l, and its k-th value (k < 8) multiplies input element 512*b + k*m + l.
// The packer applies that in-dimension permutation to every row, so the lane's 8 inputs
// are x[512*b + k*m + l]: consecutive lanes read consecutive LDS words (no bank conflicts)
// and each lane keeps its inputs in registers for all rows of a phase.
template <int NL>
struct XV {
  float v[NL][8];
};

__device__ __forceinline__ int block_lanes(int k, int b) {
  const int rem = k - 512 * b;
  return rem >= 512 ? 64 : (rem > 0 ? rem / 8 : 0);
}

// The lane's inputs of a K-long vector held in LDS in lane-major order (lane_major<K>).
template <int NL>
__device__ __forceinline__ void load_x(XV<NL>& xv, const float* x, int k, int lane) {
#pragma unroll
  for (int j = 0; j < NL; ++j) {
    const int m = block_lanes(k, j);
    const int sw = (lane >> 3) & 1;   // this lane's halves are stored swapped (lane_major)
    const float4* p = reinterpret_cast<const float4*>(x + 512 * j + 8 * (lane < m ? lane : 0));
    const float4 a = p[sw], b = p[1 - sw];
    const bool on = lane < m;
    xv.v[j][0] = on ? a.x : 0.f;
    xv.v[j][1] = on ? a.y : 0.f;
    xv.v[j][2] = on ? a.z : 0.f;
    xv.v[j][3] = on ? a.w : 0.f;
    xv.v[j][4] = on ? b.x : 0.f;
    xv.v[j][5] = on ? b.y : 0.f;
    xv.v[j][6] = on ? b.z : 0.f;
    xv.v[j][7] = on ? b.w : 0.f;
  }
}

// Dot products of R rows with the lane's inputs from the rows' 16-byte pieces w (lanes past a
// short last block hold bytes beyond the row, zeroed here); the R wave sums run interleaved.
template <int NL, int R>
__device__ __forceinline__ void dot_frags(const uint4 (&w)[R][NL], const XV<NL>& xv, int k, int lane,
                                          float (&out)[R]) {
#pragma unroll
  for (int i = 0; i < R; ++i) {
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < NL; ++j) {
      uint4 u = w[i][j];
      if (lane >= block_lanes(k, j)) u = make_uint4(0, 0, 0, 0);
      acc += bf_lo(u.x) * xv.v[j][0];
      acc += bf_hi(u.x) * xv.v[j][1];
      acc += bf_lo(u.y) * xv.v[j][2];
      acc += bf_hi(u.y) * xv.v[j][3];
      acc += bf_lo(u.z) * xv.v[j][4];
      acc += bf_hi(u.z) * xv.v[j][5];
      acc += bf_lo(u.w) * xv.v[j][6];
      acc += bf_hi(u.w) * xv.v[j][7];
    }
    out[i] = acc;
  }
  wave_sum_n<R>(out);
}

// Dot products of R rows (in LDS) with the lane's inputs: every 16-byte piece of every row
// is read before the first multiply.  Lanes past a short last block read in-bounds LDS bytes
// beyond the row.
template <int NL, int R>
__device__ __forceinline__ void dot_rows(const uint8_t* const (&rows)[R], const XV<NL>& xv, int k, int lane,
                                         float (&out)[R]) {
  uint4 w[R][NL];
#pragma unroll
  for (int i = 0; i < R; ++i)
#pragma unroll
    for (int j = 0; j < NL; ++j) w[i][j] = *reinterpret_cast<const uint4*>(rows[i] + 1024 * j + 16 * lane);
  dot_frags<NL, R>(w, xv, k, lane, out);
}

// The value through an empty asm: the compiler can neither fold it nor hoist what depends on it
// out of a loop (where it would hold registers for the whole loop).
__device__ __forceinline__ int opaque(int v) {
  asm volatile("" : "+v"(v));
  return v;
}

// Loads the 16-byte pieces of R rows of the output projection (rows r + S i, clamped to r1 - 1)
// straight from memory, with the streaming policy; lanes past a short last block read the
// row's first piece instead (zeroed by dot_frags).  The addresses are formed at the call.
template <int NL, int R, int S>
__device__ __forceinline__ void load_frags(const uint16_t* outp, int D, int r, int r1, int lane_, uint4 (&w)[R][NL]) {
  const int lane = opaque(lane_);
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const uint8_t* row = reinterpret_cast<const uint8_t*>(outp + int64_t(min(r + S * i, r1 - 1)) * D);
#pragma unroll
    for (int j = 0; j < NL; ++j) {
      const int off = lane < block_lanes(D, j) ? 1024 * j + 16 * lane : 0;
      typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
      const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(row + off));
      w[i][j] = make_uint4(v[0], v[1], v[2], v[3]);
    }
  }
}

// dot_rows with one more wave sum taken in the same reduction chain: out[R] = sum over the
// wave of `extra` (the lane's partial sum of squares of a folded RMSNorm).
template <int NL, int R>
__device__ __forceinline__ void dot_rows_x(const uint8_t* const (&rows)[R], const XV<NL>& xv, int k, int lane,
                                           float extra, float (&out)[R + 1]) {
  uint4 w[R][NL];
#pragma unroll
  for (int i = 0; i < R; ++i)
#pragma unroll
    for (int j = 0; j < NL; ++j) w[i][j] = *reinterpret_cast<const uint4*>(rows[i] + 1024 * j + 16 * lane);
#pragma unroll
  for (int i = 0; i < R; ++i) {
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < NL; ++j) {
      uint4 u = w[i][j];
      if (lane >= block_lanes(k, j)) u = make_uint4(0, 0, 0, 0);
      acc += bf_lo(u.x) * xv.v[j][0];
      acc += bf_hi(u.x) * xv.v[j][1];
      acc += bf_lo(u.y) * xv.v[j][2];
      acc += bf_hi(u.y) * xv.v[j][3];
      acc += bf_lo(u.z) * xv.v[j][4];
      acc += bf_hi(u.z) * xv.v[j][5];
      acc += bf_lo(u.w) * xv.v[j][6];
      acc += bf_hi(u.w) * xv.v[j][7];
    }
    out[i] = acc;
  }
  out[R] = extra;
  wave_sum_n<R + 1>(out);
}

// RMSNorm folded into R row dot products (model.py:94-98): the rows multiply sc * h, the sum
// of squares of h is reduced in the same chain, and the outputs are scaled by
// 1 / sqrt(mean(h^2) + eps) afterwards, so the dot products do not wait for the norm.
template <int NL, int R>
__device__ __forceinline__ void normed_dots(const uint8_t* const (&rows)[R], const XV<NL>& h, const XV<NL>& sc, int k,
                                            int lane, float (&out)[R]) {
  XV<NL> x;
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < NL; ++j)
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      ss += h.v[j][q] * h.v[j][q];
      x.v[j][q] = sc.v[j][q] * h.v[j][q];
    }
  float t[R + 1];
  dot_rows_x<NL, R>(rows, x, k, lane, ss, t);
  const float inv = 1.f / sqrtf(t[R] / float(k) + 1e-5f);
#pragma unroll
  for (int i = 0; i < R; ++i) out[i] = t[i] * inv;
}

__device__ __forceinline__ void split(int total, int parts, int idx, int& lo, int& hi) {
  lo = int((int64_t(total) * idx) / parts);
  hi = int((int64_t(total) * (idx + 1)) / parts);
}

__device__ __forceinline__ uint64_t argmax_key(float v, int idx) {
  uint32_t u = __float_as_uint(v);
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return (uint64_t(u) << 32) | uint64_t(0xffffffffu - uint32_t(idx));
}

__device__ __forceinline__ uint64_t* layer_x(const Args& a, int l) { return a.xw + int64_t(l) * a.lay.x_layer; }
__device__ __forceinline__ const uint16_t* layer_w(const Args& a, int l) { return a.w + int64_t(l) * a.lay.layer_elems; }
__device__ __forceinline__ uint16_t* layer_k(const Args& a, int l) { return a.kv + int64_t(l) * 2 * a.KV * a.ctx * kDh; }

// Token words: the last arriver of step s stores (epoch + s | argmax) to kTokReps replicas, which
// the next step's workgroups poll (a replica per 16 workgroups: fewer pollers per address).
constexpr int kTokReps = 16;
__device__ __forceinline__ uint64_t* tok_words(const Args& a) { return reinterpret_cast<uint64_t*>(a.ctrl + 16); }
// Wait for step s's token (tag epoch + s) on replica `rep`; returns it (0 if the wait ran out).
__device__ __forceinline__ int poll_token(const Args& a, int s, int rep, int lane, bool& bad) {
  const uint32_t want = a.epoch + uint32_t(s);
  const uint64_t* src = tok_words(a) + rep % kTokReps;
  uint64_t w = ld_tag(src);
  uint32_t spins = 0;
  while (!bad && uint32_t(w >> 32) != want) {
    spin_step(spins, a.ctrl, lane, bad);
    w = ld_tag(src);
  }
  return uint32_t(w >> 32) == want ? int(uint32_t(w)) : 0;
}

// ---------------------------------------------------------------- row workgroups
// Shared state of a row workgroup (LDS pointers, row ranges).
struct RowCtx {
  int wr, lane, wv;
  int qp0, qp1, or0, or1, f0, f1, v0, v1;   // QKV pairs, O/down rows, gate/up pairs, vocabulary rows
  uint8_t* ring;
  float* xatt;    // attention vector (input of the O rows)
  float* xhd1;    // O output (gathered)
  float* xact;    // SwiGLU activation (input of the down rows)
  float* xhd2;    // down output (gathered)
  float* xa;      // gathered attention partials
  int* ctr;       // [0] worker barrier, [4] ring jobs consumed (worker bumps), [5] ring jobs loaded,
                  // [6] the step's input token
  float* red_v;   // argmax per worker wave
  int* red_i;
};
enum { kCtrBar = 0, kCtrUsed = 4, kCtrLoaded = 5, kCtrTok = 6 };

// Loader wave of a row workgroup.  Jobs in order, per step: per layer the QKV, O, gate/up and
// down rows of this workgroup, into their fixed ring regions (the worker waves stream the logit
// rows themselves).  Job j may overwrite its region once the job that last used it has been
// consumed by all compute waves (a step's first job: every job of the previous step).  Job
// indices run on across the steps of a launch, as do the LDS counters.
template <int D, int FF, bool MULTI>
__device__ void row_loader(const Args& a, const RowCtx& c) {
  const Layout& lay = a.lay;
  const int lane = c.lane;
  Dma<kDmaLayer, MSD_DMA_AUX> d;
  Dma<kDmaLayer, kAuxKeep> dk;
  Dma<kDmaFirst, kAuxKeep> d0;
  const int njobs = 4 * a.L;
  const int nsteps = MULTI ? a.nsteps : 1;
  for (int st = 0; st < nsteps; ++st) {
    const int base = st * njobs;
    for (int j = 0; j < njobs; ++j) {
      const uint16_t* src;
      int64_t bytes;
      int off, need;
      {
        const int l = j / 4, p = j % 4;
        const uint16_t* w = layer_w(a, l);
        if (p == 0) { src = w + lay.off_qkv + int64_t(2 * c.qp0) * D; bytes = int64_t(2 * (c.qp1 - c.qp0)) * D * 2; off = a.ring_q; }
        else if (p == 1) { src = w + lay.off_o + int64_t(c.or0) * D; bytes = int64_t(c.or1 - c.or0) * D * 2; off = a.ring_o; }
        else if (p == 2) { src = w + lay.off_gu + int64_t(2 * c.f0) * D; bytes = int64_t(2 * (c.f1 - c.f0)) * D * 2; off = a.ring_g; }
        else { src = w + lay.off_dn + int64_t(c.or0) * FF; bytes = int64_t(c.or1 - c.or0) * FF * 2; off = a.ring_d; }
        // job j - 4 (same region, previous layer) consumed; a step's first layer: the whole
        // previous step
        need = l == 0 ? base : base + j - 3;
      }
      if (need > 0 && lds_ld(c.ctr + kCtrUsed) < kWavesR * need) lds_wait(c.ctr + kCtrUsed, kWavesR * need, a.ctrl);
      if (bytes > 0) {
        if (j < 4 && a.keep > 0) {
          dma_copy(d0, reinterpret_cast<const uint8_t*>(src), c.ring + off, bytes, lane);
          d0.drain();
        } else if (j < 4 * a.keep) {
          dma_copy(dk, reinterpret_cast<const uint8_t*>(src), c.ring + off, bytes, lane);
          dk.drain();
        } else {
          dma_copy(d, reinterpret_cast<const uint8_t*>(src), c.ring + off, bytes, lane);
          d.drain();
        }
      }
      lds_set(c.ctr + kCtrLoaded, base + j + 1, lane);
      MSD_TRACE_POINT(st == 0, j / 4, 28 + (j % 4));
    }
  }
}

// Worker waves of a row workgroup (8 waves; the loader wave streams the weights).  Every
// worker keeps the residual stream h in registers in the lane layout of the row dot
// products (lane l holds elements 512 j + k m + l), so each takes the RMSNorms itself with
// one wave reduction.  Per phase every worker takes the dot products of its rows
// (workgroup-local items w, w + 8, ...; at most QPW QKV pairs, ORW O/down rows and GPW
// gate/up pairs), stores the outputs to the exchange words, and once all workers have
// stored (so this workgroup's stores never queue behind its own polls) the workers gather
// the next vector, each an eighth of its words, into LDS.  Workgroup-local barriers are LDS
// counters among the 8 workers.
template <int D, int FF, int QPW, int ORW, int GPW, bool MULTI>
__device__ void row_worker(const Args& a, const RowCtx& c, int token) {
  constexpr int NLD = (D + 511) / 512;
  constexpr int NLF = (FF + 511) / 512;
  constexpr int HPW = (D + 64 * kWavesR - 1) / (64 * kWavesR);    // d-vector words per lane
  constexpr int NKF = (FF + 64 * kWavesR - 1) / (64 * kWavesR);   // act words per lane
  constexpr int H = D / kDh;
  constexpr int NKA2 = (2 * H * kPart + 64 * kWavesR - 1) / (64 * kWavesR);   // 2 splits
  const int lane = c.lane, wv = c.wv;
  const Layout& lay = a.lay;
  bool bad = false;
  int bars = 0;
  auto bar = [&]() { wsync(c.ctr + kCtrBar, bars, kWavesR, lane, a.ctrl); };
  const int64_t myrep = int64_t(c.wr % kRep) * lay.x_rep;
  const int natt = a.H * a.nsplit;
  const int nq = c.qp1 - c.qp0, no = c.or1 - c.or0, ng = c.f1 - c.f0;
  float cs[QPW], sn[QPW];   // rotary factors of this wave's QKV pairs (q/k rows) at the step's position
  // residual stream and RMSNorm scales in the lane layout
  auto load_vec = [&](XV<NLD>& v, const uint16_t* src) {
#pragma unroll
    for (int j = 0; j < NLD; ++j) {
      const int m = block_lanes(D, j);
#pragma unroll
      for (int q = 0; q < 8; ++q) v.v[j][q] = (lane < m) ? bf2f(src[512 * j + q * m + lane]) : 0.f;
    }
  };
  XV<NLD> h, sc;
  auto add_res = [&](const float* buf) {   // h += gathered output
    XV<NLD> t;
    load_x(t, buf, D, lane);
#pragma unroll
    for (int j = 0; j < NLD; ++j)
#pragma unroll
      for (int q = 0; q < 8; ++q) h.v[j][q] = h.v[j][q] + t.v[j][q];
  };
  // x = sc * h * (1 / sqrt(mean(h^2) + eps)): model.py:94-98, with the reciprocal taken once
  // as the reference kernel does (multi_sm_decode.py:122-126 multiplies by rsqrt)
  auto norm = [&](XV<NLD>& x) {
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < NLD; ++j)
#pragma unroll
      for (int q = 0; q < 8; ++q) ss += h.v[j][q] * h.v[j][q];
    ss = wave_sum(ss);
    const float inv = 1.f / sqrtf(ss / float(D) + 1e-5f);
#pragma unroll
    for (int j = 0; j < NLD; ++j)
#pragma unroll
      for (int q = 0; q < 8; ++q) x.v[j][q] = sc.v[j][q] * (h.v[j][q] * inv);
  };
  auto weights = [&](int job) { lds_wait(c.ctr + kCtrLoaded, job + 1, a.ctrl); };
  auto release = [&]() { lds_bump(c.ctr + kCtrUsed, lane); };
  // LDS row of workgroup-local item rel (the region's first row when rel is past the end)
  auto at = [&](int region, int rel, int n, int item_bytes) {
    return c.ring + region + int64_t(rel < n ? rel : 0) * item_bytes;
  };
  auto count = [&](int n, int cap) {   // this wave's items among n (items w, w + 8, ...)
    return n > wv ? min(cap, (n - wv + kWavesR - 1) / kWavesR) : 0;
  };
  const int njobs = 4 * a.L;
  const int nsteps = MULTI ? a.nsteps : 1;

  for (int st = 0; st < nsteps; ++st) {
    const int pos = a.pos + st;
    const uint32_t tag = a.epoch + uint32_t(st);
    const int jb = st * njobs;   // this step's first ring job
    if (st > 0) {
      // the input token is the previous step's argmax, published by its last arriver
      if (wv == 0) {
        const int t = poll_token(a, st - 1, c.wr, lane, bad);
        if (lane == 0) {
          c.ctr[kCtrTok] = t;
          if (c.wr == 0) {   // step start (as the kernel entry does for step 0)
            __hip_atomic_store(a.ctrl + 1, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(reinterpret_cast<uint64_t*>(a.ctrl + 2), uint64_t(0), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
            atomicAnd(a.ctrl, ~kStatusBadToken);
            put_out(a.next_token + 2 * st + 1, int32_t(kStatusUnfinished));
            __builtin_amdgcn_s_waitcnt(0);
          }
        }
      }
      bar();
      token = __hip_atomic_load(c.ctr + kCtrTok, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
#pragma unroll
    for (int i = 0; i < QPW; ++i) {
      cs[i] = 1.f;
      sn[i] = 0.f;
      const int rel = wv + kWavesR * i;
      if (rel < nq) {
        const int row = 2 * (c.qp0 + rel);
        if (row / kDh < a.H + a.KV) {
          const float* rope = a.rope + int64_t(pos) * kDh + (row % kDh) / 2;
          cs[i] = rope[0];
          sn[i] = rope[kDh / 2];
        }
      }
    }
    load_vec(h, a.emb + int64_t(token) * D);
    load_vec(sc, layer_w(a, 0) + lay.off_ln1);

    for (int l = 0; l < a.L; ++l) {
      uint64_t* X = layer_x(a, l);
      uint16_t* kcache = layer_k(a, l);
      uint16_t* vcache = kcache + int64_t(a.KV) * a.ctx * kDh;
      // ---- h += down output of the previous layer; x = rmsnorm1(h); QKV rows, RoPE, KV write
      //      (multi_sm_decode.py:121-180)
      if (l > 0) {
        gather_x<kWavesR, HPW, 0, kFirstPoll, D>(layer_x(a, l - 1) + lay.x_hd2 + myrep, D, c.xhd2, tag, a.ctrl, wv, lane, bad);
        bar();
        add_res(c.xhd2);
        MSD_TRACE_POINT(wv == 0, l - 1, 6);
      }
      weights(jb + 4 * l);
      MSD_TRACE_POINT(wv == 0, l, 16);
      {
        MSD_TRACE_POINT(wv == 0, l, 11);
        const uint8_t* rows[2 * QPW];
#pragma unroll
        for (int i = 0; i < QPW; ++i) {
          rows[2 * i] = at(a.ring_q, wv + kWavesR * i, nq, 2 * D * 2);
          rows[2 * i + 1] = rows[2 * i] + D * 2;
        }
        float sd[2 * QPW] = {};
        // idle waves leave the SIMD to others
        if (count(nq, QPW) > 0) normed_dots<NLD, 2 * QPW>(rows, h, sc, D, lane, sd);
        MSD_TRACE_POINT(wv == 0, l, 14);
        release();
        float y[2 * QPW];
        int ix[2 * QPW];
#pragma unroll
        for (int i = 0; i < QPW; ++i) {
          const int rel = wv + kWavesR * i;
          const int row = 2 * (c.qp0 + (rel < nq ? rel : 0));
          const int head = row / kDh;
          const int rr = row % kDh;
          const float s0 = sd[2 * i], s1 = sd[2 * i + 1];
          if (head < a.H + a.KV) {  // q or k rows (i, i+32): rotate-half RoPE (model.py:110-117)
            y[2 * i] = s0 * cs[i] - s1 * sn[i];
            y[2 * i + 1] = s0 * sn[i] + s1 * cs[i];
            ix[2 * i] = head * kDh + rr / 2;
            ix[2 * i + 1] = ix[2 * i] + kDh / 2;
          } else {
            y[2 * i] = s0;
            y[2 * i + 1] = s1;
            ix[2 * i] = head * kDh + rr;
            ix[2 * i + 1] = ix[2 * i] + 1;
          }
        }
        store_out<2 * QPW>(X + lay.x_qkv, y, ix, 2 * count(nq, QPW), false, lay.x_rep, tag, lane);
        {
          // K (post-RoPE) and V rows of the cache at pos, bf16 (multi_sm_decode.py:179-180), after
          // the exchange stores: the attention workgroups wait for k and v, not for the cache
#pragma unroll
          for (int i = 0; i < QPW; ++i) {
            const int rel = wv + kWavesR * i;
            const int row = 2 * (c.qp0 + (rel < nq ? rel : 0));
            const int head = row / kDh;
            if (rel < nq && head >= a.H && lane == 0) {
              const bool isv = head >= a.H + a.KV;
              const int kvh = isv ? head - a.H - a.KV : head - a.H;
              uint16_t* cp = (isv ? vcache : kcache) + (int64_t(kvh) * a.ctx + pos) * kDh;
              if constexpr (MULTI) {
                __hip_atomic_store(cp + (ix[2 * i] - head * kDh), f2bf(y[2 * i]), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(cp + (ix[2 * i + 1] - head * kDh), f2bf(y[2 * i + 1]), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
              } else {
                cp[ix[2 * i] - head * kDh] = f2bf(y[2 * i]);
                cp[ix[2 * i + 1] - head * kDh] = f2bf(y[2 * i + 1]);
              }
            }
          }
        }
      }
      load_vec(sc, layer_w(a, l) + lay.off_ln2);   // scale of the next norm
      if constexpr (kStoreBar) bar();   // every QKV output of this workgroup is issued
      MSD_TRACE_POINT(wv == 0, l, 17);
      // ---- attention vector (multi_sm_decode.py:243-259): with one split the attention
      //      workgroups publish each head's normalised output, gathered straight into xatt;
      //      with several, the (head, split) partials are merged here by log-sum-exp
      if (a.nsplit == 1) {
        gather_x<kWavesR, HPW, 0, kAttFirstPoll, D>(X + lay.x_att + myrep, D, c.xatt, tag, a.ctrl, wv, lane, bad);
        MSD_TRACE_POINT(wv == 0, l, 3);
      } else {
        // in pieces of at most two splits' words (four splits: two pieces)
        const int nw = natt * kPart, piece = 2 * a.H * kPart;
        for (int b = 0; b < nw; b += piece)
          gather_x<kWavesR, NKA2, 0, kAttFirstPoll>(X + lay.x_att + myrep + b, min(piece, nw - b), c.xa + b, tag,
                                                    a.ctrl, wv, lane, bad);
        MSD_TRACE_POINT(wv == 0, l, 3);
        bar();
        MSD_TRACE_POINT(wv == 0, l, 4);
        for (int i = wv * 64 + lane; i < D; i += kWavesR * 64) {
          const int hd = i / kDh, dim = i % kDh;
          float M = -INFINITY;
          for (int s = 0; s < a.nsplit; ++s) {
            const float* ps = c.xa + (hd * a.nsplit + s) * kPart;
            if (ps[1] > 0.f) M = fmaxf(M, ps[0]);
          }
          float num = 0.f, den = 0.f;
          for (int s = 0; s < a.nsplit; ++s) {
            const float* ps = c.xa + (hd * a.nsplit + s) * kPart;
            if (ps[1] > 0.f) {
              const float wgt = expf(ps[0] - M);
              num += wgt * ps[2 + dim];
              den += wgt * ps[1];
            }
          }
          c.xatt[lane_major<D>(i)] = den > 0.f ? num / den : 0.f;
        }
      }
      bar();
      MSD_TRACE_POINT(wv == 0, l, 1);
      // ---- O rows (multi_sm_decode.py:223-232)
      weights(jb + 4 * l + 1);
      MSD_TRACE_POINT(wv == 0, l, 18);
      {
        XV<NLD> xv;
        load_x(xv, c.xatt, D, lane);
        const uint8_t* rows[ORW];
        int ix[ORW];
#pragma unroll
        for (int i = 0; i < ORW; ++i) {
          rows[i] = at(a.ring_o, wv + kWavesR * i, no, D * 2);
          ix[i] = int(lay.x_hd1) + c.or0 + wv + kWavesR * i;
        }
        float y[ORW] = {};
        if (count(no, ORW) > 0) dot_rows<NLD, ORW>(rows, xv, D, lane, y);
        release();
        store_out<ORW>(X, y, ix, count(no, ORW), true, lay.x_rep, tag, lane);
      }
      if constexpr (kStoreBar) bar();
      MSD_TRACE_POINT(wv == 0, l, 19);
      // ---- h += O output; x = rmsnorm2(h); gate/up rows + SwiGLU (multi_sm_decode.py:262-289, model.py:159)
      gather_x<kWavesR, HPW, 0, kFirstPoll, D>(X + lay.x_hd1 + myrep, D, c.xhd1, tag, a.ctrl, wv, lane, bad);
      bar();
      MSD_TRACE_POINT(wv == 0, l, 2);
      add_res(c.xhd1);
      weights(jb + 4 * l + 2);
      MSD_TRACE_POINT(wv == 0, l, 20);
      MSD_TRACE_WAVE(l, 0);
      {
        MSD_TRACE_POINT(wv == 0, l, 8);
        MSD_TRACE_WAVE(l, 1);
        const uint8_t* rows[2 * GPW];
        int ix[GPW];
#pragma unroll
        for (int i = 0; i < GPW; ++i) {
          rows[2 * i] = at(a.ring_g, wv + kWavesR * i, ng, 2 * D * 2);
          rows[2 * i + 1] = rows[2 * i] + D * 2;
          ix[i] = int(lay.x_act) + c.f0 + wv + kWavesR * i;
        }
        float gu[2 * GPW] = {};
        if (count(ng, GPW) > 0) normed_dots<NLD, 2 * GPW>(rows, h, sc, D, lane, gu);
        MSD_TRACE_POINT(wv == 0, l, 9);
        MSD_TRACE_WAVE(l, 2);
        release();
        float y[GPW];
#pragma unroll
        for (int i = 0; i < GPW; ++i) {
          const float gt = gu[2 * i], up = gu[2 * i + 1];
          y[i] = (gt * (1.f / (1.f + expf(-gt)))) * up;
        }
        store_out<GPW>(X, y, ix, count(ng, GPW), true, lay.x_rep, tag, lane);
        MSD_TRACE_POINT(wv == 0, l, 10);
        MSD_TRACE_WAVE(l, 3);
      }
      if constexpr (kStoreBar) bar();
      MSD_TRACE_WAVE(l, 4);
      MSD_TRACE_POINT(wv == 0, l, 21);
      // ---- act -> LDS; down rows (multi_sm_decode.py:273-291)
      gather_x<kWavesR, NKF, 0, kFirstPoll, FF>(X + lay.x_act + myrep, a.ff, c.xact, tag, a.ctrl, wv, lane, bad);
      bar();
      MSD_TRACE_POINT(wv == 0, l, 5);
      weights(jb + 4 * l + 3);
      MSD_TRACE_POINT(wv == 0, l, 22);
      {
        XV<NLF> xv;
        load_x(xv, c.xact, FF, lane);
        const uint8_t* rows[ORW];
        int ix[ORW];
#pragma unroll
        for (int i = 0; i < ORW; ++i) {
          rows[i] = at(a.ring_d, wv + kWavesR * i, no, FF * 2);
          ix[i] = int(lay.x_hd2) + c.or0 + wv + kWavesR * i;
        }
        float y[ORW] = {};
        if (count(no, ORW) > 0) dot_rows<NLF, ORW>(rows, xv, FF, lane, y);
        MSD_TRACE_POINT(wv == 0, l, 15);
        release();
        store_out<ORW>(X, y, ix, count(no, ORW), true, lay.x_rep, tag, lane);
      }
      load_vec(sc, l + 1 < a.L ? layer_w(a, l + 1) + lay.off_ln1 : a.lnf);   // scale of the next norm
      if constexpr (kStoreBar) bar();
      MSD_TRACE_POINT(wv == 0, l, 23);
    }
    // ---- h += last down output; x = final rmsnorm(h); tied logits over this workgroup's
    //      vocabulary rows (multi_sm_decode.py:314-337).  Each worker wave streams its rows
    //      (v0 + w, v0 + w + 8, ...) from memory straight into registers, RB rows per batch with
    //      the next batch in flight (two register sets taken in turn); the first batch is
    //      requested before the last down vector is gathered, as it does not depend on it.  A
    //      launch of several steps holds more state across the step loop: one row per batch.
    constexpr int RB = MULTI ? 1 : 2;    // rows per batch
    constexpr int SB = kWavesR * RB;     // rows between a wave's consecutive batches
    uint4 wa[RB][NLD], wb[RB][NLD];
    if (c.v0 + wv < c.v1) load_frags<NLD, RB, kWavesR>(a.outp, D, c.v0 + wv, c.v1, lane, wa);
    gather_x<kWavesR, HPW, 0, kFirstPoll, D>(layer_x(a, a.L - 1) + lay.x_hd2 + myrep, D, c.xhd2, tag, a.ctrl, wv, lane, bad);
    bar();
    MSD_TRACE_POINT(wv == 0, a.L - 1, 6);
    add_res(c.xhd2);
    XV<NLD> xv;
    norm(xv);
    float best = -INFINITY;
    int besti = 0x7fffffff;
    auto take = [&](const uint4 (&w)[RB][NLD], int r) {   // rows r + kWavesR i
      float y[RB];
      dot_frags<NLD, RB>(w, xv, D, lane, y);
#pragma unroll
      for (int i = 0; i < RB; ++i) {
        const int row = r + kWavesR * i;
        if (row < c.v1) {
          if (lane == 0) a.logits[st * a.logits_stride + row] = y[i];
          if (y[i] > best) { best = y[i]; besti = row; }
        }
      }
    };
    for (int r = c.v0 + wv; r < c.v1; r += 2 * SB) {
      if (r + SB < c.v1) load_frags<NLD, RB, kWavesR>(a.outp, D, r + SB, c.v1, lane, wb);
      take(wa, r);
      if (r + SB >= c.v1) break;
      if (r + 2 * SB < c.v1) load_frags<NLD, RB, kWavesR>(a.outp, D, r + 2 * SB, c.v1, lane, wa);
      take(wb, r + SB);
    }
    MSD_TRACE_POINT(wv == 0, a.L, 1);
    if (lane == 0) {
      c.red_v[wv] = best;
      c.red_i[wv] = besti;
    }
    // every store of this wave (cache rows, logits) completes before the arrival below, so the
    // next step of the launch, which starts after the last arrival, sees them
    if constexpr (MULTI) __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    bar();
    MSD_TRACE_POINT(wv == 0, a.L, 12);
    if (wv == 0 && lane == 0) {   // argmax: larger value wins, ties -> lower index (np.argmax)
      float bv = c.red_v[0];
      int bi = c.red_i[0];
      for (int w = 1; w < kWavesR; ++w) {
        const float v = c.red_v[w];
        const int i = c.red_i[w];
        if (v > bv || (v == bv && i < bi)) { bv = v; bi = i; }
      }
      uint64_t* keyp = reinterpret_cast<uint64_t*>(a.ctrl + 2);
      if (bi != 0x7fffffff)
        __hip_atomic_fetch_max(keyp, argmax_key(bv, bi), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      // the max above completes before the arrival below is issued
      __builtin_amdgcn_s_waitcnt(0);
      // The counter and the key were reset by workgroup 0 at the start of this step (before
      // any of its outputs, which every arrival here depends on), so exactly one arrival sees
      // GR - 1, whatever the counter held before the step.
      const uint32_t old = __hip_atomic_fetch_add(a.ctrl + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (old == uint32_t(a.GR - 1)) {   // last arriver publishes the token and the status
        const uint64_t key = __hip_atomic_load(keyp, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const uint32_t tok = 0xffffffffu - uint32_t(key & 0xffffffffu);
        put_out(a.next_token + 2 * st, int32_t(tok));
        put_out(a.next_token + 2 * st + 1, int32_t(ld_status(a.ctrl)));
        if (MULTI && st + 1 < nsteps)
          for (int r = 0; r < kTokReps; ++r) st_tag(tok_words(a) + r, __uint_as_float(tok), tag);
      }
    }
  }   // steps
}

// ---------------------------------------------------------------- attention workgroups
// One query head h and one split s of the context: cached positions [lo, lo + cap) below
// pos, plus the current position when it falls in the split (multi_sm_decode.py:182-221).
struct AttCtx {
  int h, g, split, item, lane, wv;
  bool has_cur;
  int64_t part;     // word offset of this head's output (one split) or (head, split)'s partials
  uint8_t* K;       // cap rows of kKRowB bytes (bf16 K, post-RoPE)
  uint8_t* V;       // cap rows of kVRowB bytes
  uint16_t* apw;    // [kWavesA][3][64]: each wave's q as three bf16 parts (A-operand staging)
  float* pw;        // [kWavesA][64]: each wave's softmax weights in P.V order
  float* ow;        // [2][kWavesA][64] block outputs (double-buffered by layer parity)
  float* mw;        // [2][kWavesA] block maxima
  float* lw;        // [2][kWavesA] block sums
  float* kvl;       // [2][2][64] the current position's k and v (double-buffered by layer parity)
  int* ctr;         // [0] wave sync, [1] KV layers loaded, [2] KV layers consumed (wave bumps),
                    // [3] layers whose current k and v are in kvl, [4] layers whose q wave 0 has
                    // received
};

// Loader wave of an attention workgroup: per layer, once every attention wave has
// finished with the previous layer's rows, DMA this split's cached K rows (kKSlots slots of
// 16 bytes per row; those past the 8th are padding) and V rows (8 slots) into LDS.
template <class DMA>
__device__ __forceinline__ void att_copy(DMA& d, const Args& a, const AttCtx& c, int l, int lo, int ncached) {
  const int lane = c.lane;
  const uint16_t* kc = layer_k(a, l) + (int64_t(c.g) * a.ctx + lo) * kDh;
  const uint16_t* vc = kc + int64_t(a.KV) * a.ctx * kDh;
  const int nk = cdiv(ncached * kKSlots, 64);
  for (int t = 0; t < nk; ++t) {
    const int i = 64 * t + lane;
    const int r = min(i / kKSlots, ncached - 1), p = min(i % kKSlots, 7);
    d.issue(kc + r * kDh + p * 8, c.K + t * 1024);
  }
  const int nv = cdiv(ncached, 8);
  for (int t = 0; t < nv; ++t) {
    const int i = 64 * t + lane;
    const int r = min(i / 8, ncached - 1), p = i % 8;
    d.issue(vc + r * kDh + p * 8, c.V + t * 1024);
  }
  d.drain();
}

// One more cached row, row `r` of this split (whose rows 0 .. r - 1 att_copy has placed), to its
// place after them: K at kKRowB r (lanes 0..kKSlots-1, one 16-byte slot each, those past the 8th
// repeating it) and V at 128 r (lanes 0..7).  Issued after att_copy's drain, so these writes land
// last.
template <class DMA>
__device__ __forceinline__ void att_copy_row(DMA& d, const Args& a, const AttCtx& c, int l, int lo, int r) {
  const int lane = c.lane;
  const uint16_t* kc = layer_k(a, l) + (int64_t(c.g) * a.ctx + lo + r) * kDh;
  const uint16_t* vc = kc + int64_t(a.KV) * a.ctx * kDh;
  if (lane < kKSlots) d.issue(kc + min(lane, 7) * 8, c.K + kKRowB * r);
  if (lane < 8) d.issue(vc + lane * 8, c.V + 128 * r);
  d.drain();
}

// This workgroup's cached positions at position pos: [0, pos) is cut into nsplit equal ranges
// (at most cap each); the last split also takes the current position.
__device__ __forceinline__ void att_range(const Args& a, const AttCtx& c, int pos, int& lo, int& ncached) {
  const int chunk = cdiv(pos, a.nsplit);
  lo = c.split * chunk;
  ncached = max(0, min(pos - lo, chunk));
}

// Device-scope DMA policy for the cached rows when a launch runs several steps: rows written by
// an earlier step of the same launch are then read from memory, not from a cache.
constexpr int kAuxDevice = 16;

template <bool MULTI>
__device__ void att_loader(const Args& a, const AttCtx& c) {
  const int lane = c.lane;
  Dma<kDmaKV> d;
  Dma<kDmaKV, kAuxDevice> dd;
  bool bad = false;
  const int nsteps = MULTI ? a.nsteps : 1;
  for (int st = 0; st < nsteps; ++st) {
    int lo, ncached;
    att_range(a, c, a.pos + st, lo, ncached);
    // The previous step's cache rows are complete once its token is published (every row
    // workgroup waits for its stores before arriving).  Only its own row (position pos + st - 1)
    // needs that token: the older rows were covered by the tokens already seen, so the first
    // layer's older rows are copied before the poll, during the previous step's logits.
    const int newest = st > 0 && a.pos + st - 1 >= lo && a.pos + st - 1 < lo + ncached ? 1 : 0;
    for (int l = 0; l < a.L; ++l) {
      const int gl = st * a.L + l;   // layers run on across the steps of a launch
      if (gl > 0) lds_wait(c.ctr + 2, kWavesA * gl, a.ctrl);
      if (MULTI && st > 0 && l == 0) {
        if (ncached - newest > 0) att_copy(dd, a, c, l, lo, ncached - newest);
        poll_token(a, st - 1, c.item, lane, bad);
        if (newest) att_copy_row(dd, a, c, l, lo, ncached - 1);
      } else if (ncached > 0) {
        if (MULTI) att_copy(dd, a, c, l, lo, ncached);
        else att_copy(d, a, c, l, lo, ncached);
      }
      lds_set(c.ctr + 1, gl + 1, lane);
      MSD_TRACE_POINT(true, l, 28);
      if (c.has_cur) {
        // the current position's k and v of layer l for the waves' merge, polled once q of the
        // layer has arrived (they are posted with it) while the waves take the cached blocks
        lds_wait(c.ctr + 4, gl + 1, a.ctrl);
        const uint32_t tag = a.epoch + uint32_t(st);
        const uint64_t* ks = layer_x(a, l) + a.lay.x_qkv + (a.H + c.g) * kDh + lane;
        const uint64_t* vs = layer_x(a, l) + a.lay.x_qkv + (a.H + a.KV + c.g) * kDh + lane;
        uint64_t kw = ld_tag(ks), vw = ld_tag(vs);
        uint32_t spins = 0;
        while (!bad) {
          const bool kok = uint32_t(kw >> 32) == tag, vok = uint32_t(vw >> 32) == tag;
          if (__all(kok && vok)) break;
          if (!kok) kw = ld_tag(ks);
          if (!vok) vw = ld_tag(vs);
          spin_step(spins, a.ctrl, lane, bad);
        }
        float* kv = c.kvl + (gl & 1) * 2 * kDh;
        kv[lane] = __uint_as_float(uint32_t(kw));
        kv[kDh + lane] = __uint_as_float(uint32_t(vw));
        lds_set(c.ctr + 3, gl + 1, lane);
      }
    }
  }
}

// Sum / max over lanes 0..7 (three DPP steps; lanes 8.. must not matter), read from lane 7.
// For a value that is zero (or -inf) outside lanes 0..7 the sum equals wave_sum's bit for bit.
__device__ __forceinline__ float sum8(float v) {
  v += dpp_f(v, 0x111);
  v += dpp_f(v, 0x112);
  v += dpp_f(v, 0x114);
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 7));
}
// Sum / max over lanes 0..15 (one DPP row), read from lane 15.
__device__ __forceinline__ float sum16(float v) {
  v += dpp_f(v, 0x111);
  v += dpp_f(v, 0x112);
  v += dpp_f(v, 0x114);
  v += dpp_f(v, 0x118);
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 15));
}
__device__ __forceinline__ float max16(float v) {
  v = fmaxf(v, dppm_f(v, 0x111));
  v = fmaxf(v, dppm_f(v, 0x112));
  v = fmaxf(v, dppm_f(v, 0x114));
  v = fmaxf(v, dppm_f(v, 0x118));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 15));
}
__device__ __forceinline__ float max8(float v) {
  v = fmaxf(v, dppm_f(v, 0x111));
  v = fmaxf(v, dppm_f(v, 0x112));
  v = fmaxf(v, dppm_f(v, 0x114));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 7));
}

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ bf16x8 as_bf16x8(uint4 u) { return __builtin_bit_cast(bf16x8, u); }

// Attention waves.  Per layer every wave polls the head's q itself (lane = dim), takes a
// block of the cached positions (block size a multiple of 16, at most 64, so that all waves
// share the rows) and computes
//   scores on the matrix cores: v_mfma_f32_16x16x32_bf16 with A = the three bf16 parts of q
//     in rows 0..2 (zero elsewhere) and B = 16 K rows from LDS, so lanes 0..15 receive the
//     three partial scores of 16 positions in one tile (two products per 64 dims);
//   softmax over the block (wave max / sum);
//   P.V on the vector units: lane (g, dq) = (lane / 16, lane % 16) accumulates dims
//     4 dq .. 4 dq + 3 over positions 4 i + g (two lane groups read two consecutive 128-byte V
//     rows per half-wave: no bank conflicts), then the four groups are summed.
// The wave then polls the new k and v (un-rounded, multi_sm_decode.py:197,205), meets the
// others, and every wave merges the blocks and the current position by log-sum-exp and
// stores one replica: with one split the normalised head output (the row workgroups'
// merge, multi_sm_decode.py:243-259, done here), else (max, sum, unnormalised output).
template <bool MULTI>
__device__ void att_waves(const Args& a, const AttCtx& c) {
  const int lane = c.lane, wv = c.wv;
  const Layout& lay = a.lay;
  bool bad = false;
  int ws = 0;
  const int m16 = lane & 15, kb = lane >> 4;
  uint16_t* apw = c.apw + wv * 3 * kDh;
  float* pw = c.pw + wv * kDh;
  const int nsteps = MULTI ? a.nsteps : 1;
  for (int st = 0; st < nsteps; ++st) {
  int lo, ncached;
  att_range(a, c, a.pos + st, lo, ncached);
  const uint32_t tag = a.epoch + uint32_t(st);
  for (int l = 0; l < a.L; ++l) {
    const int gl = st * a.L + l;   // layers run on across the steps of a launch
    uint64_t* X = layer_x(a, l);
    float* ow = c.ow + (gl & 1) * kWavesA * kDh;   // double-buffered: a wave may start the next
    float* mw = c.mw + (gl & 1) * kWavesA;         // layer while another still merges this one
    float* lw = c.lw + (gl & 1) * kWavesA;
    float qv[1];
    poll_words<1, 1>(X + lay.x_qkv + c.h * kDh, kDh, tag, qv, a.ctrl, 0, lane, bad);
    if (wv == 0 && c.has_cur) lds_set(c.ctr + 4, gl + 1, lane);   // the loader polls k and v now
    MSD_TRACE_POINT(wv == 0, l, 24);
    MSD_TRACE_WAVE(l, 0);
    {   // q = hi + mid + lo exactly, three bf16 parts taken by truncation (each holds the next
        // 8 significant bits), so bf16 products summed in f32 reproduce the f32 products.
        // Staged before the loads below: a wait for q must not wait for them.
      const float x = qv[0];
      const uint32_t hb = __float_as_uint(x) & 0xffff0000u;
      const float r1 = x - __uint_as_float(hb);
      const uint32_t mb = __float_as_uint(r1) & 0xffff0000u;
      const uint32_t lb = __float_as_uint(r1 - __uint_as_float(mb));
      apw[lane] = uint16_t(hb >> 16);
      apw[kDh + lane] = uint16_t(mb >> 16);
      apw[2 * kDh + lane] = uint16_t(lb >> 16);
    }
    lds_wait(c.ctr + 1, gl + 1, a.ctrl);   // cached rows of layer l are in LDS
    MSD_TRACE_POINT(wv == 0, l, 25);
    MSD_TRACE_WAVE(l, 1);
    // block of this wave: tiles [t0, t1) of 16 cached positions, the tiles split evenly over
    // the waves (at most 4 each: ncached <= 512); waves w and w + 4 share a SIMD, and the
    // even split keeps every SIMD's tile count within one of the others'
    int t0, t1;
    split(cdiv(ncached, 16), kWavesA, wv, t0, t1);
    float m = -INFINITY, lsum = 0.f;
    float o[4] = {0.f, 0.f, 0.f, 0.f};
    const int r0 = 16 * t0;
    if (t1 > t0) {
      const int np = min(16 * (t1 - t0), ncached - r0);
      // q parts in the A layout: lane row m16 < 3 holds part m16 of dims 32 ch + 8 kb .. + 8
      __builtin_amdgcn_s_waitcnt(0xc07f);
      __builtin_amdgcn_wave_barrier();
      uint4 aq[2];
#pragma unroll
      for (int ch = 0; ch < 2; ++ch) {
        const uint4 u = *reinterpret_cast<const uint4*>(apw + (m16 < 3 ? m16 : 0) * kDh + 32 * ch + 8 * kb);
        aq[ch] = m16 < 3 ? u : make_uint4(0u, 0u, 0u, 0u);
      }
      // scores: tile t covers positions r0 + 16 t .. + 16 (rows past the cached ones re-read
      // the last cached row and are masked)
      uint4 kk[4][2];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int row = min(r0 + 16 * t + m16, ncached - 1);
        const uint8_t* kr = c.K + row * kKRowB + 16 * kb;
        kk[t][0] = *reinterpret_cast<const uint4*>(kr);
        kk[t][1] = *reinterpret_cast<const uint4*>(kr + 64);
      }
      // all four tiles are computed (independent chains the matrix core overlaps) and the
      // positions past the block masked; the scores sit in lanes 0..15
      float sv[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(aq[0]), as_bf16x8(kk[t][0]), acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(aq[1]), as_bf16x8(kk[t][1]), acc, 0, 0, 0);
        sv[t] = (lane < 16 && 16 * t + lane < np) ? ((acc[0] + acc[1]) + acc[2]) * 0.125f : -INFINITY;
      }
      m = max16(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3])));
      float e[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) e[t] = expf(sv[t] - m);   // 0 for masked positions
      lsum = sum16((e[0] + e[1]) + (e[2] + e[3]));
      // weights to LDS in the P.V order: position q at slot (q % 4) * 16 + q / 4
      if (lane < 16) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int q = 16 * t + lane;
          pw[(q & 3) * 16 + (q >> 2)] = e[t];
        }
      }
      MSD_TRACE_POINT(wv == 0, l, 29);
      MSD_TRACE_WAVE(l, 2);
      __builtin_amdgcn_s_waitcnt(0xc07f);
      __builtin_amdgcn_wave_barrier();
      const int g = kb, dq = m16;
      // all reads first (one LDS round trip); steps past the block (at most 4 of 4 positions
      // per group: np <= 64) use weight 0 on the last row, which adds exact zeros (fewer
      // steps for small blocks measured slower)
      const uint8_t* vb = c.V + r0 * kVRowB + 8 * dq;
      float4 p4[4];
      uint2 vv[4][4];
#pragma unroll
      for (int it = 0; it < 4; ++it) {
        p4[it] = *reinterpret_cast<const float4*>(pw + g * 16 + 4 * it);
#pragma unroll
        for (int k = 0; k < 4; ++k)
          vv[it][k] = *reinterpret_cast<const uint2*>(vb + min(4 * (4 * it + k) + g, np - 1) * kVRowB);
      }
#pragma unroll
      for (int it = 0; it < 4; ++it) {
        const float pk[4] = {p4[it].x, p4[it].y, p4[it].z, p4[it].w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          o[0] += pk[k] * bf_lo(vv[it][k].x);
          o[1] += pk[k] * bf_hi(vv[it][k].x);
          o[2] += pk[k] * bf_lo(vv[it][k].y);
          o[3] += pk[k] * bf_hi(vv[it][k].y);
        }
      }
      // sum the four position groups (rows of 16 lanes): lane l adds lane l ^ 16, then l ^ 32,
      // with the row-swapping permutes (no LDS traffic); a + b in either order, as before
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(o[j]), __float_as_uint(o[j]), false, false);
        o[j] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(o[j]), __float_as_uint(o[j]), false, false);
        o[j] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
      }
      MSD_TRACE_POINT(wv == 0, l, 30);
      MSD_TRACE_WAVE(l, 3);
    }
    lds_bump(c.ctr + 2, lane);   // this wave is done with the cached rows of layer l
    if (lane < 16) *reinterpret_cast<float4*>(ow + wv * kDh + 4 * lane) = make_float4(o[0], o[1], o[2], o[3]);
    if (lane == 0) {
      mw[wv] = m;
      lw[wv] = lsum;
    }
    // the current position's k and v, polled by the loader wave
    float kv2[2] = {0.f, 0.f};
    if (c.has_cur) {
      lds_wait(c.ctr + 3, gl + 1, a.ctrl);
      const float* kv = c.kvl + (gl & 1) * 2 * kDh;
      kv2[0] = kv[lane];
      kv2[1] = kv[kDh + lane];
    }
    // score of the current position (un-rounded k), taken while the other waves finish
    const float scur = c.has_cur ? wave_sum(qv[0] * kv2[0]) * 0.125f : -INFINITY;
    MSD_TRACE_WAVE(l, 4);
    wsync(c.ctr, ws, kWavesA, lane, a.ctrl);
    MSD_TRACE_POINT(wv == 0, l, 26);
    MSD_TRACE_WAVE(l, 5);
    {   // merge the blocks and the current position (log-sum-exp).  Lane w < 8 holds block
        // w's max and sum.
      const float mv = lane < kWavesA ? mw[lane] : -INFINITY;
      const float lv = lane < kWavesA ? lw[lane] : 0.f;
      const float M = fmaxf(max8(lv > 0.f ? mv : -INFINITY), scur);
      float Ls = 0.f, O = 0.f;
      if (M != -INFINITY) {
        const float f = lv > 0.f ? expf(mv - M) : 0.f;   // block weights, one exp per lane
        Ls = sum8(f * lv);
#pragma unroll
        for (int w = 0; w < kWavesA; ++w)
          O += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(f), w)) * ow[w * kDh + lane];
        if (c.has_cur) {
          const float fc = expf(scur - M);
          Ls += fc;
          O += fc * kv2[1];
        }
      }
      if (a.nsplit == 1) {
        const float y = Ls > 0.f ? O * (1.f / Ls) : 0.f;
        for (int r = wv; r < kRep; r += kWavesA) st_tag(X + lay.x_att + c.part + r * lay.x_rep + lane, y, tag);
      } else {
        for (int r = wv; r < kRep; r += kWavesA) {   // replicas wv, wv + 8, ...
          uint64_t* dst = X + lay.x_att + c.part + r * lay.x_rep;
          st_tag(dst + 2 + lane, O, tag);
          if (lane < 2) st_tag(dst + lane, lane == 0 ? M : Ls, tag);
        }
      }
      MSD_TRACE_POINT(wv == 0, l, 27);
      MSD_TRACE_WAVE(l, 6);
    }
  }
  }   // steps
}

// ---------------------------------------------------------------- kernel
// MULTI: several greedy steps per launch (a.nsteps); otherwise one step, without the stores and
// waits only the steps of one launch need of each other.
template <int D, int FF, int QPW, int ORW, int GPW, bool MULTI>
__global__ __launch_bounds__(kThreadsWG, 1) void decode_step_kernel(Args a) {
  extern __shared__ __align__(16) uint8_t smem[];
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // wave-uniform
  const int wg = blockIdx.x;

  if (wg >= a.GR) {   // ------------------------------------------ attention workgroup
    const int i = wg - a.GR;
    // heads of one KV group on as few XCDs as possible (workgroup w runs on XCD w % 8)
    int item = i;
    if (a.NA % 8 == 0 && a.GR % 8 == 0) item = (i % 8) * (a.NA / 8) + i / 8;
    AttCtx c;
    c.item = item;
    c.h = item / a.nsplit;
    c.split = item % a.nsplit;
    c.g = c.h / (a.H / a.KV);
    c.has_cur = c.split == a.nsplit - 1;
    c.lane = lane;
    c.wv = wv;
    c.part = a.nsplit == 1 ? int64_t(c.h) * kDh : int64_t(item) * kPart;
    c.K = smem;
    c.V = c.K + cdiv(a.cap * kKSlots, 64) * 1024;
    c.apw = reinterpret_cast<uint16_t*>(c.V + cdiv(a.cap, 8) * 1024);
    c.pw = reinterpret_cast<float*>(c.apw + kWavesA * 3 * kDh);
    c.ow = c.pw + kWavesA * kDh;
    c.mw = c.ow + 2 * kWavesA * kDh;
    c.lw = c.mw + 2 * kWavesA;
    c.kvl = c.lw + 2 * kWavesA;
    c.ctr = reinterpret_cast<int*>(c.kvl + 4 * kDh);
    if (threadIdx.x < 8) c.ctr[threadIdx.x] = 0;
    __syncthreads();   // the only workgroup barrier; the roles below meet on LDS counters
    if (wv == kLoader) att_loader<MULTI>(a, c);
    else if (wv < kWavesA) att_waves<MULTI>(a, c);
    return;
  }

  // --------------------------------------------------------------- row workgroup
  RowCtx c;
  c.wr = wg;
  c.lane = lane;
  c.wv = wv;
  const int nqkv = (a.H + 2 * a.KV) * kDh;
  split(nqkv / 2, a.GR, wg, c.qp0, c.qp1);
  split(D, a.GR, wg, c.or0, c.or1);
  split(a.ff, a.GR, wg, c.f0, c.f1);
  split(a.V, a.GR, wg, c.v0, c.v1);
  c.ring = smem;
  c.xatt = reinterpret_cast<float*>(smem + a.ring_bytes);
  c.xhd1 = c.xatt + D;
  c.xhd2 = c.xhd1 + D;
  c.xact = c.xhd2 + D;
  // the (head, split) partials: their own region with two splits; with more they share the
  // O-output, down-output and activation vectors, none of which is live from the QKV stores'
  // barrier to the O gather (the merge ends in a barrier before that gather writes xhd1)
  c.xa = a.nsplit > 2 ? c.xhd1 : c.xact + ((FF + 3) & ~3);
  c.ctr = reinterpret_cast<int*>(c.xact + ((FF + 3) & ~3) + (a.nsplit > 2 ? 0 : ((a.H * a.nsplit * kPart + 3) & ~3)));
  c.red_v = reinterpret_cast<float*>(c.ctr + 8);
  c.red_i = reinterpret_cast<int*>(c.red_v + kWavesR);
  if (threadIdx.x < 8) c.ctr[threadIdx.x] = 0;
  int token = a.token_dev ? *a.token_dev : a.token;
  const bool bad_token = token < 0 || token >= a.V;
  if (bad_token) token = token < 0 ? 0 : a.V - 1;   // clamped for addressing, reported below
  if (wg == 0 && threadIdx.x == 0) {
    // Start of the step: the arrival counter and the argmax key start from zero, the
    // bad-token bit of the status word describes this step's token, and the status output
    // holds a sentinel until the last arriver overwrites it, so a step whose arrivals never
    // complete still reports a non-zero status.  The stores complete before this workgroup
    // publishes anything, and every arrival waits for its outputs.
    __hip_atomic_store(a.ctrl + 1, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(reinterpret_cast<uint64_t*>(a.ctrl + 2), uint64_t(0), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
    if (bad_token) atomicOr(a.ctrl, kStatusBadToken);
    else atomicAnd(a.ctrl, ~kStatusBadToken);
    put_out(a.next_token + 1, int32_t(kStatusUnfinished));
    __builtin_amdgcn_s_waitcnt(0);
  }
  __syncthreads();   // the only workgroup barrier; the roles below meet on LDS counters

  if (wv == kLoader) {
    row_loader<D, FF, MULTI>(a, c);
  } else if (wv < kWavesR) {
    // the worker waves issue ahead of the loader wave on a shared SIMD (measured: 316.5 -> 314.6 us
    // per token; a higher loader priority costs 2.5-4 us, the attention waves' gains nothing)
    if constexpr (kWorkerPrio > 0) __builtin_amdgcn_s_setprio(kWorkerPrio);
    row_worker<D, FF, QPW, ORW, GPW, MULTI>(a, c, token);
  }
}

// ---------------------------------------------------------------- host side
struct Plan {   // per-config launch parameters
  int nsplit, cap, NA, GR;
  int qpw, orw, gpw;   // QKV pairs, O/down rows and gate/up pairs per compute wave (at most)
  int ring_q, ring_o, ring_g, ring_d, ring_bytes;
  size_t lds;
};

// Instantiated shapes: (d_model, d_ff, per-wave caps of QKV pairs, O/down rows and gate/up
// pairs).  The reference's configurations (d_ff = 8d/3 rounded up to 128, model.py:13-20, for
// d = 256, 512, 768, 1024) and the tiny benchmark configuration (d 256, d_ff 704); on 256
// workgroups every one of them needs at most the listed rows per wave, with up to one KV head
// per query head.
#if MSD_ROW_WAVES >= 12
#define MSD_SHAPES(X)        \
  X(256, 704, 1, 1, 1)       \
  X(256, 768, 1, 1, 1)       \
  X(512, 1408, 1, 1, 1)      \
  X(768, 2048, 1, 1, 1)      \
  X(1024, 2816, 1, 1, 1)
#elif MSD_ROW_WAVES >= 8
#define MSD_SHAPES(X)        \
  X(256, 704, 1, 1, 1)       \
  X(256, 768, 1, 1, 1)       \
  X(512, 1408, 1, 1, 1)      \
  X(768, 2048, 1, 1, 2)      \
  X(1024, 2816, 1, 1, 2)
#else
#define MSD_SHAPES(X)        \
  X(256, 704, 1, 1, 1)       \
  X(256, 768, 1, 1, 1)       \
  X(512, 1408, 1, 1, 2)      \
  X(768, 2048, 1, 1, 3)      \
  X(1024, 2816, 1, 2, 3)
#endif

struct Shape {
  int d, ff, qpw, orw, gpw;
};
static const Shape kShapes[] = {
#define MSD_SHAPE_ENTRY(D, FF, Q, O, G) {D, FF, Q, O, G},
    MSD_SHAPES(MSD_SHAPE_ENTRY)
#undef MSD_SHAPE_ENTRY
};

static const Shape* find_shape(int d, int ff) {
  for (const Shape& sh : kShapes)
    if (sh.d == d && sh.ff == ff) return &sh;
  return nullptr;
}

static bool config_ok(const msd_config* c) {
  if (!c) return false;
  if (c->d_head != kDh || c->n_heads <= 0 || c->n_kv_heads <= 0 || c->n_layers <= 0) return false;
  if (c->n_heads * kDh != c->d_model || c->n_heads % c->n_kv_heads != 0) return false;
  if (c->d_ff <= 0 || c->d_ff % 16 != 0 || c->vocab_size <= 0 || c->context_len <= 0) return false;
  if (c->context_len > kMaxCtx) return false;
  return find_shape(c->d_model, c->d_ff) != nullptr;
}

constexpr int kMaxLds = 160 * 1024;
// At least this much LDS per workgroup, so that no two workgroups of a step share a
// compute unit: the grid then spreads over every CU.
constexpr int kMinLds = 84 * 1024;

// Shapes for n_workgroups workgroups; false if unsupported.
static bool make_plan(const msd_config* c, int G, Plan* p) {
  if (!config_ok(c) || G <= 0) return false;
  const int D = c->d_model, ff = c->d_ff, H = c->n_heads, KV = c->n_kv_heads;
  const int nqkv = (H + 2 * KV) * kDh;
  p->cap = att_cap(c->context_len);
  p->nsplit = att_splits(c->context_len);
  p->NA = H * p->nsplit;
  p->GR = G - p->NA;
  // every row workgroup owns at least one O/down row and one gate/up pair: its own outputs
  // are then part of every vector it gathers, which orders its LDS buffer reuse
  if (p->GR < 8 || p->GR > D || p->GR > ff) return false;
  const int qpairs = cdiv(nqkv / 2, p->GR), orows = cdiv(D, p->GR), gpairs = cdiv(ff, p->GR);
  p->qpw = cdiv(qpairs, kWavesR);
  p->orw = cdiv(orows, kWavesR);
  p->gpw = cdiv(gpairs, kWavesR);
  if (2 * p->qpw > kMbox || p->orw > kMbox || p->gpw > kMbox) return false;
  auto kb = [](int64_t b) { return int((b + 1023) / 1024 * 1024); };
  p->ring_q = 0;
  p->ring_o = p->ring_q + kb(int64_t(2) * qpairs * D * 2);
  p->ring_g = p->ring_o + kb(int64_t(orows) * D * 2);
  p->ring_d = p->ring_g + kb(int64_t(2) * gpairs * D * 2);
  const int ring = p->ring_d + kb(int64_t(orows) * ff * 2);
  const int natt = H * p->nsplit * kPart;
  // more than two splits: the partials alias xhd1 | xhd2 | xact (2 D + d_ff floats)
  if (p->nsplit > 2 && natt > 2 * D + ff) return false;
  const int row_other = 4 * (3 * D + ((ff + 3) & ~3) + (p->nsplit > 2 ? 0 : ((natt + 3) & ~3)) + 8 + 2 * kWavesR);
  const int att_lds = cdiv(p->cap * kKSlots, 64) * 1024 + cdiv(p->cap, 8) * 1024 +
                      2 * 3 * kWavesA * kDh + 4 * (3 * kWavesA * kDh + 4 * kWavesA + 4 * kDh + 8);
  p->ring_bytes = ring;
  p->lds = size_t(std::max(std::max(att_lds, ring + row_other), kMinLds));
  return p->lds <= size_t(kMaxLds);
}

// Workgroups of the step that the device can hold at once (compute units x workgroups per
// unit at this LDS size): every workgroup waits on others, so a grid larger than this could
// never finish (its waits would run out instead).  Cached per device and LDS size.
static int resident_capacity(const void* fn, size_t lds) {
  struct Entry {
    const void* fn;
    size_t lds;
    int dev, cap;
  };
  static std::mutex mu;
  static std::vector<Entry> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return -1;
  std::lock_guard<std::mutex> lk(mu);
  for (const Entry& e : cache)
    if (e.fn == fn && e.lds == lds && e.dev == dev) return e.cap;
  int cus = 0, per_cu = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return -1;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kThreadsWG, lds) != hipSuccess) return -1;
  cache.push_back({fn, lds, dev, cus * per_cu});
  return cus * per_cu;
}

template <int D, int FF, int QPW, int ORW, int GPW, bool MULTI>
static hipError_t launch_t(const Args& a, int grid, size_t lds, hipStream_t s, bool* not_resident) {
  const void* fn = reinterpret_cast<const void*>(&decode_step_kernel<D, FF, QPW, ORW, GPW, MULTI>);
  if (hipError_t e = msdc::ensure_dynamic_lds(fn, lds); e != hipSuccess) return e;
  const int cap = resident_capacity(fn, lds);
  if (cap < 0) return hipErrorInvalidValue;
  if (grid > cap) {
    *not_resident = true;
    return hipSuccess;
  }
  hipLaunchKernelGGL((decode_step_kernel<D, FF, QPW, ORW, GPW, MULTI>), dim3(grid), dim3(kThreadsWG), lds, s, a);
  return hipGetLastError();
}

// The plan's per-wave row counts must fit the instance compiled for the shape.
static bool plan_instantiated(const msd_config* c, const Plan& p) {
  const Shape* sh = find_shape(c->d_model, c->d_ff);
  return sh && p.qpw <= sh->qpw && p.orw <= sh->orw && p.gpw <= sh->gpw;
}

static hipError_t launch(const Args& a, int d, int ff, int grid, size_t lds, hipStream_t s, bool* not_resident) {
#define MSD_SHAPE_LAUNCH(D, FF, Q, O, G)                                                     \
  if (d == D && ff == FF)                                                                    \
    return a.nsteps > 1 ? launch_t<D, FF, Q, O, G, true>(a, grid, lds, s, not_resident)      \
                        : launch_t<D, FF, Q, O, G, false>(a, grid, lds, s, not_resident);
  MSD_SHAPES(MSD_SHAPE_LAUNCH)
#undef MSD_SHAPE_LAUNCH
  return hipErrorInvalidValue;
}

}  // namespace msd

hipError_t msdc::ensure_dynamic_lds(const void* fn, size_t lds) {
  struct Entry {
    const void* fn;
    int dev;
    size_t lds;
  };
  static std::mutex mu;
  static std::vector<Entry> set;
  int dev = 0;
  if (hipError_t e = hipGetDevice(&dev); e != hipSuccess) return e;
  std::lock_guard<std::mutex> lk(mu);
  Entry* hit = nullptr;
  for (Entry& x : set)
    if (x.fn == fn && x.dev == dev) hit = &x;
  if (hit && hit->lds >= lds) return hipSuccess;
  if (hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, int(lds)); e != hipSuccess)
    return e;
  if (hit)
    hit->lds = lds;
  else
    set.push_back({fn, dev, lds});
  return hipSuccess;
}

bool msdc::decode_supported(const msd_config* cfg, int n_workgroups) {
  msd::Plan p;
  return msd::config_ok(cfg) && msd::make_plan(cfg, n_workgroups, &p) && msd::plan_instantiated(cfg, p);
}

using namespace msd;

extern "C" int64_t msd_packed_weight_elems(const msd_config* cfg) {
  if (!config_ok(cfg)) return MSD_E_CONFIG;
  return make_layout(cfg->d_model, cfg->n_heads, cfg->n_kv_heads, cfg->d_ff, cfg->context_len).layer_elems *
         cfg->n_layers;
}

extern "C" int64_t msd_workspace_bytes(const msd_config* cfg, int32_t n_workgroups) {
  Plan p;
  if (!config_ok(cfg)) return MSD_E_CONFIG;
  if (!make_plan(cfg, n_workgroups, &p) || !plan_instantiated(cfg, p)) return MSD_E_CONFIG;
  const Layout t = make_layout(cfg->d_model, cfg->n_heads, cfg->n_kv_heads, cfg->d_ff, cfg->context_len);
  return t.ctrl_bytes + t.x_layer * cfg->n_layers * int64_t(sizeof(uint64_t));
}

extern "C" int32_t msd_default_workgroups(int32_t device) {
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess) return MSD_E_HIP;
  return n;
}

static int32_t decode_impl(const msd_config* cfg, const void* token_emb, const void* output_proj,
                           const void* packed_w, const void* lnf_s, const float* rope, int32_t token_id,
                           const int32_t* token_dev, int32_t pos, int32_t n_steps, void* kv, void* workspace,
                           uint32_t epoch, float* logits, int64_t logits_stride, int32_t* next_token,
                           int32_t n_workgroups, hipStream_t stream) {
  Plan p;
  if (!config_ok(cfg)) return MSD_E_CONFIG;
  if (n_workgroups <= 0 || n_workgroups > 4096) return MSD_E_ARG;
  if (!make_plan(cfg, n_workgroups, &p) || !plan_instantiated(cfg, p)) return MSD_E_CONFIG;
  if (!token_emb || !output_proj || !packed_w || !lnf_s || !rope || !kv || !workspace || !logits || !next_token)
    return MSD_E_ARG;
  if (n_steps <= 0 || pos < 0 || int64_t(pos) + n_steps > cfg->context_len) return MSD_E_ARG;
  if (!token_dev && (token_id < 0 || token_id >= cfg->vocab_size)) return MSD_E_ARG;
  if (epoch == 0 || uint64_t(epoch) + uint64_t(n_steps - 1) > 0xffffffffull) return MSD_E_ARG;
  const uintptr_t al = reinterpret_cast<uintptr_t>(token_emb) | reinterpret_cast<uintptr_t>(packed_w) |
                       reinterpret_cast<uintptr_t>(output_proj) |
                       reinterpret_cast<uintptr_t>(kv) | reinterpret_cast<uintptr_t>(workspace);
  if (al & 15) return MSD_E_ARG;
  Args a;
  a.emb = static_cast<const uint16_t*>(token_emb);
  a.outp = static_cast<const uint16_t*>(output_proj);
  a.w = static_cast<const uint16_t*>(packed_w);
  a.lnf = static_cast<const uint16_t*>(lnf_s);
  a.rope = rope;
  a.kv = static_cast<uint16_t*>(kv);
  a.logits = logits;
  a.next_token = next_token;
  a.token_dev = token_dev;
  a.ctrl = static_cast<uint32_t*>(workspace);
  a.lay = make_layout(cfg->d_model, cfg->n_heads, cfg->n_kv_heads, cfg->d_ff, cfg->context_len);
  a.xw = reinterpret_cast<uint64_t*>(static_cast<char*>(workspace) + a.lay.ctrl_bytes);
  a.token = token_id;
  a.pos = pos;
  a.epoch = epoch;
  a.nsteps = n_steps;
  a.logits_stride = logits_stride;
  a.H = cfg->n_heads;
  a.KV = cfg->n_kv_heads;
  a.L = cfg->n_layers;
  a.ff = cfg->d_ff;
  a.V = cfg->vocab_size;
  a.ctx = cfg->context_len;
  a.nsplit = p.nsplit;
  a.cap = p.cap;
  a.NA = p.NA;
  a.GR = p.GR;
  a.ring_q = p.ring_q;
  a.ring_o = p.ring_o;
  a.ring_g = p.ring_g;
  a.ring_d = p.ring_d;
  a.ring_bytes = p.ring_bytes;
  a.keep = int(std::min<int64_t>(cfg->n_layers, kKeepBytes / (a.lay.layer_elems * 2)));
  bool not_resident = false;
  const hipError_t e = launch(a, cfg->d_model, cfg->d_ff, n_workgroups, p.lds, stream, &not_resident);
  if (not_resident) return MSD_E_CONFIG;
  return e == hipSuccess ? MSD_OK : MSD_E_HIP;
}

extern "C" int32_t msd_decode_step(const msd_config* cfg, const void* token_emb, const void* output_proj,
                                   const void* packed_w, const void* lnf_s, const float* rope, int32_t token_id,
                                   const int32_t* token_dev, int32_t pos, void* kv, void* workspace,
                                   uint32_t epoch, float* logits, int32_t* next_token,
                                   int32_t n_workgroups, void* stream) {
  return decode_impl(cfg, token_emb, output_proj, packed_w, lnf_s, rope, token_id, token_dev, pos, 1, kv, workspace,
                     epoch, logits, 0, next_token, n_workgroups, static_cast<hipStream_t>(stream));
}

extern "C" int32_t msd_decode_steps(const msd_config* cfg, const void* token_emb, const void* output_proj,
                                    const void* packed_w, const void* lnf_s, const float* rope, int32_t token_id,
                                    const int32_t* token_dev, int32_t pos, int32_t n_steps, void* kv,
                                    void* workspace, uint32_t epoch, float* logits, int32_t all_logits,
                                    int32_t* tokens_out, int32_t n_workgroups, void* stream) {
  if (!cfg) return MSD_E_CONFIG;
  return decode_impl(cfg, token_emb, output_proj, packed_w, lnf_s, rope, token_id, token_dev, pos, n_steps, kv,
                     workspace, epoch, logits, all_logits ? int64_t(cfg->vocab_size) : 0, tokens_out, n_workgroups,
                     static_cast<hipStream_t>(stream));
}

// Decode workspaces in uncached device memory, pooled per (device, size) and never freed.
namespace {
struct WsBlock {
  int dev;
  int64_t bytes;
  void* ptr;
  bool used;
};
std::mutex g_ws_mu;
std::vector<WsBlock> g_ws;
}  // namespace

extern "C" int32_t msd_workspace_acquire(int32_t device, int64_t bytes, void** out) {
  if (!out || bytes <= 0) return MSD_E_ARG;
  *out = nullptr;
  std::lock_guard<std::mutex> lk(g_ws_mu);
  int prev = 0;
  if (hipGetDevice(&prev) != hipSuccess) return MSD_E_HIP;
  if (prev != device && hipSetDevice(device) != hipSuccess) return MSD_E_HIP;
  WsBlock* blk = nullptr;
  for (auto& b : g_ws)
    if (!b.used && b.dev == device && b.bytes == bytes) {
      blk = &b;
      break;
    }
  hipError_t e = hipSuccess;
  if (blk) {
    e = hipDeviceSynchronize();   // the previous owner's steps may still be queued
  } else {
    void* p = nullptr;
    e = hipExtMallocWithFlags(&p, size_t(bytes), hipDeviceMallocUncached);
    if (e == hipSuccess) {
      g_ws.push_back({device, bytes, p, false});
      blk = &g_ws.back();
    }
  }
  if (e == hipSuccess) e = hipMemset(blk->ptr, 0, size_t(bytes));
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (prev != device) (void)hipSetDevice(prev);
  if (e != hipSuccess) return MSD_E_HIP;
  blk->used = true;
  *out = blk->ptr;
  return MSD_OK;
}

extern "C" int32_t msd_workspace_release(void* workspace) {
  std::lock_guard<std::mutex> lk(g_ws_mu);
  for (auto& b : g_ws)
    if (b.ptr == workspace && b.used) {
      b.used = false;
      return MSD_OK;
    }
  return MSD_E_ARG;
}

extern "C" int32_t msd_check_status(void* workspace, void* stream) {
  if (!workspace) return MSD_E_ARG;
  hipStream_t s = static_cast<hipStream_t>(stream);
  uint32_t st = 0;
  if (hipMemcpyAsync(&st, workspace, sizeof(st), hipMemcpyDeviceToHost, s) != hipSuccess) return MSD_E_HIP;
  if (hipStreamSynchronize(s) != hipSuccess) return MSD_E_HIP;
  if (st == 0) return MSD_OK;
  const uint32_t zero = 0;
  if (hipMemcpyAsync(workspace, &zero, sizeof(zero), hipMemcpyHostToDevice, s) != hipSuccess) return MSD_E_HIP;
  if (hipStreamSynchronize(s) != hipSuccess) return MSD_E_HIP;
  if (st & kStatusTimeout) return MSD_E_TIMEOUT;
  return MSD_E_ARG;
}

#ifdef MSD_TRACE
extern "C" int msd_trace_waves_copy(void* host) {
  return hipMemcpyFromSymbol(host, HIP_SYMBOL(msd::msd_trace_waves), sizeof(uint64_t) * 4096 * 16 * 8) == hipSuccess ? 0 : -1;
}
extern "C" int msd_trace_copy(void* host) {
  return hipMemcpyFromSymbol(host, HIP_SYMBOL(msd::msd_trace_buffer),
                             sizeof(uint64_t) * kTraceLayers * kTraceWgs * kTraceSlots) == hipSuccess ? 0 : -1;
}
#endif
