// Fused whole-model decode step for gfx950 (MI355X): one persistent launch per token.
//
// Reference path replaced (zahlmann/transformer): kernels/multi_sm_decode.py:35-357
// (_multi_sm_decode) behind multi_sm_decode_nlayer (:369-432).  The maths follows
// model.py:94-191; the decode-step semantics (f32 residual stream, K/V written to the
// cache as bf16 at `pos`, the current position attending with its un-rounded K/V,
// argmax resolving ties to the lowest index) follow kernels/multi_sm_decode.py.
//
// Execution model
//   * grid = one workgroup per compute unit (256 on MI355X), 256 threads (4 wave64s);
//     every workgroup is resident for the whole step (1 workgroup per CU, launched on an
//     otherwise idle device), so workgroups may wait on each other.
//   * weights are bf16 in an (out, in) row layout: every output element is one
//     contiguous dot product, read with 128-bit loads (each lane 8 bf16 per load) and
//     reduced across the wave; bf16 is widened to f32 in registers and all activation
//     arithmetic is f32.
//   * every workgroup keeps its own copy of the residual stream h (d floats in LDS) and
//     recomputes the RMSNorms redundantly; only projection outputs cross workgroups.
//   * cross-workgroup exchange uses tagged 64-bit words: (f32 value | 32-bit epoch tag),
//     written with device-scope atomic stores and polled with device-scope atomic loads.
//     A word carries its own validity, so no separate flag, fence or barrier is needed;
//     each (layer, exchange) has its own buffer so tags only need to differ per step.
//   * per layer: QKV rows (+RoPE, KV write) -> attention over position chunks per KV head
//     -> chunk merge -> O rows (+residual) -> gate/up rows (+SwiGLU) -> down rows
//     (+residual); then final RMSNorm, vocabulary rows of the tied embedding, argmax via
//     a 64-bit atomic max of (ordered value, inverted index) and a last-arriver counter.
//   * every wait is bounded: a workgroup that exceeds the spin bound sets the status word
//     and stops waiting; the others see the status and stop as well, so a broken step
//     still drains the grid.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

#include "../../include/msdecode.h"

namespace msd {

// Optional phase timestamps for profiling builds (-DMSD_TRACE): lane 0 of the first exchange
// wave and of compute wave 0 record s_memrealtime (100 MHz) at phase boundaries of one layer
// into msd_trace_buffer[workgroup][slot].  Compiled out otherwise.
#ifdef MSD_TRACE
__device__ uint64_t msd_trace_buffer[4096 * 32];
#define MSD_TRACE_POINT(cond, slot)                                                        \
  do {                                                                                    \
    if ((cond) && l == MSD_TRACE_LAYER && c.lane == 0)                                    \
      msd_trace_buffer[c.wg * 32 + (slot)] = __builtin_amdgcn_s_memrealtime();           \
  } while (0)
#else
#define MSD_TRACE_POINT(cond, slot) \
  do {                              \
  } while (0)
#endif

constexpr int kDh = 64;          // head dimension (fixed)
constexpr int kChunkMax = 64;    // attention positions per chunk (one per lane of a wave)
constexpr int kPartStride = 66;  // per (chunk, head): m, l, o[64]
// LDS row stride of cached K rows (floats): 16-byte aligned rows whose 128-bit reads by 16
// consecutive lanes (one LDS pass) start 4 banks apart, so they never conflict.
constexpr int kKPad = kDh + 4;
constexpr uint32_t kSpinLimit = 1u << 20;

constexpr int kWavesC = 4;      // compute waves per workgroup
constexpr int kWavesX = 4;      // exchange waves per workgroup

constexpr uint32_t kStatusTimeout = 1u;
constexpr uint32_t kStatusBadToken = 2u;

// ---------------------------------------------------------------- layout
struct Layout {
  // packed weights, per layer (bf16 elements)
  int64_t off_ln1, off_ln2, off_qkv, off_o, off_gu, off_dn, layer_elems;
  // exchange words per layer (uint64)
  int64_t x_qkv, x_part, x_attn, x_hd1, x_act, x_hd2, x_layer;
  int64_t x_rep;   // word stride between the replicas of the all-gathered vectors
  int64_t ctrl_bytes;
  // producer flags: flags[(layer * kNumEx + exchange) * G + producer_workgroup] (uint32)
  int64_t flag_words;   // uint32 flags per layer
};

// Replicas of every exchange vector that all workgroups gather (workgroup w reads replica
// w % kRep, its XCD under the round-robin dispatch of workgroups to XCDs).
constexpr int kRep = 8;

// exchanges of a layer (index into the flag arrays)
enum { kExQkv = 0, kExPart = 1, kExAttn = 2, kExHd1 = 3, kExAct = 4, kExHd2 = 5, kNumEx = 6 };

__host__ __device__ inline int64_t align64(int64_t v) { return (v + 63) & ~int64_t(63); }

// attention chunks per KV head: enough that a chunk of the full context fits a wave
__host__ __device__ inline int n_chunks(int ctx) { return (ctx + kChunkMax - 1) / kChunkMax; }

__host__ __device__ inline Layout make_layout(int d, int H, int KV, int ff, int ctx, int G = 0) {
  Layout t;
  const int64_t nqkv = int64_t(H + 2 * KV) * kDh;
  t.off_ln1 = 0;
  t.off_ln2 = d;
  t.off_qkv = 2 * int64_t(d);
  t.off_o = t.off_qkv + nqkv * d;
  t.off_gu = t.off_o + int64_t(d) * d;
  t.off_dn = t.off_gu + 2 * int64_t(ff) * d;
  t.layer_elems = t.off_dn + int64_t(d) * ff;
  const int GQ = H / KV;
  t.x_qkv = 0;
  t.x_part = t.x_qkv + align64(nqkv);
  t.x_attn = t.x_part + align64(int64_t(KV) * n_chunks(ctx) * GQ * kPartStride);
  t.x_hd1 = t.x_attn + align64(d);
  t.x_act = t.x_hd1 + align64(d);
  t.x_hd2 = t.x_act + align64(ff);
  // attn, hd1, act and hd2 are read by every workgroup: kRep replicas (at a stride that is
  // not a multiple of 4 KB) spread those reads over the memory channels
  const int64_t rep_words = t.x_hd2 + align64(d) - t.x_attn;
  t.x_rep = ((rep_words + 511) & ~int64_t(511)) + 32;
  t.x_layer = t.x_attn + kRep * t.x_rep;
  t.ctrl_bytes = 256;
  t.flag_words = int64_t(kNumEx) * G;
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
  int32_t* next_token;
  const int32_t* token_dev;
  uint32_t* ctrl;   // [0] status, [1] arrival counter, [2..3] argmax key (u64)
  uint64_t* xw;     // exchange words, n_layers * x_layer
  uint32_t* flags;  // producer flags, n_layers * flag_words
  int token, pos;
  uint32_t epoch;
  int H, KV, L, ff, V, ctx, nch;
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
__device__ __forceinline__ float dpp_f(float v, int ctrl, int row_mask) {
  switch (ctrl) {   // the control word must be a compile-time constant
    case 0x111: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x111, 0xf, 0xf, true));
    case 0x112: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x112, 0xf, 0xf, true));
    case 0x114: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x114, 0xf, 0xf, true));
    case 0x118: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x118, 0xf, 0xf, true));
    case 0x142: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x142, 0xa, 0xf, true));
    default: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x143, 0xc, 0xf, true));
  }
  (void)row_mask;
}
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_f(v, 0x111, 0xf);
  v += dpp_f(v, 0x112, 0xf);
  v += dpp_f(v, 0x114, 0xf);
  v += dpp_f(v, 0x118, 0xf);
  v += dpp_f(v, 0x142, 0xa);
  v += dpp_f(v, 0x143, 0xc);
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

__device__ __forceinline__ void st_tag(uint64_t* p, float v, uint32_t tag) {
  __hip_atomic_store(p, (uint64_t(tag) << 32) | __float_as_uint(v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld_tag(const uint64_t* p) {
  return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_flag(uint32_t* p, uint32_t tag) {
  __hip_atomic_store(p, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ld_flag(const uint32_t* p) {
  return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ld_status(uint32_t* ctrl) {
  return __hip_atomic_load(ctrl, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Poll NW tagged words per lane (word k of lane at src[idx(k)]) until every tag equals
// `tag`.  A bounded spin: after kSpinLimit rounds, or when another workgroup has reported a
// timeout in the status word, the wave stops waiting and `bad` is set.
constexpr int kXW = 12;   // words per lane per exchange wave and batch (3072 words per batch)

// The exchange waves share a gather: 64-word blocks are dealt round-robin to the
// kWavesX waves (block b -> wave b % kWavesX), so wave ew, lane j handles words
// 64 * (kWavesX * k + ew) + j.
__device__ __forceinline__ int xidx(int k, int ew, int lane) { return 64 * (kWavesX * k + ew) + lane; }

__device__ void gather_x(const uint64_t* src, int n, float* dst, uint32_t tag, uint32_t* ctrl,
                         int ew, int lane, bool& bad) {
  for (int base = 0; base < n; base += 64 * kWavesX * kXW) {
    uint64_t w[kXW];
#pragma unroll
    for (int k = 0; k < kXW; ++k) {
      const int i = base + xidx(k, ew, lane);
      w[k] = (i < n) ? ld_tag(src + i) : (uint64_t(tag) << 32);
    }
    uint32_t spins = 0;
    while (!bad) {
      bool ok = true;
#pragma unroll
      for (int k = 0; k < kXW; ++k) {
        if (uint32_t(w[k] >> 32) != tag) {
          ok = false;
          w[k] = ld_tag(src + base + xidx(k, ew, lane));
        }
      }
      if (__all(ok)) break;
      ++spins;
      if ((spins & 255u) == 0 && (ld_status(ctrl) & kStatusTimeout)) bad = true;
      if (spins > kSpinLimit) {
        if (lane == 0) atomicOr(ctrl, kStatusTimeout);
        bad = true;
      }
    }
#pragma unroll
    for (int k = 0; k < kXW; ++k) {
      const int i = base + xidx(k, ew, lane);
      if (i < n) dst[i] = __uint_as_float(uint32_t(w[k]));
    }
  }
}

// Producer-flag gating of gathers.  With MSD_FLAG_POLL defined, consumers first wait for the
// producers' flags and then read the data; otherwise they poll the tagged data words
// directly (one round trip less; the flags are still raised).
#ifdef MSD_FLAG_POLL
constexpr bool kFlagPoll = true;
#else
constexpr bool kFlagPoll = false;
#endif

// Wait until the producer flags f[0..n) all equal `tag` (one wave; bounded spin).  A
// producer raises its flag after issuing its tagged data words, so a consumer polls n
// 4-byte flags instead of all data words; the data words are still validated by their tags.
__device__ void poll_flags(const uint32_t* f, int n, uint32_t tag, uint32_t* ctrl, int lane, bool& bad) {
  if (!kFlagPoll) return;
  for (int base = 0; base < n; base += 64 * 4) {
    uint32_t v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int i = base + lane + 64 * k;
      v[k] = (i < n) ? ld_flag(f + i) : tag;
    }
    uint32_t spins = 0;
    while (!bad) {
      bool ok = true;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        if (v[k] != tag) {
          ok = false;
          v[k] = ld_flag(f + base + lane + 64 * k);
        }
      }
      if (__all(ok)) break;
      ++spins;
      if ((spins & 255u) == 0 && (ld_status(ctrl) & kStatusTimeout)) bad = true;
      if (spins > kSpinLimit) {
        if (lane == 0) atomicOr(ctrl, kStatusTimeout);
        bad = true;
      }
    }
  }
}

// LDS spin-wait until *ctr >= target (intra-workgroup hand-off between wave roles).
__device__ __forceinline__ void lds_wait(int* ctr, int target) {
  while (__hip_atomic_load(ctr, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < target) __builtin_amdgcn_s_sleep(1);
}
__device__ __forceinline__ void lds_bump(int* ctr, int lane) {
  __builtin_amdgcn_s_waitcnt(0xc07f);   // this wave's LDS writes are done (lgkmcnt(0))
  if (lane == 0) __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Synchronise the exchange waves only (the compute waves are not involved): every wave
// bumps an LDS counter and waits for the other waves' bumps.  `phase` counts calls.
__device__ __forceinline__ void xsync(int* ctr, int& phase, int lane) {
  phase += kWavesX;
  __builtin_amdgcn_s_waitcnt(0xc07f);   // this wave's LDS writes are done (lgkmcnt(0))
  if (lane == 0) __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
  while (__hip_atomic_load(ctr, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < phase) __builtin_amdgcn_s_sleep(1);
}

// Row layout for the matrix-vector products.  A row of K bf16 values is cut into blocks of
// 512 (the last block may be shorter: S = 8*m values, m lanes); in block b, lane l holds the
// 16 bytes at packed offset 512*b + 8*l, and its k-th value (k < 8) multiplies input element
// 512*b + k*m + l.  The packer applies that in-dimension permutation to every row, so the
// lane's 8 inputs are x[512*b + k*m + l]: consecutive lanes read consecutive LDS words
// (no bank conflicts) and each lane keeps its inputs in registers for all rows of a phase.
template <int NL>
struct Row {
  uint4 v[NL];
};
template <int NL>
struct XV {
  float v[NL][8];
};

__device__ __forceinline__ int block_lanes(int k, int b) {
  const int rem = k - 512 * b;
  return rem >= 512 ? 64 : (rem > 0 ? rem / 8 : 0);
}

template <int NL>
__device__ __forceinline__ void load_row(Row<NL>& r, const uint16_t* row, int k, int lane) {
  const uint4* p = reinterpret_cast<const uint4*>(row);
#pragma unroll
  for (int j = 0; j < NL; ++j) r.v[j] = (lane < block_lanes(k, j)) ? p[j * 64 + lane] : make_uint4(0, 0, 0, 0);
}

template <int NL>
__device__ __forceinline__ void load_x(XV<NL>& xv, const float* x, int k, int lane) {
#pragma unroll
  for (int j = 0; j < NL; ++j) {
    const int m = block_lanes(k, j);
#pragma unroll
    for (int q = 0; q < 8; ++q) xv.v[j][q] = (lane < m) ? x[512 * j + q * m + lane] : 0.f;
  }
}

template <int NL>
__device__ __forceinline__ float dot_row(const Row<NL>& r, const XV<NL>& xv) {
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < NL; ++j) {
    const uint4 w = r.v[j];
    acc += bf_lo(w.x) * xv.v[j][0];
    acc += bf_hi(w.x) * xv.v[j][1];
    acc += bf_lo(w.y) * xv.v[j][2];
    acc += bf_hi(w.y) * xv.v[j][3];
    acc += bf_lo(w.z) * xv.v[j][4];
    acc += bf_hi(w.z) * xv.v[j][5];
    acc += bf_lo(w.w) * xv.v[j][6];
    acc += bf_hi(w.w) * xv.v[j][7];
  }
  return wave_sum(acc);
}

// Same as dot_row, with the lane's inputs read from LDS block by block (single-row phases).
template <int NL>
__device__ __forceinline__ float dot_row_lds(const Row<NL>& r, const float* x, int k, int lane) {
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < NL; ++j) {
    const int m = block_lanes(k, j);
    float xv[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) xv[q] = (lane < m) ? x[512 * j + q * m + lane] : 0.f;
    const uint4 w = r.v[j];
    acc += bf_lo(w.x) * xv[0];
    acc += bf_hi(w.x) * xv[1];
    acc += bf_lo(w.y) * xv[2];
    acc += bf_hi(w.y) * xv[3];
    acc += bf_lo(w.z) * xv[4];
    acc += bf_hi(w.z) * xv[5];
    acc += bf_lo(w.w) * xv[6];
    acc += bf_hi(w.w) * xv[7];
  }
  return wave_sum(acc);
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

// ---------------------------------------------------------------- kernel
// Workgroup = 4 compute waves + 1 exchange wave.
//   compute waves: own fixed output rows of every projection; the weights of a phase for
//     layer l+1 are loaded into registers right after the phase of layer l used them, so
//     weight streaming runs a whole layer ahead of the dependency chain.
//   exchange wave: waits for the inputs of the next phase (tagged words), keeps the
//     residual stream h in its registers, applies the residual adds and RMSNorms, and
//     writes the next phase's input vector into one of two LDS buffers (alternating).
// Phases per layer (all waves meet at a workgroup barrier between phases):
//   B0: x0 = rmsnorm1(h)         | compute: QKV rows (+RoPE, KV write)   | exch: q/k/v of the head group (attention WGs)
//   B1:                          | compute: attention chunk (attention WGs) | exch: merge (merger WGs), attn -> x1
//   B2: x1 = attention output    | compute: O rows -> hd1                | exch: h += hd1, x0 = rmsnorm2(h)
//   B3: x0                       | compute: gate/up rows -> act          | exch: act -> x1
//   B4: x1 = act                 | compute: down rows -> hd2             | exch: h += hd2, x0 = rmsnorm1'(h)
constexpr int kThreadsWG = (kWavesC + kWavesX) * 64;

// Shared per-step quantities of one workgroup.
struct Ctx {
  int G, wg, lane, wv;
  int H, KV, GQ, ff, L, nch, npart, nqkv;
  int pos;
  uint32_t tag;
  bool att, merger;
  int ag, ac, q0, q1, P, ncached;
  float* sh_x0;
  float* sh_x1;
  float* sh_k;
  float* sh_v;
  float* sh_q;
  float* sh_e;
  float* sh_red;
  int* sh_sync;
  // mailbox from compute waves to the publishing exchange wave
  float* mb_val;   // kWavesC * kMbox values
  int* mb_idx;     // word index in the layer's exchange words, -1 = unused
  int* mb_out;     // compute waves: outputs written (bumped once per wave and phase)
  int* mb_pub;     // exchange wave 0: outputs published (bumped once per phase)
};

constexpr int kMbox = 4;   // outputs per compute wave and phase

__device__ __forceinline__ uint64_t* layer_x(const Args& a, int l) { return a.xw + int64_t(l) * a.lay.x_layer; }
__device__ __forceinline__ const uint16_t* layer_w(const Args& a, int l) { return a.w + int64_t(l) * a.lay.layer_elems; }
__device__ __forceinline__ uint16_t* layer_k(const Args& a, int l) { return a.kv + int64_t(l) * 2 * a.KV * a.ctx * kDh; }

// ---------------------------------------------------------------- exchange waves
// kWavesX waves.  Per phase they first publish this workgroup's outputs (exchange wave 0
// takes them from the compute waves' LDS mailbox, stores the tagged words, then raises the
// workgroup's flag), then wait for the producer flags of the next input and gather it in
// parallel (gather_x).  They keep the residual stream h (element xidx(k, ew, lane)) and
// apply the residual adds and the RMSNorms.
template <int D>
__device__ void exchange_role(const Args& a, const Ctx& c, int token) {
  constexpr int HPW = D / (64 * kWavesX);   // residual elements per lane of each exchange wave
  const int lane = c.lane, ew = c.wv - kWavesC;
  const int G = c.G;
  bool bad = false;
  int sphase = 0, pphase = 0, aphase = 0;
  float* ss_slot = c.sh_red + 32;           // per-wave partial sums of squares
  float h[HPW];
  float sc[HPW];                            // prefetched RMSNorm scale
#pragma unroll
  for (int k = 0; k < HPW; ++k) h[k] = bf2f(a.emb[int64_t(token) * D + xidx(k, ew, lane)]);
  auto flagp = [&](int l, int ex) { return a.flags + (int64_t(l) * kNumEx + ex) * G; };
  auto load_scale = [&](const uint16_t* scale) {
#pragma unroll
    for (int k = 0; k < HPW; ++k) sc[k] = bf2f(scale[xidx(k, ew, lane)]);
  };
  // x = scale * (h / sqrt(mean(h^2) + eps)) into LDS (model.py:94-98)
  auto norm_to = [&](float* x) {
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < HPW; ++k) ss += h[k] * h[k];
    ss = wave_sum(ss);
    const int slot = (sphase / kWavesX) % 2;
    if (lane == 0) ss_slot[slot * kWavesX + ew] = ss;
    xsync(c.sh_sync, sphase, lane);
    float tot = 0.f;
#pragma unroll
    for (int w = 0; w < kWavesX; ++w) tot += ss_slot[slot * kWavesX + w];
    const float r = sqrtf(tot / float(D) + 1e-5f);
#pragma unroll
    for (int k = 0; k < HPW; ++k) x[xidx(k, ew, lane)] = sc[k] * (h[k] / r);
  };
  auto add_h = [&](const uint64_t* src) {
    uint64_t wd[HPW];
#pragma unroll
    for (int k = 0; k < HPW; ++k) wd[k] = ld_tag(src + xidx(k, ew, lane));
    uint32_t spins = 0;
    while (!bad) {
      bool ok = true;
#pragma unroll
      for (int k = 0; k < HPW; ++k) {
        if (uint32_t(wd[k] >> 32) != c.tag) {
          ok = false;
          wd[k] = ld_tag(src + xidx(k, ew, lane));
        }
      }
      if (__all(ok)) break;
      ++spins;
      if ((spins & 255u) == 0 && (ld_status(a.ctrl) & kStatusTimeout)) bad = true;
      if (spins > kSpinLimit) {
        if (lane == 0) atomicOr(a.ctrl, kStatusTimeout);
        bad = true;
      }
    }
#pragma unroll
    for (int k = 0; k < HPW; ++k) h[k] = h[k] + __uint_as_float(uint32_t(wd[k]));
  };
  // exchange wave 0: publish the compute waves' outputs of this phase, then the flag
  auto publish = [&](uint64_t* X, uint32_t* flag, bool replicated) {
    ++pphase;
    if (ew != 0) return;
    lds_wait(c.mb_out, kWavesC * pphase);
    constexpr int E = kWavesC * kMbox;   // mailbox entries; 64 / E replicas per pass
    const int e = lane % E;
    const int idx = c.mb_idx[e];
    const float v = c.mb_val[e];
    if (replicated) {
      for (int r = lane / E; r < kRep; r += 64 / E)
        if (idx >= 0) st_tag(X + idx + r * a.lay.x_rep, v, c.tag);
    } else if (lane < E && idx >= 0) {
      st_tag(X + idx, v, c.tag);
    }
    if (lane == 0) st_flag(flag, c.tag);
    lds_bump(c.mb_pub, lane);
  };
  const int64_t myrep = int64_t(c.wg % kRep) * a.lay.x_rep;
  load_scale(a.w + a.lay.off_ln1);
  norm_to(c.sh_x0);
  __syncthreads();
  for (int l = 0; l < c.L; ++l) {
    const Layout& lay = a.lay;
    uint64_t* X = layer_x(a, l);
    load_scale(layer_w(a, l) + lay.off_ln2);
    // B0 .. B1: publish q/k/v rows; attention workgroups gather q of their head group and the new k, v
    publish(X, flagp(l, kExQkv) + c.wg, false);
    if (c.att) {
      poll_flags(flagp(l, kExQkv), G, c.tag, a.ctrl, lane, bad);
      gather_x(X + lay.x_qkv + int64_t(c.ag) * c.GQ * kDh, c.GQ * kDh, c.sh_q, c.tag, a.ctrl, ew, lane, bad);
      if (c.pos >= c.q0 && c.pos < c.q1 && ew < 2) {   // current position: un-rounded K/V (multi_sm_decode.py:197,205)
        const int prow = c.pos - c.q0;
        const int hh = ew == 0 ? c.H + c.ag : c.H + c.KV + c.ag;
        float* dst = ew == 0 ? c.sh_k + prow * kKPad : c.sh_v + prow * kDh;
        uint64_t w = ld_tag(X + lay.x_qkv + int64_t(hh) * kDh + lane);
        uint32_t spins = 0;
        while (!bad && uint32_t(w >> 32) != c.tag) {
          w = ld_tag(X + lay.x_qkv + int64_t(hh) * kDh + lane);
          if (++spins > kSpinLimit) {
            if (lane == 0) atomicOr(a.ctrl, kStatusTimeout);
            bad = true;
          }
        }
        dst[lane] = __uint_as_float(uint32_t(w));
      }
    }
    MSD_TRACE_POINT(ew == 0, 0);
    __syncthreads();  // B1
    MSD_TRACE_POINT(ew == 0, 1);
    // B1 .. B2: flag of this chunk's partials; merge the chunks of a KV head
    // (multi_sm_decode.py:243-259); everyone gathers the attention vector -> x1
    if (c.att) {
      ++aphase;
      if (ew == 0) {
        lds_wait(c.mb_out + 2, kWavesC * aphase);   // the compute waves issued their partials
        if (lane == 0) st_flag(flagp(l, kExPart) + c.wg, c.tag);
      }
    }
    if (c.merger) {
      poll_flags(flagp(l, kExPart) + c.ag * c.nch, c.nch, c.tag, a.ctrl, lane, bad);
      gather_x(X + lay.x_part + int64_t(c.ag) * c.npart, c.npart, c.sh_x1, c.tag, a.ctrl, ew, lane, bad);
      xsync(c.sh_sync, sphase, lane);
      for (int n = ew; n < c.GQ; n += kWavesX) {
        float M = -INFINITY;
        for (int ch = 0; ch < c.nch; ++ch) {
          const float* pc = c.sh_x1 + (ch * c.GQ + n) * kPartStride;
          if (pc[1] > 0.f) M = fmaxf(M, pc[0]);
        }
        float num = 0.f, den = 0.f;
        for (int ch = 0; ch < c.nch; ++ch) {
          const float* pc = c.sh_x1 + (ch * c.GQ + n) * kPartStride;
          if (pc[1] > 0.f) {
            const float wgt = expf(pc[0] - M);
            num += wgt * pc[2 + lane];
            den += wgt * pc[1];
          }
        }
        for (int r = 0; r < kRep; ++r)
          st_tag(X + lay.x_attn + r * lay.x_rep + (c.ag * c.GQ + n) * kDh + lane, num / den, c.tag);
      }
      xsync(c.sh_sync, sphase, lane);   // every head's words are issued, the partials in x1 are no longer read
      if (ew == 0 && lane == 0) st_flag(flagp(l, kExAttn) + c.ag, c.tag);
      MSD_TRACE_POINT(ew == 0, 2);
    }
    poll_flags(flagp(l, kExAttn), c.KV, c.tag, a.ctrl, lane, bad);
    gather_x(X + lay.x_attn + myrep, D, c.sh_x1, c.tag, a.ctrl, ew, lane, bad);
    MSD_TRACE_POINT(ew == 0, 3);
    __syncthreads();  // B2
    MSD_TRACE_POINT(ew == 0, 4);
    // B2 .. B3: publish O rows; h += O output, x0 = rmsnorm2(h)
    publish(X, flagp(l, kExHd1) + c.wg, true);
    poll_flags(flagp(l, kExHd1), G, c.tag, a.ctrl, lane, bad);
    add_h(X + lay.x_hd1 + myrep);
    MSD_TRACE_POINT(ew == 0, 5);
    norm_to(c.sh_x0);
    MSD_TRACE_POINT(ew == 0, 6);
    load_scale(l + 1 < c.L ? layer_w(a, l + 1) + lay.off_ln1 : a.lnf);
    __syncthreads();  // B3
    MSD_TRACE_POINT(ew == 0, 7);
    // B3 .. B4: publish gate/up outputs; act -> x1
    publish(X, flagp(l, kExAct) + c.wg, true);
    poll_flags(flagp(l, kExAct), G, c.tag, a.ctrl, lane, bad);
    gather_x(X + lay.x_act + myrep, c.ff, c.sh_x1, c.tag, a.ctrl, ew, lane, bad);
    MSD_TRACE_POINT(ew == 0, 8);
    __syncthreads();  // B4
    MSD_TRACE_POINT(ew == 0, 9);
    // B4 .. B0': publish down rows; h += down output, x0 = rmsnorm1 of the next layer (or the final norm)
    publish(X, flagp(l, kExHd2) + c.wg, true);
    poll_flags(flagp(l, kExHd2), G, c.tag, a.ctrl, lane, bad);
    add_h(X + lay.x_hd2 + myrep);
    MSD_TRACE_POINT(ew == 0, 10);
    norm_to(c.sh_x0);
    __syncthreads();  // B0'
    MSD_TRACE_POINT(ew == 0, 11);
  }
  __syncthreads();  // logits done
}

// ---------------------------------------------------------------- compute waves
template <int D, int FF, int FRW>
__device__ void compute_role(const Args& a, const Ctx& c) {
  constexpr int NLD = (D + 511) / 512;
  constexpr int FFL = (FF + 511) / 512;
  constexpr int ff = FF;
  const int lane = c.lane, wv = c.wv;
  const Layout& lay = a.lay;
  const int tidc = wv * 64 + lane;   // index among the compute threads
  int qp0, qp1, or0, or1, f0, f1;
  split(c.nqkv / 2, c.G, c.wg, qp0, qp1);
  split(D, c.G, c.wg, or0, or1);
  split(ff, c.G, c.wg, f0, f1);
  const int myqp = qp0 + wv, myor = or0 + wv;
  const bool has_qp = myqp < qp1, has_or = myor < or1;
  const float* rope = a.rope + int64_t(c.pos) * kDh;
  const int nkv16 = c.att ? c.ncached * 16 : 0;   // 16-byte pieces of cached K/V: 8 of K, 8 of V per row

  // Weights are loaded one phase ahead: right after a phase's dot products, the rows of
  // the next phase are requested, so the loads overlap the exchange that precedes it.
  Row<NLD> qb0, qb1, ob, gbg[FRW], gbu[FRW];
  Row<FFL> db;
  uint4 kvr[4];
  auto load_qkv = [&](int l) {
    if (has_qp) {
      load_row(qb0, layer_w(a, l) + lay.off_qkv + int64_t(2 * myqp) * D, D, lane);
      load_row(qb1, layer_w(a, l) + lay.off_qkv + int64_t(2 * myqp + 1) * D, D, lane);
    }
    // cached K/V rows of this workgroup's attention chunk (rows < pos of layer l)
    uint16_t* kc = layer_k(a, l);
    uint16_t* vc = kc + int64_t(c.KV) * a.ctx * kDh;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int t = tidc + j * (kWavesC * 64);
      if (t < nkv16) {
        const int prow = t >> 4, piece = t & 15;
        const uint16_t* src = ((piece >= 8) ? vc : kc) + (int64_t(c.ag) * a.ctx + c.q0 + prow) * kDh + (piece & 7) * 8;
        kvr[j] = *reinterpret_cast<const uint4*>(src);
      }
    }
  };
  auto load_o = [&](int l) { if (has_or) load_row(ob, layer_w(a, l) + lay.off_o + int64_t(myor) * D, D, lane); };
  auto load_gu = [&](int l) {
#pragma unroll
    for (int j = 0; j < FRW; ++j) {
      const int f = f0 + wv * FRW + j;   // contiguous gate/up pairs per wave
      if (f < f1) {
        load_row(gbg[j], layer_w(a, l) + lay.off_gu + int64_t(2 * f) * D, D, lane);
        load_row(gbu[j], layer_w(a, l) + lay.off_gu + int64_t(2 * f + 1) * D, D, lane);
      }
    }
  };
  auto load_dn = [&](int l) { if (has_or) load_row(db, layer_w(a, l) + lay.off_dn + int64_t(myor) * ff, ff, lane); };

  // Outputs go through the LDS mailbox to exchange wave 0, which stores them; the compute
  // waves request the next phase's weights only after the outputs are published, so the
  // latency-critical stores leave this CU ahead of the bulk loads.
  int cphase = 0;
  auto post = [&](int j, int idx, float v) {
    if (lane == 0) {
      c.mb_idx[wv * kMbox + j] = idx;
      c.mb_val[wv * kMbox + j] = v;
    }
  };
  auto handoff = [&]() {
    ++cphase;
    lds_bump(c.mb_out, lane);
    lds_wait(c.mb_pub, cphase);
  };

  load_qkv(0);
  __syncthreads();
  for (int l = 0; l < c.L; ++l) {
    uint64_t* X = layer_x(a, l);
    uint16_t* kcache = layer_k(a, l);
    uint16_t* vcache = kcache + int64_t(c.KV) * a.ctx * kDh;

    // ---- B0 .. B1: QKV rows, RoPE, KV write (multi_sm_decode.py:121-180)
    MSD_TRACE_POINT(wv == 0, 16);
    // Stores share the in-order vmcnt counter with loads, so every phase computes its dot
    // products first, then requests the next phase's weights, and publishes last: later
    // waits for those weights never wait behind a store.
    int i0 = 0, i1 = 0, head = 0;
    float o0 = 0.f, o1 = 0.f;
    if (has_qp) {
      XV<NLD> xv;
      load_x(xv, c.sh_x0, D, lane);
      const float s0 = dot_row(qb0, xv);
      const float s1 = dot_row(qb1, xv);
      const int row = 2 * myqp;
      head = row / kDh;
      const int rr = row % kDh;
      if (head < c.H + c.KV) {  // q or k rows (i, i+32): rotate-half RoPE (model.py:110-117)
        const int i = rr / 2;
        const float cs = rope[i], sn = rope[kDh / 2 + i];
        o0 = s0 * cs - s1 * sn;
        o1 = s0 * sn + s1 * cs;
        i0 = head * kDh + i;
        i1 = i0 + kDh / 2;
      } else {
        o0 = s0;
        o1 = s1;
        i0 = head * kDh + rr;
        i1 = i0 + 1;
      }
    }
    MSD_TRACE_POINT(wv == 0, 17);
    post(0, has_qp ? int(lay.x_qkv) + i0 : -1, o0);
    post(1, has_qp ? int(lay.x_qkv) + i1 : -1, o1);
#pragma unroll
    for (int j = 2; j < kMbox; ++j) post(j, -1, 0.f);
    handoff();
    load_o(l);
    if (has_qp && lane == 0) {
      if (head >= c.H) {  // K (post-RoPE) or V row of the cache at pos, bf16 (multi_sm_decode.py:179-180)
        const bool isv = head >= c.H + c.KV;
        const int kvh = isv ? head - c.H - c.KV : head - c.H;
        uint16_t* cp = (isv ? vcache : kcache) + (int64_t(kvh) * a.ctx + c.pos) * kDh;
        cp[i0 - head * kDh] = f2bf(o0);
        cp[i1 - head * kDh] = f2bf(o1);
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int t = tidc + j * (kWavesC * 64);
      if (t < nkv16) {   // K rows padded to kKPad floats (conflict-free 128-bit reads in the score loop)
        const int prow = t >> 4, piece = t & 15;
        float* dst = (piece >= 8) ? c.sh_v + prow * kDh + (piece & 7) * 8 : c.sh_k + prow * kKPad + (piece & 7) * 8;
        const uint4 u = kvr[j];
        dst[0] = bf_lo(u.x); dst[1] = bf_hi(u.x); dst[2] = bf_lo(u.y); dst[3] = bf_hi(u.y);
        dst[4] = bf_lo(u.z); dst[5] = bf_hi(u.z); dst[6] = bf_lo(u.w); dst[7] = bf_hi(u.w);
      }
    }
    __syncthreads();  // B1
    MSD_TRACE_POINT(wv == 0, 18);

    // ---- B1 .. B2: attention over this chunk, one head per compute wave (multi_sm_decode.py:182-221)
    if (c.att) {
      for (int n = wv; n < c.GQ; n += kWavesC) {
        // scores: lane = position; q (same for every lane) in registers, the lane's K row
        // read as 16 independent 128-bit LDS loads
        const float4* q4 = reinterpret_cast<const float4*>(c.sh_q + n * kDh);
        float s = -INFINITY;
        if (lane < c.P) {
          const float4* kr = reinterpret_cast<const float4*>(c.sh_k + lane * kKPad);
          float4 kk[kDh / 4];
#pragma unroll
          for (int j = 0; j < kDh / 4; ++j) kk[j] = kr[j];
          float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
#pragma unroll
          for (int j = 0; j < kDh / 4; ++j) {
            const float4 qq = q4[j];
            a0 += qq.x * kk[j].x;
            a1 += qq.y * kk[j].y;
            a2 += qq.z * kk[j].z;
            a3 += qq.w * kk[j].w;
          }
          s = ((a0 + a1) + (a2 + a3)) * 0.125f;
        }
        const float m = wave_max(s);
        const float e = (lane < c.P) ? expf(s - m) : 0.f;
        const float lsum = wave_sum(e);
        // o[lane = dim] = sum_p e[p] * V[p][lane]: V entries read 16 positions ahead, the
        // weights e[p] taken from lane p as wave-uniform values
        float o4[4] = {0.f, 0.f, 0.f, 0.f};
        for (int p0 = 0; p0 < c.P; p0 += 16) {
          float vv[16];
#pragma unroll
          for (int k = 0; k < 16; ++k) vv[k] = (p0 + k < c.P) ? c.sh_v[(p0 + k) * kDh + lane] : 0.f;
#pragma unroll
          for (int k = 0; k < 16; ++k) {
            const float ek = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e), p0 + k));
            o4[k & 3] += ek * vv[k];
          }
        }
        const float o = (o4[0] + o4[1]) + (o4[2] + o4[3]);
        uint64_t* part = X + lay.x_part + (int64_t(c.ag * c.nch + c.ac) * c.GQ + n) * kPartStride;
        if (lane == 0) {
          st_tag(part + 0, c.P > 0 ? m : -INFINITY, c.tag);
          st_tag(part + 1, lsum, c.tag);
        }
        st_tag(part + 2 + lane, o, c.tag);
        __builtin_amdgcn_wave_barrier();
      }
      lds_bump(c.mb_out + 2, lane);   // exchange wave 0 raises the chunk's flag after all heads
      MSD_TRACE_POINT(wv == 0, 19);
    }
    __syncthreads();  // B2
    MSD_TRACE_POINT(wv == 0, 20);

    // ---- B2 .. B3: O rows (multi_sm_decode.py:223-232)
    float yo = 0.f;
    if (has_or) {
      XV<NLD> xv;
      load_x(xv, c.sh_x1, D, lane);
      yo = dot_row(ob, xv);
    }
    MSD_TRACE_POINT(wv == 0, 21);
    post(0, has_or ? int(lay.x_hd1) + myor : -1, yo);
#pragma unroll
    for (int j = 1; j < kMbox; ++j) post(j, -1, 0.f);
    handoff();
    load_gu(l);
    __syncthreads();  // B3
    MSD_TRACE_POINT(wv == 0, 22);

    // ---- B3 .. B4: gate/up rows + SwiGLU (multi_sm_decode.py:262-289, model.py:159)
    XV<NLD> xg;
    if (f0 + wv * FRW < f1) load_x(xg, c.sh_x0, D, lane);
    float act[FRW];
#pragma unroll
    for (int j = 0; j < FRW; ++j) {
      const int f = f0 + wv * FRW + j;   // contiguous gate/up pairs per wave
      act[j] = 0.f;
      if (f < f1) {
        const float gt = dot_row(gbg[j], xg);
        const float up = dot_row(gbu[j], xg);
        act[j] = (gt * (1.f / (1.f + expf(-gt)))) * up;
      }
    }
    MSD_TRACE_POINT(wv == 0, 23);
#pragma unroll
    for (int j = 0; j < kMbox; ++j) {
      const int f = f0 + wv * FRW + j;   // contiguous gate/up pairs per wave
      post(j, (j < FRW && f < f1) ? int(lay.x_act) + f : -1, j < FRW ? act[j < FRW ? j : 0] : 0.f);
    }
    handoff();
    load_dn(l);
    __syncthreads();  // B4
    MSD_TRACE_POINT(wv == 0, 24);

    // ---- B4 .. B0': down rows (multi_sm_decode.py:273-291)
    float yd = 0.f;
    if (has_or) yd = dot_row_lds(db, c.sh_x1, ff, lane);
    MSD_TRACE_POINT(wv == 0, 25);
    post(0, has_or ? int(lay.x_hd2) + myor : -1, yd);
#pragma unroll
    for (int j = 1; j < kMbox; ++j) post(j, -1, 0.f);
    handoff();
    if (l + 1 < c.L) load_qkv(l + 1);
    __syncthreads();  // B0'
    MSD_TRACE_POINT(wv == 0, 26);
  }
  // ---- tied logits over this workgroup's vocabulary rows (multi_sm_decode.py:314-337)
  int v0, v1;
  split(a.V, c.G, c.wg, v0, v1);
  float best = -INFINITY;
  int besti = 0x7fffffff;
  constexpr int B = 4;
  XV<NLD> xv;
  load_x(xv, c.sh_x0, D, lane);
  for (int base = v0 + wv * B; base < v1; base += kWavesC * B) {
    Row<NLD> rr[B];
#pragma unroll
    for (int j = 0; j < B; ++j)
      if (base + j < v1) load_row(rr[j], a.outp + int64_t(base + j) * D, D, lane);
#pragma unroll
    for (int j = 0; j < B; ++j) {
      if (base + j < v1) {
        const float y = dot_row(rr[j], xv);
        if (lane == 0) a.logits[base + j] = y;
        if (y > best) { best = y; besti = base + j; }
      }
    }
  }
  if (lane == 0) {
    c.sh_red[wv] = best;
    reinterpret_cast<int*>(c.sh_red)[8 + wv] = besti;
  }
  __syncthreads();  // logits done
  if (wv == 0 && lane == 0) {   // argmax: larger value wins, ties -> lower index (np.argmax)
    float bv = c.sh_red[0];
    int bi = reinterpret_cast<int*>(c.sh_red)[8];
    for (int w = 1; w < kWavesC; ++w) {
      const float v = c.sh_red[w];
      const int i = reinterpret_cast<int*>(c.sh_red)[8 + w];
      if (v > bv || (v == bv && i < bi)) { bv = v; bi = i; }
    }
    uint64_t* keyp = reinterpret_cast<uint64_t*>(a.ctrl + 2);
    if (bi != 0x7fffffff)
      __hip_atomic_fetch_max(keyp, argmax_key(bv, bi), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // the max above completes before the arrival below is issued
    __builtin_amdgcn_s_waitcnt(0);
    const uint32_t old = __hip_atomic_fetch_add(a.ctrl + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if ((old % uint32_t(c.G)) == uint32_t(c.G - 1)) {   // last arriver publishes the token
      const uint64_t key = __hip_atomic_load(keyp, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      a.next_token[0] = int32_t(0xffffffffu - uint32_t(key & 0xffffffffu));
      a.next_token[1] = int32_t(ld_status(a.ctrl));
      __hip_atomic_store(keyp, uint64_t(0), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

template <int D, int FF, int FRW>
__global__ __launch_bounds__(kThreadsWG, 1) void decode_step_kernel(Args a) {
  extern __shared__ float smem[];
  Ctx c;
  c.G = gridDim.x;
  c.wg = blockIdx.x;
  c.lane = threadIdx.x & 63;
  c.wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // wave-uniform (scalar register)
  c.H = a.H;
  c.KV = a.KV;
  c.GQ = a.H / a.KV;
  c.ff = a.ff;
  c.L = a.L;
  c.nch = a.nch;
  c.npart = c.nch * c.GQ * kPartStride;
  c.nqkv = (a.H + 2 * a.KV) * kDh;
  c.pos = a.pos;
  c.tag = a.epoch;
  const int ch_max = (a.ctx + c.nch - 1) / c.nch;
  // attention: workgroup i < KV*nch handles KV head i / nch, position chunk i % nch
  c.att = c.wg < c.KV * c.nch;
  c.ag = c.wg / c.nch;
  c.ac = c.wg % c.nch;
  c.merger = c.att && c.ac == 0;
  const int npos = c.pos + 1;
  const int cs = (npos + c.nch - 1) / c.nch;
  c.q0 = min(c.ac * cs, npos);
  c.q1 = min(c.q0 + cs, npos);
  c.P = c.q1 - c.q0;
  c.ncached = max(0, min(c.q1, c.pos) - c.q0);
  const int xmax = (max(max(D, c.ff), c.npart) + 3) & ~3;   // keeps sh_k 16-byte aligned
  c.sh_x0 = smem;
  c.sh_x1 = c.sh_x0 + D;
  c.sh_k = c.sh_x1 + xmax;
  c.sh_v = c.sh_k + ch_max * kKPad;
  c.sh_q = c.sh_v + ch_max * kDh;
  c.sh_e = c.sh_q + c.GQ * kDh;
  c.sh_red = c.sh_e + kWavesC * 64;
  c.sh_sync = reinterpret_cast<int*>(c.sh_red + 64);
  c.mb_val = c.sh_red + 64 + 4;
  c.mb_idx = reinterpret_cast<int*>(c.mb_val + kWavesC * kMbox);
  c.mb_out = c.mb_idx + kWavesC * kMbox;   // [0] outputs written, [2] attention partials issued
  c.mb_pub = c.mb_out + 1;
  if (threadIdx.x == 0) {
    *c.sh_sync = 0;
    c.mb_out[0] = 0;
    c.mb_out[1] = 0;
    c.mb_out[2] = 0;
  }
  __syncthreads();

  int token = a.token_dev ? *a.token_dev : a.token;
  if (token < 0 || token >= a.V) {
    if (c.wg == 0 && threadIdx.x == 0) atomicOr(a.ctrl, kStatusBadToken);
    token = token < 0 ? 0 : a.V - 1;
  }
  if (c.wv >= kWavesC) exchange_role<D>(a, c, token);
  else compute_role<D, FF, FRW>(a, c);
}

// ---------------------------------------------------------------- host side
struct Plan {   // per-config launch parameters
  int frw;      // gate/up rows per compute wave
  int ffl;      // 16-byte pieces per lane of a d_ff row
  size_t lds;
};

static bool config_ok(const msd_config* c) {
  if (!c) return false;
  if (c->d_head != kDh || c->n_heads <= 0 || c->n_kv_heads <= 0 || c->n_layers <= 0) return false;
  if (c->n_heads * kDh != c->d_model || c->n_heads % c->n_kv_heads != 0) return false;
  if (c->d_ff <= 0 || c->d_ff % 16 != 0 || c->vocab_size <= 0 || c->context_len <= 0) return false;
  if (c->context_len > 1024) return false;
  if (c->d_model != 256 && c->d_model != 1024) return false;
  return true;
}

static int cdiv(int a, int b) { return (a + b - 1) / b; }

// Shapes the kernel instantiations cover for n_workgroups workgroups; false if unsupported.
static bool make_plan(const msd_config* c, int G, Plan* p) {
  if (!config_ok(c) || G <= 0) return false;
  const int nqkv = (c->n_heads + 2 * c->n_kv_heads) * kDh;
  if (cdiv(nqkv / 2, G) > kWavesC || cdiv(c->d_model, G) > kWavesC) return false;
  if (c->n_kv_heads * n_chunks(c->context_len) > G) return false;
  p->frw = cdiv(cdiv(c->d_ff, G), kWavesC);
  p->ffl = cdiv(c->d_ff, 512);
  const int GQ = c->n_heads / c->n_kv_heads;
  const int nch = n_chunks(c->context_len);
  const int ch_max = cdiv(c->context_len, nch);
  const int xmax = (std::max(std::max(c->d_model, c->d_ff), nch * GQ * kPartStride) + 3) & ~3;
  const size_t floats = size_t(c->d_model) + xmax + ch_max * (kKPad + kDh) + GQ * kDh + kWavesC * 64 + 64 + 4 +
                        2 * kWavesC * kMbox + 8;
  p->lds = floats * 4;
  return true;
}

// At least this much LDS per workgroup, so that no two workgroups of a step share a
// compute unit (160 KB per CU): the grid then spreads over every CU.
constexpr size_t kMinLds = 84 * 1024;

template <int D, int FF, int FRW>
static hipError_t launch_t(const Args& a, int grid, size_t lds, hipStream_t s) {
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&decode_step_kernel<D, FF, FRW>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  hipLaunchKernelGGL((decode_step_kernel<D, FF, FRW>), dim3(grid), dim3(kThreadsWG), lds, s, a);
  return hipGetLastError();
}

// Instantiated shapes (d_model, d_ff, gate/up rows per compute wave): the tiny and the
// 306M configurations on 256 workgroups, and the same shapes on fewer workgroups.
static hipError_t launch(const Args& a, const Plan& p, int d, int ff, int grid, size_t lds, hipStream_t s) {
  if (d == 256 && ff == 704 && p.frw == 1) return launch_t<256, 704, 1>(a, grid, lds, s);
  if (d == 1024 && ff == 2816 && p.frw == 3) return launch_t<1024, 2816, 3>(a, grid, lds, s);
  return hipErrorInvalidValue;
}

static bool plan_instantiated(const msd_config* c, const Plan& p) {
  return (c->d_model == 256 && c->d_ff == 704 && p.frw == 1) ||
         (c->d_model == 1024 && c->d_ff == 2816 && p.frw == 3);
}

}  // namespace msd

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
  const Layout t = make_layout(cfg->d_model, cfg->n_heads, cfg->n_kv_heads, cfg->d_ff, cfg->context_len, n_workgroups);
  return t.ctrl_bytes + t.x_layer * cfg->n_layers * int64_t(sizeof(uint64_t)) +
         t.flag_words * cfg->n_layers * int64_t(sizeof(uint32_t));
}

extern "C" int32_t msd_default_workgroups(int32_t device) {
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess) return MSD_E_HIP;
  return n;
}

extern "C" int32_t msd_decode_step(const msd_config* cfg, const void* token_emb, const void* output_proj,
                                   const void* packed_w, const void* lnf_s, const float* rope, int32_t token_id,
                                   const int32_t* token_dev, int32_t pos, void* kv, void* workspace,
                                   uint32_t epoch, float* logits, int32_t* next_token,
                                   int32_t n_workgroups, void* stream) {
  Plan p;
  if (!config_ok(cfg)) return MSD_E_CONFIG;
  if (n_workgroups <= 0 || n_workgroups > 4096) return MSD_E_ARG;
  if (!make_plan(cfg, n_workgroups, &p) || !plan_instantiated(cfg, p)) return MSD_E_CONFIG;
  if (!token_emb || !output_proj || !packed_w || !lnf_s || !rope || !kv || !workspace || !logits || !next_token)
    return MSD_E_ARG;
  if (pos < 0 || pos >= cfg->context_len) return MSD_E_ARG;
  if (!token_dev && (token_id < 0 || token_id >= cfg->vocab_size)) return MSD_E_ARG;
  if (epoch == 0) return MSD_E_ARG;
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
  a.lay = make_layout(cfg->d_model, cfg->n_heads, cfg->n_kv_heads, cfg->d_ff, cfg->context_len, n_workgroups);
  a.xw = reinterpret_cast<uint64_t*>(static_cast<char*>(workspace) + a.lay.ctrl_bytes);
  a.flags = reinterpret_cast<uint32_t*>(a.xw + a.lay.x_layer * cfg->n_layers);
  a.token = token_id;
  a.pos = pos;
  a.epoch = epoch;
  a.H = cfg->n_heads;
  a.KV = cfg->n_kv_heads;
  a.L = cfg->n_layers;
  a.ff = cfg->d_ff;
  a.V = cfg->vocab_size;
  a.ctx = cfg->context_len;
  a.nch = n_chunks(cfg->context_len);
  const size_t lds = std::max(p.lds, kMinLds);
  const hipError_t e = launch(a, p, cfg->d_model, cfg->d_ff, n_workgroups, lds, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? MSD_OK : MSD_E_HIP;
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
extern "C" int msd_trace_copy(void* host) {
  return hipMemcpyFromSymbol(host, HIP_SYMBOL(msd::msd_trace_buffer), sizeof(uint64_t) * 4096 * 32) == hipSuccess ? 0 : -1;
}
#endif
