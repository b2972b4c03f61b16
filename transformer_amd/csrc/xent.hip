// Fused output projection + cross-entropy, forward and backward, on the matrix cores (gfx950).
//
// Reference: model.py:279-379 -- _chunked_ce_fwd (chunked online logsumexp, :281-302),
// fused_cross_entropy (jax.custom_vjp, :305-312), _fused_ce_bwd (:320-361) and
// fused_output_and_loss (:367-379).  h (N, d) and weight (V, d) are bf16 (train.py:113 casts the
// parameters to bf16), targets int32 (N).  Every logit is a bf16 x bf16 dot product accumulated
// in f32 (v_mfma_f32_32x32x16_bf16); softmax statistics are f32.
//
// Forward (msd_xent_forward): one GEMM S^T = W h^T over the whole vocabulary whose epilogue never
// stores it: each 256 x 256 tile (256 vocabulary ids x 256 tokens) reduces its token columns to a
// partial (max, sum of exp(s - max)) and captures the target logits (the transposed product puts
// one token's 64 values per tile in each lane's registers, so the reduction stays in registers);
// xent_lse merges a token's partials in a fixed order (lse = max + log sum, the online logsumexp
// of :293-301), xent_mean takes the mean of lse - target logit in a fixed order (float64 sum).
// The logits never exist in memory, as in the reference, whose chunk loop materialises only one
// (N, chunk) block at a time.
//
// Backward (msd_xent_backward), per vocabulary chunk of `chunk` columns (the reference's
// chunk loop, :344-353; the chunk bounds the probability buffers):
//   1. xent_gemm<kEpiProb>: S^T = W_c h^T, then P' = (exp(S - lse) - onehot(target)) * g / N as
//      bf16, stored as PT (C x N) and P (N x C) through LDS staging;
//   2. xent_gemm<kEpiStoreBf16>: grad_W[c] = PT h   (A = PT, B = h^T: the whole reduction over
//      N rows, so the chunk's rows of grad_W are final);
//   3. xent_gemm<kEpiAccF32>: grad_h += P W_c   (A = P, B = W^T columns of the chunk), in f32
//      across chunks in order; the last chunk also writes the bf16 result.
// The target terms (:356-358) ride in P' (its -1 at the target column), so grad_h = (softmax -
// onehot) W g/N and grad_W = (softmax - onehot)^T h g/N as in the reference.  The forward's lse
// is reused instead of recomputing the logsumexp (:331-340); W^T and h^T are made once per call
// (xent_transpose) so that every GEMM reads both operands along K.
//
// GEMM (xent_gemm<TM, TN, EPI>): C = A B^T with A (M x K) and B (Nn x K) both K-contiguous bf16.
// A workgroup of GM x GN waves owns a TM x TN tile (256 x 256 with 2 x 4 waves for the forward
// logits and the backward's probability block, 128 x 128 with 2 x 2 waves for grad_W and grad_h),
// each wave a block of 32 x 32 MFMA tiles.  K advances 32 at a time through a ring of 4 LDS
// stages filled by direct DMA (global_load_lds, 16 bytes per lane), three stages in flight; a
// stage row is 64 bytes whose four 16-byte pieces are stored XOR-swizzled by the row, so the rows
// an MFMA fragment reads hit distinct banks.  Tiles are dealt to the 8 XCDs in contiguous ranges
// (workgroup i runs on XCD i % 8), so the workgroups of one XCD share operand rows in its L2.
// (XENT_DMA=0 builds the register-staged variant: two stages of K = 64, each thread's pieces
// loaded into registers before the current stage's MFMAs and stored to LDS after.)
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <math.h>

#include <algorithm>
#include <utility>

#include "../../include/msxent.h"
#include "internal.h"

namespace mxe {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));   // a native vector (HIP's uint4 is a struct)

constexpr int kBK = 64;           // K per LDS stage
// Waves of the 256 x 256 GEMMs (the logits of the forward and the backward's probability block):
// 4 (2 x 2, 128 x 128 per wave) or 8 (2 x 4, 128 x 64 per wave: two waves per SIMD)
#ifndef XENT_BIG_WAVES
#define XENT_BIG_WAVES 8
#endif
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kStatusTarget = 4;  // a target id outside [0, V) (replaced by 0)

__device__ __forceinline__ bf16x8 as_bf(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

// round to nearest even (finite inputs; NaN stays NaN)
__device__ __forceinline__ uint16_t f2bf(float x) {
  const uint32_t u = __float_as_uint(x);
  if ((u & 0x7fffffffu) > 0x7f800000u) return uint16_t((u >> 16) | 0x40);
  return uint16_t((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

// exp(x) for x <= 0 (x = -inf gives 0): the hardware base-2 exponential of x log2(e)
__device__ __forceinline__ float exp_neg(float x) { return __builtin_amdgcn_exp2f(x * kLog2e); }

// reductions over the 32 lanes of a half-wave (the lanes that hold one row of an MFMA tile)
template <int X>
__device__ __forceinline__ float swz(float v) {
  return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), (X << 10) | 0x1f));
}
__device__ __forceinline__ float half_max(float v) {
  v = fmaxf(v, swz<1>(v));
  v = fmaxf(v, swz<2>(v));
  v = fmaxf(v, swz<4>(v));
  v = fmaxf(v, swz<8>(v));
  return fmaxf(v, swz<16>(v));
}
__device__ __forceinline__ float half_sum(float v) {
  v += swz<1>(v);
  v += swz<2>(v);
  v += swz<4>(v);
  v += swz<8>(v);
  return v + swz<16>(v);
}

enum Epi { kEpiLse = 0, kEpiProb = 1, kEpiAccF32 = 2, kEpiStoreBf16 = 3 };

struct GemmArgs {
  const uint16_t* A;   // M x K, row stride lda; rows >= a_valid read row a_valid - 1
  int64_t lda;
  int a_valid;
  const uint16_t* B;   // Nn x K, row stride ldb; rows >= b_valid read row b_valid - 1
  int64_t ldb;
  int b_valid;
  int K;               // multiple of kBK
  int tiles_m, tiles_n;
  int m_valid, n_valid;     // output rows / columns that exist (the rest are padding)
  const int32_t* targets;   // kEpiLse, kEpiProb: sanitized target per token (output column)
  int vcol0;                // kEpiProb: vocabulary index of output column 0
  const float* lse;         // kEpiProb: per token
  const float* grad;        // kEpiProb: the loss gradient g (device scalar)
  float inv_n;              // kEpiProb: 1 / N
  float* part;              // kEpiLse: (max, sum) per (vocabulary tile, token): [tiles_m][ldp][2]
  int64_t ldp;
  float* tgt;               // kEpiLse: target logit per token
  uint16_t* P;              // kEpiProb: tokens x ldP
  int64_t ldP;
  uint16_t* PT;             // kEpiProb: vocabulary ids x ldPT
  int64_t ldPT;
  float* acc;               // kEpiAccF32: f32 rows x ldacc
  int64_t ldacc;
  int accumulate;           // kEpiAccF32: add to acc (else overwrite)
  uint16_t* out;            // kEpiAccF32 (when not null: bf16 of the total), kEpiStoreBf16
  int64_t ldout;
};

// 1: operand tiles reach LDS by direct DMA (global_load_lds); 0: staged through registers
#ifndef XENT_DMA
#define XENT_DMA 1
#endif

// Stages of the LDS ring: as many (TM + TN) x 64-byte stages as 160 KB holds, at most kMaxStages;
// S - 1 stages are in flight while one is read.  (Measured: 5 stages for the 256 x 256 tiles and 8
// for the 128 x 128 ones were no faster than 4 -- the operand latency is already covered.)
#ifndef XENT_MAX_STAGES
#define XENT_MAX_STAGES 4
#endif
constexpr int kMaxStages = XENT_MAX_STAGES;
template <int TM, int TN>
constexpr int ring_stages() {
  return std::min(kMaxStages, (160 * 1024) / ((TM + TN) * 64));
}
template <int TM, int TN>
constexpr int stage_bytes() { return (TM + TN) * kBK * 2; }
template <int TM, int TN>
constexpr int staging_pitch() { return TN + 8; }   // bf16 per row of the epilogue's LDS tile
template <int TM, int TN, int EPI>
constexpr size_t lds_bytes() {
#if XENT_DMA
  constexpr size_t ring = size_t(ring_stages<TM, TN>()) * (TM + TN) * 64;
  return EPI == kEpiProb ? std::max<size_t>(ring, size_t(TM) * staging_pitch<TM, TN>() * 2 + TN * 8) : ring;
#endif
  // kEpiProb: the bf16 staging tile (over the stage buffers) and the rows' lse and targets after it
  return EPI == kEpiProb
             ? std::max<size_t>(2 * stage_bytes<TM, TN>(), size_t(TM) * staging_pitch<TM, TN>() * 2 + TN * 8)
             : size_t(2 * stage_bytes<TM, TN>());
}

// Tile (tm, tn) of workgroup b.  Workgroup b runs on XCD b % 8, which takes the tile ids
// [x * per, (x + 1) * per) in order; ids then walk blocks of GB column tiles, row tile by row
// tile, so the 32 workgroups an XCD holds at a time cover 4 row tiles x 8 column tiles and
// share their operand rows in its L2.
__device__ __forceinline__ void tile_of(int b, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int total = tiles_m * tiles_n, per = (total + 7) / 8;
  const int x = b & 7, k = b >> 3;
  int t = x * per + k;
  if (t >= total || per * 8 != total) t = b;   // uneven: the plain order
  const int GB = tiles_n % 8 == 0 ? 8 : (tiles_n % 4 == 0 ? 4 : 1);
  const int blk = t / (GB * tiles_m), rem = t % (GB * tiles_m);
  tm = rem / GB;
  tn = blk * GB + rem % GB;
}

// the 16-byte pieces of one stage: global -> registers, registers -> LDS (piece u is R rows
// after piece u - 1, R = threads / 8); the piece index is a constant of each expansion, so the
// arrays stay in registers
template <int N, size_t... U>
__device__ __forceinline__ void gload_(u32x4 (&r)[N], const uint16_t* base, const uint32_t (&off)[N], int kk,
                                       std::index_sequence<U...>) {
  ((r[U] = *reinterpret_cast<const u32x4*>(base + off[U] + kk)), ...);
}
template <int N>
__device__ __forceinline__ void gload(u32x4 (&r)[N], const uint16_t* base, const uint32_t (&off)[N], int kk) {
  gload_(r, base, off, kk, std::make_index_sequence<N>{});
}
template <int R, int N, size_t... U>
__device__ __forceinline__ void lstore_(uint8_t* dst, const u32x4 (&r)[N], std::index_sequence<U...>) {
  ((*reinterpret_cast<u32x4*>(dst + R * 128 * U) = r[U]), ...);
}
template <int R, int N>
__device__ __forceinline__ void lstore(uint8_t* dst, const u32x4 (&r)[N]) {
  lstore_<R>(dst, r, std::make_index_sequence<N>{});
}
template <int R, int N, size_t... U>
__device__ __forceinline__ void piece_offsets_(uint32_t (&off)[N], int row, int valid, int64_t ld, int col,
                                               std::index_sequence<U...>) {
  ((off[U] = uint32_t(min(row + R * int(U), valid - 1)) * uint32_t(ld) + col), ...);
}

// ---- direct-to-LDS pipeline (XENT_DMA): K advances 32 at a time through a ring of S LDS stages,
// S - 1 in flight.  Each lane's global_load_lds writes 16 bytes at (stage base + 1 KB per
// instruction + 16 lane); a stage row is 64 bytes (4 pieces of 8 K values) and holds piece c at
// position c ^ ((row >> 2) & 3).  Measured with a probe of ds_read_b128 address patterns
// (SQ_LDS_BANK_CONFLICT): the fragment read of 32 rows x one piece is conflict-free with this
// swizzle and takes twice the LDS cycles with c ^ ((row >> 1) & 3) or with no swizzle.  The
// fragment reads are inline assembly with explicit waits: the compiler would otherwise wait for
// every outstanding DMA (vmcnt(0)) before each LDS read, and __syncthreads' fence would too, so
// the stage barrier is a bare s_barrier after this wave's own DMAs of the stage have landed.
constexpr int kKD = 32;   // K per DMA stage
typedef __attribute__((address_space(3))) uint8_t lds_u8;
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return uint32_t(reinterpret_cast<uintptr_t>((const lds_u8*)p));
}
// (the host pass instantiates these templates along with the kernels but never emits them, and
// an x86 compile rejects the vector-register constraints and the LDS builtin, so their bodies
// are in the device pass only)
template <int N>
__device__ __forceinline__ void wait_vm() {
#if defined(__HIP_DEVICE_COMPILE__)
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
#endif
}
// Wait until at most n (< D, wave-uniform) stages of NIW DMA instructions are outstanding.
template <int NIW, int D>
__device__ __forceinline__ void wait_stages(int n) {
  if constexpr (D > 1) {
    if (n >= D - 1) {
      wait_vm<(D - 1) * NIW>();
      return;
    }
    wait_stages<NIW, D - 1>(n);
  } else {
    wait_vm<0>();
  }
}
// The fragment reads of one K step (16) of a DMA stage: fa[i] is the A fragment of row block i
// at a + 2048 i (32 rows of 64 bytes apart), fb[j] the B fragment at b + 2048 j.  The reads are
// issued by one assembly block and waited for by wait_frags, whose "+v" operands tie the
// fragments to the wait: the compiler cannot place a use (or a copy) of a fragment before the
// wait, while the MFMAs of the other K step may run between the two.
__device__ __forceinline__ void step_reads(u32x4 (&fa)[4], u32x4 (&fb)[2], uint32_t a, uint32_t b) {
#if defined(__HIP_DEVICE_COMPILE__)
  asm volatile(
      "ds_read_b128 %0, %6 offset:0\n"
      "ds_read_b128 %1, %6 offset:2048\n"
      "ds_read_b128 %2, %6 offset:4096\n"
      "ds_read_b128 %3, %6 offset:6144\n"
      "ds_read_b128 %4, %7 offset:0\n"
      "ds_read_b128 %5, %7 offset:2048"
      : "=&v"(fa[0]), "=&v"(fa[1]), "=&v"(fa[2]), "=&v"(fa[3]), "=&v"(fb[0]), "=&v"(fb[1])
      : "v"(a), "v"(b));
#endif
}
template <int N>
__device__ __forceinline__ void wait_frags(u32x4 (&fa)[4], u32x4 (&fb)[2]) {
#if defined(__HIP_DEVICE_COMPILE__)
  asm volatile("s_waitcnt lgkmcnt(%6)"
               : "+v"(fa[0]), "+v"(fa[1]), "+v"(fa[2]), "+v"(fa[3]), "+v"(fb[0]), "+v"(fb[1])
               : "n"(N));
#endif
}
__device__ __forceinline__ void step_reads(u32x4 (&fa)[2], u32x4 (&fb)[2], uint32_t a, uint32_t b) {
#if defined(__HIP_DEVICE_COMPILE__)
  asm volatile(
      "ds_read_b128 %0, %4 offset:0\n"
      "ds_read_b128 %1, %4 offset:2048\n"
      "ds_read_b128 %2, %5 offset:0\n"
      "ds_read_b128 %3, %5 offset:2048"
      : "=&v"(fa[0]), "=&v"(fa[1]), "=&v"(fb[0]), "=&v"(fb[1])
      : "v"(a), "v"(b));
#endif
}
template <int N>
__device__ __forceinline__ void wait_frags(u32x4 (&fa)[2], u32x4 (&fb)[2]) {
#if defined(__HIP_DEVICE_COMPILE__)
  asm volatile("s_waitcnt lgkmcnt(%4)" : "+v"(fa[0]), "+v"(fa[1]), "+v"(fb[0]), "+v"(fb[1]) : "n"(N));
#endif
}
__device__ __forceinline__ void step_reads(u32x4 (&fa)[4], u32x4 (&fb)[4], uint32_t a, uint32_t b) {
#if defined(__HIP_DEVICE_COMPILE__)
  asm volatile(
      "ds_read_b128 %0, %8 offset:0\n"
      "ds_read_b128 %1, %8 offset:2048\n"
      "ds_read_b128 %2, %8 offset:4096\n"
      "ds_read_b128 %3, %8 offset:6144\n"
      "ds_read_b128 %4, %9 offset:0\n"
      "ds_read_b128 %5, %9 offset:2048\n"
      "ds_read_b128 %6, %9 offset:4096\n"
      "ds_read_b128 %7, %9 offset:6144"
      : "=&v"(fa[0]), "=&v"(fa[1]), "=&v"(fa[2]), "=&v"(fa[3]), "=&v"(fb[0]), "=&v"(fb[1]), "=&v"(fb[2]), "=&v"(fb[3])
      : "v"(a), "v"(b));
#endif
}
template <int N>
__device__ __forceinline__ void wait_frags(u32x4 (&fa)[4], u32x4 (&fb)[4]) {
#if defined(__HIP_DEVICE_COMPILE__)
  asm volatile("s_waitcnt lgkmcnt(%8)"
               : "+v"(fa[0]), "+v"(fa[1]), "+v"(fa[2]), "+v"(fa[3]), "+v"(fb[0]), "+v"(fb[1]), "+v"(fb[2]),
                 "+v"(fb[3])
               : "n"(N));
#endif
}
template <int RB, int CB>
__device__ __forceinline__ void step_reads(u32x4 (&)[RB], u32x4 (&)[CB], uint32_t, uint32_t) {
  static_assert(RB < 0, "no fragment-read block for this wave tile");
}
// The NIW DMAs of one stage for this wave: instruction u fills the 1 KB at st + 1024 (wv + NW u)
// from A (u < UA) or B, at K offset kt * kKD past this lane's element offset doff[u].
template <int NIW, int UA, int NW>
__device__ __forceinline__ void dma_stage(const uint16_t* A, const uint16_t* B, const uint32_t (&doff)[NIW], int kt,
                                          uint8_t* st, int wv) {
#if defined(__HIP_DEVICE_COMPILE__)
#pragma unroll
  for (int u = 0; u < NIW; ++u)
    __builtin_amdgcn_global_load_lds((u < UA ? A : B) + doff[u] + kt * kKD,
                                     (__attribute__((address_space(3))) void*)(st + 1024 * (wv + NW * u)), 16, 0, 0);
#endif
}
// The MFMAs of one DMA stage (K = 32): both K steps' fragment reads issued together, the first
// step's MFMAs once its reads have landed (the second step's reads land meanwhile), then the
// second step's.  The scheduling barrier keeps the compiler from moving the first step's MFMAs
// past the second wait.
template <int RB, int CB>
__device__ __forceinline__ void mma_step(f32x16 (&acc)[RB][CB], const u32x4 (&fa)[RB], const u32x4 (&fb)[CB]) {
#pragma unroll
  for (int i = 0; i < RB; ++i)
#pragma unroll
    for (int j = 0; j < CB; ++j)
      acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf(fa[i]), as_bf(fb[j]), acc[i][j], 0, 0, 0);
}
template <int TM, int RB, int CB>
__device__ __forceinline__ void mma_stage_dma(f32x16 (&acc)[RB][CB], uint32_t a0, uint32_t a1, uint32_t b0,
                                              uint32_t b1) {
  u32x4 fa[RB], fb[CB], ga[RB], gb[CB];
  step_reads(fa, fb, a0, b0);
  step_reads(ga, gb, a1, b1);
  wait_frags<RB + CB>(fa, fb);
  mma_step(acc, fa, fb);
  __builtin_amdgcn_sched_barrier(0);
  wait_frags<0>(ga, gb);
  mma_step(acc, ga, gb);
}

// The MFMAs of one LDS stage (K = 64): 4 steps of 16, each reading this wave's RB A fragments and
// CB B fragments (row fr of each 32-row block, 16-byte piece 2 ks + fh of the swizzled row).
template <int TM, int WM, int WN, int RB, int CB>
__device__ __forceinline__ void mma_stage(f32x16 (&acc)[RB][CB], const uint8_t* As, int wm, int wn, int fr, int fh) {
  const uint8_t* Bs = As + TM * 128;
#pragma unroll
  for (int ks = 0; ks < kBK / 16; ++ks) {
    const int sw = ((2 * ks + fh) ^ (fr & 7)) << 4;
    u32x4 af[RB], bf[CB];
#pragma unroll
    for (int i = 0; i < RB; ++i) af[i] = *reinterpret_cast<const u32x4*>(As + (wm * WM + i * 32 + fr) * 128 + sw);
#pragma unroll
    for (int j = 0; j < CB; ++j) bf[j] = *reinterpret_cast<const u32x4*>(Bs + (wn * WN + j * 32 + fr) * 128 + sw);
#pragma unroll
    for (int i = 0; i < RB; ++i)
#pragma unroll
      for (int j = 0; j < CB; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf(af[i]), as_bf(bf[j]), acc[i][j], 0, 0, 0);
  }
}

template <int TM, int TN, int GM, int GN, int EPI>
__global__ __launch_bounds__(64 * GM * GN) void xent_gemm(GemmArgs g) {
  extern __shared__ __align__(16) uint8_t smem[];
  constexpr int kThreads = 64 * GM * GN;    // GM x GN waves
  constexpr int WM = TM / GM, WN = TN / GN;   // wave tile
  constexpr int RB = WM / 32, CB = WN / 32;
  constexpr int STAGE = stage_bytes<TM, TN>();
  constexpr int LA = TM * 8 / kThreads, LB = TN * 8 / kThreads;   // 16-byte pieces per thread per stage
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wv / GN, wn = wv % GN;
  int tm, tn;
  tile_of(blockIdx.x, g.tiles_m, g.tiles_n, tm, tn);
  const int row0 = tm * TM, col0 = tn * TN;

  f32x16 acc[RB][CB];
#pragma unroll
  for (int i = 0; i < RB; ++i)
#pragma unroll
    for (int j = 0; j < CB; ++j) acc[i][j] = f32x16{};
  const int fr = lane & 31, fh = lane >> 5;
#if XENT_DMA
  {
    constexpr int NW = GM * GN, SD = (TM + TN) * 64, NI = (TM + TN) / 16, NIW = NI / NW, UA = TM / (16 * NW);
    static_assert(NI % NW == 0 && TM % (16 * NW) == 0, "whole DMA instructions per wave, A before B");
    constexpr int S = ring_stages<TM, TN>(), D = S - 1;
    static_assert(S >= 2 && S * SD <= 160 * 1024, "LDS ring");
    // instruction u of this wave covers stage rows 16 (wv + NW u) .. + 16: A rows for u < UA, then
    // B rows; this lane's row of it and the K piece it loads into position lane % 4
    uint32_t doff[NIW];
#pragma unroll
    for (int u = 0; u < NIW; ++u) {
      const int r = 16 * (wv + NW * u) + (lane >> 2) - (u < UA ? 0 : TM);
      const int piece = (lane & 3) ^ ((r >> 2) & 3);
      doff[u] = u < UA ? uint32_t(min(row0 + r, g.a_valid - 1)) * uint32_t(g.lda) + 8 * piece
                       : uint32_t(min(col0 + r, g.b_valid - 1)) * uint32_t(g.ldb) + 8 * piece;
    }
    const int KT = g.K / kKD;
    for (int s = 0; s < D && s < KT; ++s) dma_stage<NIW, UA, NW>(g.A, g.B, doff, s, smem + s * SD, wv);
    // this lane's fragment rows and swizzled pieces (the swizzle depends only on fr)
    const uint32_t base = lds_addr(smem);
    const uint32_t sw0 = ((0 + fh) ^ ((fr >> 2) & 3)) << 4, sw1 = ((2 + fh) ^ ((fr >> 2) & 3)) << 4;
    const uint32_t ar = (wm * WM + fr) * 64, br = TM * 64 + (wn * WN + fr) * 64;
    int rd = 0;   // ring slot of stage kt; stage kt + D goes to the slot stage kt - 1 used
    for (int kt = 0; kt < KT; ++kt) {
      wait_stages<NIW, D>(min(KT, kt + D) - kt - 1);   // stage kt landed
      __builtin_amdgcn_s_barrier();   // every wave's part of stage kt landed; stage kt - 1 read by all
      const int is = rd == 0 ? S - 1 : rd - 1;
      if (kt + D < KT) dma_stage<NIW, UA, NW>(g.A, g.B, doff, kt + D, smem + is * SD, wv);
      const uint32_t sb = base + rd * SD;
      mma_stage_dma<TM, RB, CB>(acc, sb + ar + sw0, sb + ar + sw1, sb + br + sw0, sb + br + sw1);
      rd = rd == S - 1 ? 0 : rd + 1;
    }
    __builtin_amdgcn_s_barrier();   // the epilogue reuses the ring
  }
#else
  // this thread's pieces: piece q = tid + T u (T threads) is row q / 8 = tid / 8 + (T / 8) u at
  // 16-byte column q % 8 = tid % 8, so its LDS offset is a fixed one plus (T / 8) rows per u (the
  // swizzle depends on the row only through row & 7 = (tid / 8) & 7)
  const int pr = tid >> 3, pc = tid & 7;
  const int poff = pr * 128 + ((pc ^ (pr & 7)) << 4);
  uint32_t aof[LA], bof[LB];   // element offsets of the pieces (rows clamped to the valid ones)
  constexpr int R = kThreads / 8;   // rows between a thread's pieces
  piece_offsets_<R>(aof, row0 + pr, g.a_valid, g.lda, 8 * pc, std::make_index_sequence<LA>{});
  piece_offsets_<R>(bof, col0 + pr, g.b_valid, g.ldb, 8 * pc, std::make_index_sequence<LB>{});
  u32x4 ra[LA], rb[LB];

  const int KT = g.K / kBK;
  gload(ra, g.A, aof, 0);
  gload(rb, g.B, bof, 0);
  lstore<R>(smem + poff, ra);
  lstore<R>(smem + poff + TM * 128, rb);
  __syncthreads();
  // fragment rows of this lane: row (lane & 31) of each 32-row block; its 8 K values at 16-byte
  // piece 2 ks + lane / 32 of the stage row
  for (int kt = 0; kt < KT; ++kt) {
    if (kt + 1 < KT) {
      gload(ra, g.A, aof, (kt + 1) * kBK);
      gload(rb, g.B, bof, (kt + 1) * kBK);
    }
    mma_stage<TM, WM, WN, RB, CB>(acc, smem + (kt & 1) * STAGE, wm, wn, fr, fh);
    if (kt + 1 < KT) {
      lstore<R>(smem + ((kt + 1) & 1) * STAGE + poff, ra);
      lstore<R>(smem + ((kt + 1) & 1) * STAGE + poff + TM * 128, rb);
    }
    __syncthreads();
  }

#endif

  // Output element e of acc[i][j] (32 x 32 MFMA layout): row 8 (e / 4) + 4 (lane / 32) + e % 4,
  // column lane % 32 of the block.
  auto trow = [&](int i, int e) { return wm * WM + i * 32 + 8 * (e >> 2) + 4 * fh + (e & 3); };
  auto tcol = [&](int j) { return wn * WN + j * 32 + fr; };

  if constexpr (EPI == kEpiLse) {
    // rows are vocabulary ids, columns tokens: a lane holds one token per 32-column block and 16
    // vocabulary rows per 32-row block, so a token's (max, sum) is a reduction in registers, one
    // exchange with the other half-wave and a merge of the GM waves that share the column
    float* smax = reinterpret_cast<float*>(smem);   // [GM][TN]
    float* ssum = smax + GM * TN;                    // [GM][TN]
    int* stg = reinterpret_cast<int*>(ssum + GM * TN);  // [TN] target of each token
    for (int c = tid; c < TN; c += kThreads) stg[c] = g.targets[min(col0 + c, g.n_valid - 1)];
    __syncthreads();
#pragma unroll
    for (int j = 0; j < CB; ++j) {
      const int ct = tcol(j), t = stg[ct] - row0;
      float mx = -INFINITY;
#pragma unroll
      for (int i = 0; i < RB; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int rt = trow(i, e);
          if (row0 + rt < g.m_valid) mx = fmaxf(mx, acc[i][j][e]);
          if (rt == t && col0 + ct < g.n_valid) g.tgt[col0 + ct] = acc[i][j][e];
        }
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      float s = 0.f;
      if (mx != -INFINITY) {
#pragma unroll
        for (int i = 0; i < RB; ++i)
#pragma unroll
          for (int e = 0; e < 16; ++e)
            if (row0 + trow(i, e) < g.m_valid) s += exp_neg(acc[i][j][e] - mx);
      }
      s += __shfl_xor(s, 32);
      if (fh == 0) {
        smax[wm * TN + ct] = mx;
        ssum[wm * TN + ct] = s;
      }
    }
    __syncthreads();
    for (int c = tid; c < TN; c += kThreads) {
      float m = -INFINITY;
#pragma unroll
      for (int w = 0; w < GM; ++w) m = fmaxf(m, smax[w * TN + c]);
      float s = 0.f;
#pragma unroll
      for (int w = 0; w < GM; ++w)
        if (smax[w * TN + c] != -INFINITY) s += ssum[w * TN + c] * exp_neg(smax[w * TN + c] - m);
      float2* p = reinterpret_cast<float2*>(g.part) + int64_t(tm) * g.ldp + col0 + c;
      *p = make_float2(m, s);
    }
  } else if constexpr (EPI == kEpiProb) {
    // rows are the chunk's vocabulary ids, columns tokens
    constexpr int PITCH = staging_pitch<TM, TN>(), PITCHT = TM + 8;
    static_assert(TN * PITCHT <= TM * PITCH || TM == TN, "transposed staging fits");
    uint16_t* st = reinterpret_cast<uint16_t*>(smem);   // the stage buffers are free now
    float* slse = reinterpret_cast<float*>(smem + size_t(TM) * PITCH * 2);
    int* stg = reinterpret_cast<int*>(slse + TN);
    for (int c = tid; c < TN; c += kThreads) {
      const int tok = min(col0 + c, g.n_valid - 1);
      slse[c] = g.lse[tok];
      stg[c] = g.targets[tok] - g.vcol0;
    }
    __syncthreads();
    const float scale = g.grad[0] * g.inv_n;
    // every value once, as bf16 pairs of consecutive rows (elements 2 m, 2 m + 1 of a block)
    uint32_t pk[RB][CB][8];
#pragma unroll
    for (int i = 0; i < RB; ++i)
#pragma unroll
      for (int j = 0; j < CB; ++j)
#pragma unroll
        for (int m = 0; m < 8; ++m) {
          uint32_t h2[2];
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            const int e = 2 * m + u, rt = trow(i, e), ct = tcol(j);
            float p = 0.f;
            if (row0 + rt < g.m_valid && col0 + ct < g.n_valid)
              p = (exp_neg(acc[i][j][e] - slse[ct]) - (row0 + rt == stg[ct] ? 1.f : 0.f)) * scale;
            h2[u] = f2bf(p);
          }
          pk[i][j][m] = h2[0] | (h2[1] << 16);
        }
    // row-major staging (vocabulary rows), then PT rows as 16-byte pieces
#pragma unroll
    for (int i = 0; i < RB; ++i)
#pragma unroll
      for (int j = 0; j < CB; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e)
          st[trow(i, e) * PITCH + tcol(j)] = uint16_t(pk[i][j][e >> 1] >> (16 * (e & 1)));
    __syncthreads();
    for (int q = tid; q < TM * TN / 8; q += kThreads) {
      const int r = q / (TN / 8), c8 = q % (TN / 8);
      *reinterpret_cast<u32x4*>(g.PT + int64_t(row0 + r) * g.ldPT + col0 + 8 * c8) =
          *reinterpret_cast<const u32x4*>(st + r * PITCH + 8 * c8);
    }
    __syncthreads();
    // transposed staging (token c as a stage row; the 4 consecutive vocabulary rows e4 of a lane
    // in one 8-byte write), then P rows as 16-byte pieces
#pragma unroll
    for (int i = 0; i < RB; ++i)
#pragma unroll
      for (int j = 0; j < CB; ++j)
#pragma unroll
        for (int e4 = 0; e4 < 4; ++e4)
          *reinterpret_cast<uint2*>(st + tcol(j) * PITCHT + trow(i, 4 * e4)) =
              make_uint2(pk[i][j][2 * e4], pk[i][j][2 * e4 + 1]);
    __syncthreads();
    for (int q = tid; q < TN * TM / 8; q += kThreads) {
      const int c = q / (TM / 8), r8 = q % (TM / 8);
      *reinterpret_cast<u32x4*>(g.P + int64_t(col0 + c) * g.ldP + row0 + 8 * r8) =
          *reinterpret_cast<const u32x4*>(st + c * PITCHT + 8 * r8);
    }
  } else if constexpr (EPI == kEpiAccF32) {
#pragma unroll
    for (int i = 0; i < RB; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int r = row0 + trow(i, e);
#pragma unroll
        for (int j = 0; j < CB; ++j) {
          const int c = col0 + tcol(j);
          float* p = g.acc + int64_t(r) * g.ldacc + c;
          const float v = g.accumulate ? *p + acc[i][j][e] : acc[i][j][e];
          *p = v;
          if (g.out && r < g.m_valid && c < g.n_valid) g.out[int64_t(r) * g.ldout + c] = f2bf(v);
        }
      }
  } else {   // kEpiStoreBf16
#pragma unroll
    for (int i = 0; i < RB; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int r = row0 + trow(i, e);
        if (r >= g.m_valid) continue;
#pragma unroll
        for (int j = 0; j < CB; ++j) {
          const int c = col0 + tcol(j);
          if (c < g.n_valid) g.out[int64_t(r) * g.ldout + c] = f2bf(acc[i][j][e]);
        }
      }
  }
}

// Transpose in blocks of `blk` rows (a multiple of 64): row r of src, column c goes to
// dst[(r / blk) cols blk + c blk + r % blk] -- block k is the (cols x blk) transpose of rows
// k blk .. -- with 0 for rows <= r < rows_pad (c < cols); 64 x 64 tiles.
__global__ __launch_bounds__(256) void xent_transpose(const uint16_t* src, int rows, int cols, int64_t lds,
                                                      uint16_t* dst, int rows_pad, int blk) {
  __shared__ uint16_t t[64][66];
  const int c0 = blockIdx.x * 64, r0 = blockIdx.y * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  // a 64-row tile lies in one block (blk is a multiple of 64)
  const int64_t dbase = int64_t(r0 / blk) * cols * blk + r0 % blk;
  uint16_t v[16];
#pragma unroll
  for (int k = 0; k < 16; ++k) {   // loads first, from clamped indices
    const int r = r0 + ty + 4 * k, c = c0 + tx;
    v[k] = src[int64_t(min(r, rows - 1)) * lds + min(c, cols - 1)];
  }
#pragma unroll
  for (int k = 0; k < 16; ++k) t[ty + 4 * k][tx] = r0 + ty + 4 * k < rows ? v[k] : uint16_t(0);
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const int c = c0 + ty + 4 * k, r = r0 + tx;
    if (c < cols && r < rows_pad) dst[dbase + int64_t(c) * blk + tx] = t[tx][ty + 4 * k];
  }
}

// targets into [0, V): an id outside is replaced by 0 and reported
__global__ void xent_targets(const int32_t* targets, int n, int V, int32_t* out, int32_t* status) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  int t = targets[i];
  if (t < 0 || t >= V) {
    atomicOr(status, kStatusTarget);
    t = 0;
  }
  out[i] = t;
}

// lse of each token from its vocabulary tiles' (max, sum); loss term lse - target logit.  16 lanes
// per token (a block of 256 threads takes 16 tokens): lane u merges tiles u, u + 16, ... in order,
// then the 16 partials are merged pairwise in a fixed tree (lanes u, u ^ 1, u ^ 2, u ^ 4, u ^ 8)
__device__ __forceinline__ void merge_ms(float& m, float& s, float m2, float s2) {
  if (m2 == -INFINITY) return;
  if (m == -INFINITY) {
    m = m2;
    s = s2;
    return;
  }
  const float nm = fmaxf(m, m2);
  s = s * exp_neg(m - nm) + s2 * exp_neg(m2 - nm);
  m = nm;
}
__global__ __launch_bounds__(256) void xent_lse(const float2* part, int tiles, int64_t ldp, const float* tgt, int n,
                                                float* lse, float* lrow) {
  const int u = threadIdx.x & 15;
  const int r = blockIdx.x * 16 + (threadIdx.x >> 4);
  const int rr = min(r, n - 1);
  float m = -INFINITY, s = 0.f;
  for (int t = u; t < tiles; t += 16) {
    const float2 p = part[int64_t(t) * ldp + rr];
    merge_ms(m, s, p.x, p.y);
  }
#pragma unroll
  for (int x = 1; x < 16; x <<= 1) {
    const float m2 = __shfl_xor(m, x, 16), s2 = __shfl_xor(s, x, 16);
    // both lanes of a pair merge in the same order (lower lane's partial first)
    if (u & x) {
      float mm = m2, ss = s2;
      merge_ms(mm, ss, m, s);
      m = mm;
      s = ss;
    } else {
      merge_ms(m, s, m2, s2);
    }
  }
  if (u == 0 && r < n) {
    const float l = m + logf(s);
    lse[r] = l;
    lrow[r] = l - tgt[r];
  }
}

// mean of lrow[0..n) in a fixed order: float64 partial sums per thread, then a tree
__global__ __launch_bounds__(1024) void xent_mean(const float* lrow, int n, float* loss) {
  __shared__ double s[1024];
  double a = 0.0;
  for (int i = threadIdx.x; i < n; i += 1024) a += double(lrow[i]);
  s[threadIdx.x] = a;
  __syncthreads();
  for (int w = 512; w > 0; w >>= 1) {
    if (int(threadIdx.x) < w) s[threadIdx.x] += s[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) loss[0] = float(s[0] / double(n));
}

int64_t al256(int64_t b) { return (b + 255) / 256 * 256; }
int rup(int x, int m) { return (x + m - 1) / m * m; }

struct Layout {
  int Np, Vp, C, Cp;
  int64_t tgt_idx, part, tgt, lrow, wt, ht, P, PT, dh, bytes;
};

Layout layout(int n, int V, int d, int chunk) {
  Layout L;
  L.Np = rup(n, 256);
  L.Vp = rup(V, 256);
  L.C = std::min(rup(std::max(chunk, 1), 256), L.Vp);
  L.Cp = L.C;
  int64_t o = 0;
  L.tgt_idx = o; o += al256(int64_t(L.Np) * 4);
  L.part = o;    o += al256(int64_t(L.Vp / 256) * L.Np * 8);
  L.tgt = o;     o += al256(int64_t(L.Np) * 4);
  L.lrow = o;    o += al256(int64_t(L.Np) * 4);
  L.wt = o;      o += al256(int64_t((L.Vp + L.C - 1) / L.C) * d * L.C * 2);   // chunk-major W^T
  L.ht = o;      o += al256(int64_t(d) * L.Np * 2);
  L.P = o;       o += al256(int64_t(L.Np) * L.Cp * 2);
  L.PT = o;      o += al256(int64_t(L.Cp) * L.Np * 2);
  L.dh = o;      o += al256(int64_t(L.Np) * d * 4);
  L.bytes = o;
  return L;
}

// d_model a multiple of 128 (the K step of the logits GEMM, the 128-column tiles of the gradients)
// and every operand small enough for the GEMM's 32-bit element offsets (rows x row stride < 2^31)
bool shape_ok(int n, int V, int d) {
  if (n < 1 || V < 1 || d < 128 || d % 128 || d > 65536) return false;
  const int64_t Np = rup(n, 256), Vp = rup(V, 256);
  return Np * d < (int64_t(1) << 31) && Vp * d < (int64_t(1) << 31) && Np * Vp < (int64_t(1) << 31);
}

template <int TM, int TN, int GM, int GN, int EPI>
hipError_t launch_gemm(const GemmArgs& g, hipStream_t s) {
  const void* fn = reinterpret_cast<const void*>(&xent_gemm<TM, TN, GM, GN, EPI>);
  const size_t lds = lds_bytes<TM, TN, EPI>();
  if (hipError_t e = msdc::ensure_dynamic_lds(fn, lds); e != hipSuccess) return e;
  hipLaunchKernelGGL((xent_gemm<TM, TN, GM, GN, EPI>), dim3(g.tiles_m * g.tiles_n), dim3(64 * GM * GN), lds, s, g);
  return hipGetLastError();
}
constexpr int kBigGM = 2, kBigGN = XENT_BIG_WAVES / 2;

}  // namespace mxe

using namespace mxe;

extern "C" int64_t msd_xent_workspace_bytes(int32_t n_rows, int32_t vocab, int32_t d_model, int32_t chunk) {
  if (!shape_ok(n_rows, vocab, d_model)) return MSD_E_CONFIG;
  return layout(n_rows, vocab, d_model, chunk).bytes;
}

extern "C" int32_t msd_xent_forward(const void* h, const void* weight, const int32_t* targets, int32_t n_rows,
                                    int32_t vocab, int32_t d_model, void* workspace, float* loss, float* lse,
                                    int32_t* status, void* stream) {
  if (!shape_ok(n_rows, vocab, d_model)) return MSD_E_CONFIG;
  if (!h || !weight || !targets || !workspace || !loss || !lse || !status) return MSD_E_ARG;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const Layout L = layout(n_rows, vocab, d_model, vocab);
  char* ws = static_cast<char*>(workspace);
  int32_t* tix = reinterpret_cast<int32_t*>(ws + L.tgt_idx);
  hipLaunchKernelGGL(xent_targets, dim3((n_rows + 255) / 256), dim3(256), 0, s, targets, n_rows, vocab, tix, status);
  GemmArgs g{};
  // S^T = W h^T: tile rows are vocabulary ids, columns tokens
  g.A = static_cast<const uint16_t*>(weight);
  g.lda = d_model;
  g.a_valid = vocab;
  g.B = static_cast<const uint16_t*>(h);
  g.ldb = d_model;
  g.b_valid = n_rows;
  g.K = d_model;
  g.tiles_m = L.Vp / 256;
  g.tiles_n = L.Np / 256;
  g.m_valid = vocab;
  g.n_valid = n_rows;
  g.targets = tix;
  g.part = reinterpret_cast<float*>(ws + L.part);
  g.ldp = L.Np;
  g.tgt = reinterpret_cast<float*>(ws + L.tgt);
  if (launch_gemm<256, 256, kBigGM, kBigGN, kEpiLse>(g, s) != hipSuccess) return MSD_E_HIP;
  float* lrow = reinterpret_cast<float*>(ws + L.lrow);
  hipLaunchKernelGGL(xent_lse, dim3((n_rows + 15) / 16), dim3(256), 0, s, reinterpret_cast<const float2*>(g.part),
                     g.tiles_m, int64_t(L.Np), g.tgt, n_rows, lse, lrow);
  hipLaunchKernelGGL(xent_mean, dim3(1), dim3(1024), 0, s, lrow, n_rows, loss);
  return hipGetLastError() == hipSuccess ? MSD_OK : MSD_E_HIP;
}

extern "C" int32_t msd_xent_backward(const void* h, const void* weight, const int32_t* targets, const float* lse,
                                     const float* grad_loss, int32_t n_rows, int32_t vocab, int32_t d_model,
                                     int32_t chunk, void* workspace, void* grad_h, void* grad_weight,
                                     int32_t* status, void* stream) {
  if (!shape_ok(n_rows, vocab, d_model)) return MSD_E_CONFIG;
  if (!h || !weight || !targets || !lse || !grad_loss || !workspace || !grad_h || !grad_weight || !status)
    return MSD_E_ARG;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const Layout L = layout(n_rows, vocab, d_model, chunk);
  char* ws = static_cast<char*>(workspace);
  int32_t* tix = reinterpret_cast<int32_t*>(ws + L.tgt_idx);
  uint16_t* wt = reinterpret_cast<uint16_t*>(ws + L.wt);
  uint16_t* ht = reinterpret_cast<uint16_t*>(ws + L.ht);
  uint16_t* P = reinterpret_cast<uint16_t*>(ws + L.P);
  uint16_t* PT = reinterpret_cast<uint16_t*>(ws + L.PT);
  float* dh = reinterpret_cast<float*>(ws + L.dh);
  const uint16_t* W = static_cast<const uint16_t*>(weight);
  const uint16_t* H = static_cast<const uint16_t*>(h);
  hipLaunchKernelGGL(xent_targets, dim3((n_rows + 255) / 256), dim3(256), 0, s, targets, n_rows, vocab, tix, status);
  // W^T (chunk-major: per chunk a d x C block, so a chunk's rows are C apart) and h^T (d x Np),
  // zero past V and N
  hipLaunchKernelGGL(xent_transpose, dim3((d_model + 63) / 64, L.Vp / 64), dim3(256), 0, s, W, vocab, d_model,
                     int64_t(d_model), wt, L.Vp, L.C);
  hipLaunchKernelGGL(xent_transpose, dim3((d_model + 63) / 64, L.Np / 64), dim3(256), 0, s, H, n_rows, d_model,
                     int64_t(d_model), ht, L.Np, L.Np);
  for (int v0 = 0; v0 < vocab; v0 += L.C) {
    const int cv = std::min(L.C, vocab - v0);   // valid columns of this chunk
    const int cp = rup(cv, 256);                // padded
    GemmArgs p{};
    p.A = W + int64_t(v0) * d_model;   // S^T of the chunk: rows vocabulary ids, columns tokens
    p.lda = d_model;
    p.a_valid = cv;
    p.B = H;
    p.ldb = d_model;
    p.b_valid = n_rows;
    p.K = d_model;
    p.tiles_m = cp / 256;
    p.tiles_n = L.Np / 256;
    p.m_valid = cv;
    p.n_valid = n_rows;
    p.targets = tix;
    p.vcol0 = v0;
    p.lse = lse;
    p.grad = grad_loss;
    p.inv_n = 1.0f / float(n_rows);
    p.P = P;
    p.ldP = L.Cp;
    p.PT = PT;
    p.ldPT = L.Np;
    if (launch_gemm<256, 256, kBigGM, kBigGN, kEpiProb>(p, s) != hipSuccess) return MSD_E_HIP;
    // grad_W rows of the chunk = PT (cp x Np) . (h^T)^T  (K = Np)
    GemmArgs w{};
    w.A = PT;
    w.lda = L.Np;
    w.a_valid = cp;
    w.B = ht;
    w.ldb = L.Np;
    w.b_valid = d_model;
    w.K = L.Np;
    w.tiles_m = cp / 128;
    w.tiles_n = (d_model + 127) / 128;
    w.m_valid = cv;
    w.n_valid = d_model;
    w.out = static_cast<uint16_t*>(grad_weight) + int64_t(v0) * d_model;
    w.ldout = d_model;
    if (launch_gemm<128, 128, 2, 2, kEpiStoreBf16>(w, s) != hipSuccess) return MSD_E_HIP;
    // grad_h (+)= P (Np x cp) . (W^T columns v0..v0+cp)^T  (K = cp)
    GemmArgs a{};
    a.A = P;
    a.lda = L.Cp;
    a.a_valid = L.Np;
    a.B = wt + int64_t(v0 / L.C) * d_model * L.C;   // the chunk's block of W^T: d rows of C
    a.ldb = L.C;
    a.b_valid = d_model;
    a.K = cp;
    a.tiles_m = L.Np / 128;
    a.tiles_n = d_model / 128;
    a.m_valid = n_rows;
    a.n_valid = d_model;
    a.acc = dh;
    a.ldacc = d_model;
    a.accumulate = v0 > 0;
    a.out = v0 + L.C >= vocab ? static_cast<uint16_t*>(grad_h) : nullptr;
    a.ldout = d_model;
    if (launch_gemm<128, 128, 2, 2, kEpiAccF32>(a, s) != hipSuccess) return MSD_E_HIP;
  }
  return hipGetLastError() == hipSuccess ? MSD_OK : MSD_E_HIP;
}
