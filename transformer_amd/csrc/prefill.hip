// Matrix-core forward passes on one MI355X (gfx950) over M token rows at once:
//   * prefill  — the M tokens of one prompt at positions 0..M-1 (model.py:194-231,
//                prefill_with_kv, as called by generate.py:70-90)
//   * batched decode — one token of each of M independent sequences, each at its own
//                position, over a paged KV cache (the reference's described batched paged
//                decode; kernels/multi_sm_decode.py:77-357 semantics per sequence)
// writing the KV cache rows of every layer and the logits, with every projection on the
// matrix cores.
//
// Numerics: model.py:94-191 in f32.  Each activation entering a projection (RMSNorm outputs,
// attention output, SwiGLU output, final norm) is stored as two bf16 parts, hi = bf16(x) and
// lo = bf16(x - hi), and both are multiplied with the bf16 weights on the matrix cores
// (v_mfma_f32_16x16x32_bf16) into one f32 accumulator: the projection sees x to about 2^-17
// relative, where the reference kernel rounds it to bf16 (multi_sm_decode.py:143,229,268,289,
// 320).  The residual stream, RoPE, softmax attention and SwiGLU are f32, K/V are stored to the
// cache as bf16 after RoPE (model.py:212-215).  In batched decode the current position attends
// with its un-rounded K/V (multi_sm_decode.py:197,205).
//
// KV cache: [layer][K, V][kv_head][pool positions][64] bf16 with pool positions = 16 * pages.
// A row's position p lives at page table[p / 16] * 16 + p % 16; without a table the page is
// p / 16 (the contiguous cache of one sequence is the pool with the identity table).
//
// Kernels per layer, on the caller's stream:
//   mx_norm        residual += split-K partials of the previous projection (in split order),
//                  then RMSNorm -> bf16 activations in the weights' permuted input order
//   mx_gemm        q/k/v projection, split-K partials
//   mx_qkv_fin     sum of the partials, RoPE on q/k, f32 q/k/v, bf16 K/V cache rows
//   attention      prefill: causal GQA over the prompt; batched decode: each sequence over
//                  its cached rows plus its current K/V
//   mx_gemm        O projection, split-K partials
//   mx_norm        (as above) -> ln2 activations
//   mx_gemm        gate/up projection, split-K partials
//   mx_swiglu_fin  silu(gate) * up -> bf16 in the down projection's input order
//   mx_gemm        down projection, split-K partials
// then mx_norm with the final scale, mx_gemm against the tied embedding, mx_argmax per row.
//
// GEMM: C[M x N] = A[M x K] * W[N x K]^T with A (activations) and W (packed weight rows)
// both K-contiguous.  A workgroup of four waves covers 64 columns and BM rows; each wave
// holds RB x CB 16 x 16 MFMA tiles, every operand fragment one 16-byte run along K loaded
// straight from memory (W streamed once per row tile, A from L2).  K is split across grid.z
// into enough workgroups to keep every compute unit streaming; partials are summed in split
// order by the consuming kernel.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <atomic>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <vector>

#include "../../include/msdecode.h"
#include "batched.h"
#include "internal.h"

namespace mpf {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kDh = 64;
constexpr int kPage = 16;     // positions per KV page
constexpr int kBN = 64;       // GEMM tile columns
constexpr int kBK = 32;       // K per MFMA step
constexpr int kNormThreads = 256;
constexpr int kMaxSplitK = 16;  // largest K split (partials summed by the consumers)
constexpr int kMaxRows = 1024;

__device__ __forceinline__ float bf2f(uint16_t b) { return __uint_as_float(uint32_t(b) << 16); }
__device__ __forceinline__ uint16_t f2bf(float f) {   // round to nearest even
  const uint32_t u = __float_as_uint(f);
  return uint16_t((u + (((u >> 16) & 1u) + 0x7fffu)) >> 16);
}

// An activation entering a projection as two bf16 parts, hi = bf16(x) and lo = bf16(x - hi): the
// matrix cores multiply both with the bf16 weight and add in f32, so the product carries x to
// about 2^-17 relative instead of bf16's 2^-9 (the f32 activations of model.py, not the
// reference kernel's bf16 rounding points).  The lo part lives in a second plane of the buffer.
__device__ __forceinline__ void put_split(uint16_t* hi, int64_t plane, float x) {
  const uint16_t h = f2bf(x);
  hi[0] = h;
  hi[plane] = f2bf(x - bf2f(h));
}

// Wave64 reductions with DPP row shifts and row broadcasts (fixed order, no LDS traffic);
// the result is read from lane 63 as a wave-uniform value.
template <int CTRL, int ROWMASK>
__device__ __forceinline__ float dpp(float v, float fill) {
  return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(fill), __float_as_int(v), CTRL, ROWMASK, 0xf, false));
}
// The sum over each row of 16 lanes, in every lane of the row: the butterfly lane ^ 1, ^ 2, ^ 4,
// ^ 8 with DPP (quad permutes, then the half-row and row mirrors: after each step the lanes of a
// group hold the same value, so a mirror adds the other group's sum exactly as the xor would)
// instead of LDS permutes
__device__ __forceinline__ float sum16_lanes(float v) {
  v += dpp<0xB1, 0xf>(v, 0.f);    // quad_perm [1, 0, 3, 2]: lane ^ 1
  v += dpp<0x4E, 0xf>(v, 0.f);    // quad_perm [2, 3, 0, 1]: lane ^ 2
  v += dpp<0x141, 0xf>(v, 0.f);   // row_half_mirror: the other quad of the 8
  v += dpp<0x140, 0xf>(v, 0.f);   // row_mirror: the other 8 of the row
  return v;
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
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp<0x111, 0xf>(v, -INFINITY));
  v = fmaxf(v, dpp<0x112, 0xf>(v, -INFINITY));
  v = fmaxf(v, dpp<0x114, 0xf>(v, -INFINITY));
  v = fmaxf(v, dpp<0x118, 0xf>(v, -INFINITY));
  v = fmaxf(v, dpp<0x142, 0xa>(v, -INFINITY));
  v = fmaxf(v, dpp<0x143, 0xc>(v, -INFINITY));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Position of input element i in a row of K under the packed row layout: blocks of 512
// (the last one S = 8m long); element b*512 + k*m + l sits at b*512 + 8*l + k.
__device__ __forceinline__ int perm_pos(int i, int K) {
  const int b = i >> 9, r = i & 511;
  const int S = min(512, K - (b << 9));
  const int m = S >> 3;
  const int k = r / m, l = r - k * m;
  return (b << 9) + 8 * l + k;
}
// Input element stored at position j (inverse of perm_pos).
__device__ __forceinline__ int perm_elem(int j, int K) {
  const int b = j >> 9, o = j & 511;
  const int S = min(512, K - (b << 9));
  const int m = S >> 3;
  return (b << 9) + (o & 7) * m + (o >> 3);
}

// Element (m, j) of an activation plane with rows of K (j a packed position).  ldx > 0: rows
// ldx apart.  ldx == 0: matrix-core tile order, the layout the projections read: 16 rows x 32
// positions form a tile of 64 lanes x 16 bytes in MFMA operand order (row m % 16 and positions
// 8 ((j % 32) / 8) .. + 8 in lane (m % 16) + 16 ((j % 32) / 8)), tile (m / 16, j / 32) at
// ((m / 16) (K / 32) + j / 32) 512 elements, so a wave's operand load reads 1 KB in one piece.
__device__ __forceinline__ int64_t act_index(int m, int j, int K, int ldx) {
  if (ldx > 0) return int64_t(m) * ldx + j;
  return ((int64_t(m >> 4) * (K >> 5) + (j >> 5)) * 64 + (m & 15) + 16 * ((j & 31) >> 3)) * 8 + (j & 7);
}

// Rows of a pass: row m is sequence seq(m) at position pos(m).
struct Rows {
  int M;
  const int32_t* pos;     // NULL: pos(m) = pos0 + m (prefill from pos0)
  int batched;            // seq(m) = m; else every row is sequence 0
  const int32_t* pages;   // [seq][max_pages] page table, NULL = identity
  int max_pages;
  int pool;               // pool positions (16 * pages)
  int pos0;               // position of row 0 when pos is NULL
};
__device__ __forceinline__ int row_pos(const Rows& r, int m) { return r.pos ? r.pos[m] : r.pos0 + m; }
__device__ __forceinline__ int64_t cache_row(const Rows& r, int m, int p) {
  const int seq = r.batched ? m : 0;
  const int page = r.pages ? r.pages[int64_t(seq) * r.max_pages + p / kPage] : p / kPage;
  return int64_t(page) * kPage + p % kPage;
}

// What mx_gemm_rows does with its final outputs.
enum Epi { kEpiStore = 0, kEpiSwiglu = 1, kEpiQkv = 2, kEpiResid = 3, kEpiResidNorm = 4 };
// Operands of the fused epilogues.
struct EpiArgs {
  uint16_t* act;       // SwiGLU: the down projection's input planes; ResidNorm: the next RMSNorm's
  int64_t act_plane;   // input planes (scale * h); tile order, the lo plane act_plane further
  const uint16_t* xscale;   // ResidNorm: the next RMSNorm's scales in packed order
  float* ssq;               // ResidNorm: each row's partial sum of h^2 per column group, [M][N / (16 CT)]
  const float* rope;   // QKV: RoPE table, rows, cache and the f32 q/k/v rows (as mx_qkv_fin)
  Rows rows;
  uint16_t* kc;
  uint16_t* vc;
  float* qkv;
  int H, KV;
};

struct GemmArgs {
  const uint16_t* A;   // [M][lda] bf16 (or tile order, see act_index): the hi parts; the lo
  int64_t a_plane;     // parts follow at A + a_plane
  const uint16_t* W;   // [N][K] bf16 (or tile order: tile (n / 16, k / 32) at ((n / 16) (K / 32) + k / 32) 512)
  float* out;          // partials [splits][M][N] f32, or [M][ldo] (single split)
  int M, N, K, lda, ldo, splits;
  EpiArgs e;
  const float* ssq;   // mx_gemm_rows with the norm folded in (AM 2): each row's partial sums of h^2,
  int nssq;           // [M][nssq], summed in a fixed order for the rms that divides the outputs
};

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 u) { return __builtin_bit_cast(bf16x8, u); }

// Eight f32 values as hi/lo bf16 parts (hi = bf16(x), lo = bf16(x - hi)), packed as MFMA operands.
__device__ __forceinline__ void split8(const float (&x)[8], uint4& hi, uint4& lo) {
  uint32_t h[4], l[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint16_t h0 = f2bf(x[2 * i]), h1 = f2bf(x[2 * i + 1]);
    h[i] = uint32_t(h0) | (uint32_t(h1) << 16);
    l[i] = uint32_t(f2bf(x[2 * i] - bf2f(h0))) | (uint32_t(f2bf(x[2 * i + 1] - bf2f(h1))) << 16);
  }
  hi = make_uint4(h[0], h[1], h[2], h[3]);
  lo = make_uint4(l[0], l[1], l[2], l[3]);
}

// f32 operands as hi/lo parts on the matrix cores: a b ~ ah bh + ah bl + al bh (the lo lo term,
// ~2^-16 of the product, is left out).
__device__ __forceinline__ f32x4 mfma3(uint4 ah, uint4 al, uint4 bh, uint4 bl, f32x4 c) {
  c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(ah), as_bf16x8(bh), c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(ah), as_bf16x8(bl), c, 0, 0, 0);
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(al), as_bf16x8(bh), c, 0, 0, 0);
}


// Four waves as WM x (4 / WM); a wave covers RB 16-row blocks and (WM) 16-column blocks.  TA / TW:
// the activations / weights in tile order (one 1 KB piece per operand load).
template <int RB, int WM, bool TA, bool TW>
__global__ __launch_bounds__(256) void mx_gemm(GemmArgs g) {
  constexpr int WN = 4 / WM, CB = 4 / WN, BM = 16 * RB * WM;
  constexpr int U = RB * CB <= 2 ? 8 : 4;   // K steps with loads in flight
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int wm = wv / WN, wn = wv % WN;
  const int m0 = blockIdx.y * BM + 16 * RB * wm, n0 = blockIdx.x * kBN + 16 * CB * wn;
  const int nchunks = g.K / kBK;
  const int c0 = (nchunks * int(blockIdx.z)) / g.splits, c1 = (nchunks * (int(blockIdx.z) + 1)) / g.splits;
  const int kq = 8 * (lane >> 4);   // this lane's 8-element K run within a 32 chunk
  const int r16 = lane & 15;
  // operand pointers of chunk 0; chunk c is kstep(c) elements further
  const uint16_t* arow[RB];   // hi parts (the lo parts a_plane elements further)
  bool aval[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const int m = m0 + 16 * rb + r16;
    aval[rb] = m < g.M;
    if constexpr (TA)   // tiles past the last one read the last (those rows are zeroed)
      arow[rb] = g.A + (int64_t(min(m0 + 16 * rb, g.M - 1) >> 4) * nchunks * 64 + lane) * 8;
    else
      arow[rb] = g.A + int64_t(aval[rb] ? m : 0) * g.lda + kq;
  }
  const uint16_t* wrow[CB];
#pragma unroll
  for (int cb = 0; cb < CB; ++cb)
    wrow[cb] = TW ? g.W + (int64_t((n0 + 16 * cb) >> 4) * nchunks * 64 + lane) * 8
                  : g.W + int64_t(n0 + 16 * cb + r16) * g.K + kq;
  auto kstep = [](int c, bool tiled) { return tiled ? int64_t(c) * 512 : int64_t(c) * kBK; };
  f32x4 acc[RB][CB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) acc[rb][cb] = f32x4{0.f, 0.f, 0.f, 0.f};
  auto step = [&](const uint4* a, const uint4* al, const uint4* w) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) {
        acc[rb][cb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a[rb]), as_bf16x8(w[cb]), acc[rb][cb], 0, 0, 0);
        acc[rb][cb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(al[rb]), as_bf16x8(w[cb]), acc[rb][cb], 0, 0, 0);
      }
  };
  // U chunks per round, all loads issued before the first MMA; the last round's chunks past c1
  // reload chunk c1 - 1 and are skipped (loads stay unconditional: a load under a branch is
  // waited for at the join)
  for (int c = c0; c < c1; c += U) {
    uint4 a[U][RB], al[U][RB], w[U][CB];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int ch = min(c + u, c1 - 1);
      const int64_t ka = kstep(ch, TA), kw = kstep(ch, TW);
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        const uint4 v = *reinterpret_cast<const uint4*>(arow[rb] + ka);
        const uint4 vl = *reinterpret_cast<const uint4*>(arow[rb] + g.a_plane + ka);
        a[u][rb] = aval[rb] ? v : make_uint4(0, 0, 0, 0);
        al[u][rb] = aval[rb] ? vl : make_uint4(0, 0, 0, 0);
      }
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) w[u][cb] = *reinterpret_cast<const uint4*>(wrow[cb] + kw);
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (c + u < c1) step(a[u], al[u], w[u]);
  }
  // D layout of a 16 x 16 tile: lane holds rows 4*(lane/16) + r (r < 4) of column lane % 16
  float* out = g.splits > 1 ? g.out + int64_t(blockIdx.z) * g.M * g.N : g.out;
  const int ldo = g.splits > 1 ? g.N : g.ldo;
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int cb = 0; cb < CB; ++cb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = m0 + 16 * rb + 4 * (lane >> 4) + r;
        if (row < g.M) out[int64_t(row) * ldo + n0 + 16 * cb + r16] = acc[rb][cb][r];
      }
}

// SwiGLU of a gate/up pair (packed rows 2f, 2f + 1; model.py:159).
__device__ __forceinline__ float swiglu(float g, float u) { return (g * (1.f / (1.f + expf(-g)))) * u; }

// Outputs s0, s1 of the packed q/k/v rows col, col + 1 (col even) of row m, whose position has
// RoPE factors c, sg for this pair: q and k pairs are rotated (dims i, i + 32; model.py:110-117),
// v is stored as projected; f32 q/k/v in natural head-dim order to `q`, bf16 K/V to the cache
// row cp (multi_sm_decode.py:179-180).
__device__ __forceinline__ void qkv_pair(float s0, float s1, float c, float sg, int col, int H, int KV, float* q,
                                         uint16_t* cp) {
  const int head = col / kDh, rr = col % kDh, ri = rr >> 1;
  const bool rot = head < H + KV;
  const float o0 = rot ? s0 * c - s1 * sg : s0, o1 = rot ? s0 * sg + s1 * c : s1;
  const int d0 = rot ? ri : rr, d1 = rot ? ri + kDh / 2 : rr + 1;
  q[d0] = o0;
  q[d1] = o1;
  if (head >= H) {
    cp[d0] = f2bf(o0);
    cp[d1] = f2bf(o1);
  }
}

// C = A W^T for many rows: a workgroup owns 16 RT rows x 16 CT columns over the whole of K, so it
// streams CT * 16 complete weight rows (contiguous in memory) and writes final outputs (no split-K
// partials); with RT = 2 every weight tile it loads serves 32 rows, and the last column group may
// be short (ragged: N / 16 need not be a multiple of CT).  The four waves take interleaved
// 32-wide K steps (wave w: steps w, w + 4, ...) with P steps of loads in flight, and add their
// tiles through LDS in wave order, so the result is deterministic.  Tiles are dealt XCD-aware:
// every row tile of a column tile runs on one XCD (workgroup b on XCD b mod 8), which then fetches
// that column tile's weights into its L2 once.  AM: the A operand as bf16 hi/lo rows (0) or tiles (1) as for mx_gemm, or (2) RMSNorm
// folded in (model.py:94-98): A = the hi/lo tiles of scale * h that the previous projection's
// epilogue wrote (kEpiResidNorm), and every output divided by sqrt(mean(h^2) + 1e-5), the sum of
// h^2 of each row added up from that epilogue's per-column-group partials.  TW as for mx_gemm.
// EPI: store the outputs, add them to the residual out (tile order; with kEpiResidNorm also the
// hi/lo tiles of scale * h and the row's partial sum of h^2 for the next RMSNorm), or finish them
// in place of mx_swiglu_fin / mx_qkv_fin (column pairs per thread, the same arithmetic).
template <int CT, int P, int AM, bool TW, int EPI, int RT = 1>
__global__ __launch_bounds__(256) void mx_gemm_rows(GemmArgs g) {
  static_assert(RT == 1 || (AM >= 1 && TW && (EPI == kEpiSwiglu || EPI == kEpiQkv)),
                "two row tiles per workgroup: tile-order operands and a pair epilogue");
  // the waves' partial tiles, element r of lane l's D registers at [r][l]: the epilogue reads
  // them across lanes contiguously (read as [l][r], 16 bytes apart, they took 2-4 times the LDS
  // cycles: SQ_LDS_BANK_CONFLICT)
  __shared__ float red[4][RT][CT][4][64];
  __shared__ float rrms[16 * RT];   // AM 2: each row's rms
  // wave-uniform wave index: the step count and its loop stay scalar (a per-lane loop would copy
  // the accumulators out of and back into the AGPRs around every step)
  const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n16 = g.N / 16, T = (g.M + 15) / 16, TG = (T + RT - 1) / RT, C = (n16 + CT - 1) / CT;
  const int b = blockIdx.x, slot = b >> 3;
  const int t = slot % TG, c = (slot / TG) * 8 + (b & 7);
  if (c >= C) return;
  const int m0 = 16 * RT * t, n0 = 16 * CT * c;
  const int ctn = min(CT, n16 - CT * c);   // column tiles of this group (the last group may be short)
  const int r16 = lane & 15, kq = 8 * (lane >> 4);
  const int S = g.K / kBK;
  // rows past M read row M - 1 (row layout) or whatever their tile holds (a row tile past the
  // last reads the last): an MFMA row only feeds its own output row, which is not stored
  const uint16_t* ar[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
    ar[rt] = AM >= 1 ? g.A + (int64_t(min(RT * t + rt, T - 1)) * S * 64 + lane) * 8
                     : g.A + int64_t(min(m0 + r16, g.M - 1)) * g.lda + kq;
  const uint16_t* wr = TW ? g.W + (int64_t(n0 >> 4) * S * 64 + lane) * 8 : g.W + int64_t(n0 + r16) * g.K + kq;
  // element offsets of step ks and of column tile ct
  const int64_t astep = AM >= 1 ? 512 : kBK, wstep = TW ? 512 : kBK;
  const int64_t wtile = TW ? int64_t(S) * 512 : int64_t(16) * g.K;
  const int ns = (S - wv + 3) / 4;   // K steps of this wave (S >= 4: every wave has one)
  f32x4 acc[RT][CT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) acc[rt][ct] = f32x4{0.f, 0.f, 0.f, 0.f};
  // AM 2: the partial sums of h^2 of row 16 rt + tid / 16 (column groups tid % 16 + 16 j),
  // requested now and added up after the K loop
  constexpr int kSq = 4;
  float sq[RT][kSq];
  if constexpr (AM == 2) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int64_t rrow = min(m0 + 16 * rt + int(threadIdx.x >> 4), g.M - 1);
#pragma unroll
      for (int j = 0; j < kSq; ++j) {
        const int cg = int(threadIdx.x & 15) + 16 * j;
        sq[rt][j] = g.ssq[rrow * g.nssq + min(cg, g.nssq - 1)];
      }
    }
  }
  // the residual elements this thread's epilogue updates (one per column tile: row 4 (lane / 16)
  // + wave of the tile, column 16 ct + lane % 16), requested before the K loop so that the
  // epilogue does not wait a memory round trip for them (rows past M read row M - 1)
  float hold[CT];
  if constexpr (EPI == kEpiResid || EPI == kEpiResidNorm) {
    const int row = min(m0 + 4 * (lane >> 4) + wv, g.M - 1);
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) hold[ct] = g.out[act_index(row, n0 + 16 * ct + (lane & 15), g.N, 0)];
  }
  uint4 a[P][RT], al[P][RT], w[P][CT];
  // step i of this wave, clamped to its last: loads stay unconditional, so no wait lands at a
  // branch join (a column tile past a short group's end reads its last tile)
  auto load = [&](int p, int i) {
    const int ks = wv + 4 * min(i, ns - 1);
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      a[p][rt] = *reinterpret_cast<const uint4*>(ar[rt] + ks * astep);
      al[p][rt] = *reinterpret_cast<const uint4*>(ar[rt] + g.a_plane + ks * astep);
    }
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) w[p][ct] = *reinterpret_cast<const uint4*>(wr + min(ct, ctn - 1) * wtile + ks * wstep);
  };
#pragma unroll
  for (int p = 0; p < P; ++p) load(p, p);
  // every round runs all P steps (a step past the end multiplies a zero A fragment), so the
  // accumulators stay in the AGPRs across the loop
  for (int i0 = 0; i0 < ns; i0 += P) {
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const bool live = i0 + p < ns;
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        uint4 x = a[p][rt], xl = al[p][rt];
        if (!live) x = xl = make_uint4(0, 0, 0, 0);
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
          acc[rt][ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(x), as_bf16x8(w[p][ct]), acc[rt][ct], 0, 0, 0);
          acc[rt][ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(xl), as_bf16x8(w[p][ct]), acc[rt][ct], 0, 0, 0);
        }
      }
      load(p, i0 + p + P);
    }
  }
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int ct = 0; ct < CT; ++ct)
#pragma unroll
      for (int r = 0; r < 4; ++r) red[wv][rt][ct][r][lane] = acc[rt][ct][r];
  if constexpr (AM == 2) {   // row 16 rt + tid / 16's sum of h^2 over its nssq <= 64 partials, in a fixed order
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      float sum = 0.f;
#pragma unroll
      for (int j = 0; j < kSq; ++j) sum += int(threadIdx.x & 15) + 16 * j < g.nssq ? sq[rt][j] : 0.f;
      sum = sum16_lanes(sum);
      if ((threadIdx.x & 15) == 0) rrms[16 * rt + (threadIdx.x >> 4)] = sqrtf(sum / float(g.K) + 1e-5f);
    }
  }
  __syncthreads();
  // D layout of a 16 x 16 tile: lane holds rows 4 (lane / 16) + r of column lane % 16
  if constexpr (EPI == kEpiStore || EPI == kEpiResid || EPI == kEpiResidNorm) {
    // (one row tile, whole column groups) thread tid holds row 4 (lane / 16) + wave of the tile,
    // columns 16 ct + lane % 16
    float hsq = 0.f;
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      const int r = wv, l = lane;
      float v = ((red[0][0][ct][r][l] + red[1][0][ct][r][l]) + red[2][0][ct][r][l]) + red[3][0][ct][r][l];
      if constexpr (AM == 2) v = v / rrms[4 * (l >> 4) + r];
      const int row = m0 + 4 * (l >> 4) + r, col = n0 + 16 * ct + (l & 15);
      float* o = g.out + (EPI == kEpiStore ? int64_t(row) * g.ldo + col : act_index(row, col, g.N, 0));
      if (row < g.M) {
        if constexpr (EPI == kEpiStore) {
          *o = v;
        } else {
          const float hv = hold[ct] + v;
          *o = hv;
          if constexpr (EPI == kEpiResidNorm) {
            put_split(g.e.act + act_index(row, col, g.N, 0), g.e.act_plane, bf2f(g.e.xscale[col]) * hv);
            hsq += hv * hv;
          }
        }
      }
    }
    if constexpr (EPI == kEpiResidNorm) {   // the row's 16 CT columns: 16 lanes, in a fixed order
      hsq = sum16_lanes(hsq);
      const int row = m0 + 4 * (lane >> 4) + wv;
      if ((lane & 15) == 0 && row < g.M) g.e.ssq[int64_t(row) * C + c] = hsq;
    }
  } else {
    // one column pair (lanes l, l + 1 of a row) per thread
    for (int idx = threadIdx.x; idx < RT * CT * 128; idx += 256) {
      const int tc = idx >> 7, rt = tc / CT, ct = tc % CT, e = idx & 127, r = e >> 5,
                l = 16 * ((e >> 3) & 3) + 2 * (e & 7);
      float v0 = ((red[0][rt][ct][r][l] + red[1][rt][ct][r][l]) + red[2][rt][ct][r][l]) + red[3][rt][ct][r][l];
      float v1 = ((red[0][rt][ct][r][l + 1] + red[1][rt][ct][r][l + 1]) + red[2][rt][ct][r][l + 1]) +
                 red[3][rt][ct][r][l + 1];
      if constexpr (AM == 2) {
        v0 = v0 / rrms[16 * rt + 4 * (l >> 4) + r];
        v1 = v1 / rrms[16 * rt + 4 * (l >> 4) + r];
      }
      const int row = m0 + 16 * rt + 4 * (l >> 4) + r, col = n0 + 16 * ct + (l & 15);
      if (row >= g.M || ct >= ctn) continue;
      const EpiArgs& ea = g.e;
      if constexpr (EPI == kEpiSwiglu) {
        // (the tile copy orders the gate/up pairs by the down projection's input positions)
        const int F = g.N / 2, f = col >> 1;
        put_split(ea.act + act_index(row, f, F, 0), ea.act_plane, swiglu(v0, v1));
      } else {
        const int p = row_pos(ea.rows, row);
        const int64_t crow = cache_row(ea.rows, row, p);
        const int head = col / kDh, ri = (col % kDh) >> 1;
        const float c = ea.rope[int64_t(p) * kDh + ri], sg = ea.rope[int64_t(p) * kDh + kDh / 2 + ri];
        const bool isv = head >= ea.H + ea.KV;
        const int gi = isv ? head - ea.H - ea.KV : head - ea.H;
        uint16_t* cp = (isv ? ea.vc : ea.kc) + (int64_t(gi) * ea.rows.pool + crow) * kDh;
        qkv_pair(v0, v1, c, sg, col, ea.H, ea.KV, ea.qkv + int64_t(row) * g.N + head * kDh, cp);
      }
    }
  }
}

__device__ __forceinline__ float block_sum256(float v, float* red) {
  v = wave_sum(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  const float s = (red[0] + red[1]) + (red[2] + red[3]);
  __syncthreads();
  return s;
}

// Row blockIdx.x + row0: h += sum_z part[z] (z in order), then
// xn[j] = scale[i] * (h[i] / sqrt(mean(h^2) + 1e-5)) as hi/lo bf16 parts (planes `plane` apart),
// with i the input element at position j of the packed row layout (model.py:94-98).  Every partial is requested before
// the first is added, so the sum costs one memory round trip.  With packed, h holds the row in
// packed order (element i at position perm_pos(i)) in tile order (act_index), and no partials are
// added.
__global__ __launch_bounds__(kNormThreads) void mx_norm(float* h, const float* part, int splits, int M, int d,
                                                        const uint16_t* scale, uint16_t* xn, int64_t plane,
                                                        int row0, int ldx, int packed) {
  constexpr int NE = kMaxRows / kNormThreads;
  __shared__ float red[4];
  __shared__ __align__(16) float hs[kMaxRows];
  const int m = blockIdx.x + row0;
  float* hr = h + int64_t(m) * d;
  // every load (residual, partials, the scales of this thread's outputs) is issued up front from
  // clamped indices: a load under a branch is waited for at the join.  Thread t sums elements
  // 4t..4t+3 (16-byte loads; d is a multiple of 32) and writes outputs t, t + 256, ...
  static_assert(kMaxRows == 4 * kNormThreads, "one float4 of the row per thread");
  const int n4 = 4 * threadIdx.x, n4c = min(n4, d - 4);
  const bool own = n4 < d;
  uint16_t sc[NE];
#pragma unroll
  for (int i = 0; i < NE; ++i) sc[i] = scale[perm_elem(min(int(threadIdx.x) + kNormThreads * i, d - 1), d)];
  float4 v = *reinterpret_cast<const float4*>(packed ? h + act_index(m, n4c, d, 0) : hr + n4c);
  {   // partials (none when splits == 0: then split 0 is read and ignored)
    float4 pv[kMaxSplitK];
#pragma unroll
    for (int z = 0; z < kMaxSplitK; ++z)
      pv[z] = *reinterpret_cast<const float4*>(part + (int64_t(min(z, max(splits, 1) - 1)) * M + m) * d + n4c);
#pragma unroll
    for (int z = 0; z < kMaxSplitK; ++z)
      if (z < splits) {
        v.x += pv[z].x;
        v.y += pv[z].y;
        v.z += pv[z].z;
        v.w += pv[z].w;
      }
  }
  float ss = 0.f;
  if (own) {
    if (splits) *reinterpret_cast<float4*>(hr + n4) = v;
    *reinterpret_cast<float4*>(hs + n4) = v;
    ss = ((v.x * v.x + v.y * v.y) + v.z * v.z) + v.w * v.w;
  }
  ss = block_sum256(ss, red);
  const float r = sqrtf(ss / float(d) + 1e-5f);
#pragma unroll
  for (int q = 0; q < NE; ++q) {
    const int j = threadIdx.x + kNormThreads * q;
    if (j < d)
      put_split(xn + act_index(blockIdx.x, j, d, ldx), plane, bf2f(sc[q]) * (hs[packed ? j : perm_elem(j, d)] / r));
  }
}

// Row m of the residual stream: the embedding of tokens[m] (element n at n, or with packed at its
// packed position perm_pos(n) in tile order, act_index).  With xscale (packed only) also the first
// RMSNorm's input planes, scale * h as hi/lo tiles (xn, lo plane `plane` further), and the row's
// sum of h^2 in ssq[m].
__global__ __launch_bounds__(256) void mx_embed(const uint16_t* emb, const int32_t* tokens, int d, float* h,
                                                int32_t* status, int V, int packed, const uint16_t* xscale,
                                                uint16_t* xn, int64_t plane, float* ssq) {
  __shared__ float red[4];
  const int m = blockIdx.x;
  int t = tokens[m];
  if (t < 0 || t >= V) {
    if (threadIdx.x == 0) atomicOr(status, 2);
    t = 0;
  }
  constexpr int NE = kMaxRows / 256;   // every load issued before the first store
  uint16_t e[NE];
#pragma unroll
  for (int i = 0; i < NE; ++i) e[i] = emb[int64_t(t) * d + min(int(threadIdx.x) + 256 * i, d - 1)];
  float hsq = 0.f;
#pragma unroll
  for (int i = 0; i < NE; ++i) {
    const int n = threadIdx.x + 256 * i;
    if (n < d) {
      const float hv = bf2f(e[i]);
      if (packed) {
        const int j = perm_pos(n, d);
        h[act_index(m, j, d, 0)] = hv;
        if (xscale) put_split(xn + act_index(m, j, d, 0), plane, bf2f(xscale[j]) * hv);
      } else {
        h[int64_t(m) * d + n] = hv;
      }
      hsq += hv * hv;
    }
  }
  if (xscale) {
    hsq = block_sum256(hsq, red);
    if (threadIdx.x == 0) ssq[m] = hsq;
  }
}

// Row blockIdx.x: q/k/v = sum_z part[z] (z in order) over the packed q/k/v rows; RoPE on the
// q and k pairs (packed rows 2i, 2i+1 = dims i, i+32; model.py:110-117) at the row's
// position; f32 q/k/v in natural head-dim order to qkv; bf16 K/V to the cache.
__global__ __launch_bounds__(256) void mx_qkv_fin(const float* part, int splits, int M, int H, int KV,
                                                  const float* rope, Rows rows, uint16_t* kc, uint16_t* vc,
                                                  float* qkv) {
  const int m = blockIdx.x, nq = (H + 2 * KV) * kDh;
  const int t = blockIdx.y * 256 + threadIdx.x;
  if (t >= nq / 4) return;
  const int col = 4 * t;   // column pairs (col, col + 1) and (col + 2, col + 3), one head
  float4 pv[kMaxSplitK];
#pragma unroll
  for (int z = 0; z < kMaxSplitK; ++z)
    pv[z] = *reinterpret_cast<const float4*>(part + (int64_t(min(z, splits - 1)) * M + m) * nq + col);
  // the loads that depend on the position (RoPE row, cache row) are issued together, for every
  // column (a load under a branch is waited for at the join)
  const int p = row_pos(rows, m);
  const int64_t crow = cache_row(rows, m, p);
  const int ri = (col % kDh) >> 1;
  const float2 cs = *reinterpret_cast<const float2*>(rope + int64_t(p) * kDh + ri);
  const float2 sn = *reinterpret_cast<const float2*>(rope + int64_t(p) * kDh + kDh / 2 + ri);
  float4 sv = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int z = 0; z < kMaxSplitK; ++z)
    if (z < splits) {
      sv.x += pv[z].x;
      sv.y += pv[z].y;
      sv.z += pv[z].z;
      sv.w += pv[z].w;
    }
  const int head = col / kDh;
  float* q = qkv + int64_t(m) * nq + head * kDh;
  const bool isv = head >= H + KV;
  const int g = isv ? head - H - KV : head - H;
  uint16_t* cp = (isv ? vc : kc) + (int64_t(g) * rows.pool + crow) * kDh;
  qkv_pair(sv.x, sv.y, cs.x, sn.x, col, H, KV, q, cp);
  qkv_pair(sv.z, sv.w, cs.y, sn.y, col + 2, H, KV, q, cp);
}

// Row blockIdx.x: act_f = silu(gate_f) * up_f over the summed partials (gate/up are the packed
// rows 2f, 2f+1; model.py:159), as hi/lo bf16 parts at the down projection's input position of f.
__global__ __launch_bounds__(256) void mx_swiglu_fin(const float* part, int splits, int M, int F, uint16_t* act,
                                                     int64_t plane, int ldx) {
  const int m = blockIdx.x, f = 2 * (blockIdx.y * 256 + threadIdx.x);   // outputs f and f + 1 (F is even)
  if (f >= F) return;
  float4 pv[kMaxSplitK];
#pragma unroll
  for (int z = 0; z < kMaxSplitK; ++z)
    pv[z] = *reinterpret_cast<const float4*>(part + (int64_t(min(z, splits - 1)) * M + m) * (2 * F) + 2 * f);
  float g0 = 0.f, u0 = 0.f, g1 = 0.f, u1 = 0.f;
#pragma unroll
  for (int z = 0; z < kMaxSplitK; ++z)
    if (z < splits) {
      g0 += pv[z].x;
      u0 += pv[z].y;
      g1 += pv[z].z;
      u1 += pv[z].w;
    }
  put_split(act + act_index(m, perm_pos(f, F), F, ldx), plane, swiglu(g0, u0));
  put_split(act + act_index(m, perm_pos(f + 1, F), F, ldx), plane, swiglu(g1, u1));
}

// Reductions over the 16 lanes of a DPP row, every lane receiving the result (rotations by 1, 2,
// 4, 8).  The sum's rounding may differ between the lanes of a row; callers read one lane.
template <int CTRL>
__device__ __forceinline__ float dpp_ror(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_ror<0x121>(v));
  v = fmaxf(v, dpp_ror<0x122>(v));
  v = fmaxf(v, dpp_ror<0x124>(v));
  return fmaxf(v, dpp_ror<0x128>(v));
}
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_ror<0x121>(v);
  v += dpp_ror<0x122>(v);
  v += dpp_ror<0x124>(v);
  return v + dpp_ror<0x128>(v);
}

// Prefill: causal GQA attention of query block blockIdx.y (16 rows) for head blockIdx.x on the
// matrix cores.  The key range 0..q0+15 is cut into 32-key chunks, wave w taking chunks w, w + 4,
// ...: S = Q K^T (16 x 32) and O += P V (16 x 64) run on v_mfma_f32_16x16x32_bf16 with every f32
// operand as hi/lo bf16 parts (mfma3), the softmax is online per query row in f32, and the four
// waves' (max, sum, O) are merged by log-sum-exp at the end.  Scale 1/sqrt(64) (model.py:98).
// MFMA operand lanes: A[i][8 (l / 16) ..] = row i = l % 16; B[8 (l / 16) ..][n] with n = l % 16;
// D: rows 4 (l / 16) + r of column l % 16.
// The head outputs go to the O projection's input planes at their packed positions, or with
// natural at their element index (the tile copy's O columns are in natural order).
__global__ __launch_bounds__(256) void mx_attention_prefill(const float* qkv, int M, int H, int KV, uint16_t* att,
                                                            int64_t plane, int ldx, int natural) {
  constexpr int PS = 36;   // row stride (floats) of a wave's P tile in LDS: 16-byte reads of 16 rows spread over banks
  __shared__ __align__(16) float sp[4][16 * PS];
  __shared__ float sm[4][16], sl[4][16];
  __shared__ float so[4][16][kDh + 4];
  const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r16 = lane & 15, kq = lane >> 4;
  const int h = blockIdx.x, g = h / (H / KV);
  const int nqkv = (H + 2 * KV) * kDh, d = H * kDh;
  const int q0 = blockIdx.y * 16;
  const int nk = min(q0 + 16, M), nch = (nk + 31) / 32;
  // Q fragments (rows past M read row M - 1: their outputs are not stored)
  uint4 qh[2], ql[2];
  {
    const float* qr = qkv + int64_t(min(q0 + r16, M - 1)) * nqkv + h * kDh + 8 * kq;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const float4 a = *reinterpret_cast<const float4*>(qr + 32 * ks);
      const float4 b = *reinterpret_cast<const float4*>(qr + 32 * ks + 4);
      const float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
      split8(x, qh[ks], ql[ks]);
    }
  }
  float m[4], l[4];   // rows 4 kq + r: running max and sum (alike in the 16 lanes of the row)
  f32x4 o[4];         // O columns 16 dt + r16
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    m[r] = -INFINITY;
    l[r] = 0.f;
    o[r] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  float* P = sp[wv];
  for (int c = wv; c < nch; c += 4) {
    const int kb = 32 * c;
    // K rows (B of S: key kb + 16 t + r16, dims 32 ks + 8 kq ..) and V values (B of P V: keys
    // kb + 8 kq + e, dim 16 dt + r16), all requested before the first MFMA; keys past M read
    // row M - 1 and are masked
    float kf[2][2][8], vf[4][8];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const float* kr = qkv + int64_t(min(kb + 16 * t + r16, M - 1)) * nqkv + (H + g) * kDh + 8 * kq;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const float4 a = *reinterpret_cast<const float4*>(kr + 32 * ks);
        const float4 b = *reinterpret_cast<const float4*>(kr + 32 * ks + 4);
        kf[t][ks][0] = a.x; kf[t][ks][1] = a.y; kf[t][ks][2] = a.z; kf[t][ks][3] = a.w;
        kf[t][ks][4] = b.x; kf[t][ks][5] = b.y; kf[t][ks][6] = b.z; kf[t][ks][7] = b.w;
      }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float* vr = qkv + int64_t(min(kb + 8 * kq + e, M - 1)) * nqkv + (H + KV + g) * kDh + r16;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) vf[dt][e] = vr[16 * dt];
    }
    f32x4 s[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      s[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        uint4 kh, kl;
        split8(kf[t][ks], kh, kl);
        s[t] = mfma3(qh[ks], ql[ks], kh, kl, s[t]);
      }
    }
    // scale, causal mask, online softmax of rows 4 kq + r over keys kb + 16 t + r16
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = q0 + 4 * kq + r;
      const int j0 = kb + r16, j1 = kb + 16 + r16;
      const float v0 = (j0 <= i && j0 < M) ? s[0][r] * 0.125f : -INFINITY;
      const float v1 = (j1 <= i && j1 < M) ? s[1][r] * 0.125f : -INFINITY;
      const float mn = fmaxf(m[r], row16_max(fmaxf(v0, v1)));
      const float p0 = mn == -INFINITY ? 0.f : expf(v0 - mn), p1 = mn == -INFINITY ? 0.f : expf(v1 - mn);
      const float alpha = m[r] == -INFINITY ? 0.f : expf(m[r] - mn);
      l[r] = l[r] * alpha + row16_sum(p0 + p1);
      m[r] = mn;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) o[dt][r] *= alpha;
      P[(4 * kq + r) * PS + r16] = p0;
      P[(4 * kq + r) * PS + 16 + r16] = p1;
    }
    __builtin_amdgcn_wave_barrier();
    uint4 ph, pl;
    {
      const float4 a = *reinterpret_cast<const float4*>(P + r16 * PS + 8 * kq);
      const float4 b = *reinterpret_cast<const float4*>(P + r16 * PS + 8 * kq + 4);
      const float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
      split8(x, ph, pl);
    }
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      uint4 vh, vl;
      split8(vf[dt], vh, vl);
      o[dt] = mfma3(ph, pl, vh, vl, o[dt]);
    }
    __builtin_amdgcn_wave_barrier();
  }
  // merge the waves by log-sum-exp
  if (r16 == 0)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      sm[wv][4 * kq + r] = m[r];
      sl[wv][4 * kq + r] = l[r];
    }
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int r = 0; r < 4; ++r) so[wv][4 * kq + r][16 * dt + r16] = o[dt][r];
  __syncthreads();
  const int qi = threadIdx.x >> 4, d4 = 4 * (threadIdx.x & 15);
  float mx = -INFINITY;
#pragma unroll
  for (int w = 0; w < 4; ++w) mx = fmaxf(mx, sm[w][qi]);
  float L = 0.f, O[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const float wt = sm[w][qi] == -INFINITY ? 0.f : expf(sm[w][qi] - mx);
    L += sl[w][qi] * wt;
#pragma unroll
    for (int e = 0; e < 4; ++e) O[e] += so[w][qi][d4 + e] * wt;
  }
  const int i = q0 + qi;
  if (i < M)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int el = h * kDh + d4 + e;
      put_split(att + act_index(i, natural ? el : perm_pos(el, d), d, ldx), plane, O[e] / L);
    }
}

// Batched decode: row m (one sequence at position p = pos(m)) and head blockIdx.y attend over
// the cached rows 0..p-1 of the sequence (bf16, through its page table) and the row's
// current, un-rounded K/V (multi_sm_decode.py:182-221).  Wave w takes positions
// [64w, 64w + 64) (contexts up to 512): each lane looks its position's cache row up, then the
// wave requests its K rows (lane = position) and all its V values (lane = dimension) at once,
// so the block costs two memory round trips; each wave keeps its own maximum and sum and the
// waves' states are merged in LDS at the end.
constexpr int kAttnWaves = 8;
// Positions mx_attention_decode covers: wave w takes the 64-position blocks w, w + 8, ...
constexpr int kAttnMaxCtx = 2048;
__global__ __launch_bounds__(64 * kAttnWaves) void mx_attention_decode(const float* qkv, Rows rows, int H, int KV,
                                                                       const uint16_t* kc, const uint16_t* vc,
                                                                       uint16_t* att, int64_t plane, int ldx,
                                                                       int natural) {
  __shared__ float sq[kDh], skc[kDh], svc[kDh];   // q, and the current position's f32 k and v
  __shared__ float sp[kAttnWaves][64];
  __shared__ int srow[kAttnWaves][64];
  __shared__ float so[kAttnWaves][kDh];
  __shared__ float sml[kAttnWaves][2];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int m = blockIdx.x, h = blockIdx.y, g = h / (H / KV);
  const int nqkv = (H + 2 * KV) * kDh, d = H * kDh;
  // q, the page-table entries of the first block and p are loaded together: the page-table load
  // does not wait for p (every entry of a row is a sanitized page; p only selects which rows are
  // cached positions), and no load sits under a branch (it would be waited for at the join)
  const float* qr = qkv + int64_t(m) * nqkv;
  const int qsel = min(int(threadIdx.x) / kDh, 2);   // threads 0..63: q, 64..127: k, others: v
  const float qv = qr[(qsel == 0 ? h : (qsel == 1 ? H + g : H + KV + g)) * kDh + (threadIdx.x & (kDh - 1))];
  auto row_of = [&](int j) { return cache_row(rows, m, rows.pages ? min(j, rows.max_pages * kPage - 1) : j); };
  int64_t cr = row_of(64 * wv + lane);
  const int p = row_pos(rows, m);
  if (threadIdx.x < 3 * kDh) (qsel == 0 ? sq : (qsel == 1 ? skc : svc))[threadIdx.x & (kDh - 1)] = qv;
  const uint16_t* kg = kc + int64_t(g) * rows.pool * kDh;
  const uint16_t* vg = vc + int64_t(g) * rows.pool * kDh;
  __syncthreads();
  float mx = -INFINITY, ls = 0.f, o = 0.f;
  // blocks wv, wv + 8, ... up to the one holding p (each holds at least one position <= p);
  // the first is taken as it is, later ones merged by log-sum-exp
  for (int blk = wv; 64 * blk <= p; blk += kAttnWaves) {
    const int j0 = 64 * blk, j = j0 + lane;
    if (blk != wv) cr = row_of(j);
    srow[wv][lane] = j < p ? int(cr) : 0;
    __builtin_amdgcn_wave_barrier();
    uint4 ku[kDh / 8];
    const uint4* kr = reinterpret_cast<const uint4*>(kg + int64_t(srow[wv][lane]) * kDh);
#pragma unroll
    for (int e8 = 0; e8 < kDh / 8; ++e8) ku[e8] = kr[e8];
    uint16_t vv[64];
#pragma unroll
    for (int jj = 0; jj < 64; ++jj) vv[jj] = vg[int64_t(srow[wv][jj]) * kDh + lane];
    float s = -INFINITY;
    if (j < p) {
      float a0 = 0.f, a1 = 0.f;
#pragma unroll
      for (int e8 = 0; e8 < kDh / 8; ++e8) {
        const uint32_t wds[4] = {ku[e8].x, ku[e8].y, ku[e8].z, ku[e8].w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          a0 += sq[8 * e8 + 2 * q] * __uint_as_float(wds[q] << 16);
          a1 += sq[8 * e8 + 2 * q + 1] * __uint_as_float(wds[q] & 0xffff0000u);
        }
      }
      s = (a0 + a1) * 0.125f;
    } else if (j == p) {   // current position: f32 K from this row's projection
      float a0 = 0.f, a1 = 0.f;
      for (int e = 0; e < kDh; e += 2) {
        a0 += sq[e] * skc[e];
        a1 += sq[e + 1] * skc[e + 1];
      }
      s = (a0 + a1) * 0.125f;
    }
    const float bmx = wave_max(s);
    const float e = (s == -INFINITY) ? 0.f : expf(s - bmx);
    const float bls = wave_sum(e);
    sp[wv][lane] = e;
    __builtin_amdgcn_wave_barrier();
    const float vcur = svc[lane];
    float o4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int jj = 0; jj < 64; ++jj) {
      const float v = j0 + jj < p ? bf2f(vv[jj]) : (j0 + jj == p ? vcur : 0.f);
      o4[jj & 3] += sp[wv][jj] * v;
    }
    const float bo = (o4[0] + o4[1]) + (o4[2] + o4[3]);
    if (blk == wv) {
      mx = bmx;
      ls = bls;
      o = bo;
    } else {
      const float M = fmaxf(mx, bmx);
      const float a0 = expf(mx - M), a1 = expf(bmx - M);
      ls = ls * a0 + bls * a1;
      o = o * a0 + bo * a1;
      mx = M;
    }
    __builtin_amdgcn_wave_barrier();   // srow and sp are rewritten by the next block
  }
  so[wv][lane] = o;
  if (lane == 0) {
    sml[wv][0] = mx;
    sml[wv][1] = ls;
  }
  __syncthreads();
  if (wv == 0) {
    float M = -INFINITY;
    for (int w = 0; w < kAttnWaves; ++w) M = fmaxf(M, sml[w][0]);
    float num = 0.f, den = 0.f;
    for (int w = 0; w < kAttnWaves; ++w) {
      if (sml[w][0] == -INFINITY) continue;
      const float a = expf(sml[w][0] - M);
      num += a * so[w][lane];
      den += a * sml[w][1];
    }
    put_split(att + act_index(m, natural ? h * kDh + lane : perm_pos(h * kDh + lane, d), d, ldx), plane, num / den);
  }
}

// argmax of each row of logits (lowest index on ties): out[2*row] = index, out[2*row+1] = status
__global__ __launch_bounds__(1024) void mx_argmax(const float* logits, int V, int ld, int32_t* out,
                                                  const int32_t* status) {
  __shared__ uint64_t red[16];
  const float* lr = logits + int64_t(blockIdx.x) * ld;
  uint64_t best = 0;
  constexpr int kBatch = 16;   // loads in flight per thread (clamped, so none sits under a branch)
  for (int j0 = threadIdx.x; j0 < V; j0 += kBatch * 1024) {
    float x[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) x[u] = lr[min(j0 + 1024 * u, V - 1)];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int j = j0 + 1024 * u;
      uint32_t b = __float_as_uint(x[u]);
      b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
      const uint64_t key = (uint64_t(b) << 32) | uint64_t(0xffffffffu - uint32_t(j));
      best = j < V && key > best ? key : best;
    }
  }
  for (int o = 32; o; o >>= 1) {
    const uint64_t w = __shfl_xor(best, o);
    best = w > best ? w : best;
  }
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint64_t b = red[0];
    for (int i = 1; i < 16; ++i) b = red[i] > b ? red[i] : b;
    out[2 * blockIdx.x] = int32_t(0xffffffffu - uint32_t(b & 0xffffffffu));
    out[2 * blockIdx.x + 1] = *status;
  }
}

// Copies the rows' positions and page tables into the workspace, which is what every later
// kernel addresses the cache with: a position outside [0, ctx) or past the table, and a table
// entry outside the pool, is replaced by 0 (status bit 2), so no access leaves the pool.
// pos == NULL: every row is at fixed_pos (the last position of a prefill).
__global__ void mx_sanitize_rows(const int32_t* pos, int fixed_pos, const int32_t* pages, int M, int max_pages,
                                 int ctx, int pool_pages, int32_t* pos_out, int32_t* pages_out, int32_t* status) {
  const int m = blockIdx.x * blockDim.x + threadIdx.x;
  if (m >= M) return;
  int p = pos ? pos[m] : fixed_pos;
  bool bad = p < 0 || p >= ctx || p / kPage >= max_pages;
  if (bad) p = 0;
  constexpr int kBatch = 8;   // page-table loads in flight (clamped indices, stores after)
  for (int i0 = 0; i0 < max_pages; i0 += kBatch) {
    int pv[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) pv[u] = pages[int64_t(m) * max_pages + min(i0 + u, max_pages - 1)];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int i = i0 + u;
      int pg = pv[u];
      if (pg < 0 || pg >= pool_pages) {
        if (i < max_pages && i <= p / kPage) bad = true;
        pg = 0;
      }
      if (i < max_pages) pages_out[int64_t(m) * max_pages + i] = pg;
    }
  }
  if (pos_out) pos_out[m] = p;
  if (bad) atomicOr(status, 4);
}

// One 16-byte piece per thread of the tile copy of an N x K matrix W (rows in packed order): piece
// p is lane p % 64 of tile p / 64 = (n / 16) (K / 32) + k / 32, i.e. row n = 16 (tile / (K / 32)) +
// lane % 16 at positions 32 (tile % (K / 32)) + 8 (lane / 16) .. + 8.  Row orders (rowperm): 1 = row
// n of the copy is row perm_elem(n, N) of W, so output column n is element perm_elem(n) of an
// N-long vector, i.e. its packed position n (the O and down projections, whose outputs add to the
// residual); 2 = row pair n / 2 is pair perm_elem(n / 2, N / 2) (gate/up: output pair f is then the
// down projection's input at its packed position f).  With natk, column k of the copy is input
// element k (W's column perm_pos(k)): the O projection, whose input the attention writes in
// natural order.  Either way an epilogue's consecutive outputs land on consecutive positions.
__global__ __launch_bounds__(256) void mx_pack_tiles(const uint16_t* W, int N, int K, int rowperm, int natk,
                                                     uint16_t* T) {
  const int64_t p = int64_t(blockIdx.x) * 256 + threadIdx.x;
  const int S = K / kBK;
  if (p >= int64_t(N) * S * 64) return;
  const int lane = int(p & 63);
  const int64_t tile = p >> 6;
  const int n = int(16 * (tile / S)) + (lane & 15);
  const int64_t src = rowperm == 1 ? perm_elem(n, N) : (rowperm == 2 ? 2 * perm_elem(n >> 1, N / 2) + (n & 1) : n);
  const int k = kBK * int(tile % S) + 8 * (lane >> 4);
  if (natk) {
    uint16_t v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = W[src * K + perm_pos(k + e, K)];
#pragma unroll
    for (int e = 0; e < 8; ++e) T[p * 8 + e] = v[e];
  } else {
    *reinterpret_cast<uint4*>(T + p * 8) = *reinterpret_cast<const uint4*>(W + src * K + k);
  }
}

// A layer's two RMSNorm scales in packed order: out[j] = scale[perm_elem(j, d)] for [ln1 | ln2].
__global__ __launch_bounds__(256) void mx_pack_scales(const uint16_t* ln, int d, uint16_t* out) {
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j >= 2 * d) return;
  const int half = j >= d ? d : 0;
  out[j] = ln[half + perm_elem(j - half, d)];
}

// ---------------------------------------------------------------- host side
struct Layout {
  size_t h, xn, ssq, qkv, att, act, part, status, rowpos, pages, bytes;
};

static size_t al256(size_t x) { return (x + 255) & ~size_t(255); }


// Widest projection mx_gemm_rows takes with weights in row order: wider ones (the 306M gate/up,
// 5632 outputs) run faster on the split-K kernel (measured: 128-token prefill 1.95 -> 1.79 ms).
// With the weights in tile order it takes every width (gate/up at 128 rows: 18.7 -> 10.1 us).
constexpr int kRowsMaxN = 4096;

// Column tiles (of 16) per workgroup of mx_gemm_rows: the widest that still gives about one
// workgroup per compute unit; 0 when the projection has too few output tiles for it (few rows),
// or too short a K for every wave to take a step, and the split-K kernel runs instead.
// With the weights in tile order (tw) every projection takes it (the fused epilogues and the
// folded norms live there): the widest that gives about one workgroup per compute unit, else 1.
// (Workgroups owning 2 or 4 row tiles, which read each weight tile for 32 or 64 rows, measured
// slower: 128-token prefill 1.16 -> 1.36 / 1.70 ms.)
static int rows_ct(int M, int N, int K, bool tw) {
  const int T = (M + 15) / 16, n16 = N / 16;
  if (K / kBK < 4) return 0;
  if (!tw && (M < 48 || N > kRowsMaxN)) return 0;
  for (int ct : {8, 6, 4, 3, 2, 1})
    if (n16 % ct == 0 && T * (n16 / ct) >= 224) return ct;
  return tw ? 1 : 0;
}

// Workgroups owning two row tiles (tile-order weights, pair epilogues): when one row tile per
// workgroup needs more workgroups than compute units, the column tiles (6, 8 or 4, the last group
// ragged) of a grid of 224-256 workgroups, else 0.  Every weight tile then serves 32 rows, and one
// pass over the CUs does the whole projection (128-token gate/up, 352 column tiles: 13.3 -> 9.2 us
// in a microbenchmark with weights that miss the last-level cache).
static int rows_ct2(int M, int N, int K, bool tw) {
  const int ct1 = rows_ct(M, N, K, tw), T = (M + 15) / 16, n16 = N / 16;
  if (!tw || ct1 <= 0 || T < 2 || T * (n16 / ct1) <= 256) return 0;
  for (int ct : {6, 8, 4}) {
    const int wg = ((T + 1) / 2) * ((n16 + ct - 1) / ct);
    if (wg >= 224 && wg <= 256) return ct;
  }
  return 0;
}

// K splits of a projection: 1 for mx_gemm_rows, else enough split-K workgroups to occupy every
// compute unit, at least 4 K steps each
static int splits_for(int M, int N, int K, int bm, bool tw) {
  if (rows_ct(M, N, K, tw) > 0) return 1;
  const int tiles = (N / kBN) * ((M + bm - 1) / bm);
  int s = 1;
  while (tiles * s < 256 && (K / kBK) / (2 * s) >= 4 && 2 * s <= kMaxSplitK) s *= 2;
  return s;
}

static int bm_for(int M) { return M <= 16 ? 16 : (M <= 64 ? 64 : 128); }

static size_t part_floats(const msd_config* c, int M) {
  const int d = c->d_model, ff = c->d_ff, nqkv = (c->n_heads + 2 * c->n_kv_heads) * kDh;
  const int bm = bm_for(M);
  size_t mx = 0;
  for (bool tw : {false, true}) {
    mx = std::max(mx, size_t(splits_for(M, nqkv, d, bm, tw)) * nqkv);
    mx = std::max(mx, size_t(splits_for(M, d, d, bm, tw)) * d);
    mx = std::max(mx, size_t(splits_for(M, 2 * ff, d, bm, tw)) * 2 * ff);
    mx = std::max(mx, size_t(splits_for(M, d, ff, bm, tw)) * d);
  }
  return mx * M;
}

static int pad16(int M) { return (M + 15) & ~15; }

static Layout layout(const msd_config* c, int M) {
  const int d = c->d_model, ff = c->d_ff, nqkv = (c->n_heads + 2 * c->n_kv_heads) * kDh;
  Layout L;
  size_t o = 0;
  L.h = o;      o += al256(size_t(pad16(M)) * d * 4);   // rows padded to whole tiles (tile order)
  // activation planes (hi and lo) in tile order, rows padded to whole tiles
  L.xn = o;     o += al256(size_t(pad16(M)) * d * 2 * 2);
  L.ssq = o;    o += al256(size_t(M) * (d / 16) * 4);   // partial sums of h^2: at most d / 16 per row
  L.qkv = o;    o += al256(size_t(M) * nqkv * 4);
  L.att = o;    o += al256(size_t(pad16(M)) * d * 2 * 2);
  L.act = o;    o += al256(size_t(pad16(M)) * ff * 2 * 2);
  L.part = o;   o += al256(part_floats(c, M) * 4);
  L.status = o; o += 256;
  L.rowpos = o; o += al256(size_t(M) * 4);
  L.pages = o;  o += al256(size_t(M) * ((c->context_len + kPage - 1) / kPage) * 4);
  L.bytes = o;
  return L;
}

static bool mx_config_ok(const msd_config* c) {
  if (!c || c->d_head != kDh || c->n_heads <= 0 || c->n_kv_heads <= 0 || c->n_layers <= 0) return false;
  if (c->n_heads * kDh != c->d_model || c->n_heads % c->n_kv_heads) return false;
  if (c->d_model % kBN || (2 * c->d_ff) % kBN || c->vocab_size % kBN || c->d_ff % 8) return false;
  if (c->d_model % kBK || c->d_ff % kBK || c->context_len <= 0 || c->d_model > kMaxRows) return false;
  return true;
}

template <int AM, bool TW, int EPI = kEpiStore>
static void launch_rows(int ct, dim3 grid, hipStream_t s, const GemmArgs& g) {
  switch (ct) {
    case 8: hipLaunchKernelGGL((mx_gemm_rows<8, 3, AM, TW, EPI>), grid, dim3(256), 0, s, g); break;
    case 6: hipLaunchKernelGGL((mx_gemm_rows<6, 3, AM, TW, EPI>), grid, dim3(256), 0, s, g); break;
    case 4: hipLaunchKernelGGL((mx_gemm_rows<4, 4, AM, TW, EPI>), grid, dim3(256), 0, s, g); break;
    case 3: hipLaunchKernelGGL((mx_gemm_rows<3, 4, AM, TW, EPI>), grid, dim3(256), 0, s, g); break;
    case 2: hipLaunchKernelGGL((mx_gemm_rows<2, 4, AM, TW, EPI>), grid, dim3(256), 0, s, g); break;
    default: hipLaunchKernelGGL((mx_gemm_rows<1, 4, AM, TW, EPI>), grid, dim3(256), 0, s, g); break;
  }
}

template <int AM, int EPI>
static void launch_rows2(int ct, dim3 grid, hipStream_t s, const GemmArgs& g) {
  switch (ct) {
    case 8: hipLaunchKernelGGL((mx_gemm_rows<8, 2, AM, true, EPI, 2>), grid, dim3(256), 0, s, g); break;
    case 6: hipLaunchKernelGGL((mx_gemm_rows<6, 2, AM, true, EPI, 2>), grid, dim3(256), 0, s, g); break;
    default: hipLaunchKernelGGL((mx_gemm_rows<4, 2, AM, true, EPI, 2>), grid, dim3(256), 0, s, g); break;
  }
}

template <bool TA, bool TW>
static void launch_splitk(int bm, dim3 grid, hipStream_t s, const GemmArgs& g) {
  if (bm == 16) hipLaunchKernelGGL((mx_gemm<1, 1, TA, TW>), grid, dim3(256), 0, s, g);
  else if (bm == 64) hipLaunchKernelGGL((mx_gemm<2, 2, TA, TW>), grid, dim3(256), 0, s, g);
  else hipLaunchKernelGGL((mx_gemm<4, 2, TA, TW>), grid, dim3(256), 0, s, g);
}

// C = A W^T split over K: partials [splits][M][N] (pass ldo = N), or with splits == 1 rows
// of stride ldo.  lda == 0: A in tile order (act_index); tw: W in tile order (msd_pack_tiles).
// ssq: A is the scale * h planes of an RMSNorm folded into mx_gemm_rows, whose rms comes from the
// nssq partial sums of h^2 per row in ssq.  epi / ea: the epilogue of mx_gemm_rows (tile-order
// weights only).
// rows_ok: mx_gemm_rows may run (single split only).  The tied logits pass false: one row and
// every row then come from the same kernel and summation order, so the last row's logits are
// bitwise the same either way.
static hipError_t gemm(const uint16_t* A, int64_t a_plane, int lda, const uint16_t* W, bool tw, int M, int N, int K,
                       float* out, int ldo, int splits, hipStream_t s, bool rows_ok = true, int epi = kEpiStore,
                       const EpiArgs* ea = nullptr, const float* ssq = nullptr, int nssq = 0) {
  GemmArgs g{A, a_plane, W, out, M, N, K, lda, ldo, splits, ea ? *ea : EpiArgs{}, ssq, nssq};
  const int am = ssq ? 2 : (lda == 0 ? 1 : 0);
  const int ct = splits == 1 && rows_ok && am > 0 ? rows_ct(M, N, K, tw) : 0;
  if ((epi != kEpiStore || am == 2) && !(ct > 0 && tw)) return hipErrorInvalidValue;
  if ((epi == kEpiQkv || epi == kEpiSwiglu || epi == kEpiResidNorm) && !ea) return hipErrorInvalidValue;
  if (am == 2 && (lda != 0 || nssq < 1 || nssq > 64)) return hipErrorInvalidValue;
  if (epi == kEpiResidNorm && (!ea->act || !ea->xscale || !ea->ssq || N / (16 * ct) > 64)) return hipErrorInvalidValue;
  const int ct2 = ct > 0 && (epi == kEpiSwiglu || epi == kEpiQkv) ? rows_ct2(M, N, K, tw) : 0;
  if (ct2 > 0) {
    const int TG = ((M + 15) / 16 + 1) / 2, C = (N / 16 + ct2 - 1) / ct2;
    const dim3 grid(8 * ((C + 7) / 8) * TG);
    if (am == 2 && epi == kEpiQkv) launch_rows2<2, kEpiQkv>(ct2, grid, s, g);
    else if (am == 2 && epi == kEpiSwiglu) launch_rows2<2, kEpiSwiglu>(ct2, grid, s, g);
    else return hipErrorInvalidValue;
    return hipGetLastError();
  }
  if (ct > 0) {
    const int T = (M + 15) / 16, C = N / (16 * ct);
    const dim3 grid(8 * ((C + 7) / 8) * T);
    if (am == 2 && epi == kEpiQkv) launch_rows<2, true, kEpiQkv>(ct, grid, s, g);
    else if (am == 2 && epi == kEpiSwiglu) launch_rows<2, true, kEpiSwiglu>(ct, grid, s, g);
    else if (am == 1 && tw && epi == kEpiResid) launch_rows<1, true, kEpiResid>(ct, grid, s, g);
    else if (am == 1 && tw && epi == kEpiResidNorm) launch_rows<1, true, kEpiResidNorm>(ct, grid, s, g);
    else if (am == 1 && !tw && epi == kEpiStore) launch_rows<1, false>(ct, grid, s, g);
    else return hipErrorInvalidValue;
    return hipGetLastError();
  }
  const int bm = bm_for(M);
  const dim3 grid(N / kBN, (M + bm - 1) / bm, splits);
  if (am == 1) launch_splitk<true, false>(bm, grid, s, g);
  else launch_splitk<false, false>(bm, grid, s, g);
  return hipGetLastError();
}

struct Weights {
  const uint16_t* emb;
  const uint16_t* outp;
  const uint16_t* w;
  const uint16_t* lnf;
  const float* rope;
  const uint16_t* tiles;   // the projections in tile order (msd_pack_tiles), or NULL
};

// Elements of one layer in the tile copy: QKV, O, gate/up, down, each N x K in tile order (the
// O and down rows permuted so that their outputs come in packed order), then the two RMSNorm
// scales in packed order; layer after layer.
static int64_t tile_layer_elems(const msd_config* c) {
  const int64_t d = c->d_model, ff = c->d_ff, nqkv = int64_t(c->n_heads + 2 * c->n_kv_heads) * kDh;
  return nqkv * d + d * d + 2 * ff * d + d * ff + 2 * d;
}

// Element offset of the first layer's packed RMSNorm1 scales in the tile copy.
static int64_t first_norm_scales(const msd_config* c) {
  const int64_t d = c->d_model, ff = c->d_ff, nqkv = int64_t(c->n_heads + 2 * c->n_kv_heads) * kDh;
  return nqkv * d + d * d + 2 * ff * d + d * ff;
}

// The layer stack over M rows whose residual stream is already in h; leaves the last
// projection's partials pending (returned split count).
static int run_layers(const msd_config* cfg, const Weights& wt, const Rows& rows, uint16_t* kv, const Layout& L,
                      char* ws, bool prefill, hipStream_t s, hipError_t& err) {
  const int M = rows.M, d = cfg->d_model, ff = cfg->d_ff, H = cfg->n_heads, KV = cfg->n_kv_heads;
  const int nqkv = (H + 2 * KV) * kDh;
  float* h = reinterpret_cast<float*>(ws + L.h);
  uint16_t* xn = reinterpret_cast<uint16_t*>(ws + L.xn);
  float* qkv = reinterpret_cast<float*>(ws + L.qkv);
  uint16_t* att = reinterpret_cast<uint16_t*>(ws + L.att);
  uint16_t* act = reinterpret_cast<uint16_t*>(ws + L.act);
  float* part = reinterpret_cast<float*>(ws + L.part);
  float* ssq = reinterpret_cast<float*>(ws + L.ssq);
  const int64_t off_ln2 = d, off_qkv = 2 * int64_t(d), off_o = off_qkv + int64_t(nqkv) * d,
                off_gu = off_o + int64_t(d) * d, off_dn = off_gu + 2 * int64_t(ff) * d,
                layer = off_dn + int64_t(d) * ff;
  const int bm = bm_for(M);
  const bool tw = wt.tiles != nullptr;
  const int sq = splits_for(M, nqkv, d, bm, tw), so = splits_for(M, d, d, bm, tw),
            sg = splits_for(M, 2 * ff, d, bm, tw), sd = splits_for(M, d, ff, bm, tw);
  // the tile copy's per-layer offsets
  const int64_t toff_o = int64_t(nqkv) * d, toff_gu = toff_o + int64_t(d) * d, toff_dn = toff_gu + 2 * int64_t(ff) * d,
                toff_sc = toff_dn + int64_t(d) * ff;
  // partial sums of h^2 per row that the O and down epilogues leave (one per column group); the
  // first layer's come from mx_embed (one per row)
  const int cg_o = tw ? d / (16 * rows_ct(M, d, d, true)) : 0, cg_d = tw ? d / (16 * rows_ct(M, d, ff, true)) : 0;
  int pending = 0;
  err = hipSuccess;
  for (int l = 0; l < cfg->n_layers && err == hipSuccess; ++l) {
    const uint16_t* Wl = wt.w + int64_t(l) * layer;
    uint16_t* kc = kv + int64_t(l) * 2 * KV * rows.pool * kDh;
    uint16_t* vc = kc + int64_t(KV) * rows.pool * kDh;
    // activation planes in tile order (ldx 0), the lo planes after the hi planes
    const int64_t pd = int64_t(pad16(M)) * d, pf = int64_t(pad16(M)) * ff;
    if (tw) {
      // Five kernels per layer over the tile copy, h in packed order: QKV with RMSNorm1 folded in
      // and q/k/v, RoPE and the cache rows in its epilogue; attention; O adding to h and writing
      // RMSNorm2's input planes; gate/up with RMSNorm2 folded in and SwiGLU in its epilogue; down
      // adding to h and writing the next layer's RMSNorm1 input planes.
      const uint16_t* Tl = wt.tiles + int64_t(l) * tile_layer_elems(cfg);
      const bool last = l + 1 == cfg->n_layers;
      EpiArgs eq{};
      eq.rope = wt.rope;
      eq.rows = rows;
      eq.kc = kc;
      eq.vc = vc;
      eq.qkv = qkv;
      eq.H = H;
      eq.KV = KV;
      if ((err = gemm(xn, pd, 0, Tl, true, M, nqkv, d, nullptr, 0, 1, s, true, kEpiQkv, &eq, ssq, l == 0 ? 1 : cg_d)) !=
          hipSuccess)
        break;
      if (prefill)
        hipLaunchKernelGGL(mx_attention_prefill, dim3(H, (M + 15) / 16), dim3(256), 0, s, qkv, M, H, KV, att, pd, 0, 1);
      else
        hipLaunchKernelGGL(mx_attention_decode, dim3(M, H), dim3(64 * kAttnWaves), 0, s, qkv, rows, H, KV, kc, vc,
                           att, pd, 0, 1);
      EpiArgs en{};   // the next RMSNorm's input planes and partial sums of h^2
      en.act = xn;
      en.act_plane = pd;
      en.ssq = ssq;
      en.xscale = Tl + toff_sc + d;
      if ((err = gemm(att, pd, 0, Tl + toff_o, true, M, d, d, h, d, 1, s, true, kEpiResidNorm, &en)) != hipSuccess)
        break;
      EpiArgs eg{};
      eg.act = act;
      eg.act_plane = pf;
      if ((err = gemm(xn, pd, 0, Tl + toff_gu, true, M, 2 * ff, d, nullptr, 0, 1, s, true, kEpiSwiglu, &eg, ssq, cg_o)) !=
          hipSuccess)
        break;
      if (!last) en.xscale = Tl + tile_layer_elems(cfg) + toff_sc;   // the next layer's RMSNorm1
      if ((err = gemm(act, pf, 0, Tl + toff_dn, true, M, d, ff, h, d, 1, s, true, last ? kEpiResid : kEpiResidNorm,
                      last ? nullptr : &en)) != hipSuccess)
        break;
      continue;
    }
    hipLaunchKernelGGL(mx_norm, dim3(M), dim3(kNormThreads), 0, s, h, part, pending, M, d, Wl, xn, pd, 0, 0, 0);
    if ((err = gemm(xn, pd, 0, Wl + off_qkv, false, M, nqkv, d, part, nqkv, sq, s)) != hipSuccess) break;
    hipLaunchKernelGGL(mx_qkv_fin, dim3(M, (nqkv / 4 + 255) / 256), dim3(256), 0, s, part, sq, M, H, KV, wt.rope, rows,
                       kc, vc, qkv);
    if (prefill)
      hipLaunchKernelGGL(mx_attention_prefill, dim3(H, (M + 15) / 16), dim3(256), 0, s, qkv, M, H, KV, att, pd, 0, 0);
    else
      hipLaunchKernelGGL(mx_attention_decode, dim3(M, H), dim3(64 * kAttnWaves), 0, s, qkv, rows, H, KV, kc, vc, att,
                         pd, 0, 0);
    if ((err = gemm(att, pd, 0, Wl + off_o, false, M, d, d, part, d, so, s)) != hipSuccess) break;
    hipLaunchKernelGGL(mx_norm, dim3(M), dim3(kNormThreads), 0, s, h, part, so, M, d, Wl + off_ln2, xn, pd, 0, 0, 0);
    if ((err = gemm(xn, pd, 0, Wl + off_gu, false, M, 2 * ff, d, part, 2 * ff, sg, s)) != hipSuccess) break;
    hipLaunchKernelGGL(mx_swiglu_fin, dim3(M, (ff / 2 + 255) / 256), dim3(256), 0, s, part, sg, M, ff, act, pf, 0);
    if ((err = gemm(act, pf, 0, Wl + off_dn, false, M, d, ff, part, d, sd, s)) != hipSuccess) break;
    pending = sd;
  }
  if (err == hipSuccess) err = hipGetLastError();
  return pending;
}

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

__global__ void mx_clear_status(int32_t* status) { *status = 0; }
__global__ void mx_copy_f32(const float* src, float* dst, int n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) dst[i] = src[i];
}

// ---- Replaying a pass's launches from a graph (opt-in) ----
// A pass is ~130 dependent launches; enqueueing them costs the host ~0.35 ms per pass (306M),
// replaying them from a graph ~0.07 ms.  The device runs the replay ~1 % slower (128-token
// prefill 1.037-1.047 vs 1.022-1.032 ms; 16 tokens 0.797 vs 0.787 ms), so graphs are for callers
// whose host thread is the bottleneck and are off unless asked for (msd_set_launch_graphs, or
// MSD_LAUNCH_GRAPHS=1 in the environment).  The key holds every value a launch bakes in (shape, device pointers, sizes); buffer
// contents are read when the kernels run, so a replay with new tokens or weights in the same
// buffers is exact.  Captured on a private stream of the device (capture runs nothing) and launched
// on the caller's stream; a stream that is itself being captured gets the launches directly.
// The status word is cleared by a kernel, not a memset node.
constexpr size_t kGraphCache = 16;   // graphs kept per process (least recently used is dropped)

struct GraphEntry {
  std::vector<char> key;
  int dev;
  hipGraphExec_t exec;
  hipEvent_t done;   // recorded after the latest replay: waited for before the graph is dropped
  uint64_t used;
};

static std::atomic<int> g_use_graphs{-1};   // -1: not read yet (MSD_LAUNCH_GRAPHS=1 switches them on)

static bool graphs_on() {
  int v = g_use_graphs.load();
  if (v < 0) {
    const char* e = std::getenv("MSD_LAUNCH_GRAPHS");
    int want = e && e[0] == '1' ? 1 : 0;
    g_use_graphs.compare_exchange_strong(v, want);
    v = g_use_graphs.load();
  }
  return v != 0;
}

struct KeyBuf {
  std::vector<char> b;
  template <class T>
  KeyBuf& add(const T& v) {
    const char* p = reinterpret_cast<const char*>(&v);
    b.insert(b.end(), p, p + sizeof(T));
    return *this;
  }
  KeyBuf& cfg(const msd_config* c) {
    return add(c->vocab_size).add(c->d_model).add(c->n_heads).add(c->n_kv_heads).add(c->n_layers).add(c->d_head)
        .add(c->d_ff).add(c->context_len);
  }
};

template <class F>
static int32_t launch_graphed(const std::vector<char>& key, hipStream_t s, F&& body) {
  if (!graphs_on()) return body(s);
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &cs) != hipSuccess) return MSD_E_HIP;
  if (cs != hipStreamCaptureStatusNone) return body(s);
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return MSD_E_HIP;
  static std::mutex mu;
  static std::vector<GraphEntry> cache;
  static std::vector<hipStream_t> capture_streams;
  static uint64_t tick = 0;
  std::lock_guard<std::mutex> lock(mu);
  GraphEntry* e = nullptr;
  for (GraphEntry& c : cache)
    if (c.dev == dev && c.key == key) e = &c;
  if (!e) {
    if (int(capture_streams.size()) <= dev) capture_streams.resize(dev + 1, nullptr);
    if (!capture_streams[dev] && hipStreamCreateWithFlags(&capture_streams[dev], hipStreamNonBlocking) != hipSuccess)
      return MSD_E_HIP;
    hipStream_t cap = capture_streams[dev];
    if (hipStreamBeginCapture(cap, hipStreamCaptureModeRelaxed) != hipSuccess) return MSD_E_HIP;
    const int32_t rc = body(cap);
    hipGraph_t g = nullptr;
    const hipError_t ec = hipStreamEndCapture(cap, &g);
    if (rc != MSD_OK || ec != hipSuccess) {
      if (g) (void)hipGraphDestroy(g);
      (void)hipGetLastError();
      return rc != MSD_OK ? rc : MSD_E_HIP;
    }
    hipGraphExec_t ex = nullptr;
    const hipError_t ei = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (ei != hipSuccess) return MSD_E_HIP;
    hipEvent_t ev = nullptr;
    if (hipEventCreateWithFlags(&ev, hipEventDisableTiming) != hipSuccess) {
      (void)hipGraphExecDestroy(ex);
      return MSD_E_HIP;
    }
    if (cache.size() >= kGraphCache) {
      auto lru = std::min_element(cache.begin(), cache.end(),
                                  [](const GraphEntry& a, const GraphEntry& b) { return a.used < b.used; });
      // cleanup of an evicted entry: its failures leave nothing to undo
      (void)hipEventSynchronize(lru->done);
      (void)hipGraphExecDestroy(lru->exec);
      (void)hipEventDestroy(lru->done);
      cache.erase(lru);
    }
    cache.push_back(GraphEntry{key, dev, ex, ev, 0});
    e = &cache.back();
  }
  e->used = ++tick;
  if (hipGraphLaunch(e->exec, s) != hipSuccess || hipEventRecord(e->done, s) != hipSuccess) return MSD_E_HIP;
  return MSD_OK;
}

}  // namespace mpf

using namespace mpf;

extern "C" int64_t msd_prefill_workspace_bytes(const msd_config* cfg, int32_t n_tokens) {
  if (!mx_config_ok(cfg)) return MSD_E_CONFIG;
  if (n_tokens <= 0 || n_tokens > cfg->context_len) return MSD_E_ARG;
  return int64_t(layout(cfg, n_tokens).bytes);
}

// The forward pass over tokens[0..n_tokens) at positions start..start+n_tokens-1.  With
// start == 0 this is the prompt prefill (causal attention within the pass, f32 keys and values
// of the pass, model.py:194-231).  With start > 0 it is the verification of draft tokens over an
// existing cache: every row attends like a decode step at its position (cached rows 0..p-1 as
// stored bf16, including the draft rows this pass has just written, and its own un-rounded K/V,
// multi_sm_decode.py:182-221), so row i's logits are those the sequential decode steps would
// give after accepting rows 0..i-1.  argmax_all (optional) receives every row's
// (argmax, status) pair.
static int32_t prefill_impl(const msd_config* cfg, const Weights& wt, const int32_t* tokens, int32_t n_tokens,
                            int32_t start, const int32_t* page_table, int32_t max_pages, int32_t pool_pages,
                            void* kv, void* workspace, float* logits_last, float* logits_all, int32_t* next_token,
                            int32_t* argmax_all, hipStream_t s) {
  if (!mx_config_ok(cfg)) return MSD_E_CONFIG;
  const int M = n_tokens;
  if (M <= 0 || start < 0 || start + M > cfg->context_len) return MSD_E_ARG;
  if (start > 0 && cfg->context_len > kAttnMaxCtx) return MSD_E_CONFIG;   // decode attention
  if (argmax_all && !logits_all) return MSD_E_ARG;
  if (!wt.emb || !wt.outp || !wt.w || !wt.lnf || !wt.rope || !tokens || !kv || !workspace || !logits_last ||
      !next_token)
    return MSD_E_ARG;
  if (!aligned16(wt.emb) || !aligned16(wt.outp) || !aligned16(wt.w) || !aligned16(kv) || !aligned16(workspace) ||
      !aligned16(wt.tiles))
    return MSD_E_ARG;
  if (page_table && (max_pages * kPage < start + M || max_pages > (cfg->context_len + kPage - 1) / kPage ||
                     pool_pages <= 0))
    return MSD_E_ARG;
  KeyBuf key;
  key.add('p').cfg(cfg).add(wt).add(tokens).add(M).add(start).add(page_table).add(max_pages).add(pool_pages).add(kv)
      .add(workspace).add(logits_last).add(logits_all).add(next_token).add(argmax_all);
  return launch_graphed(key.b, s, [&](hipStream_t s) -> int32_t {
  const int d = cfg->d_model, V = cfg->vocab_size;
  const Layout L = layout(cfg, M);
  char* ws = static_cast<char*>(workspace);
  float* h = reinterpret_cast<float*>(ws + L.h);
  uint16_t* xn = reinterpret_cast<uint16_t*>(ws + L.xn);
  float* part = reinterpret_cast<float*>(ws + L.part);
  int32_t* status = reinterpret_cast<int32_t*>(ws + L.status);
  int32_t* pages = reinterpret_cast<int32_t*>(ws + L.pages);
  hipLaunchKernelGGL(mx_clear_status, dim3(1), dim3(1), 0, s, status);
  if (page_table)
    hipLaunchKernelGGL(mx_sanitize_rows, dim3(1), dim3(64), 0, s, nullptr, start + M - 1, page_table, 1, max_pages,
                       cfg->context_len, pool_pages, nullptr, pages, status);
  Rows rows{M, nullptr, 0, page_table ? pages : nullptr, max_pages, page_table ? pool_pages * kPage : cfg->context_len,
            start};
  const int packed = wt.tiles != nullptr;   // the tile path keeps h in packed order
  // with the tile copy also the first layer's RMSNorm1 input planes and sums of h^2
  hipLaunchKernelGGL(mx_embed, dim3(M), dim3(256), 0, s, wt.emb, tokens, d, h, status, V, packed,
                     packed ? wt.tiles + first_norm_scales(cfg) : nullptr, xn, int64_t(pad16(M)) * d,
                     reinterpret_cast<float*>(ws + L.ssq));
  hipError_t err;
  const int pending = run_layers(cfg, wt, rows, static_cast<uint16_t*>(kv), L, ws, start == 0, s, err);
  if (err != hipSuccess) return MSD_E_HIP;
  // final norm of the rows whose logits are wanted, then the tied output projection
  const int r0 = logits_all ? 0 : M - 1, nr = M - r0;
  hipLaunchKernelGGL(mx_norm, dim3(nr), dim3(kNormThreads), 0, s, h, part, pending, M, d, wt.lnf, xn,
                     int64_t(nr) * d, r0, d, packed);
  if (gemm(xn, int64_t(nr) * d, d, wt.outp, false, nr, V, d, logits_all ? logits_all : logits_last, V, 1, s, false) !=
      hipSuccess)
    return MSD_E_HIP;
  const float* last = logits_all ? logits_all + int64_t(M - 1) * V : logits_last;
  if (logits_all && last != logits_last)
    hipLaunchKernelGGL(mx_copy_f32, dim3((V + 255) / 256), dim3(256), 0, s, last, logits_last, V);
  if (argmax_all)   // every row (next_token points at the last row's pair)
    hipLaunchKernelGGL(mx_argmax, dim3(M), dim3(1024), 0, s, logits_all, V, V, argmax_all, status);
  else
    hipLaunchKernelGGL(mx_argmax, dim3(1), dim3(1024), 0, s, logits_last, V, V, next_token, status);
  return hipGetLastError() == hipSuccess ? MSD_OK : MSD_E_HIP;
  });
}

extern "C" int64_t msd_tiles_bytes(const msd_config* cfg) {
  if (!mx_config_ok(cfg)) return MSD_E_CONFIG;
  return tile_layer_elems(cfg) * cfg->n_layers * 2;
}

extern "C" int32_t msd_pack_tiles(const msd_config* cfg, const void* packed_w, void* tiles, void* stream) {
  if (!mx_config_ok(cfg)) return MSD_E_CONFIG;
  if (!packed_w || !tiles || !aligned16(packed_w) || !aligned16(tiles)) return MSD_E_ARG;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int d = cfg->d_model, ff = cfg->d_ff, nqkv = (cfg->n_heads + 2 * cfg->n_kv_heads) * kDh;
  const int64_t off_qkv = 2 * int64_t(d), off_o = off_qkv + int64_t(nqkv) * d, off_gu = off_o + int64_t(d) * d,
                off_dn = off_gu + 2 * int64_t(ff) * d, layer = off_dn + int64_t(d) * ff;
  const int64_t dst_o = int64_t(nqkv) * d, dst_gu = dst_o + int64_t(d) * d, dst_dn = dst_gu + 2 * int64_t(ff) * d,
                dst_sc = dst_dn + int64_t(d) * ff;
  const struct { int64_t src, dst; int N, K, rowperm, natk; } mats[4] = {
      {off_qkv, 0, nqkv, d, 0, 0}, {off_o, dst_o, d, d, 1, 1}, {off_gu, dst_gu, 2 * ff, d, 2, 0},
      {off_dn, dst_dn, d, ff, 1, 0}};
  const uint16_t* w = static_cast<const uint16_t*>(packed_w);
  uint16_t* t = static_cast<uint16_t*>(tiles);
  for (int l = 0; l < cfg->n_layers; ++l) {
    uint16_t* tl = t + l * tile_layer_elems(cfg);
    for (const auto& m : mats) {
      const int64_t pieces = int64_t(m.N) * m.K / 8;
      hipLaunchKernelGGL(mx_pack_tiles, dim3(unsigned((pieces + 255) / 256)), dim3(256), 0, s, w + l * layer + m.src,
                         m.N, m.K, m.rowperm, m.natk, tl + m.dst);
    }
    hipLaunchKernelGGL(mx_pack_scales, dim3((2 * d + 255) / 256), dim3(256), 0, s, w + l * layer, d, tl + dst_sc);
  }
  return hipGetLastError() == hipSuccess ? MSD_OK : MSD_E_HIP;
}

extern "C" int32_t msd_prefill(const msd_config* cfg, const void* token_emb, const void* output_proj,
                               const void* packed_w, const void* tiles, const void* lnf_s, const float* rope,
                               const int32_t* tokens, int32_t n_tokens, void* kv, void* workspace, float* logits_last,
                               float* logits_all, int32_t* next_token, void* stream) {
  const Weights wt{static_cast<const uint16_t*>(token_emb), static_cast<const uint16_t*>(output_proj),
                   static_cast<const uint16_t*>(packed_w), static_cast<const uint16_t*>(lnf_s), rope,
                   static_cast<const uint16_t*>(tiles)};
  return prefill_impl(cfg, wt, tokens, n_tokens, 0, nullptr, 0, 0, kv, workspace, logits_last, logits_all, next_token,
                      nullptr, static_cast<hipStream_t>(stream));
}

extern "C" int32_t msd_prefill_paged(const msd_config* cfg, const void* token_emb, const void* output_proj,
                                     const void* packed_w, const void* tiles, const void* lnf_s, const float* rope,
                                     const int32_t* tokens, int32_t n_tokens, const int32_t* page_table,
                                     int32_t max_pages, void* kv_pool, int32_t pool_pages, void* workspace,
                                     float* logits_last, int32_t* next_token, void* stream) {
  if (!page_table) return MSD_E_ARG;
  const Weights wt{static_cast<const uint16_t*>(token_emb), static_cast<const uint16_t*>(output_proj),
                   static_cast<const uint16_t*>(packed_w), static_cast<const uint16_t*>(lnf_s), rope,
                   static_cast<const uint16_t*>(tiles)};
  return prefill_impl(cfg, wt, tokens, n_tokens, 0, page_table, max_pages, pool_pages, kv_pool, workspace, logits_last,
                      nullptr, next_token, nullptr, static_cast<hipStream_t>(stream));
}

extern "C" int64_t msd_verify_workspace_bytes(const msd_config* cfg, int32_t n_tokens) {
  return msd_prefill_workspace_bytes(cfg, n_tokens);
}

extern "C" int32_t msd_verify(const msd_config* cfg, const void* token_emb, const void* output_proj,
                              const void* packed_w, const void* tiles, const void* lnf_s, const float* rope,
                              const int32_t* tokens, int32_t n_tokens, int32_t start_pos, void* kv, void* workspace,
                              float* logits, int32_t* argmax, void* stream) {
  if (!cfg || !logits || !argmax || n_tokens <= 0 || start_pos < 1) return MSD_E_ARG;
  const Weights wt{static_cast<const uint16_t*>(token_emb), static_cast<const uint16_t*>(output_proj),
                   static_cast<const uint16_t*>(packed_w), static_cast<const uint16_t*>(lnf_s), rope,
                   static_cast<const uint16_t*>(tiles)};
  // the last row's logits land in logits (as part of logits_all); its argmax again in argmax[2(n-1)]
  return prefill_impl(cfg, wt, tokens, n_tokens, start_pos, nullptr, 0, 0, kv, workspace,
                      logits + int64_t(n_tokens - 1) * cfg->vocab_size, logits, argmax + 2 * (n_tokens - 1), argmax,
                      static_cast<hipStream_t>(stream));
}

// The batched workspace: the persistent step's region (fixed size per shape, first, so that
// its epoch and flags stay put whatever the batch), then the multi-kernel step's buffers.
static int64_t batch_region(const msd_config* cfg) { return (mbd::region_bytes(cfg) + 255) & ~int64_t(255); }

extern "C" int64_t msd_batch_workspace_bytes(const msd_config* cfg, int32_t batch) {
  if (!mx_config_ok(cfg)) return MSD_E_CONFIG;
  if (batch <= 0 || batch > kMaxRows) return MSD_E_ARG;
  return batch_region(cfg) + int64_t(layout(cfg, batch).bytes);
}

extern "C" int32_t msd_batch_decode_step(const msd_config* cfg, const void* token_emb, const void* output_proj,
                                         const void* packed_w, const void* tiles, const void* lnf_s, const float* rope,
                                         const int32_t* tokens, const int32_t* positions, int32_t batch,
                                         const int32_t* page_tables, int32_t max_pages, void* kv_pool,
                                         int32_t pool_pages, void* workspace, float* logits,
                                         int32_t* next_tokens, void* stream) {
  if (!mx_config_ok(cfg)) return MSD_E_CONFIG;
  const int M = batch;
  if (M <= 0 || M > kMaxRows) return MSD_E_ARG;
  if (!token_emb || !output_proj || !packed_w || !lnf_s || !rope || !tokens || !positions || !page_tables ||
      !kv_pool || !workspace || !logits || !next_tokens)
    return MSD_E_ARG;
  if (!aligned16(token_emb) || !aligned16(output_proj) || !aligned16(packed_w) || !aligned16(kv_pool) ||
      !aligned16(workspace) || !aligned16(tiles))
    return MSD_E_ARG;
  if (max_pages <= 0 || max_pages > (cfg->context_len + kPage - 1) / kPage || pool_pages <= 0) return MSD_E_ARG;
  if (cfg->context_len > kAttnMaxCtx) return MSD_E_CONFIG;   // decode attention
  hipStream_t s = static_cast<hipStream_t>(stream);
  {   // up to 8 sequences: one persistent launch when the shape and the device allow it
    const mbd::StepArgs sa{cfg, static_cast<const uint16_t*>(token_emb), static_cast<const uint16_t*>(output_proj),
                           static_cast<const uint16_t*>(packed_w), static_cast<const uint16_t*>(lnf_s), rope, tokens,
                           positions, batch, page_tables, max_pages, static_cast<uint16_t*>(kv_pool), pool_pages,
                           workspace, logits, next_tokens, s};
    const int32_t rc = mbd::try_step(sa);
    if (rc != 1) return rc;
  }
  const Weights wt{static_cast<const uint16_t*>(token_emb), static_cast<const uint16_t*>(output_proj),
                   static_cast<const uint16_t*>(packed_w), static_cast<const uint16_t*>(lnf_s), rope,
                   static_cast<const uint16_t*>(tiles)};
  KeyBuf key;
  key.add('b').cfg(cfg).add(wt).add(tokens).add(positions).add(M).add(page_tables).add(max_pages).add(kv_pool)
      .add(pool_pages).add(workspace).add(logits).add(next_tokens);
  return launch_graphed(key.b, s, [&](hipStream_t s) -> int32_t {
  const int d = cfg->d_model, V = cfg->vocab_size;
  const Layout L = layout(cfg, M);
  char* ws = static_cast<char*>(workspace) + batch_region(cfg);
  float* h = reinterpret_cast<float*>(ws + L.h);
  uint16_t* xn = reinterpret_cast<uint16_t*>(ws + L.xn);
  float* part = reinterpret_cast<float*>(ws + L.part);
  int32_t* status = reinterpret_cast<int32_t*>(ws + L.status);
  int32_t* rowpos = reinterpret_cast<int32_t*>(ws + L.rowpos);
  int32_t* pages = reinterpret_cast<int32_t*>(ws + L.pages);
  hipLaunchKernelGGL(mx_clear_status, dim3(1), dim3(1), 0, s, status);
  hipLaunchKernelGGL(mx_sanitize_rows, dim3((M + 255) / 256), dim3(256), 0, s, positions, 0, page_tables, M, max_pages,
                     cfg->context_len, pool_pages, rowpos, pages, status);
  Rows rows{M, rowpos, 1, pages, max_pages, pool_pages * kPage, 0};
  const int packed = wt.tiles != nullptr;
  // with the tile copy also the first layer's RMSNorm1 input planes and sums of h^2
  hipLaunchKernelGGL(mx_embed, dim3(M), dim3(256), 0, s, wt.emb, tokens, d, h, status, V, packed,
                     packed ? wt.tiles + first_norm_scales(cfg) : nullptr, xn, int64_t(pad16(M)) * d,
                     reinterpret_cast<float*>(ws + L.ssq));
  hipError_t err;
  const int pending = run_layers(cfg, wt, rows, static_cast<uint16_t*>(kv_pool), L, ws, false, s, err);
  if (err != hipSuccess) return MSD_E_HIP;
  hipLaunchKernelGGL(mx_norm, dim3(M), dim3(kNormThreads), 0, s, h, part, pending, M, d, wt.lnf, xn, int64_t(M) * d, 0,
                     d, packed);
  if (gemm(xn, int64_t(M) * d, d, wt.outp, false, M, V, d, logits, V, 1, s, false) != hipSuccess) return MSD_E_HIP;
  hipLaunchKernelGGL(mx_argmax, dim3(M), dim3(1024), 0, s, logits, V, V, next_tokens, status);
  return hipGetLastError() == hipSuccess ? MSD_OK : MSD_E_HIP;
  });
}

extern "C" int32_t msd_config_support(const msd_config* cfg, int32_t n_workgroups) {
  if (!cfg) return MSD_E_ARG;
  const int G = n_workgroups > 0 ? n_workgroups : 256;
  int32_t paths = 0;
  if (msdc::decode_supported(cfg, G)) paths |= MSD_PATH_DECODE;
  if (mx_config_ok(cfg)) {
    paths |= MSD_PATH_PREFILL;
    if (cfg->context_len <= kAttnMaxCtx) paths |= MSD_PATH_VERIFY | MSD_PATH_BATCHED;
    if ((paths & MSD_PATH_BATCHED) && mbd::region_bytes(cfg) > 0) paths |= MSD_PATH_BATCHED_STEP;
  }
  if (msdc::sample_supported(cfg->vocab_size)) paths |= MSD_PATH_SAMPLE;
  return paths;
}

extern "C" int32_t msd_set_launch_graphs(int32_t enabled) {
  graphs_on();
  return g_use_graphs.exchange(enabled ? 1 : 0);
}
