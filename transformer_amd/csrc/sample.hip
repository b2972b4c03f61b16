// Sampling tail of token generation on one MI355X (gfx950): repetition penalty, temperature,
// softmax, top-p (nucleus) filtering and the inverse-CDF draw of one token.
//
// Follows generate.py:28-65 (sample_token) with numpy's float arithmetic reproduced step by
// step, so that the drawn token matches the host code on the same logits and uniform:
//   * penalty and temperature in float32 (generate.py:33-46; NEP 50 casts the Python floats
//     to float32), applied once per distinct previously generated id (a 0/1 byte per id);
//   * max shift, exp, and normalisation by numpy's float32 `sum` (generate.py:48-51), whose
//     reduction order is reproduced exactly: buffers of 8192 entries summed in turn, each by
//     numpy's pairwise recursion (blocks of <= 128 entries with 8 interleaved accumulators);
//     exp is the correctly rounded float32 value, computed in float64;
//   * the descending sort of the probabilities with equal values in ascending id order
//     (generate.py:55), the float32 sequential `cumsum` of the sorted values and
//     `searchsorted(cumsum, top_p)` compared in float64 (generate.py:56-58), the pairwise
//     float32 sum of the kept values and their float32 renormalisation (generate.py:59-61);
//   * RandomState.choice(keep, p=filtered) on a supplied uniform u (generate.py:62-65):
//     searchsorted(cdf / cdf[-1], u, 'right') with cdf the float64 cumulative sum.
//
// The sort runs on the penalised logits instead of the probabilities, so it can start in the
// first kernel: a probability is a nondecreasing function of its logit, so the sorted sequence of
// probability values (and with it the cutoff, the sums and the drawn position) is the same; only
// ids of equal probability can come out in a different order, and the draw maps its position to
// the right id of such a run afterwards (tie_fixup).
//
// Kernels, all on the caller's stream:
//   sample_greedy_kernel   temperature 0: argmax of the penalised logits (1 workgroup)
//   sample_max_kernel      512 ids per workgroup: penalised, scaled logits and their maxima;
//                          nucleus: the sort keys (logit order) and first digit counts
//   sample_leaf_kernel     one wave per leaf of numpy's pairwise sum (<= 128 ids): correctly
//                          rounded exponentials and the leaf's sum; nucleus: radix pass 0 in
//                          workgroups of its own
//   sample_norm_kernel     512 ids per workgroup: the pairwise trees over the leaf sums and the
//                          normalisation; nucleus: radix pass 1 in workgroups of its own
//   sample_full_kernel     top_p >= 1: inverse CDF over all ids (1 workgroup)
//   sample_radix_kernel    passes 2 and 3 of the stable LSD sort (8 bits each) of (logit key, id),
//                          tiles of 512 entries per workgroup; each pass counts the next pass's
//                          digits, the last writes the probabilities in sorted order
//   sample_table_kernel    per 64-entry chunk of the sorted probabilities: exact ulp totals for
//                          the cumsum walk, equal-neighbour bits, pairwise leaves of full buffers
//   sample_nucleus_kernel  1 workgroup: the cumsum cutoff walk, renormalisation, draw and the
//                          id of the drawn position
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <math.h>

#include <algorithm>
#include <mutex>

#include "../../include/msdecode.h"
#include "internal.h"

// Every float operation below is a separately rounded IEEE operation (no contraction).
#pragma clang fp contract(off)

namespace mss {

constexpr int kT = 1024;                    // threads of the single-workgroup kernels
constexpr int kWaves = kT / 64;
constexpr int kVMax = 32768;                // largest vocabulary: 32 entries per thread
constexpr int kPer = kVMax / kT;
static_assert(kPer == 32, "a thread of the single-workgroup kernels holds one 32-bit word of entry flags");
constexpr int kTile = 512;                  // radix tile: entries per scatter workgroup
constexpr int kTileThreads = 256;
constexpr int kRounds = kTile / kTileThreads;
constexpr int kMaxTiles = kVMax / kTile;
constexpr int kHistWords = kMaxTiles * 256;  // one pass's [tile][digit] counts
constexpr int kPasses = 4;
constexpr int kRedChunk = 8192;             // numpy's reduction buffer (np.getbufsize())
constexpr int kPwBlock = 128;               // numpy's pairwise-sum block
constexpr int kSlots = 255;                 // heap slots of one buffer's pairwise tree (depth <= 7)
// Large LDS arrays keep entry j at j + j/32: a thread's 32 consecutive entries then start on
// a different bank from its neighbours'.
constexpr size_t kLdsBig = size_t(kVMax + kVMax / 32) * sizeof(float);

enum Mode { kGreedy = 0, kFull = 1, kNucleus = 2 };

struct SArgs {
  const float* logits;
  uint8_t* seen;          // [V] 1 = generated before (penalised); the drawn id is marked
  const double* u;        // one uniform draw in [0, 1)
  int32_t* token_out;
  float* probs_out;       // optional [V]: normalised probabilities in id order
  int32_t* kept_out;      // optional: number of ids kept by the nucleus
  float* lg;              // [V] penalised, scaled logits in id order
  float* ex;              // [V] exp(l - max) in id order
  float* pr;              // [V] probabilities in id order
  float* sp;              // [V] probabilities in sorted order (written by the last radix pass)
  uint32_t* eqw;          // [kVMax / 32] bit i of word w: sorted entry 32w + i equals entry 32w + i + 1
  float* pre;             // [kVMax / 128] numpy's pairwise leaf sums of the full 8192-entry buffers
                          // of the sorted probabilities
  uint32_t* keys[2];      // radix ping-pong: order-preserving bits of the penalised logits
  uint32_t* ids[2];
  uint32_t* hist;         // [kPasses][kMaxTiles][256]
  int* table;             // [3][kVMax / 64]: chunk totals, binades, odd-start changes
  float* tmax;            // [kVMax / 512]: maxima of the penalised, scaled logits per tile
  float* lsum;            // [kVMax / 8192][256]: numpy's pairwise leaf sums by buffer and heap slot
  int V;
  int ntiles;             // tiles of kTile ids
  int nleaf;              // workgroups of the pairwise-leaf role of sample_leaf_kernel
  int mode;
  int use_pen;
  float pen;
  int scale;              // temperature != 1
  float temp;
  float t32;              // smallest float32 >= top_p
};

// ---------------------------------------------------------------- wave/block helpers
__device__ inline int lane_id() { return threadIdx.x & 63; }

// Inclusive prefix sum over the 64 lanes (row shifts within rows of 16, then row broadcasts).
__device__ inline int wave_incl_scan(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false);   // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false);   // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false);   // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false);   // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);   // row_bcast:15 -> rows 1, 3
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);   // row_bcast:31 -> rows 2, 3
  return v;
}

__device__ inline int readlane_i(int v, int l) { return __builtin_amdgcn_readlane(v, l); }
__device__ inline float readlane_f(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

__device__ inline float wave_max(float v) {
  for (int o = 32; o; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}

__device__ inline uint64_t wave_max_u64(uint64_t v) {
  for (int o = 32; o; o >>= 1) {
    const uint64_t w = __shfl_xor(v, o);
    v = w > v ? w : v;
  }
  return v;
}

// float -> unsigned with the same order
__device__ inline uint32_t ordered(float f) {
  const uint32_t b = __float_as_uint(f);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ inline int pad(int j) { return j + (j >> 5); }

__device__ inline int binade(float s) { return int((__float_as_uint(s) >> 23) & 0xffu) - 127; }

struct BlockScratch {   // small shared scratch of the 1024-thread kernels
  float vals[kT];       // pairwise-tree node sums
  double dw[kWaves];
  uint64_t kw[kWaves];
  double dthr;          // inverse CDF threshold
  int i0;
};

__device__ uint64_t block_max_u64(uint64_t v, BlockScratch& b) {
  v = wave_max_u64(v);
  if (lane_id() == 0) b.kw[threadIdx.x >> 6] = v;
  __syncthreads();
  uint64_t m = b.kw[0];
  for (int i = 1; i < kWaves; ++i) m = b.kw[i] > m ? b.kw[i] : m;
  __syncthreads();
  return m;
}

// Sum of the float64 values of all threads with lower index (thread order).
__device__ double block_excl_scan_f64(double v, BlockScratch& b) {
  const int lane = lane_id(), w = threadIdx.x >> 6;
  double incl = v;
  for (int o = 1; o < 64; o <<= 1) {
    const double t = __shfl_up(incl, o);
    if (lane >= o) incl += t;
  }
  double excl = __shfl_up(incl, 1);
  if (lane == 0) excl = 0.0;
  if (lane == 63) b.dw[w] = incl;
  __syncthreads();
  double off = 0.0;
  for (int i = 0; i < w; ++i) off += b.dw[i];
  __syncthreads();
  return w == 0 ? excl : (lane == 0 ? off : off + excl);
}

// ---------------------------------------------------------------- numpy's float32 sum
// Node (start, len) of heap slot `slot` of numpy's pairwise recursion over n entries: a node of
// more than 128 entries splits into n2 = n/2 rounded down to a multiple of 8, and n - n2.
__device__ bool pw_node(int n, int slot, int& start, int& len) {
  const int id = slot + 1;
  const int depth = 31 - __clz(id);
  start = 0;
  len = n;
  for (int b = depth - 1; b >= 0; --b) {
    if (len <= kPwBlock) return false;
    int n2 = len / 2;
    n2 -= n2 % 8;
    if ((id >> b) & 1) {
      start += n2;
      len -= n2;
    } else {
      len = n2;
    }
  }
  return true;
}

// numpy's pairwise leaf: < 8 entries summed in order from 0; otherwise 8 interleaved
// accumulators over the multiple-of-8 prefix, combined as ((r0+r1)+(r2+r3))+((r4+r5)+(r6+r7)),
// then the remaining entries added in order.
__device__ float pw_leaf(const float* a, int start, int n) {
  if (n < 8) {
    float r = 0.f;
    for (int i = 0; i < n; ++i) r += a[pad(start + i)];
    return r;
  }
  float r0 = a[pad(start)], r1 = a[pad(start + 1)], r2 = a[pad(start + 2)], r3 = a[pad(start + 3)];
  float r4 = a[pad(start + 4)], r5 = a[pad(start + 5)], r6 = a[pad(start + 6)], r7 = a[pad(start + 7)];
  const int lim = n - (n % 8);
  int i = 8;
  for (; i < lim; i += 8) {
    const int j = start + i;
    r0 += a[pad(j)];
    r1 += a[pad(j + 1)];
    r2 += a[pad(j + 2)];
    r3 += a[pad(j + 3)];
    r4 += a[pad(j + 4)];
    r5 += a[pad(j + 5)];
    r6 += a[pad(j + 6)];
    r7 += a[pad(j + 7)];
  }
  float res = ((r0 + r1) + (r2 + r3)) + ((r4 + r5) + (r6 + r7));
  for (; i < n; ++i) res += a[pad(start + i)];
  return res;
}

// numpy's float32 sum of a[0..n) (n <= 32768, padded LDS layout); every thread gets the result.
// Buffers of 8192 entries are reduced by the pairwise recursion (thread 256*k + slot evaluates
// heap slot `slot` of buffer k; leaves first, then inner nodes by decreasing depth) and their
// results added in buffer order to 0.
// `pre` (optional): the leaf sums of full buffers, pre[64 k + j] = pw_leaf of entries
// [8192 k + 128 j, +128) -- the leaves of a full buffer are exactly these 64 blocks.
__device__ float np_sum(const float* a, int n, BlockScratch& b, const float* pre = nullptr) {
  const int t = threadIdx.x, k = t >> 8, slot = t & 255;
  const int nbuf = (n + kRedChunk - 1) / kRedChunk;
  const int bn = k < nbuf ? min(kRedChunk, n - k * kRedChunk) : 0;
  int start = 0, len = 0;
  const bool valid = k < nbuf && slot < kSlots && pw_node(bn, slot, start, len);
  const bool leaf = valid && len <= kPwBlock;
  if (leaf)
    b.vals[t] = pre && bn == kRedChunk ? pre[k * (kRedChunk / kPwBlock) + start / kPwBlock]
                                       : pw_leaf(a, k * kRedChunk + start, len);
  __syncthreads();
  const int depth = 31 - __clz(slot + 1);
  for (int d = 6; d >= 0; --d) {
    if (valid && !leaf && depth == d) b.vals[t] = b.vals[(k << 8) + 2 * slot + 1] + b.vals[(k << 8) + 2 * slot + 2];
    __syncthreads();
  }
  float s = 0.f;
  for (int i = 0; i < nbuf; ++i) s += b.vals[i << 8];
  __syncthreads();
  return s;
}

// ---------------------------------------------------------------- inverse CDF draw
// The largest double x with x / total <= u (float64 division): the division by total > 0 is
// correctly rounded and so nondecreasing in x, and fl(u * total) lies within an ulp or two of
// that boundary, so a few steps of one ulp from it find x.  cdf[i] / total <= u then holds
// exactly when cdf[i] <= x.
__device__ double cdf_threshold(double total, double u) {
  double x = u * total;
  for (int i = 0; i < 16 && x / total > u; ++i) x = nextafter(x, -INFINITY);
  for (int i = 0; i < 16; ++i) {
    const double y = nextafter(x, INFINITY);
    if (!(y / total <= u)) break;
    x = y;
  }
  return x;
}

// RandomState.choice on one uniform: the number of i < n with cdf[i] / cdf[n-1] <= u, where
// cdf is the float64 running sum of w[i] = (divide ? v[i] / div : v[i]) (float32 values,
// padded LDS layout, read once into registers).  The float64 sums are exact whenever the float32
// terms span fewer than 29 binades below the total, and then every partial sum equals the
// sequential one in any order: thread t sums its entries [32t, 32t+32), a block scan gives the
// sum of all earlier entries, and their sum is cdf at the thread's last entry.  cdf is
// nondecreasing, so each thread tests its last entry against the threshold of cdf_threshold and
// only the thread whose range crosses it adds its entries one by one.  Threads past n (whole
// waves for a small nucleus) skip the divisions.
__device__ __forceinline__ int inverse_cdf(const float* v, int n, bool divide, float div, double u,
                                           BlockScratch& b) {
  __shared__ uint8_t flag[kT];
  const int t = threadIdx.x, base = t * kPer;
  const int cnt = max(0, min(kPer, n - base));
  float w[kPer];
  double tot = 0.0;
  if (cnt > 0) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) w[i] = v[pad(min(base + i, kVMax - 1))];
    if (divide) {
#pragma unroll
      for (int i = 0; i < kPer; ++i) w[i] = w[i] / div;
    }
#pragma unroll
    for (int i = 0; i < kPer; ++i)
      if (i < cnt) tot += double(w[i]);
  }
  const double excl = block_excl_scan_f64(tot, b);
  const double r = excl + tot;
  if (cnt > 0 && base + cnt == n) b.dthr = cdf_threshold(r, u);   // r = cdf[n-1] here
  if (t == 0) b.i0 = n;   // no range crosses: every entry is <= the threshold
  __syncthreads();
  const double thr = b.dthr;
  const bool below = cnt > 0 && r <= thr;
  flag[t] = below;
  __syncthreads();
  // cdf is nondecreasing: every range before the crossing one is entirely below, so the count
  // is the crossing range's base plus its entries below
  if (cnt > 0 && !below && (t == 0 || flag[t - 1])) {   // the range that crosses u
    double rr = excl;
    int c = 0;
#pragma unroll
    for (int i = 0; i < kPer; ++i)
      if (i < cnt) {
        rr += double(w[i]);
        if (rr <= thr) ++c;
      }
    b.i0 = base + c;
  }
  __syncthreads();
  const int cs = b.i0;
  __syncthreads();
  return min(cs, n - 1);
}

// ---------------------------------------------------------------- nucleus cutoff
// Adding x to a float32 running sum s that stays in the binade [2^E, 2^(E+1)) adds
// round-half-even(x / ulp) ulps, ulp = 2^(E-23).  With y = x / ulp: y - floor(y) != 1/2 adds
// rint(y) whatever s is; at a tie the addition adds floor(y) plus 1 when the sum so far plus
// floor(y) is odd.  Over a run of entries that stays in the binade, let b_i be the parity of
// the start value plus all entries' base counts (rint or floor) up to tie i: the cumulative
// parity of the tie adjustments after tie i equals b_i, so tie i adds b_i XOR b_(previous tie).
// Every running sum of a 64-entry chunk is therefore an exact integer prefix, computed in
// parallel across the wave.

constexpr int kChunks = kVMax / 64;

// Inclusive prefix (in ulps of binade E) of the exact increments of this wave's 64 entries
// added to start value S; tm / bm: masks of the tie lanes and of their parities b.
__device__ int chunk_prefix(float x, bool valid, int S, int E, uint64_t& tm, uint64_t& bm) {
  const int lane = lane_id();
  const float y = ldexpf(x, 23 - E);
  const float fl = floorf(y);
  const bool tie = valid && (y - fl) == 0.5f;
  const int base = valid ? (tie ? int(fl) : int(rintf(y))) : 0;
  const int pb = wave_incl_scan(base);
  const bool b = tie && ((S + pb) & 1);
  tm = __ballot(tie);
  bm = __ballot(b);
  const uint64_t prev = tm & ((1ull << lane) - 1);
  const bool bprev = prev ? ((bm >> (63 - __clzll(prev))) & 1ull) != 0 : false;
  const uint64_t am = __ballot(tie && (b != bprev));
  return pb + __popcll(am & ((2ull << lane) - 1));
}

// One wave: with cumsum the float32 running sum of the descending probabilities p[0..n),
// padded LDS layout, returns searchsorted(cumsum, top_p) + 1 -- one past the first i with
// cumsum[i] >= top_p (n + 1 when there is none).  t32 is the smallest float32 >= top_p, so
// cumsum[i] >= top_p (compared in float64) exactly when cumsum[i] >= t32.
// Whole chunks come from the table while the sum stays in the table's binade and below top_p;
// otherwise the current chunk's exact prefixes are formed in parallel up to the first entry
// where the sum would leave the binade or reach top_p, which is added with an ordinary float32
// addition before the walk resumes after it.  (p is sorted descending, so every later x <= s
// and x / ulp < 2^24.)
__device__ int nucleus_cutoff(const float* p, int n, float t32, const int* ttot, const int* tex, const int* tdl) {
  const int lane = lane_id();
  float s = p[pad(0)];
  if (s >= t32) return 1;
  const int te = binade(t32);
  int k = 1;
  while (k < n) {
    const int E = binade(s);
    const int S = int(ldexpf(s, 23 - E));
    const int lim = te == E ? int(ldexpf(t32, 23 - E)) : (1 << 24);
    // the LDS reads of both paths are issued together, from clamped indices
    const int end = min(n, (k & ~63) + 64);   // the rest of the current chunk
    const bool valid = k + lane < end;
    const float xl = p[pad(min(k + lane, n - 1))];
    const int cc = (k >> 6) + lane;
    const int ccl = min(cc, kChunks - 1);
    const int tvl = ttot[ccl], tel = tex[ccl], tdv = tdl[ccl];
    if ((k & 63) == 0) {
      // up to 64 whole chunks at once, lane = chunk k/64 + lane.  A chunk with ties leaves the
      // sum's parity at the parity of its even-start total whatever it started with; one
      // without ties flips it by that parity.  So each lane's start parity follows from the
      // chunks since the last chunk with ties, and an inclusive scan of the totals gives the
      // sum after every chunk; the run stops before the first chunk outside the table's
      // binade or whose sum would reach the binade's end or top_p.
      const bool in = (cc + 1) * 64 <= n;
      const int tv = in ? tvl : -1;
      const bool good = tv >= 0 && tel == E;
      const int dv = good ? tdv : 0;
      const uint64_t gm = __ballot(good);
      const int ngood = ~gm == 0 ? 64 : __ffsll(static_cast<unsigned long long>(~gm)) - 1;
      if (ngood > 0) {
        const uint64_t pe = __ballot(good && (tv & 1)), pd = __ballot(good && dv != 0);
        const uint64_t lt = (1ull << lane) - 1;
        const uint64_t pdl = pd & lt;
        int pb;
        if (pdl) {
          const int j0 = 63 - __clzll(pdl);
          pb = __popcll(pe & lt & ~((1ull << j0) - 1)) & 1;
        } else {
          pb = (S & 1) ^ (__popcll(pe & lt) & 1);
        }
        const int tot = good ? min(tv + (pb ? dv : 0), 1 << 24) : (1 << 24);
        const int P = wave_incl_scan(tot);
        const uint64_t stop = __ballot(lane >= ngood || S + P >= lim);
        const int nadv = stop ? __ffsll(static_cast<unsigned long long>(stop)) - 1 : 64;
        if (nadv > 0) {
          s = ldexpf(float(S + readlane_i(P, nadv - 1)), E - 23);
          k += 64 * nadv;
          continue;
        }
      }
    }
    const float x = valid ? xl : 0.f;
    uint64_t tm, bm;
    const int pi = chunk_prefix(x, valid, S, E, tm, bm);
    const uint64_t m = __ballot(valid && S + pi >= lim);
    if (m == 0) {
      s = ldexpf(float(S + readlane_i(pi, 63)), E - 23);
      k = end;
      continue;
    }
    const int f = __ffsll(static_cast<unsigned long long>(m)) - 1;
    const int jf = k + f;
    const float sp = f == 0 ? s : ldexpf(float(S + readlane_i(pi, f - 1)), E - 23);
    const float sn = sp + readlane_f(x, f);
    if (sn >= t32) return jf + 1;
    s = sn;
    k = jf + 1;
  }
  return n + 1;
}

// ---------------------------------------------------------------- kernels
__device__ void finish(const SArgs& a, int token) {
  if (threadIdx.x == 0) {
    a.token_out[0] = token;
    a.seen[token] = 1;
  }
}

// Penalised logit v of an id with history flag `seen` (generate.py:33-39), divided by the
// temperature when scaled (generate.py:45-46); float32 operations as numpy performs them.
// Callers load v and seen from a clamped index, unconditionally, and issue all their loads
// before the first use: a load under a branch makes the compiler wait for it at the join.
__device__ __forceinline__ float penalised(const SArgs& a, float v, uint8_t seen, bool scaled) {
  if (a.use_pen && seen) v = v > 0.f ? v / a.pen : v * a.pen;
  if (scaled && a.scale) v = v / a.temp;
  return v;
}

// temperature == 0: argmax of the penalised logits, lowest id on ties (generate.py:41-42)
__global__ __launch_bounds__(kT) void sample_greedy_kernel(SArgs a) {
  __shared__ BlockScratch b;
  const int t = threadIdx.x;
  constexpr int kHalf = kPer / 2;   // 16 ids per thread in flight at a time
  uint64_t best = 0;
  for (int h = 0; h < 2; ++h) {
    float l[kHalf];
    uint8_t sn[kHalf];
#pragma unroll
    for (int i = 0; i < kHalf; ++i) {
      const int jc = min(t + kT * (h * kHalf + i), a.V - 1);
      l[i] = a.logits[jc];
      sn[i] = a.seen[jc];
    }
#pragma unroll
    for (int i = 0; i < kHalf; ++i) {
      const int j = t + kT * (h * kHalf + i);
      l[i] = penalised(a, l[i], sn[i], false);
      const uint64_t key = (uint64_t(ordered(l[i])) << 32) | uint32_t(0xffffffffu - uint32_t(j));
      best = j < a.V && key > best ? key : best;
    }
  }
  best = block_max_u64(best, b);
  finish(a, int(0xffffffffu - uint32_t(best & 0xffffffffu)));
}

// Softmax, first step (generate.py:33-48): workgroup w takes ids [512w, 512w+512), stores the
// penalised, scaled logits (to lg) and their maximum (to tmax[w]).  For the nucleus it also starts
// the sort (generate.py:55): the sort keys are the order-preserving bits of those logits with the
// ids in order, and this tile's counts of the first radix digit; the counts of the later passes
// are cleared here for the scatters to fill.
__global__ __launch_bounds__(kTile) void sample_max_kernel(SArgs a) {
  __shared__ float wm[kTile / 64];
  __shared__ uint32_t hl[256];
  const int t = threadIdx.x, w = blockIdx.x, j = w * kTile + t;
  const bool nuc = a.mode == kNucleus;
  if (nuc && t < 256) hl[t] = 0;
  const int jc = min(j, a.V - 1);
  const float lv = a.logits[jc];
  const uint8_t sn = a.seen[jc];
  const float pv = penalised(a, lv, sn, true);
  const float l = j < a.V ? pv : -INFINITY;
  const uint32_t key = ordered(l);
  if (j < a.V) {
    a.lg[j] = l;
    if (nuc) {
      a.keys[0][j] = key;
      a.ids[0][j] = uint32_t(j);
    }
  }
  const float m = wave_max(l);
  if (lane_id() == 0) wm[t >> 6] = m;
  __syncthreads();
  if (nuc && j < a.V) atomicAdd(&hl[255u - (key & 255u)], 1u);
  if (t == 0) {
    float mm = wm[0];
    for (int i = 1; i < kTile / 64; ++i) mm = fmaxf(mm, wm[i]);
    a.tmax[w] = mm;
  }
  __syncthreads();
  if (nuc && t < 256) {
    a.hist[w * 256 + t] = hl[t];
    for (int p = 1; p < kPasses; ++p) a.hist[p * kHistWords + w * 256 + t] = 0;
  }
}

// numpy's pairwise leaf of 128 entries held by one wave (x0: entry lane, x1: entry lane + 64):
// accumulator r_k = e[k] + e[k + 8] + ... + e[k + 120] in order on lane k < 8, combined as
// ((r0 + r1) + (r2 + r3)) + ((r4 + r5) + (r6 + r7)).  Wave-uniform result.
__device__ float leaf128(float x0, float x1) {
  const int lane = lane_id();
  float r = x0;
#pragma unroll
  for (int q = 1; q < 16; ++q) {
    const int idx = lane + 8 * q;
    r += q < 8 ? __shfl(x0, idx & 63) : __shfl(x1, idx & 63);
  }
  return ((readlane_f(r, 0) + readlane_f(r, 1)) + (readlane_f(r, 2) + readlane_f(r, 3))) +
         ((readlane_f(r, 4) + readlane_f(r, 5)) + (readlane_f(r, 6) + readlane_f(r, 7)));
}

// Softmax numerator (generate.py:49-50) and the leaves of numpy's float32 sum: wave g takes heap
// slot g % 255 of reduction buffer g / 255 and, when that node is a leaf (<= 128 ids), writes
// the correctly rounded exp(l - max) of its ids (to ex) and the leaf's pairwise sum (to
// lsum[256 * buffer + slot]).  The leaves of a buffer partition it, so every id is covered once.
// For the nucleus, the workgroups after the first nleaf run the sort's first radix pass.
constexpr int kLeafWaves = 4;
static_assert(64 * kLeafWaves == kTileThreads, "the leaf launch also runs radix workgroups");

__device__ void radix_pass(const SArgs& a, int pass, int w);

__global__ __launch_bounds__(64 * kLeafWaves) void sample_leaf_kernel(SArgs a) {
  if (int(blockIdx.x) >= a.nleaf) {   // the nucleus' first radix pass runs beside the leaves
    radix_pass(a, 0, int(blockIdx.x) - a.nleaf);
    return;
  }
  const int lane = lane_id();
  const int g = blockIdx.x * kLeafWaves + (threadIdx.x >> 6);
  const int k = g / kSlots, slot = g - k * kSlots;
  const int V = a.V;
  if (k * kRedChunk >= V) return;
  const int bn = min(kRedChunk, V - k * kRedChunk);
  int start = 0, len = 0;
  if (!pw_node(bn, slot, start, len) || len > kPwBlock) return;
  const int ntiles = (V + kTile - 1) / kTile;
  const int j0 = k * kRedChunk + start;
  const float* lg = a.lg;
  float* eo = a.ex;
  const float l0 = lg[j0 + min(lane, len - 1)], l1 = lg[j0 + min(lane + 64, len - 1)];
  const float tm = a.tmax[min(lane, ntiles - 1)];
  const float m = wave_max(lane < ntiles ? tm : -INFINITY);
  float x0 = 0.f, x1 = 0.f;   // e of leaf entries lane and lane + 64
  if (lane < len) {
    x0 = float(exp(double(l0 - m)));
    eo[j0 + lane] = x0;
  }
  if (lane + 64 < len) {
    x1 = float(exp(double(l1 - m)));
    eo[j0 + lane + 64] = x1;
  }
  float res = 0.f;
  int i = 0;
  if (len >= 8) {
    // lanes 0..7: accumulator r_lane = e[lane] + e[lane + 8] + ... in order
    const int lim = len - len % 8;
    float r = x0;
#pragma unroll
    for (int q = 1; q < 16; ++q) {
      const int idx = lane + 8 * q;
      const float v = q < 8 ? __shfl(x0, idx & 63) : __shfl(x1, idx & 63);
      if (idx < lim) r += v;
    }
    res = ((readlane_f(r, 0) + readlane_f(r, 1)) + (readlane_f(r, 2) + readlane_f(r, 3))) +
          ((readlane_f(r, 4) + readlane_f(r, 5)) + (readlane_f(r, 6) + readlane_f(r, 7)));
    i = lim;
  }
  for (; i < len; ++i) res += readlane_f(i < 64 ? x0 : x1, i & 63);
  if (lane == 0) a.lsum[k * 256 + slot] = res;
}

// Normalisation (generate.py:51): p = e / sum with numpy's sum = the buffer sums added in order
// to 0, each buffer's sum its pairwise tree over the leaf sums (inner nodes by decreasing
// depth; every workgroup evaluates the tree identically).  Workgroup w takes ids
// [512w, 512w+512), two per thread: the probabilities in id order (to pr, optionally to
// probs_out).  For the nucleus, the workgroups after the first ntiles run the second radix pass.
constexpr int kMaxBufs = kVMax / kRedChunk;
constexpr int kNormThreads = 256;
static_assert(kNormThreads == kTileThreads, "the normalisation launch also runs radix workgroups");

__global__ __launch_bounds__(kNormThreads) void sample_norm_kernel(SArgs a) {
  if (int(blockIdx.x) >= a.ntiles) {
    radix_pass(a, 1, int(blockIdx.x) - a.ntiles);
    return;
  }
  __shared__ float node[kMaxBufs * 256];
  const int t = threadIdx.x, w = blockIdx.x, V = a.V;
  const int nbuf = (V + kRedChunk - 1) / kRedChunk;
  constexpr int kNodeRounds = kMaxBufs * 256 / kNormThreads;
  constexpr int kIds = kTile / kNormThreads;
  int depth[kNodeRounds];
  bool inner[kNodeRounds];
  float e[kIds], ls[kNodeRounds];
#pragma unroll
  for (int r = 0; r < kIds; ++r) e[r] = a.ex[min(w * kTile + t + kNormThreads * r, V - 1)];
#pragma unroll
  for (int r = 0; r < kNodeRounds; ++r) ls[r] = a.lsum[t + kNormThreads * r];
#pragma unroll
  for (int r = 0; r < kNodeRounds; ++r) {
    const int q = t + kNormThreads * r, k = q >> 8, slot = q & 255;
    int start = 0, len = 0;
    const bool valid = k < nbuf && slot < kSlots && pw_node(min(kRedChunk, V - k * kRedChunk), slot, start, len);
    inner[r] = valid && len > kPwBlock;
    depth[r] = 31 - __clz(slot + 1);
    if (valid && len <= kPwBlock) node[q] = ls[r];
  }
  __syncthreads();
  for (int d = 6; d >= 0; --d) {
#pragma unroll
    for (int r = 0; r < kNodeRounds; ++r) {
      const int q = t + kNormThreads * r, kb = q & ~255, slot = q & 255;
      if (inner[r] && depth[r] == d) node[q] = node[kb + 2 * slot + 1] + node[kb + 2 * slot + 2];
    }
    __syncthreads();
  }
  float total = 0.f;
  for (int q = 0; q < nbuf; ++q) total += node[q << 8];
#pragma unroll
  for (int r = 0; r < kIds; ++r) {
    const int j = w * kTile + t + kNormThreads * r;
    if (j < V) {
      const float pj = e[r] / total;
      a.pr[j] = pj;
      if (a.probs_out) a.probs_out[j] = pj;
    }
  }
}

// top_p >= 1: RandomState.choice over all ids in id order (generate.py:65)
__global__ __launch_bounds__(kT) void sample_full_kernel(SArgs a) {
  extern __shared__ float sh_p[];   // probabilities in id order, padded layout
  __shared__ BlockScratch b;
  const int t = threadIdx.x, V = a.V;
  uint32_t kv[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) kv[i] = __float_as_uint(a.pr[min(t + kT * i, V - 1)]);
#pragma unroll
  for (int i = 0; i < kPer; ++i)
    if (t + kT * i < V) sh_p[pad(t + kT * i)] = __uint_as_float(kv[i]);
  __syncthreads();
  finish(a, inverse_cdf(sh_p, V, false, 1.f, a.u[0], b));
}

// Table for whole chunks c (entries [64c, 64c+64)) of the sorted probabilities whose float32
// running sum is certain to stay in one binade E: the float64 sums before and after the chunk
// lie inside [2^E, 2^(E+1)) with a margin of 4e-3 relative (more than 32768 float32 roundings
// can move a sum).  table[c] = the chunk's increment in ulps for an even start value (-1: take
// it entry by entry), table[kChunks + c] = E, table[2 kChunks + c] = the change for an odd
// start value (only the first tie's adjustment flips).  Workgroup w takes chunks
// [16w, 16w + 16), one wave per chunk (the last chunk may be partial: no table entry).  Each wave
// also marks the entries equal to their successor (eqw) and, when its index g is a leaf of a full
// 8192-entry buffer, stores numpy's pairwise leaf sum of entries [128 g, 128 g + 128) (pre): the
// renormalising sum of the kept prefix reuses the leaves of its full buffers.
constexpr int kTabChunks = kWaves;   // one chunk per wave

__global__ __launch_bounds__(kT) void sample_table_kernel(SArgs a) {
  __shared__ double red[kWaves];
  __shared__ double csum[kTabChunks];
  const int t = threadIdx.x, lane = lane_id(), wv = t >> 6;
  const int n = a.V, nch = n / 64, nall = (n + 63) / 64;
  const int c0 = blockIdx.x * kTabChunks;
  const float* p = a.sp;
  // float64 sum of the entries before this workgroup's chunks (at most 31 per thread, all
  // requested at once; the order is irrelevant: only the binade with its margin is used)
  float pv[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const float v = p[min(t + kT * i, n - 1)];
    pv[i] = t + kT * i < 64 * c0 ? v : 0.f;
  }
  const int c = c0 + wv, g = blockIdx.x * kWaves + wv;
  const float xl = p[min(64 * c + lane, n - 1)], xn = p[min(64 * c + lane + 1, n - 1)];
  const float y0 = p[min(128 * g + lane, n - 1)], y1 = p[min(128 * g + 64 + lane, n - 1)];
  double pre = 0.0;
#pragma unroll
  for (int i = 0; i < kPer; ++i) pre += double(pv[i]);
  for (int o = 32; o; o >>= 1) pre += __shfl_xor(pre, o);
  if (lane == 0) red[wv] = pre;
  const float x = c < nch ? xl : 0.f;
  double v = x;
  for (int o = 32; o; o >>= 1) v += __shfl_xor(v, o);
  if (lane == 0) csum[wv] = v;
  if (c < nall) {
    const uint64_t eq = __ballot(64 * c + lane + 1 < n && xl == xn);
    if (lane < 2) a.eqw[2 * c + lane] = uint32_t(eq >> (32 * lane));
  }
  if (g < kVMax / kPwBlock && (g / (kRedChunk / kPwBlock) + 1) * kRedChunk <= n) {
    const float s = leaf128(y0, y1);
    if (lane == 0) a.pre[g] = s;
  }
  __syncthreads();
  if (c >= nch) return;
  double ps = 0.0;
  for (int q = 0; q < kWaves; ++q) ps += red[q];
  for (int q = 0; q < wv; ++q) ps += csum[q];
  const double pe = ps + csum[wv];
  const int E = ps > 0.0 ? ilogb(ps) : 0;
  const bool ok = ps > 0.0 && ps >= ldexp(1.0, E) * (1.0 + 4e-3) && pe <= ldexp(1.0, E + 1) * (1.0 - 4e-3);
  int tv = -1, dv = 0;
  if (ok && __ballot(!(ldexpf(x, 23 - E) < 16777216.f)) == 0) {
    uint64_t tm, bm;
    const int pi = chunk_prefix(x, true, 0, E, tm, bm);
    tv = readlane_i(pi, 63);
    if (tm) dv = 1 - 2 * int((bm >> (__ffsll(static_cast<unsigned long long>(tm)) - 1)) & 1ull);
  }
  if (lane == 0) {
    a.table[c] = tv;
    a.table[kChunks + c] = E;
    a.table[2 * kChunks + c] = dv;
  }
}

// One stable LSD pass over digit `pass` (bits 8*pass..8*pass+7, descending order) from
// keys/ids[pass & 1] to keys/ids[(pass + 1) & 1], by workgroup w (256 threads) of the launch that
// runs it.  Tile w holds entries [512w, 512w+512), moved in order: an entry's destination is the
// number of entries with a larger digit, plus those with the same digit in earlier tiles, earlier
// rounds of this tile, earlier waves of this round and lower lanes of this wave.  The last pass
// also writes each entry's probability to its sorted position (sp).
__device__ void radix_pass(const SArgs& a, int pass, int w) {
  __shared__ uint32_t base[256], run[256], wcnt[kTileThreads / 64][256], wtot[kTileThreads / 64];
  const int t = threadIdx.x, wv = t >> 6, lane = lane_id();
  const int V = a.V, ntiles = (V + kTile - 1) / kTile;
  const bool last = pass == kPasses - 1;
  const uint32_t* kin = a.keys[pass & 1];
  const uint32_t* iin = a.ids[pass & 1];
  uint32_t key[kRounds], id[kRounds];   // this thread's entries, requested with the counts
#pragma unroll
  for (int r = 0; r < kRounds; ++r) {
    const int e = w * kTile + r * kTileThreads + t;
    key[r] = kin[min(e, V - 1)];
    id[r] = iin[min(e, V - 1)];
  }
  float pv[kRounds] = {};
  if (last) {
#pragma unroll
    for (int r = 0; r < kRounds; ++r) pv[r] = a.pr[min(id[r], uint32_t(V - 1))];
  }
  const uint32_t* H = a.hist + pass * kHistWords;
  uint32_t tot = 0, part = 0;
#pragma unroll
  for (int i = 0; i < kMaxTiles; ++i) {
    const uint32_t hl = H[min(i, ntiles - 1) * 256 + t];
    const uint32_t h = i < ntiles ? hl : 0u;
    tot += h;
    part += i < w ? h : 0u;
  }
  const int inc = wave_incl_scan(int(tot));
  if (lane == 63) wtot[wv] = uint32_t(inc);
  __syncthreads();
  uint32_t off = 0;
  for (int i = 0; i < wv; ++i) off += wtot[i];
  base[t] = off + uint32_t(inc) - tot + part;
  run[t] = 0;
  uint32_t* kout = a.keys[(pass + 1) & 1];
  uint32_t* iout = a.ids[(pass + 1) & 1];
  const int shift = 8 * pass;
  const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
#pragma unroll
  for (int r = 0; r < kRounds; ++r) {
    for (int i = 0; i < kTileThreads / 64; ++i) wcnt[i][t] = 0;
    __syncthreads();
    const bool valid = w * kTile + r * kTileThreads + t < V;
    const uint32_t dig = 255u - ((key[r] >> shift) & 255u);
    uint64_t peers = __ballot(valid);
    for (int bit = 0; bit < 8; ++bit) {
      const bool on = (dig >> bit) & 1u;
      const uint64_t bb = __ballot(on);
      peers &= on ? bb : ~bb;
    }
    const int rk = __popcll(peers & below);
    if (valid && rk == 0) wcnt[wv][dig] = uint32_t(__popcll(peers));
    __syncthreads();
    uint32_t acc = 0;
    for (int i = 0; i < kTileThreads / 64; ++i) {   // exclusive prefix over waves, digit t
      const uint32_t c = wcnt[i][t];
      wcnt[i][t] = acc;
      acc += c;
    }
    __syncthreads();
    const uint32_t pos = base[dig] + run[dig] + wcnt[wv][dig] + uint32_t(rk);
    if (valid && pos < uint32_t(V)) {   // always true when the counts are consistent
      kout[pos] = key[r];
      iout[pos] = id[r];
      if (last) a.sp[pos] = pv[r];
      if (pass + 1 < kPasses) {
        const uint32_t nd = 255u - ((key[r] >> (shift + 8)) & 255u);
        atomicAdd(&a.hist[(pass + 1) * kHistWords + (pos / kTile) * 256 + nd], 1u);
      }
    }
    __syncthreads();
    run[t] += acc;
  }
}

__global__ __launch_bounds__(kTileThreads) void sample_radix_kernel(SArgs a, int pass) {
  radix_pass(a, pass, blockIdx.x);
}

// The id at sorted position pos in numpy's order.  The radix sort orders the ids by their
// penalised logits, which gives the probabilities in the same sequence of values (a probability is
// a nondecreasing function of its logit: rounding, exp and the division by the total all keep
// order), so the cutoff, the sums and the drawn position are numpy's; but ids of equal probability
// come out in the order of their logits, where numpy's stable sort has them in ascending id order.
// So the answer is the (pos - ra)-th smallest id of the run [ra, rb) of entries equal to entry
// pos.  eqw (LDS copy, kVMax / 32 words; bit n - 1 is clear: the last entry has no successor)
// locates the run -- wave 0 scans 64 words per step outward from pos -- and is then reused as a
// bitmap of the run's ids.
__device__ int tie_fixup(const SArgs& a, uint32_t* eqw, int pos, BlockScratch& b) {
  const int t = threadIdx.x, lane = lane_id();
  const uint32_t* ids = a.ids[kPasses & 1];
  if (t < 64) {
    const int wp = pos >> 5, bp = pos & 31;
    // ra = 1 + the largest i < pos with bit i clear (0 when there is none)
    const uint32_t below = bp ? ~eqw[wp] & ((1u << bp) - 1u) : 0u;
    int ra = -1;
    if (below) {
      ra = 32 * wp + 31 - __clz(below) + 1;
    } else {
      for (int w1 = wp - 1; w1 >= 0 && ra < 0; w1 -= 64) {
        const int w = w1 - lane;
        const uint32_t c = w >= 0 ? ~eqw[max(w, 0)] : 0u;
        const uint64_t m = __ballot(c != 0u);
        if (m) {
          const int l = __ffsll(static_cast<unsigned long long>(m)) - 1;
          const uint32_t cl = uint32_t(__builtin_amdgcn_readlane(int(c), l));
          ra = 32 * (w1 - l) + 31 - __clz(cl) + 1;
        }
      }
      if (ra < 0) ra = 0;
    }
    // rb = 1 + the smallest i >= pos with bit i clear
    const uint32_t from = ~eqw[wp] & ~((1u << bp) - 1u);
    int rb = -1;
    if (from) {
      rb = 32 * wp + __ffs(from) - 1 + 1;
    } else {
      for (int w1 = wp + 1; rb < 0 && w1 < kVMax / 32; w1 += 64) {   // bit n - 1 is clear
        const int w = min(w1 + lane, kVMax / 32 - 1);
        const uint32_t c = ~eqw[w];
        const uint64_t m = __ballot(c != 0u);
        if (m) {
          const int l = __ffsll(static_cast<unsigned long long>(m)) - 1;
          const uint32_t cl = uint32_t(__builtin_amdgcn_readlane(int(c), l));
          rb = 32 * min(w1 + l, kVMax / 32 - 1) + __ffs(cl) - 1 + 1;
        }
      }
    }
    if (rb < 0) rb = a.V;
    if (lane == 0) {
      b.kw[0] = uint64_t(ra);
      b.kw[1] = uint64_t(rb);
    }
  }
  __syncthreads();
  const int ra = int(b.kw[0]), rb = int(b.kw[1]);
  __syncthreads();
  if (rb - ra == 1) return int(ids[pos]);
  eqw[t] = 0u;
  __syncthreads();
  for (int i = ra + t; i < rb; i += kT) {
    const uint32_t id = ids[i];
    atomicOr(&eqw[id >> 5], 1u << (id & 31u));
  }
  __syncthreads();
  const uint32_t m0 = eqw[t];
  const int c = __popc(m0), k = pos - ra;
  const int ex = int(block_excl_scan_f64(double(c), b));
  if (k >= ex && k < ex + c) {
    uint32_t m = m0;
    for (int q = 0; q < k - ex; ++q) m &= m - 1u;   // clear the lowest set bits
    b.i0 = 32 * t + __ffs(m) - 1;
  }
  __syncthreads();
  const int r = b.i0;
  __syncthreads();
  return r;
}

__global__ __launch_bounds__(kT) void sample_nucleus_kernel(SArgs a) {
  extern __shared__ float sh_p[];   // sorted probabilities, padded layout
  __shared__ BlockScratch b;
  __shared__ int ttot[kChunks], tex[kChunks], tdl[kChunks];
  __shared__ float pre[kVMax / kPwBlock];   // leaf sums of the full 8192-entry buffers
  __shared__ uint32_t eqw[kVMax / 32];      // equal-successor bits of the sorted entries
  const int t = threadIdx.x, V = a.V, nw = 2 * ((V + 63) / 64);
  uint32_t kv[kPer];   // every load issued before the first LDS store
#pragma unroll
  for (int i = 0; i < kPer; ++i) kv[i] = __float_as_uint(a.sp[min(t + kT * i, V - 1)]);
  const uint32_t ew = a.eqw[min(t, nw - 1)];
  const float pl = a.pre[min(t, kVMax / kPwBlock - 1)];
  for (int c = t; c < V / 64; c += kT) {
    ttot[c] = a.table[c];
    tex[c] = a.table[kChunks + c];
    tdl[c] = a.table[2 * kChunks + c];
  }
#pragma unroll
  for (int i = 0; i < kPer; ++i)
    if (t + kT * i < V) sh_p[pad(t + kT * i)] = __uint_as_float(kv[i]);
  eqw[t] = t < nw ? ew : 0u;
  if (t < kVMax / kPwBlock) pre[t] = pl;
  __syncthreads();
  if (t < 64) {
    const int c = nucleus_cutoff(sh_p, V, a.t32, ttot, tex, tdl);
    if (t == 0) b.i0 = c;
  }
  __syncthreads();
  const int kept = min(b.i0, V);
  const float fsum = np_sum(sh_p, kept, b, pre);
  const int pos = inverse_cdf(sh_p, kept, true, fsum, a.u[0], b);
  if (t == 0 && a.kept_out) a.kept_out[0] = kept;
  finish(a, tie_fixup(a, eqw, pos, b));
}

// ---------------------------------------------------------------- host side
struct SLayout {
  size_t lg, ex, pr, sp, keys0, keys1, ids0, ids1, hist, table, tmax, lsum, eqw, pre, bytes;
};

constexpr size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

constexpr SLayout slayout(int V) {
  SLayout s{};
  const size_t arr = align256(size_t(V) * sizeof(uint32_t));
  s.lg = 0;
  s.ex = arr;
  s.pr = 2 * arr;
  s.sp = 3 * arr;
  s.keys0 = 4 * arr;
  s.keys1 = 5 * arr;
  s.ids0 = 6 * arr;
  s.ids1 = 7 * arr;
  s.hist = 8 * arr;
  s.table = s.hist + align256(size_t(kPasses) * kHistWords * sizeof(uint32_t));
  s.tmax = s.table + align256(size_t(3) * (kVMax / 64) * sizeof(int));
  s.lsum = s.tmax + align256(size_t(kMaxTiles) * sizeof(float));
  s.eqw = s.lsum + align256(size_t(kVMax / kRedChunk) * 256 * sizeof(float));
  s.pre = s.eqw + align256(size_t(kVMax / 32) * sizeof(uint32_t));
  s.bytes = s.pre + size_t(kVMax / kPwBlock) * sizeof(float);
  return s;
}

static hipError_t set_big_lds() {
  const void* big[] = {reinterpret_cast<const void*>(&sample_full_kernel),
                       reinterpret_cast<const void*>(&sample_nucleus_kernel)};
  for (const void* k : big)
    if (const hipError_t e = msdc::ensure_dynamic_lds(k, kLdsBig); e != hipSuccess) return e;
  return hipSuccess;
}

}  // namespace mss

using namespace mss;

extern "C" int64_t msd_sample_workspace_bytes(int32_t vocab) {
  if (vocab <= 0 || vocab > kVMax) return MSD_E_CONFIG;
  return int64_t(slayout(vocab).bytes);
}

namespace mss {

// Scratch of msd_sample_token_noalloc: the workspace of the largest vocabulary, one copy per
// device (its address is taken once per device with hipGetSymbolAddress; host code never
// passes the symbol itself to a kernel).  Every call on a device shares it.
constexpr size_t kScratchBytes = slayout(kVMax).bytes;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

static int32_t sample_impl(const float* logits, int32_t vocab, double temperature, double top_p,
                           double rep_penalty, uint8_t* seen, const double* uniform, int32_t* token_out,
                           float* probs_out, int32_t* kept_out, void* workspace, void* stream) {
  if (vocab <= 0 || vocab > kVMax) return MSD_E_CONFIG;
  if (!logits || !seen || !token_out || !workspace) return MSD_E_ARG;
  if (!(temperature >= 0.0) || !isfinite(temperature) || !isfinite(rep_penalty) || rep_penalty == 0.0 ||
      isnan(top_p))
    return MSD_E_ARG;
  if (reinterpret_cast<uintptr_t>(workspace) & 255) return MSD_E_ARG;
  SArgs a;
  a.mode = temperature == 0.0 ? kGreedy : (top_p < 1.0 ? kNucleus : kFull);
  if (a.mode != kGreedy && !uniform) return MSD_E_ARG;
  const SLayout L = slayout(vocab);
  char* ws = static_cast<char*>(workspace);
  a.logits = logits;
  a.seen = seen;
  a.u = uniform;
  a.token_out = token_out;
  a.probs_out = probs_out;
  a.kept_out = kept_out;
  a.lg = reinterpret_cast<float*>(ws + L.lg);
  a.ex = reinterpret_cast<float*>(ws + L.ex);
  a.pr = reinterpret_cast<float*>(ws + L.pr);
  a.sp = reinterpret_cast<float*>(ws + L.sp);
  a.eqw = reinterpret_cast<uint32_t*>(ws + L.eqw);
  a.pre = reinterpret_cast<float*>(ws + L.pre);
  a.keys[0] = reinterpret_cast<uint32_t*>(ws + L.keys0);
  a.keys[1] = reinterpret_cast<uint32_t*>(ws + L.keys1);
  a.ids[0] = reinterpret_cast<uint32_t*>(ws + L.ids0);
  a.ids[1] = reinterpret_cast<uint32_t*>(ws + L.ids1);
  a.hist = reinterpret_cast<uint32_t*>(ws + L.hist);
  a.table = reinterpret_cast<int*>(ws + L.table);
  a.tmax = reinterpret_cast<float*>(ws + L.tmax);
  a.lsum = reinterpret_cast<float*>(ws + L.lsum);
  a.V = vocab;
  a.use_pen = rep_penalty != 1.0;
  a.pen = float(rep_penalty);
  a.scale = temperature != 1.0;
  a.temp = float(temperature);
  float t32 = float(top_p);
  if (double(t32) < top_p) t32 = nextafterf(t32, INFINITY);
  a.t32 = t32;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (set_big_lds() != hipSuccess) return MSD_E_HIP;
  if (a.mode == kGreedy) {
    hipLaunchKernelGGL(sample_greedy_kernel, dim3(1), dim3(kT), 0, s, a);
    return hipGetLastError() == hipSuccess ? MSD_OK : MSD_E_HIP;
  }
  const int ntiles = (vocab + kTile - 1) / kTile;
  const int nbuf = (vocab + kRedChunk - 1) / kRedChunk;
  const bool nuc = a.mode == kNucleus;
  a.ntiles = ntiles;
  a.nleaf = (nbuf * kSlots + kLeafWaves - 1) / kLeafWaves;
  // the nucleus' first two radix passes ride in the leaf and normalisation launches
  hipLaunchKernelGGL(sample_max_kernel, dim3(ntiles), dim3(kTile), 0, s, a);
  hipLaunchKernelGGL(sample_leaf_kernel, dim3(a.nleaf + (nuc ? ntiles : 0)), dim3(64 * kLeafWaves), 0, s, a);
  hipLaunchKernelGGL(sample_norm_kernel, dim3(nuc ? 2 * ntiles : ntiles), dim3(kNormThreads), 0, s, a);
  if (hipGetLastError() != hipSuccess) return MSD_E_HIP;
  if (!nuc) {
    hipLaunchKernelGGL(sample_full_kernel, dim3(1), dim3(kT), kLdsBig, s, a);
    return hipGetLastError() == hipSuccess ? MSD_OK : MSD_E_HIP;
  }
  for (int p = 2; p < kPasses; ++p) {
    hipLaunchKernelGGL(sample_radix_kernel, dim3(ntiles), dim3(kTileThreads), 0, s, a, p);
    if (hipGetLastError() != hipSuccess) return MSD_E_HIP;
  }
  hipLaunchKernelGGL(sample_table_kernel, dim3(((vocab + 63) / 64 + kTabChunks - 1) / kTabChunks), dim3(kT), 0, s, a);
  if (hipGetLastError() != hipSuccess) return MSD_E_HIP;
  hipLaunchKernelGGL(sample_nucleus_kernel, dim3(1), dim3(kT), kLdsBig, s, a);
  if (hipGetLastError() != hipSuccess) return MSD_E_HIP;
  return MSD_OK;
}

}  // namespace mss

bool msdc::sample_supported(int vocab) { return vocab >= 1 && vocab <= kVMax; }

extern "C" int32_t msd_sample_token(const float* logits, int32_t vocab, double temperature, double top_p,
                                    double rep_penalty, uint8_t* seen, const double* uniform,
                                    int32_t* token_out, float* probs_out, int32_t* kept_out,
                                    void* workspace, void* stream) {
  return sample_impl(logits, vocab, temperature, top_p, rep_penalty, seen, uniform, token_out, probs_out,
                     kept_out, workspace, stream);
}

namespace {
std::mutex g_scratch_mu;
void* g_scratch_ptr[64] = {};   // device address of `scratch` per device, taken once
}  // namespace

extern "C" int32_t msd_sample_token_noalloc(const float* logits, int32_t vocab, double temperature, double top_p,
                                            double rep_penalty, uint8_t* seen, const double* uniform,
                                            int32_t* token_out, float* probs_out, int32_t* kept_out,
                                            void* stream) {
  if (vocab <= 0 || vocab > kVMax || slayout(vocab).bytes > kScratchBytes) return MSD_E_CONFIG;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return MSD_E_HIP;
  void* ws = nullptr;
  {
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
      void* p = nullptr;
      if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return MSD_E_HIP;
      g_scratch_ptr[dev] = p;
    }
    ws = g_scratch_ptr[dev];
  }
  return sample_impl(logits, vocab, temperature, top_p, rep_penalty, seen, uniform, token_out, probs_out, kept_out,
                     ws, stream);
}
