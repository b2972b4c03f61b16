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

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kDh = 64;          // head dimension (fixed)
constexpr int kChunks = 16;      // attention position chunks per KV head
constexpr int kPartStride = 66;  // per (chunk, head): m, l, o[64]
constexpr uint32_t kSpinLimit = 1u << 20;

constexpr uint32_t kStatusTimeout = 1u;
constexpr uint32_t kStatusBadToken = 2u;

// ---------------------------------------------------------------- layout
struct Layout {
  // packed weights, per layer (bf16 elements)
  int64_t off_ln1, off_ln2, off_qkv, off_o, off_gu, off_dn, layer_elems;
  // exchange words per layer (uint64)
  int64_t x_qkv, x_part, x_attn, x_hd1, x_act, x_hd2, x_layer;
  int64_t ctrl_bytes;
};

__host__ __device__ inline int64_t align64(int64_t v) { return (v + 63) & ~int64_t(63); }

__host__ __device__ inline Layout make_layout(int d, int H, int KV, int ff) {
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
  t.x_attn = t.x_part + align64(int64_t(KV) * kChunks * GQ * kPartStride);
  t.x_hd1 = t.x_attn + align64(d);
  t.x_act = t.x_hd1 + align64(d);
  t.x_hd2 = t.x_act + align64(ff);
  t.x_layer = t.x_hd2 + align64(d);
  t.ctrl_bytes = 256;
  return t;
}

struct Args {
  const uint16_t* emb;
  const uint16_t* w;
  const uint16_t* lnf;
  const float* rope;
  uint16_t* kv;
  float* logits;
  int32_t* next_token;
  const int32_t* token_dev;
  uint32_t* ctrl;   // [0] status, [1] arrival counter, [2..3] argmax key (u64)
  uint64_t* xw;     // exchange words, n_layers * x_layer
  int token, pos;
  uint32_t epoch;
  int H, KV, L, ff, V, ctx;
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

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

__device__ __forceinline__ void st_tag(uint64_t* p, float v, uint32_t tag) {
  __hip_atomic_store(p, (uint64_t(tag) << 32) | __float_as_uint(v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld_tag(const uint64_t* p) {
  return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ld_status(uint32_t* ctrl) {
  return __hip_atomic_load(ctrl, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Gather n tagged words into LDS floats; all threads of the workgroup participate.
// `bad` (workgroup-uniform after the call) records a timeout or an abort seen in the status.
__device__ void gather(const uint64_t* src, int n, float* dst, uint32_t tag, uint32_t* ctrl,
                       int* sh_flag, bool& bad) {
  constexpr int PT = 8;
  const int tid = threadIdx.x;
  for (int base = 0; base < n; base += kThreads * PT) {
    uint64_t w[PT];
#pragma unroll
    for (int j = 0; j < PT; ++j) {
      const int i = base + tid + j * kThreads;
      w[j] = (i < n) ? ld_tag(src + i) : (uint64_t(tag) << 32);
    }
    uint32_t spins = 0;
    bool mybad = bad;
    while (!mybad) {
      bool ok = true;
#pragma unroll
      for (int j = 0; j < PT; ++j) {
        if (uint32_t(w[j] >> 32) != tag) {
          ok = false;
          w[j] = ld_tag(src + base + tid + j * kThreads);
        }
      }
      if (ok) break;
      ++spins;
      if ((spins & 255u) == 0 && (ld_status(ctrl) & kStatusTimeout)) mybad = true;
      if (spins > kSpinLimit) {
        atomicOr(ctrl, kStatusTimeout);
        mybad = true;
      }
    }
#pragma unroll
    for (int j = 0; j < PT; ++j) {
      const int i = base + tid + j * kThreads;
      if (i < n) dst[i] = __uint_as_float(uint32_t(w[j]));
    }
    if (mybad) *sh_flag = 1;
  }
  __syncthreads();
  bad = bad || (*sh_flag != 0);
}

// x = scale * (h / sqrt(mean(h^2) + 1e-5))   (model.py:94-98), all threads
__device__ void rmsnorm(const float* h, const uint16_t* scale, float* x, int d, float* red) {
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  float ss = 0.f;
  for (int i = tid; i < d; i += kThreads) ss += h[i] * h[i];
  ss = wave_sum(ss);
  if (lane == 0) red[wv] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) tot += red[w];
  const float r = sqrtf(tot / float(d) + 1e-5f);
  for (int i = tid; i < d; i += kThreads) x[i] = bf2f(scale[i]) * (h[i] / r);
  __syncthreads();
}

// One row of K bf16 held as NL 16-byte pieces per lane (piece j covers elements
// [(j*64 + lane)*8, +8)); dot with x (LDS floats), reduced over the wave.
template <int NL>
struct Row {
  uint4 v[NL];
};

template <int NL>
__device__ __forceinline__ void load_row(Row<NL>& r, const uint16_t* row, int k, int lane) {
  const uint4* p = reinterpret_cast<const uint4*>(row);
  const int n16 = k >> 3;
#pragma unroll
  for (int j = 0; j < NL; ++j) {
    const int i = j * 64 + lane;
    r.v[j] = (i < n16) ? p[i] : make_uint4(0, 0, 0, 0);
  }
}

template <int NL>
__device__ __forceinline__ float dot_row(const Row<NL>& r, const float* x, int k, int lane) {
  const int n16 = k >> 3;
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < NL; ++j) {
    const int i = j * 64 + lane;
    if (i < n16) {
      const float4 a = *reinterpret_cast<const float4*>(x + i * 8);
      const float4 b = *reinterpret_cast<const float4*>(x + i * 8 + 4);
      const uint4 w = r.v[j];
      acc += bf_lo(w.x) * a.x;
      acc += bf_hi(w.x) * a.y;
      acc += bf_lo(w.y) * a.z;
      acc += bf_hi(w.y) * a.w;
      acc += bf_lo(w.z) * b.x;
      acc += bf_hi(w.z) * b.y;
      acc += bf_lo(w.w) * b.z;
      acc += bf_hi(w.w) * b.w;
    }
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
// D = d_model (compile time), FFL = 16-byte pieces per lane for a d_ff-long row.
template <int D, int FFL>
__global__ __launch_bounds__(kThreads, 1) void decode_step_kernel(Args a) {
  constexpr int NLD = (D + 511) / 512;  // pieces per lane for a d-long row
  extern __shared__ float smem[];
  const int G = gridDim.x, wg = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int H = a.H, KV = a.KV, GQ = H / KV, ff = a.ff;
  const Layout& lay = a.lay;
  const int ch_max = (a.ctx + kChunks - 1) / kChunks;

  // LDS carve-up
  float* sh_h = smem;                                      // D
  float* sh_x = sh_h + D;                                  // xmax
  const int xmax = max(max(D, ff), kChunks * GQ * kPartStride);
  float* sh_k = sh_x + xmax;                               // ch_max * 64
  float* sh_v = sh_k + ch_max * kDh;                       // ch_max * 64
  float* sh_q = sh_v + ch_max * kDh;                       // GQ*64 + 128 (q, k_new, v_new)
  float* sh_e = sh_q + GQ * kDh + 2 * kDh;                 // kWaves * 64
  float* sh_red = sh_e + kWaves * 64;                      // 64
  int* sh_flag = reinterpret_cast<int*>(sh_red + 64);      // 1

  if (tid == 0) *sh_flag = 0;
  bool bad = false;
  const uint32_t tag = a.epoch;
  const int pos = a.pos;

  int token = a.token_dev ? *a.token_dev : a.token;
  if (token < 0 || token >= a.V) {
    if (wg == 0 && tid == 0) atomicOr(a.ctrl, kStatusBadToken);
    token = token < 0 ? 0 : a.V - 1;
  }
  // embedding gather (multi_sm_decode.py:88)
  for (int i = tid; i < D; i += kThreads) sh_h[i] = bf2f(a.emb[int64_t(token) * D + i]);
  __syncthreads();

  const int nqkv = (H + 2 * KV) * kDh;
  const float* rope = a.rope + int64_t(pos) * kDh;

  for (int l = 0; l < a.L; ++l) {
    const uint16_t* W = a.w + int64_t(l) * lay.layer_elems;
    uint64_t* X = a.xw + int64_t(l) * lay.x_layer;
    uint16_t* kcache = a.kv + int64_t(l) * 2 * KV * a.ctx * kDh;
    uint16_t* vcache = kcache + int64_t(KV) * a.ctx * kDh;

    // ---------------- QKV rows, RoPE, KV write (multi_sm_decode.py:121-180)
    {
      int p0, p1;
      split(nqkv / 2, G, wg, p0, p1);
      const int npairs = p1 - p0;
      // prefetch this wave's first pair before the norm
      Row<NLD> r0, r1;
      const int pf = p0 + wv;
      if (pf < p1) {
        load_row(r0, W + lay.off_qkv + int64_t(2 * pf) * D, D, lane);
        load_row(r1, W + lay.off_qkv + int64_t(2 * pf + 1) * D, D, lane);
      }
      rmsnorm(sh_h, W + lay.off_ln1, sh_x, D, sh_red);
      for (int p = pf; p < p1; p += kWaves) {
        if (p != pf) {
          load_row(r0, W + lay.off_qkv + int64_t(2 * p) * D, D, lane);
          load_row(r1, W + lay.off_qkv + int64_t(2 * p + 1) * D, D, lane);
        }
        const float s0 = dot_row(r0, sh_x, D, lane);
        const float s1 = dot_row(r1, sh_x, D, lane);
        const int row = 2 * p;
        const int head = row / kDh, rr = row % kDh;
        int i0, i1;
        float o0, o1;
        if (head < H + KV) {  // q or k: packed rows (i, i+32), rotate-half (model.py:110-117)
          const int i = rr / 2;
          const float c = rope[i], s = rope[kDh / 2 + i];
          o0 = s0 * c - s1 * s;
          o1 = s0 * s + s1 * c;
          i0 = head * kDh + i;
          i1 = i0 + kDh / 2;
        } else {
          o0 = s0;
          o1 = s1;
          i0 = head * kDh + rr;
          i1 = i0 + 1;
        }
        if (lane == 0) {
          st_tag(X + lay.x_qkv + i0, o0, tag);
          st_tag(X + lay.x_qkv + i1, o1, tag);
          if (head >= H) {  // K (post-RoPE) or V row of the cache at pos, bf16 (:179-180)
            const bool isv = head >= H + KV;
            const int kvh = isv ? head - H - KV : head - H;
            uint16_t* c = (isv ? vcache : kcache) + (int64_t(kvh) * a.ctx + pos) * kDh;
            c[i0 - head * kDh] = f2bf(o0);
            c[i1 - head * kDh] = f2bf(o1);
          }
        }
      }
      (void)npairs;
    }

    // ---------------- attention over a chunk of positions for one KV head (:182-221)
    const int n_att = KV * kChunks;
    if (wg < n_att) {
      const int g = wg / kChunks, c = wg % kChunks;
      const int npos = pos + 1;
      const int cs = (npos + kChunks - 1) / kChunks;
      const int q0 = c * cs, q1 = min(q0 + cs, npos);
      const int P = max(0, q1 - q0);
      // cached rows [q0, min(q1, pos)) -> LDS f32 (these do not depend on this step)
      const int nc = max(0, min(q1, pos) - q0);
      for (int t = tid; t < nc * 16; t += kThreads) {
        const int prow = t >> 4, piece = t & 15;   // 8 pieces of K, 8 of V per row
        const bool isv = piece >= 8;
        const uint16_t* src = (isv ? vcache : kcache) + (int64_t(g) * a.ctx + q0 + prow) * kDh + (piece & 7) * 8;
        const uint4 u = *reinterpret_cast<const uint4*>(src);
        float* dst = (isv ? sh_v : sh_k) + prow * kDh + (piece & 7) * 8;
        dst[0] = bf_lo(u.x); dst[1] = bf_hi(u.x); dst[2] = bf_lo(u.y); dst[3] = bf_hi(u.y);
        dst[4] = bf_lo(u.z); dst[5] = bf_hi(u.z); dst[6] = bf_lo(u.w); dst[7] = bf_hi(u.w);
      }
      // q for the GQ heads of group g, and the new k, v (f32, un-rounded: :197, :205)
      gather(X + lay.x_qkv + int64_t(g) * GQ * kDh, GQ * kDh, sh_q, tag, a.ctrl, sh_flag, bad);
      gather(X + lay.x_qkv + int64_t(H + g) * kDh, kDh, sh_q + GQ * kDh, tag, a.ctrl, sh_flag, bad);
      gather(X + lay.x_qkv + int64_t(H + KV + g) * kDh, kDh, sh_q + GQ * kDh + kDh, tag, a.ctrl, sh_flag, bad);
      if (pos >= q0 && pos < q1) {
        const int prow = pos - q0;
        for (int j = tid; j < kDh; j += kThreads) {
          sh_k[prow * kDh + j] = sh_q[GQ * kDh + j];
          sh_v[prow * kDh + j] = sh_q[GQ * kDh + kDh + j];
        }
      }
      __syncthreads();
      for (int n = wv; n < GQ; n += kWaves) {
        const float* q = sh_q + n * kDh;
        float s = -INFINITY;
        if (lane < P) {
          float acc = 0.f;
          const float* kr = sh_k + lane * kDh;
#pragma unroll 16
          for (int j = 0; j < kDh; ++j) acc += q[j] * kr[j];
          s = acc * 0.125f;
        }
        const float m = wave_max(s);
        const float e = (lane < P) ? expf(s - m) : 0.f;
        const float lsum = wave_sum(e);
        sh_e[wv * 64 + lane] = e;
        __builtin_amdgcn_wave_barrier();
        float o = 0.f;
        for (int p = 0; p < P; ++p) o += sh_e[wv * 64 + p] * sh_v[p * kDh + lane];
        uint64_t* part = X + lay.x_part + (int64_t(g * kChunks + c) * GQ + n) * kPartStride;
        if (lane == 0) {
          st_tag(part + 0, P > 0 ? m : -INFINITY, tag);
          st_tag(part + 1, lsum, tag);
        }
        st_tag(part + 2 + lane, o, tag);
        __builtin_amdgcn_wave_barrier();
      }
    }

    // ---------------- merge the chunks of one KV head (:243-259 LSE merge)
    if (wg < n_att && (wg % kChunks) == 0) {
      const int g = wg / kChunks;
      gather(X + lay.x_part + int64_t(g) * kChunks * GQ * kPartStride, kChunks * GQ * kPartStride,
             sh_x, tag, a.ctrl, sh_flag, bad);
      for (int n = wv; n < GQ; n += kWaves) {
        float M = -INFINITY;
        for (int c = 0; c < kChunks; ++c) {
          const float* pc = sh_x + (c * GQ + n) * kPartStride;
          if (pc[1] > 0.f) M = fmaxf(M, pc[0]);
        }
        float num = 0.f, den = 0.f;
        for (int c = 0; c < kChunks; ++c) {
          const float* pc = sh_x + (c * GQ + n) * kPartStride;
          if (pc[1] > 0.f) {
            const float wgt = expf(pc[0] - M);
            num += wgt * pc[2 + lane];
            den += wgt * pc[1];
          }
        }
        st_tag(X + lay.x_attn + (g * GQ + n) * kDh + lane, num / den, tag);
      }
      __syncthreads();
    }

    // ---------------- O projection rows + residual (:223-232, :244-260)
    {
      int r0, r1;
      split(D, G, wg, r0, r1);
      Row<NLD> rw;
      const int rf = r0 + wv;
      if (rf < r1) load_row(rw, W + lay.off_o + int64_t(rf) * D, D, lane);
      gather(X + lay.x_attn, D, sh_x, tag, a.ctrl, sh_flag, bad);
      for (int r = rf; r < r1; r += kWaves) {
        if (r != rf) load_row(rw, W + lay.off_o + int64_t(r) * D, D, lane);
        const float y = dot_row(rw, sh_x, D, lane);
        if (lane == 0) st_tag(X + lay.x_hd1 + r, y, tag);
      }
      gather(X + lay.x_hd1, D, sh_x, tag, a.ctrl, sh_flag, bad);
      for (int i = tid; i < D; i += kThreads) sh_h[i] = sh_h[i] + sh_x[i];
      __syncthreads();
    }

    // ---------------- gate/up rows + SwiGLU (:262-289, model.py:159)
    {
      int f0, f1;
      split(ff, G, wg, f0, f1);
      Row<NLD> rg, ru;
      const int ffirst = f0 + wv;
      if (ffirst < f1) {
        load_row(rg, W + lay.off_gu + int64_t(2 * ffirst) * D, D, lane);
        load_row(ru, W + lay.off_gu + int64_t(2 * ffirst + 1) * D, D, lane);
      }
      rmsnorm(sh_h, W + lay.off_ln2, sh_x, D, sh_red);
      for (int f = ffirst; f < f1; f += kWaves) {
        if (f != ffirst) {
          load_row(rg, W + lay.off_gu + int64_t(2 * f) * D, D, lane);
          load_row(ru, W + lay.off_gu + int64_t(2 * f + 1) * D, D, lane);
        }
        const float gt = dot_row(rg, sh_x, D, lane);
        const float up = dot_row(ru, sh_x, D, lane);
        const float act = (gt * (1.f / (1.f + expf(-gt)))) * up;
        if (lane == 0) st_tag(X + lay.x_act + f, act, tag);
      }
    }

    // ---------------- down rows + residual (:273-305)
    {
      int r0, r1;
      split(D, G, wg, r0, r1);
      Row<FFL> rw;
      const int rf = r0 + wv;
      if (rf < r1) load_row(rw, W + lay.off_dn + int64_t(rf) * ff, ff, lane);
      gather(X + lay.x_act, ff, sh_x, tag, a.ctrl, sh_flag, bad);
      for (int r = rf; r < r1; r += kWaves) {
        if (r != rf) load_row(rw, W + lay.off_dn + int64_t(r) * ff, ff, lane);
        const float y = dot_row(rw, sh_x, ff, lane);
        if (lane == 0) st_tag(X + lay.x_hd2 + r, y, tag);
      }
      gather(X + lay.x_hd2, D, sh_x, tag, a.ctrl, sh_flag, bad);
      for (int i = tid; i < D; i += kThreads) sh_h[i] = sh_h[i] + sh_x[i];
      __syncthreads();
    }
  }

  // ---------------- final RMSNorm, tied logits, argmax (:314-357, model.py:185-191)
  rmsnorm(sh_h, a.lnf, sh_x, D, sh_red);
  {
    int v0, v1;
    split(a.V, G, wg, v0, v1);
    float best = -INFINITY;
    int besti = 0x7fffffff;
    constexpr int B = 4;
    for (int base = v0 + wv * B; base < v1; base += kWaves * B) {
      Row<NLD> rr[B];
#pragma unroll
      for (int j = 0; j < B; ++j)
        if (base + j < v1) load_row(rr[j], a.emb + int64_t(base + j) * D, D, lane);
#pragma unroll
      for (int j = 0; j < B; ++j) {
        if (base + j < v1) {
          const float y = dot_row(rr[j], sh_x, D, lane);
          if (lane == 0) a.logits[base + j] = y;
          if (y > best) { best = y; besti = base + j; }
        }
      }
    }
    // combine waves: larger value wins, ties -> lower index
    if (lane == 0) {
      sh_red[wv] = best;
      reinterpret_cast<int*>(sh_red)[8 + wv] = besti;
    }
    __syncthreads();
    if (tid == 0) {
      float bv = sh_red[0];
      int bi = reinterpret_cast<int*>(sh_red)[8];
      for (int w = 1; w < kWaves; ++w) {
        const float v = sh_red[w];
        const int i = reinterpret_cast<int*>(sh_red)[8 + w];
        if (v > bv || (v == bv && i < bi)) { bv = v; bi = i; }
      }
      uint64_t* keyp = reinterpret_cast<uint64_t*>(a.ctrl + 2);
      if (bi != 0x7fffffff)
        __hip_atomic_fetch_max(keyp, argmax_key(bv, bi), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      // the max above returns before the arrival below is issued
      __builtin_amdgcn_s_waitcnt(0);
      const uint32_t old = __hip_atomic_fetch_add(a.ctrl + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if ((old % uint32_t(G)) == uint32_t(G - 1)) {   // last arriver publishes the token
        const uint64_t key = __hip_atomic_load(keyp, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        a.next_token[0] = int32_t(0xffffffffu - uint32_t(key & 0xffffffffu));
        a.next_token[1] = int32_t(ld_status(a.ctrl));
        __hip_atomic_store(keyp, uint64_t(0), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
  (void)bad;
}

// ---------------------------------------------------------------- host side
static bool config_ok(const msd_config* c) {
  if (!c) return false;
  if (c->d_head != kDh || c->n_heads <= 0 || c->n_kv_heads <= 0 || c->n_layers <= 0) return false;
  if (c->n_heads * kDh != c->d_model || c->n_heads % c->n_kv_heads != 0) return false;
  if (c->d_ff <= 0 || c->d_ff % 16 != 0 || c->vocab_size <= 0 || c->context_len <= 0) return false;
  if ((c->context_len + kChunks - 1) / kChunks > 64) return false;   // chunk fits a wave
  if (c->d_model != 256 && c->d_model != 1024) return false;
  if ((c->d_ff + 511) / 512 > 8) return false;
  return true;
}

static size_t lds_bytes(const msd_config* c) {
  const int GQ = c->n_heads / c->n_kv_heads;
  const int ch_max = (c->context_len + kChunks - 1) / kChunks;
  const int xmax = std::max(std::max(c->d_model, c->d_ff), kChunks * GQ * kPartStride);
  const size_t floats = size_t(c->d_model) + xmax + 2 * ch_max * kDh + GQ * kDh + 2 * kDh + kWaves * 64 + 64 + 4;
  return floats * 4;
}

// At least this much LDS per workgroup, so that no two workgroups of a step share a
// compute unit (160 KB per CU): the grid then spreads over every CU.
constexpr size_t kMinLds = 84 * 1024;

template <int D, int FFL>
static hipError_t launch_t(const Args& a, int grid, size_t lds, hipStream_t s) {
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&decode_step_kernel<D, FFL>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  hipLaunchKernelGGL((decode_step_kernel<D, FFL>), dim3(grid), dim3(kThreads), lds, s, a);
  return hipGetLastError();
}

template <int D>
static hipError_t launch_ff(const Args& a, int grid, size_t lds, hipStream_t s) {
  switch ((a.ff + 511) / 512) {
    case 1: return launch_t<D, 1>(a, grid, lds, s);
    case 2: return launch_t<D, 2>(a, grid, lds, s);
    case 3: return launch_t<D, 3>(a, grid, lds, s);
    case 4: return launch_t<D, 4>(a, grid, lds, s);
    case 5: return launch_t<D, 5>(a, grid, lds, s);
    case 6: return launch_t<D, 6>(a, grid, lds, s);
    case 7: return launch_t<D, 7>(a, grid, lds, s);
    case 8: return launch_t<D, 8>(a, grid, lds, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace msd

using namespace msd;

extern "C" int64_t msd_packed_weight_elems(const msd_config* cfg) {
  if (!config_ok(cfg)) return MSD_E_CONFIG;
  return make_layout(cfg->d_model, cfg->n_heads, cfg->n_kv_heads, cfg->d_ff).layer_elems * cfg->n_layers;
}

extern "C" int64_t msd_workspace_bytes(const msd_config* cfg, int32_t n_workgroups) {
  if (!config_ok(cfg)) return MSD_E_CONFIG;
  if (n_workgroups < cfg->n_kv_heads * kChunks) return MSD_E_ARG;
  const Layout t = make_layout(cfg->d_model, cfg->n_heads, cfg->n_kv_heads, cfg->d_ff);
  return t.ctrl_bytes + t.x_layer * cfg->n_layers * int64_t(sizeof(uint64_t));
}

extern "C" int32_t msd_default_workgroups(int32_t device) {
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess) return MSD_E_HIP;
  return n;
}

extern "C" int32_t msd_decode_step(const msd_config* cfg, const void* token_emb, const void* packed_w,
                                   const void* lnf_s, const float* rope, int32_t token_id,
                                   const int32_t* token_dev, int32_t pos, void* kv, void* workspace,
                                   uint32_t epoch, float* logits, int32_t* next_token,
                                   int32_t n_workgroups, void* stream) {
  if (!config_ok(cfg)) return MSD_E_CONFIG;
  if (!token_emb || !packed_w || !lnf_s || !rope || !kv || !workspace || !logits || !next_token) return MSD_E_ARG;
  if (pos < 0 || pos >= cfg->context_len) return MSD_E_ARG;
  if (!token_dev && (token_id < 0 || token_id >= cfg->vocab_size)) return MSD_E_ARG;
  if (n_workgroups < cfg->n_kv_heads * kChunks || n_workgroups > 4096) return MSD_E_ARG;
  if (epoch == 0) return MSD_E_ARG;
  const uintptr_t al = reinterpret_cast<uintptr_t>(token_emb) | reinterpret_cast<uintptr_t>(packed_w) |
                       reinterpret_cast<uintptr_t>(kv) | reinterpret_cast<uintptr_t>(workspace);
  if (al & 15) return MSD_E_ARG;
  Args a;
  a.emb = static_cast<const uint16_t*>(token_emb);
  a.w = static_cast<const uint16_t*>(packed_w);
  a.lnf = static_cast<const uint16_t*>(lnf_s);
  a.rope = rope;
  a.kv = static_cast<uint16_t*>(kv);
  a.logits = logits;
  a.next_token = next_token;
  a.token_dev = token_dev;
  a.ctrl = static_cast<uint32_t*>(workspace);
  a.lay = make_layout(cfg->d_model, cfg->n_heads, cfg->n_kv_heads, cfg->d_ff);
  a.xw = reinterpret_cast<uint64_t*>(static_cast<char*>(workspace) + a.lay.ctrl_bytes);
  a.token = token_id;
  a.pos = pos;
  a.epoch = epoch;
  a.H = cfg->n_heads;
  a.KV = cfg->n_kv_heads;
  a.L = cfg->n_layers;
  a.ff = cfg->d_ff;
  a.V = cfg->vocab_size;
  a.ctx = cfg->context_len;
  const size_t lds = std::max(lds_bytes(cfg), kMinLds);
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e;
  switch (cfg->d_model) {
    case 256: e = launch_ff<256>(a, n_workgroups, lds, s); break;
    case 1024: e = launch_ff<1024>(a, n_workgroups, lds, s); break;
    default: return MSD_E_CONFIG;
  }
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
