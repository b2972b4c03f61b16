// Multi-token prefill on one MI355X (gfx950): the full forward over a prompt of M tokens,
// writing the KV cache rows 0..M-1 and the logits of the last position (optionally of all
// positions), with every projection on the matrix cores.
//
// Reference: model.py:194-231 (prefill_with_kv), called by generate.py:70-90 (_prefill).
// The maths is model.py:94-191 with the activations entering each projection rounded to
// bf16 (RMSNorm outputs, attention output, SwiGLU output, final norm), the projections as
// bf16 x bf16 products accumulated in f32 (v_mfma_f32_16x16x32_bf16), the residual stream,
// RoPE, softmax attention and SwiGLU in f32, and K/V stored to the cache as bf16 after RoPE
// (model.py:212-215).
//
// Kernels per layer, on the caller's stream:
//   pf_norm        residual += split-K partials of the previous projection (in split order),
//                  then RMSNorm -> bf16 activations in the weights' permuted input order
//   pf_gemm<QKV>   q/k/v projection; RoPE on q/k pairs, f32 q/k/v, bf16 K/V cache rows
//   pf_attention   causal GQA attention, f32, online softmax over key chunks of 64
//   pf_gemm<PART>  O projection, split-K partials
//   pf_norm        (as above) -> ln2 activations
//   pf_gemm<SWIGLU> gate/up projection; silu(gate) * up -> bf16 in down's input order
//   pf_gemm<PART>  down projection, split-K partials
// then pf_norm with the final scale, pf_gemm<LOGITS> against the tied embedding, pf_argmax.
//
// GEMM: C[M x N] = A[M x K] * W[N x K]^T with A (activations) and W (packed weight rows)
// both K-contiguous.  Workgroup tile 64 x 64, four waves as 2 x 2 blocks of 32 x 32, each
// four 16 x 16 MFMA tiles; every operand fragment is one 16-byte run along K loaded
// straight from memory (A from L2, W streamed once).  K is split across grid.z where the
// consumer sums the partials.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

#include "../../include/msdecode.h"

namespace mpf {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kDh = 64;
constexpr int kBM = 64;       // GEMM tile rows (tokens)
constexpr int kBN = 64;       // GEMM tile columns (output features)
constexpr int kBK = 32;       // K per MFMA step
constexpr int kSplitO = 4;    // K splits of the O projection
constexpr int kSplitDn = 8;   // K splits of the down projection
constexpr int kMaxSplit = 8;
constexpr int kNormThreads = 256;
constexpr int kAttnQ = 64;    // queries per attention workgroup (16 per wave)
constexpr int kKStride = kDh + 4;

enum Epi { kEpiQkv = 0, kEpiPart = 1, kEpiSwiglu = 2, kEpiLogits = 3 };

__device__ __forceinline__ float bf2f(uint16_t b) { return __uint_as_float(uint32_t(b) << 16); }
__device__ __forceinline__ uint16_t f2bf(float f) {   // round to nearest even
  const uint32_t u = __float_as_uint(f);
  return uint16_t((u + (((u >> 16) & 1u) + 0x7fffu)) >> 16);
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

struct GemmArgs {
  const uint16_t* A;   // [M][K] bf16
  const uint16_t* W;   // [N][K] bf16
  int M, N, K, lda;
  int splits;
  // epilogue targets
  float* out;          // QKV: [M][N] f32 natural order; PART: [splits][M][N]; LOGITS: [M][N]
  int ldo;
  uint16_t* act;       // SWIGLU: [M][N/2] bf16 in the down projection's input order
  uint16_t* kcache;    // QKV: this layer's K cache [KV][ctx][64]
  uint16_t* vcache;
  const float* rope;   // [ctx][64]: cos | sin
  int H, KV, ctx;
};

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 u) { return __builtin_bit_cast(bf16x8, u); }

template <int EPI>
__global__ __launch_bounds__(256) void pf_gemm(GemmArgs g) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int wm = wv >> 1, wn = wv & 1;
  const int m0 = blockIdx.y * kBM + 32 * wm, n0 = blockIdx.x * kBN + 32 * wn;
  const int nchunks = g.K / kBK;
  const int c0 = (nchunks * int(blockIdx.z)) / g.splits, c1 = (nchunks * (int(blockIdx.z) + 1)) / g.splits;
  const int kq = 8 * (lane >> 4);   // this lane's 8-element K run within a 32 chunk
  const int r16 = lane & 15;
  const uint16_t* arow[2];
  bool aval[2];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    const int m = m0 + 16 * rb + r16;
    aval[rb] = m < g.M;
    arow[rb] = g.A + int64_t(aval[rb] ? m : 0) * g.lda + kq;
  }
  const uint16_t* wrow[2];
#pragma unroll
  for (int cb = 0; cb < 2; ++cb) wrow[cb] = g.W + int64_t(n0 + 16 * cb + r16) * g.K + kq;
  f32x4 acc[2][2];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb)
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) acc[rb][cb] = f32x4{0.f, 0.f, 0.f, 0.f};
  constexpr int U = 4;   // chunks in flight
  int c = c0;
  for (; c + U <= c1; c += U) {
    uint4 a[U][2], w[U][2];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = (c + u) * kBK;
#pragma unroll
      for (int rb = 0; rb < 2; ++rb)
        a[u][rb] = aval[rb] ? *reinterpret_cast<const uint4*>(arow[rb] + k) : make_uint4(0, 0, 0, 0);
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) w[u][cb] = *reinterpret_cast<const uint4*>(wrow[cb] + k);
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int rb = 0; rb < 2; ++rb)
#pragma unroll
        for (int cb = 0; cb < 2; ++cb)
          acc[rb][cb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a[u][rb]), as_bf16x8(w[u][cb]),
                                                                acc[rb][cb], 0, 0, 0);
  }
  for (; c < c1; ++c) {
    const int k = c * kBK;
    uint4 a[2], w[2];
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
      a[rb] = aval[rb] ? *reinterpret_cast<const uint4*>(arow[rb] + k) : make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) w[cb] = *reinterpret_cast<const uint4*>(wrow[cb] + k);
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
      for (int cb = 0; cb < 2; ++cb)
        acc[rb][cb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a[rb]), as_bf16x8(w[cb]), acc[rb][cb], 0, 0, 0);
  }
  // D layout of a 16 x 16 tile: lane holds rows 4*(lane/16) + r (r < 4) of column lane % 16
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
      const int col = n0 + 16 * cb + r16;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = m0 + 16 * rb + 4 * (lane >> 4) + r;
        const float v = acc[rb][cb][r];
        if (EPI == kEpiPart) {
          if (row < g.M) g.out[(int64_t(blockIdx.z) * g.M + row) * g.ldo + col] = v;
        } else if (EPI == kEpiLogits) {
          if (row < g.M) g.out[int64_t(row) * g.ldo + col] = v;
        } else if (EPI == kEpiSwiglu) {
          // columns (2f, 2f+1) are gate and up of d_ff index f, held by lanes l, l^1
          const float up = __shfl_xor(v, 1);
          if (row < g.M && (col & 1) == 0) {
            const float gt = v;
            const float a = (gt * (1.f / (1.f + expf(-gt)))) * up;
            const int f = col >> 1, F = g.N >> 1;
            g.act[int64_t(row) * F + perm_pos(f, F)] = f2bf(a);
          }
        } else {   // kEpiQkv
          const float other = __shfl_xor(v, 1);
          if (row < g.M) {
            const int head = col / kDh, rr = col % kDh;
            float o;
            int dim;
            if (head < g.H + g.KV) {   // rotate-half RoPE on the pair (i, i + 32) (model.py:110-117)
              const int i = rr >> 1;
              const float cs = g.rope[int64_t(row) * kDh + i], sn = g.rope[int64_t(row) * kDh + kDh / 2 + i];
              if ((rr & 1) == 0) {
                o = v * cs - other * sn;
                dim = i;
              } else {
                o = other * sn + v * cs;
                dim = i + kDh / 2;
              }
            } else {
              o = v;
              dim = rr;
            }
            g.out[int64_t(row) * g.ldo + head * kDh + dim] = o;
            if (head >= g.H) {
              const bool isv = head >= g.H + g.KV;
              const int kvh = isv ? head - g.H - g.KV : head - g.H;
              uint16_t* cp = (isv ? g.vcache : g.kcache) + (int64_t(kvh) * g.ctx + row) * kDh + dim;
              *cp = f2bf(o);
            }
          }
        }
      }
    }
  }
}

__device__ __forceinline__ float block_sum256(float v, float* red) {
  for (int o = 32; o; o >>= 1) v += __shfl_xor(v, o);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  const float s = (red[0] + red[1]) + (red[2] + red[3]);
  __syncthreads();
  return s;
}

// One row m per workgroup: h[m] += sum_z part[z][m] (z in order), then
// xn[m][j] = bf16(scale[i] * (h[m][i] / sqrt(mean(h[m]^2) + 1e-5))) with i the input element
// at position j of the packed row layout (model.py:94-98).
__global__ __launch_bounds__(kNormThreads) void pf_norm(float* h, const float* part, int splits, int M, int d,
                                                        const uint16_t* scale, uint16_t* xn, int row0) {
  __shared__ float red[4];
  const int m = blockIdx.x + row0;
  float* hr = h + int64_t(m) * d;
  float ss = 0.f;
  for (int n = threadIdx.x; n < d; n += kNormThreads) {
    float v = hr[n];
    for (int z = 0; z < splits; ++z) v += part[(int64_t(z) * M + m) * d + n];
    if (splits) hr[n] = v;
    ss += v * v;
  }
  ss = block_sum256(ss, red);
  const float r = sqrtf(ss / float(d) + 1e-5f);
  __syncthreads();   // the h writes above are visible to the whole workgroup
  for (int j = threadIdx.x; j < d; j += kNormThreads) {
    const int i = perm_elem(j, d);
    xn[int64_t(blockIdx.x) * d + j] = f2bf(bf2f(scale[i]) * (hr[i] / r));
  }
}

__global__ __launch_bounds__(256) void pf_embed(const uint16_t* emb, const int32_t* tokens, int d, float* h,
                                                int32_t* status, int V) {
  const int m = blockIdx.x;
  int t = tokens[m];
  if (t < 0 || t >= V) {
    if (threadIdx.x == 0) atomicOr(status, 2);
    t = 0;
  }
  for (int n = threadIdx.x; n < d; n += 256) h[int64_t(m) * d + n] = bf2f(emb[int64_t(t) * d + n]);
}

// Causal GQA attention of query block blockIdx.y (64 rows) for head blockIdx.x.  Each wave
// owns 16 queries; key chunks of 64 rows go through LDS, with an online softmax per query
// (scores: lane = key; output: lane = dimension).  Scale 1/sqrt(64) (model.py:98).
__global__ __launch_bounds__(256) void pf_attention(const float* qkv, int M, int H, int KV, uint16_t* att) {
  __shared__ float sk[64 * kKStride];
  __shared__ float sv[64 * kDh];
  __shared__ float sq[kAttnQ * kDh];
  __shared__ float sp[4][16][64];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int h = blockIdx.x, g = h / (H / KV);
  const int nqkv = (H + 2 * KV) * kDh, d = H * kDh;
  const int q0 = blockIdx.y * kAttnQ;
  for (int t = threadIdx.x; t < kAttnQ * kDh; t += 256) {
    const int i = q0 + t / kDh;
    sq[t] = i < M ? qkv[int64_t(i) * nqkv + h * kDh + (t % kDh)] : 0.f;
  }
  float mx[16], ls[16], o[16];
#pragma unroll
  for (int t = 0; t < 16; ++t) {
    mx[t] = -INFINITY;
    ls[t] = 0.f;
    o[t] = 0.f;
  }
  const int nchunk = min((q0 + kAttnQ + 63) / 64, (M + 63) / 64);
  for (int c = 0; c < nchunk; ++c) {
    __syncthreads();
    for (int t = threadIdx.x; t < 64 * kDh; t += 256) {
      const int j = 64 * c + t / kDh, e = t % kDh;
      const bool ok = j < M;
      sk[(t / kDh) * kKStride + e] = ok ? qkv[int64_t(j) * nqkv + (H + g) * kDh + e] : 0.f;
      sv[t] = ok ? qkv[int64_t(j) * nqkv + (H + KV + g) * kDh + e] : 0.f;
    }
    __syncthreads();
    const int j = 64 * c + lane;
    float s[16];
#pragma unroll
    for (int t = 0; t < 16; ++t) s[t] = 0.f;
    const float4* kr = reinterpret_cast<const float4*>(sk + lane * kKStride);
#pragma unroll 4
    for (int e4 = 0; e4 < kDh / 4; ++e4) {
      const float4 kk = kr[e4];
#pragma unroll
      for (int t = 0; t < 16; ++t) {
        const float4 qq = *reinterpret_cast<const float4*>(sq + (16 * wv + t) * kDh + 4 * e4);
        s[t] += qq.x * kk.x + qq.y * kk.y + qq.z * kk.z + qq.w * kk.w;
      }
    }
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      const int i = q0 + 16 * wv + t;
      float sc = (j <= i && j < M) ? s[t] * 0.125f : -INFINITY;
      float cm = sc;
      for (int off = 32; off; off >>= 1) cm = fmaxf(cm, __shfl_xor(cm, off));
      const float mn = fmaxf(mx[t], cm);
      const float p = (mn == -INFINITY) ? 0.f : expf(sc - mn);
      float ps = p;
      for (int off = 32; off; off >>= 1) ps += __shfl_xor(ps, off);
      const float alpha = (mx[t] == -INFINITY) ? 0.f : expf(mx[t] - mn);
      ls[t] = ls[t] * alpha + ps;
      o[t] *= alpha;
      mx[t] = mn;
      sp[wv][t][lane] = p;
    }
    __builtin_amdgcn_wave_barrier();
    for (int jj = 0; jj < 64; ++jj) {
      const float vv = sv[jj * kDh + lane];
#pragma unroll
      for (int t = 0; t < 16; ++t) o[t] += sp[wv][t][jj] * vv;
    }
    __builtin_amdgcn_wave_barrier();
  }
#pragma unroll
  for (int t = 0; t < 16; ++t) {
    const int i = q0 + 16 * wv + t;
    if (i < M) att[int64_t(i) * d + perm_pos(h * kDh + lane, d)] = f2bf(o[t] / ls[t]);
  }
}

// argmax over one row of logits (lowest index on ties), one workgroup of 1024 threads
__global__ __launch_bounds__(1024) void pf_argmax(const float* logits, int V, int32_t* out, const int32_t* status) {
  __shared__ uint64_t red[16];
  uint64_t best = 0;
  for (int j = threadIdx.x; j < V; j += 1024) {
    uint32_t u = __float_as_uint(logits[j]);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    const uint64_t key = (uint64_t(u) << 32) | uint64_t(0xffffffffu - uint32_t(j));
    best = key > best ? key : best;
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
    out[0] = int32_t(0xffffffffu - uint32_t(b & 0xffffffffu));
    out[1] = *status;
  }
}

// ---------------------------------------------------------------- host side
struct PfLayout {
  size_t h, xn, qkv, att, act, part, status, bytes;
};

static size_t al256(size_t x) { return (x + 255) & ~size_t(255); }

static PfLayout pf_layout(const msd_config* c, int M) {
  const int d = c->d_model, ff = c->d_ff, nqkv = (c->n_heads + 2 * c->n_kv_heads) * kDh;
  PfLayout L;
  size_t o = 0;
  L.h = o;      o += al256(size_t(M) * d * 4);
  L.xn = o;     o += al256(size_t(M) * d * 2);
  L.qkv = o;    o += al256(size_t(M) * nqkv * 4);
  L.att = o;    o += al256(size_t(M) * d * 2);
  L.act = o;    o += al256(size_t(M) * ff * 2);
  L.part = o;   o += al256(size_t(kMaxSplit) * M * d * 4);
  L.status = o; o += 256;
  L.bytes = o;
  return L;
}

static bool pf_config_ok(const msd_config* c) {
  if (!c || c->d_head != kDh || c->n_heads <= 0 || c->n_kv_heads <= 0 || c->n_layers <= 0) return false;
  if (c->n_heads * kDh != c->d_model || c->n_heads % c->n_kv_heads) return false;
  if (c->d_model % kBN || (2 * c->d_ff) % kBN || c->vocab_size % kBN || c->d_ff % 8) return false;
  if (c->d_model % kBK || c->d_ff % kBK || c->context_len <= 0) return false;
  return true;
}

template <int EPI>
static hipError_t gemm(const GemmArgs& g, hipStream_t s) {
  const dim3 grid(g.N / kBN, (g.M + kBM - 1) / kBM, g.splits);
  hipLaunchKernelGGL(pf_gemm<EPI>, grid, dim3(256), 0, s, g);
  return hipGetLastError();
}

}  // namespace mpf

using namespace mpf;

extern "C" int64_t msd_prefill_workspace_bytes(const msd_config* cfg, int32_t n_tokens) {
  if (!pf_config_ok(cfg)) return MSD_E_CONFIG;
  if (n_tokens <= 0 || n_tokens > cfg->context_len) return MSD_E_ARG;
  return int64_t(pf_layout(cfg, n_tokens).bytes);
}

extern "C" int32_t msd_prefill(const msd_config* cfg, const void* token_emb, const void* output_proj,
                               const void* packed_w, const void* lnf_s, const float* rope, const int32_t* tokens,
                               int32_t n_tokens, void* kv, void* workspace, float* logits_last,
                               float* logits_all, int32_t* next_token, void* stream) {
  if (!pf_config_ok(cfg)) return MSD_E_CONFIG;
  const int M = n_tokens;
  if (M <= 0 || M > cfg->context_len) return MSD_E_ARG;
  if (!token_emb || !output_proj || !packed_w || !lnf_s || !rope || !tokens || !kv || !workspace || !logits_last ||
      !next_token)
    return MSD_E_ARG;
  const uintptr_t al = reinterpret_cast<uintptr_t>(token_emb) | reinterpret_cast<uintptr_t>(output_proj) |
                       reinterpret_cast<uintptr_t>(packed_w) | reinterpret_cast<uintptr_t>(kv) |
                       reinterpret_cast<uintptr_t>(workspace);
  if (al & 15) return MSD_E_ARG;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int d = cfg->d_model, ff = cfg->d_ff, H = cfg->n_heads, KV = cfg->n_kv_heads, ctx = cfg->context_len;
  const int nqkv = (H + 2 * KV) * kDh, V = cfg->vocab_size;
  const PfLayout L = pf_layout(cfg, M);
  char* ws = static_cast<char*>(workspace);
  float* hbuf = reinterpret_cast<float*>(ws + L.h);
  uint16_t* xn = reinterpret_cast<uint16_t*>(ws + L.xn);
  float* qkv = reinterpret_cast<float*>(ws + L.qkv);
  uint16_t* att = reinterpret_cast<uint16_t*>(ws + L.att);
  uint16_t* act = reinterpret_cast<uint16_t*>(ws + L.act);
  float* part = reinterpret_cast<float*>(ws + L.part);
  int32_t* status = reinterpret_cast<int32_t*>(ws + L.status);
  // per-layer packed offsets (same layout as the decode step)
  const int64_t off_ln2 = d, off_qkv = 2 * int64_t(d), off_o = off_qkv + int64_t(nqkv) * d,
                off_gu = off_o + int64_t(d) * d, off_dn = off_gu + 2 * int64_t(ff) * d,
                layer = off_dn + int64_t(d) * ff;
  const uint16_t* W = static_cast<const uint16_t*>(packed_w);
  uint16_t* kvb = static_cast<uint16_t*>(kv);
  if (hipMemsetAsync(status, 0, 4, s) != hipSuccess) return MSD_E_HIP;
  hipLaunchKernelGGL(pf_embed, dim3(M), dim3(256), 0, s, static_cast<const uint16_t*>(token_emb), tokens, d, hbuf,
                     status, V);
  int splits = 0;   // partials pending in `part` for the next norm
  for (int l = 0; l < cfg->n_layers; ++l) {
    const uint16_t* Wl = W + int64_t(l) * layer;
    uint16_t* kc = kvb + int64_t(l) * 2 * KV * ctx * kDh;
    uint16_t* vc = kc + int64_t(KV) * ctx * kDh;
    hipLaunchKernelGGL(pf_norm, dim3(M), dim3(kNormThreads), 0, s, hbuf, part, splits, M, d, Wl, xn, 0);
    GemmArgs g{};
    g.A = xn; g.lda = d; g.M = M; g.K = d; g.splits = 1;
    g.W = Wl + off_qkv; g.N = nqkv; g.out = qkv; g.ldo = nqkv;
    g.kcache = kc; g.vcache = vc; g.rope = rope; g.H = H; g.KV = KV; g.ctx = ctx;
    if (gemm<kEpiQkv>(g, s) != hipSuccess) return MSD_E_HIP;
    hipLaunchKernelGGL(pf_attention, dim3(H, (M + kAttnQ - 1) / kAttnQ), dim3(256), 0, s, qkv, M, H, KV, att);
    GemmArgs go{};
    go.A = att; go.lda = d; go.M = M; go.K = d; go.splits = kSplitO;
    go.W = Wl + off_o; go.N = d; go.out = part; go.ldo = d;
    if (gemm<kEpiPart>(go, s) != hipSuccess) return MSD_E_HIP;
    hipLaunchKernelGGL(pf_norm, dim3(M), dim3(kNormThreads), 0, s, hbuf, part, kSplitO, M, d, Wl + off_ln2, xn, 0);
    GemmArgs gg{};
    gg.A = xn; gg.lda = d; gg.M = M; gg.K = d; gg.splits = 1;
    gg.W = Wl + off_gu; gg.N = 2 * ff; gg.act = act;
    if (gemm<kEpiSwiglu>(gg, s) != hipSuccess) return MSD_E_HIP;
    GemmArgs gd{};
    gd.A = act; gd.lda = ff; gd.M = M; gd.K = ff; gd.splits = std::min(kSplitDn, ff / kBK);
    gd.W = Wl + off_dn; gd.N = d; gd.out = part; gd.ldo = d;
    if (gemm<kEpiPart>(gd, s) != hipSuccess) return MSD_E_HIP;
    splits = gd.splits;
  }
  // final norm of the rows whose logits are wanted, then the tied output projection
  const int r0 = logits_all ? 0 : M - 1, nr = M - r0;
  hipLaunchKernelGGL(pf_norm, dim3(nr), dim3(kNormThreads), 0, s, hbuf, part, splits, M, d,
                     static_cast<const uint16_t*>(lnf_s), xn, r0);
  GemmArgs gl{};
  gl.A = xn; gl.lda = d; gl.M = nr; gl.K = d; gl.splits = 1;
  gl.W = static_cast<const uint16_t*>(output_proj); gl.N = V;
  gl.out = logits_all ? logits_all : logits_last; gl.ldo = V;
  if (gemm<kEpiLogits>(gl, s) != hipSuccess) return MSD_E_HIP;
  const float* last = logits_all ? logits_all + int64_t(M - 1) * V : logits_last;
  if (logits_all && hipMemcpyAsync(logits_last, last, size_t(V) * 4, hipMemcpyDeviceToDevice, s) != hipSuccess)
    return MSD_E_HIP;
  hipLaunchKernelGGL(pf_argmax, dim3(1), dim3(1024), 0, s, logits_last, V, next_token, status);
  return hipGetLastError() == hipSuccess ? MSD_OK : MSD_E_HIP;
}
