// Exchange-latency probe: what one cross-workgroup hop of the decode step costs on this device,
// with no weights, no arithmetic and nothing else running.
//
//   * ping-pong: workgroups a and b take turns storing an incrementing word and polling for the
//     other's (device-scope relaxed atomics, the decode step's exchange accesses); the round trip
//     is two store -> poll visibilities.  Run for a and b on the same XCD and on different XCDs,
//     in uncached device memory (the decode step's exchange workspace) and in ordinary memory.
//   * all-gather: 256 workgroups of 256 threads each store their share of an NW-word vector of
//     tagged 64-bit words (tag = iteration) and poll the whole vector until every tag is current,
//     as the decode step's gathers do (NW = 1024: a d_model vector; 2816: the FFN activation;
//     8192 / 22528: the same for 8 sequences), after a first-poll delay of 0 / 0.2 / 0.4 us.
//   * relay: as the 1024-word all-gather, but one workgroup per XCD polls the vector and copies it
//     into a buffer of its XCD that the other workgroups of the XCD poll.
//
// Every wait is bounded (a gather that runs out of spins stops and is reported as failed).
// Build and run:  hipcc -O3 --offload-arch=gfx950 -Xclang -target-feature -Xclang -packed-fp32-ops
//                 exchange_latency.hip -o exchange_latency && ./exchange_latency
#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <vector>

constexpr int kGroups = 256;   // one workgroup per CU
constexpr int kRounds = 1000;  // gathers per timing
constexpr double kTickUs = 0.01;   // s_memrealtime runs at 100 MHz

__device__ __forceinline__ uint32_t xcc_id() {
  uint32_t v;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
  return v & 0xf;
}
__device__ __forceinline__ uint64_t now() { return __builtin_amdgcn_s_memrealtime(); }
__device__ __forceinline__ uint32_t ld32(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld64(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st64(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// out: [0] ticks of a's loop, [1] a's failed waits, [2] a's XCC, [3] b's XCC, [4] b's failed waits
__global__ void pingpong(uint32_t* flags, int a, int b, int n, uint64_t* out) {
  const int w = blockIdx.x;
  if ((w != a && w != b) || threadIdx.x != 0) return;
  uint32_t* mine = flags + (w == a ? 0 : 64);
  const uint32_t* theirs = flags + (w == a ? 64 : 0);
  uint32_t fails = 0;
  const uint64_t t0 = now();
  for (int i = 1; i <= n; ++i) {
    if (w == a) __hip_atomic_store(mine, uint32_t(i), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    uint32_t spins = 0;
    while (ld32(theirs) != uint32_t(i) && ++spins < (1u << 20)) {}
    if (spins >= (1u << 20)) { ++fails; break; }
    if (w == b) __hip_atomic_store(mine, uint32_t(i), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  const uint64_t t1 = now();
  if (w == a) { out[0] = t1 - t0; out[1] = fails; out[2] = xcc_id(); }
  else { out[3] = xcc_id(); out[4] = fails; }
}

// Poll the NW words at src (thread t reads words t, t + 256, ...) until all carry tag >= it.
template <int NW>
__device__ __forceinline__ bool poll_all(const uint64_t* src, uint32_t it, int t, uint64_t (&v)[NW / 256]) {
  for (uint32_t spins = 0; spins < (1u << 16); ++spins) {
#pragma unroll
    for (int j = 0; j < NW / 256; ++j) v[j] = ld64(src + 256 * j + t);
    bool ok = true;
#pragma unroll
    for (int j = 0; j < NW / 256; ++j) ok = ok && uint32_t(v[j] >> 32) >= it;
    if (ok) return true;
  }
  return false;
}

// out[2 w] = ticks of workgroup w's loop, out[2 w + 1] = its failed waits
template <int NW>
__global__ __launch_bounds__(256) void gather(uint64_t* X, int rounds, int first_delay, uint64_t* out) {
  const int w = blockIdx.x, t = threadIdx.x, G = gridDim.x;
  __shared__ int bad;
  if (t == 0) bad = 0;
  __syncthreads();
  uint32_t fails = 0;
  const int o0 = int((int64_t(NW) * w) / G), o1 = int((int64_t(NW) * (w + 1)) / G);
  const uint64_t t0 = now();
  for (int i = 1; i <= rounds; ++i) {
    for (int o = o0 + t; o < o1; o += 256) st64(X + o, (uint64_t(i) << 32) | uint32_t(o));
    const uint64_t ts = now();
    while (now() - ts < uint64_t(first_delay)) {}
    uint64_t v[NW / 256];
    if (!poll_all<NW>(X, uint32_t(i), t, v)) { ++fails; bad = 1; }
    __syncthreads();
    if (bad) break;
    __syncthreads();
  }
  const uint64_t t1 = now();
  if (t == 0) { out[2 * w] = t1 - t0; out[2 * w + 1] = fails; }
}

// The first workgroup of each XCD to arrive relays the 1024-word vector into L + 1024 * xcc.
__global__ __launch_bounds__(256) void gather_relay(uint64_t* X, uint64_t* L, uint32_t* elect, int rounds,
                                                    int first_delay, uint64_t* out) {
  constexpr int NW = 1024;
  const int w = blockIdx.x, t = threadIdx.x, G = gridDim.x;
  __shared__ int role, bad;
  if (t == 0) { role = int(atomicAdd(elect + xcc_id(), 1u)); bad = 0; }
  __syncthreads();
  uint64_t* loc = L + NW * xcc_id();
  uint32_t fails = 0;
  const int o0 = (NW * w) / G, o1 = (NW * (w + 1)) / G;
  const uint64_t t0 = now();
  for (int i = 1; i <= rounds; ++i) {
    for (int o = o0 + t; o < o1; o += 256) st64(X + o, (uint64_t(i) << 32) | uint32_t(o));
    uint64_t v[NW / 256];
    if (role == 0) {
      if (!poll_all<NW>(X, uint32_t(i), t, v)) { ++fails; bad = 1; }
#pragma unroll
      for (int j = 0; j < NW / 256; ++j) st64(loc + 256 * j + t, v[j]);
    } else {
      const uint64_t ts = now();
      while (now() - ts < uint64_t(first_delay)) {}
      if (!poll_all<NW>(loc, uint32_t(i), t, v)) { ++fails; bad = 1; }
    }
    __syncthreads();
    if (bad) break;
    __syncthreads();
  }
  const uint64_t t1 = now();
  if (t == 0) { out[2 * w] = t1 - t0; out[2 * w + 1] = fails; }
}

#define CK(x)                                                                  \
  do {                                                                         \
    hipError_t e_ = (x);                                                       \
    if (e_ != hipSuccess) {                                                    \
      std::printf("%s: %s\n", #x, hipGetErrorString(e_));                      \
      return 1;                                                                \
    }                                                                          \
  } while (0)

int main() {
  // Uncached allocations are kept until the process ends (never freed after a kernel read them).
  uint32_t *flags_uc, *flags_ord, *elect;
  uint64_t *out, *X_uc, *X_ord, *L;
  constexpr int kMaxWords = 22528;
  CK(hipExtMallocWithFlags((void**)&flags_uc, 4096, hipDeviceMallocUncached));
  CK(hipMalloc(&flags_ord, 4096));
  CK(hipMalloc(&out, 2 * kGroups * 8));
  CK(hipExtMallocWithFlags((void**)&X_uc, kMaxWords * 8, hipDeviceMallocUncached));
  CK(hipMalloc(&X_ord, kMaxWords * 8));
  CK(hipMalloc(&L, 16 * 1024 * 8));
  CK(hipMalloc(&elect, 16 * 4));
  std::vector<uint64_t> h(2 * kGroups);

  const int n_pp = 2000;
  struct Case { const char* name; uint32_t* flags; int a, b; };
  // workgroups are dealt to the XCDs round-robin: 0 and 8 share one, 0 and 1 do not
  const Case cases[] = {{"uncached, same XCD", flags_uc, 0, 8}, {"uncached, other XCD", flags_uc, 0, 1},
                        {"ordinary, same XCD", flags_ord, 0, 8}, {"ordinary, other XCD", flags_ord, 0, 1}};
  for (const Case& c : cases) {
    CK(hipMemset(c.flags, 0, 1024));
    CK(hipMemset(out, 0, 64));
    hipLaunchKernelGGL(pingpong, dim3(64), dim3(64), 0, 0, c.flags, c.a, c.b, n_pp, out);
    CK(hipGetLastError());
    CK(hipDeviceSynchronize());
    CK(hipMemcpy(h.data(), out, 5 * 8, hipMemcpyDeviceToHost));
    std::printf("ping-pong %-20s (XCC %llu / %llu, failed waits %llu): round trip %.3f us\n", c.name,
                (unsigned long long)h[2], (unsigned long long)h[3], (unsigned long long)(h[1] + h[4]),
                double(h[0]) * kTickUs / n_pp);
  }

  auto report = [&](const char* what, int delay) -> int {
    CK(hipGetLastError());
    CK(hipDeviceSynchronize());
    CK(hipMemcpy(h.data(), out, 2 * kGroups * 8, hipMemcpyDeviceToHost));
    uint64_t mx = 0, fails = 0;
    for (int w = 0; w < kGroups; ++w) { mx = std::max(mx, h[2 * w]); fails += h[2 * w + 1]; }
    std::printf("%-40s first-poll delay %.1f us: %.3f us per gather (failed waits %llu)\n", what,
                delay * kTickUs, double(mx) * kTickUs / kRounds, (unsigned long long)fails);
    return 0;
  };
  auto run = [&](auto kern, uint64_t* X, int words, const char* what, int delay) -> int {
    CK(hipMemset(X, 0, size_t(words) * 8));
    CK(hipMemset(out, 0, 2 * kGroups * 8));
    hipLaunchKernelGGL(kern, dim3(kGroups), dim3(256), 0, 0, X, kRounds, delay, out);
    return report(what, delay);
  };
  for (int d : {0, 20, 40}) {
    if (run(gather<1024>, X_uc, 1024, "all-gather 1024 words, uncached", d)) return 1;
    if (run(gather<1024>, X_ord, 1024, "all-gather 1024 words, ordinary", d)) return 1;
  }
  for (int d : {20, 40}) {
    CK(hipMemset(X_uc, 0, 1024 * 8));
    CK(hipMemset(L, 0, 16 * 1024 * 8));
    CK(hipMemset(elect, 0, 16 * 4));
    CK(hipMemset(out, 0, 2 * kGroups * 8));
    hipLaunchKernelGGL(gather_relay, dim3(kGroups), dim3(256), 0, 0, X_uc, L, elect, kRounds, d, out);
    if (report("all-gather 1024 words, relay per XCD", d)) return 1;
  }
  if (run(gather<2816>, X_uc, 2816, "all-gather 2816 words, uncached", 40)) return 1;
  if (run(gather<8192>, X_uc, 8192, "all-gather 8192 words, uncached", 40)) return 1;
  if (run(gather<22528>, X_uc, 22528, "all-gather 22528 words, uncached", 40)) return 1;
  return 0;
}
