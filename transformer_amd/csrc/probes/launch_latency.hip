// Launch-latency probe: what a kernel boundary costs on this device, with nothing else running.
//
//   * an empty kernel of 256 workgroups, launched 400 times back to back on one stream;
//   * a dependent chain: 400 launches of a kernel whose 256 workgroups each read n floats that the
//     previous launch wrote and write n floats (n = 1, 64, 512), launched one by one on a stream;
//   * the same chain captured once in a HIP graph and replayed.
//
// Times are HIP events around the 400 launches.  Launched one by one, short kernels are bound
// by the host's enqueue cost; the graph replay shows the device's own cost of a dependent launch.
// Build and run:  hipcc -O3 --offload-arch=gfx950 -Xclang -target-feature -Xclang -packed-fp32-ops
//                 launch_latency.hip -o launch_latency && ./launch_latency
#include <hip/hip_runtime.h>
#include <cstdio>
__global__ void empty_k() {}
// each of G workgroups reads n floats written by the previous launch and writes n floats
__global__ __launch_bounds__(256) void chain_k(const float* __restrict__ in, float* __restrict__ out, int n) {
  const int base = blockIdx.x * n;
  for (int i = threadIdx.x; i < n; i += 256) out[base + i] = in[base + i] * 1.0001f + 1.f;
}
#define CK(x) do { hipError_t e_ = (x); if (e_ != hipSuccess) { printf("%s: %s\n", #x, hipGetErrorString(e_)); return 1; } } while (0)
int main() {
  float *a, *b;
  const int G = 256, nmax = 512;
  CK(hipMalloc(&a, G * nmax * 4)); CK(hipMalloc(&b, G * nmax * 4));
  CK(hipMemset(a, 0, G * nmax * 4)); CK(hipMemset(b, 0, G * nmax * 4));
  hipEvent_t e0, e1; CK(hipEventCreate(&e0)); CK(hipEventCreate(&e1));
  const int R = 400;
  for (int rep = 0; rep < 2; ++rep) {
    float ms;
    CK(hipEventRecord(e0, 0));
    for (int i = 0; i < R; ++i) hipLaunchKernelGGL(empty_k, dim3(G), dim3(256), 0, 0);
    CK(hipEventRecord(e1, 0)); CK(hipEventSynchronize(e1)); CK(hipEventElapsedTime(&ms, e0, e1));
    printf("empty kernel, %d WGs: %.2f us per launch\n", G, ms * 1000 / R);
    for (int n : {1, 64, 512}) {
      CK(hipEventRecord(e0, 0));
      for (int i = 0; i < R; ++i) hipLaunchKernelGGL(chain_k, dim3(G), dim3(256), 0, 0, (i & 1) ? b : a, (i & 1) ? a : b, n);
      CK(hipEventRecord(e1, 0)); CK(hipEventSynchronize(e1)); CK(hipEventElapsedTime(&ms, e0, e1));
      printf("dependent chain, %d WGs x %d floats read+written: %.2f us per launch\n", G, n, ms * 1000 / R);
    }
  }
  // the same dependent chain captured once in a graph and replayed
  hipStream_t st; CK(hipStreamCreate(&st));
  for (int n : {1, 64}) {
    hipGraph_t gr; hipGraphExec_t ge;
    CK(hipStreamBeginCapture(st, hipStreamCaptureModeGlobal));
    for (int i = 0; i < R; ++i) hipLaunchKernelGGL(chain_k, dim3(G), dim3(256), 0, st, (i & 1) ? b : a, (i & 1) ? a : b, n);
    CK(hipStreamEndCapture(st, &gr));
    CK(hipGraphInstantiate(&ge, gr, nullptr, nullptr, 0));
    for (int rep = 0; rep < 3; ++rep) {
      float ms;
      CK(hipEventRecord(e0, st)); CK(hipGraphLaunch(ge, st)); CK(hipEventRecord(e1, st));
      CK(hipEventSynchronize(e1)); CK(hipEventElapsedTime(&ms, e0, e1));
      printf("graph replay, dependent chain, %d WGs x %d floats: %.2f us per kernel\n", G, n, ms * 1000 / R);
    }
  }
  CK(hipGetLastError());
  return 0;
}
