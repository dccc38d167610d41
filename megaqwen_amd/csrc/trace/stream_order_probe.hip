// Do two kernel launches on one HIP stream overlap? Kernel A (256 workgroups, one per CU by
// its LDS use) has workgroup 0 spin for a fixed time (bounded by the s_memrealtime clock,
// 100 MHz) and then record the clock; kernel B, launched right after A on the same stream,
// records the clock at the start of each of its 256 workgroups. If a B workgroup could start
// on a CU that A had released while A's last workgroup still ran, some B start would precede
// A's end. Run as ordinary launches and as a captured two-node HIP graph, 20 times each.
// A profiling tool (built by `python -m megaqwen_amd.build --trace`), not part of the library.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include <algorithm>
#include <vector>

#define CK(x)                                                                     \
  do {                                                                            \
    hipError_t e_ = (x);                                                          \
    if (e_ != hipSuccess) {                                                       \
      printf("HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__);       \
      return 1;                                                                   \
    }                                                                             \
  } while (0)

__device__ __forceinline__ uint64_t now() { return __builtin_amdgcn_s_memrealtime(); }

// 96 KB of LDS: one workgroup per CU
__global__ void __launch_bounds__(512) kernel_a(uint64_t* t, uint64_t spin) {
  __shared__ uint32_t pad[24576];
  pad[threadIdx.x] = threadIdx.x;
  __syncthreads();
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    const uint64_t t0 = now();
    uint64_t t1 = t0;
    while (t1 - t0 < spin) {
      __builtin_amdgcn_s_sleep(8);
      t1 = now();
    }
    t[0] = now();
  }
  if (pad[(threadIdx.x + 1) & 511] == 0xdeadbeefu) t[1] = 1;
}

__global__ void __launch_bounds__(512) kernel_b(uint64_t* t) {
  __shared__ uint32_t pad[24576];
  const uint64_t t0 = now();
  pad[threadIdx.x] = threadIdx.x;
  __syncthreads();
  if (threadIdx.x == 0) t[2 + blockIdx.x] = t0;
  if (pad[(threadIdx.x + 1) & 511] == 0xdeadbeefu) t[1] = 1;
}

int main() {
  const uint64_t spin = 3000;  // 30 us
  uint64_t* T;
  CK(hipMalloc(&T, (2 + 256) * 8));
  std::vector<uint64_t> h(2 + 256);
  hipStream_t s;
  CK(hipStreamCreate(&s));
  hipGraph_t gr;
  hipGraphExec_t ge;
  CK(hipStreamBeginCapture(s, hipStreamCaptureModeGlobal));
  hipLaunchKernelGGL(kernel_a, dim3(256), dim3(512), 0, s, T, spin);
  hipLaunchKernelGGL(kernel_b, dim3(256), dim3(512), 0, s, T);
  CK(hipStreamEndCapture(s, &gr));
  CK(hipGraphInstantiate(&ge, gr, nullptr, nullptr, 0));
  for (int graph = 0; graph < 2; graph++) {
    int early = 0;
    double dmin = 1e30, dmax = -1e30;
    for (int rep = 0; rep < 20; rep++) {
      CK(hipMemset(T, 0, (2 + 256) * 8));
      CK(hipDeviceSynchronize());
      if (graph) {
        CK(hipGraphLaunch(ge, s));
      } else {
        hipLaunchKernelGGL(kernel_a, dim3(256), dim3(512), 0, s, T, spin);
        hipLaunchKernelGGL(kernel_b, dim3(256), dim3(512), 0, s, T);
      }
      CK(hipStreamSynchronize(s));
      CK(hipMemcpy(h.data(), T, h.size() * 8, hipMemcpyDeviceToHost));
      uint64_t bmin = ~0ull;
      for (int i = 0; i < 256; i++) bmin = std::min(bmin, h[2 + i]);
      const double d = (double)(int64_t)(bmin - h[0]) * 0.01;  // us
      dmin = std::min(dmin, d);
      dmax = std::max(dmax, d);
      early += bmin < h[0];
    }
    printf("%s: B's first workgroup started %.2f .. %.2f us after A's last workgroup recorded its end; "
           "%d of 20 launches overlapped\n",
           graph ? "HIP graph of two kernel nodes" : "two ordinary launches", dmin, dmax, early);
  }
  return 0;
}
