// Plain device copy of a known size: the calibration for HBM traffic
// counters (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE should read 256 MiB per
// dispatch) and the achievable copy bandwidth of the GPU.
// Build: hipcc --offload-arch=gfx950 -O3 -o copy_calibration copy_calibration.hip
#include <hip/hip_runtime.h>

#include <cstdio>

#define CHECK(x)                                                               \
  do {                                                                         \
    hipError_t e_ = (x);                                                       \
    if (e_ != hipSuccess) {                                                    \
      std::printf("HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__); \
      return 1;                                                                \
    }                                                                          \
  } while (0)

__global__ __launch_bounds__(256) void k_copy(const int4 *__restrict__ src,
                                              int4 *__restrict__ dst, long n) {
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (long)gridDim.x * blockDim.x)
    dst[i] = src[i];
}

int main() {
  const size_t bytes = size_t(256) << 20;  // 256 MiB, larger than the 256 MB MALL
  const long n = (long)(bytes / sizeof(int4));
  int4 *a = nullptr, *b = nullptr;
  CHECK(hipMalloc(&a, bytes));
  CHECK(hipMalloc(&b, bytes));
  CHECK(hipMemset(a, 1, bytes));
  CHECK(hipMemset(b, 0, bytes));
  int cus = 0;
  CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0));
  const unsigned grid = (unsigned)cus * 16;
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));
  for (int rep = 0; rep < 6; ++rep) {
    // Alternate directions so no dispatch finds its source in a cache.
    const int4 *s = (rep & 1) ? b : a;
    int4 *d = (rep & 1) ? a : b;
    CHECK(hipEventRecord(e0));
    hipLaunchKernelGGL(k_copy, dim3(grid), dim3(256), 0, 0, s, d, n);
    CHECK(hipGetLastError());
    CHECK(hipEventRecord(e1));
    CHECK(hipEventSynchronize(e1));
    float ms = 0.f;
    CHECK(hipEventElapsedTime(&ms, e0, e1));
    std::printf("copy %zu MiB: %.3f ms, %.1f GB/s (read + write)\n", bytes >> 20, ms,
                2.0 * (double)bytes / (ms * 1e-3) / 1e9);
  }
  CHECK(hipFree(a));
  CHECK(hipFree(b));
  return 0;
}
