// LDS accumulate rates on gfx950 for the layouts a (g,h) int64 histogram can
// take: updates (one (g,h) pair = two ds_add_u64) per clock per CU, with
// uniform random bins over 256.
//
//   copies C : lane l adds into copy l % C of its bin, words bin*C + c
//              (g and h in separate arrays); one feature per lane group.
//   slots S  : lane l owns slot l % S (a feature, or a feature's copy), words
//              bin*S + slot, so a slot's words all sit in one bank pair and a
//              wave's 64 lanes spread evenly over the banks whatever the bins.
//
// Build: hipcc --offload-arch=gfx950 -O3 -o lds_slots lds_slots.hip
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>

#define CHECK(x)                                                               \
  do {                                                                         \
    hipError_t e = (x);                                                        \
    if (e != hipSuccess) {                                                     \
      printf("err %s line %d\n", hipGetErrorString(e), __LINE__);              \
      return 1;                                                                \
    }                                                                          \
  } while (0)

// W = words per bin (C or S); the array holds 256 * W words for g, then the
// same for h.  Lane l adds at bin * W + (l % W).
template <int W>
__global__ __launch_bounds__(256) void k_acc(int iters, unsigned long long *out) {
  extern __shared__ unsigned long long h[];
  for (int i = threadIdx.x; i < 2 * 256 * W; i += 256) h[i] = 0;
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int sub = lane % W;
  uint32_t s[8];
  for (int q = 0; q < 8; ++q) s[q] = (blockIdx.x * 256 + threadIdx.x) * 2654435761u + q * 40503u + 1u;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      s[q] ^= s[q] << 13;
      s[q] ^= s[q] >> 17;
      s[q] ^= s[q] << 5;
      const uint32_t bin = (s[q] >> 8) & 255u;
      __hip_atomic_fetch_add(&h[bin * W + sub], (unsigned long long)s[q], __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_WORKGROUP);
      __hip_atomic_fetch_add(&h[256 * W + bin * W + sub], (unsigned long long)q,
                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
  }
  __syncthreads();
  unsigned long long acc = 0;
  for (int i = threadIdx.x; i < 2 * 256 * W; i += 256) acc += h[i];
  atomicAdd(out, acc);
}

template <int W>
int run(const char *name, int cu, int clk_khz, unsigned long long *d) {
  const size_t lds = 2 * 256 * W * sizeof(unsigned long long);
  int per_cu = (int)(160 * 1024 / lds);
  if (per_cu > 8) per_cu = 8;
  const int blocks = cu * per_cu, iters = 128;
  hipEvent_t a, b;
  CHECK(hipEventCreate(&a));
  CHECK(hipEventCreate(&b));
  CHECK(hipFuncSetAttribute(reinterpret_cast<const void *>(&k_acc<W>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
  for (int rep = 0; rep < 2; ++rep) {
    CHECK(hipEventRecord(a));
    hipLaunchKernelGGL(k_acc<W>, dim3(blocks), dim3(256), lds, 0, iters, d);
    CHECK(hipGetLastError());
    CHECK(hipEventRecord(b));
    CHECK(hipEventSynchronize(b));
    float ms;
    CHECK(hipEventElapsedTime(&ms, a, b));
    if (rep == 1) {
      const double upd = (double)blocks * 256 * iters * 8;
      printf("%-28s LDS %6zu B  blocks/CU %d  %7.3f ms  %5.2f updates/clk/CU\n", name, lds, per_cu,
             ms, upd / (ms * 1e-3) / (clk_khz * 1e3) / cu);
    }
  }
  CHECK(hipEventDestroy(a));
  CHECK(hipEventDestroy(b));
  return 0;
}

int main() {
  unsigned long long *d;
  CHECK(hipMalloc(&d, 8));
  int cu = 0, clk = 0;
  CHECK(hipDeviceGetAttribute(&cu, hipDeviceAttributeMultiprocessorCount, 0));
  CHECK(hipDeviceGetAttribute(&clk, hipDeviceAttributeClockRate, 0));
  printf("CUs %d, clock %d kHz\n", cu, clk);
  if (run<1>("W=1  (C=1)", cu, clk, d)) return 1;
  if (run<2>("W=2  (C=2)", cu, clk, d)) return 1;
  if (run<4>("W=4  (C=4)", cu, clk, d)) return 1;
  if (run<8>("W=8  (C=8 or 8 slots)", cu, clk, d)) return 1;
  if (run<16>("W=16 (16 slots)", cu, clk, d)) return 1;
  if (run<32>("W=32 (32 slots)", cu, clk, d)) return 1;
  CHECK(hipFree(d));
  return 0;
}
