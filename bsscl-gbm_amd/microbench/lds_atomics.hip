// LDS accumulate throughput on gfx950: updates per clock per CU for the ways a
// histogram bin can be accumulated (2x u64, 2x u32, native f32/f64, packed
// u64), with 256 and 16 distinct bins per block.  Each block owns a 4-feature
// histogram in LDS; bins come from 8 independent xorshift streams.
// Build: hipcc --offload-arch=gfx950 -O3 -munsafe-fp-atomics -o lds_atomics lds_atomics.hip
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdint>
#define CHECK(x) do { hipError_t e=(x); if(e!=hipSuccess){printf("err %s line %d\n", hipGetErrorString(e), __LINE__); return 1;} } while(0)
// Bins from 8 independent xorshift streams, masked to a power of two.
template<int MODE>
__global__ __launch_bounds__(256) void k(int iters, unsigned long long* out, uint32_t mask) {
  __shared__ unsigned long long h[4*512];
  for (int i=threadIdx.x;i<4*512;i+=256) h[i]=0;
  __syncthreads();
  uint32_t s[8];
  for (int q=0;q<8;++q) s[q] = (blockIdx.x*256+threadIdx.x)*2654435761u + q*40503u + 1u;
  for (int it=0; it<iters; ++it) {
#pragma unroll
    for (int q=0;q<8;++q) {
      s[q] ^= s[q]<<13; s[q] ^= s[q]>>17; s[q] ^= s[q]<<5;
      const uint32_t bin = (s[q]>>8) & mask;
      if (MODE==0) { __hip_atomic_fetch_add(&h[2*bin], (unsigned long long)s[q], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP); __hip_atomic_fetch_add(&h[2*bin+1], (unsigned long long)q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP); }
      if (MODE==1) { unsigned* h32=(unsigned*)h; __hip_atomic_fetch_add(&h32[2*bin], s[q], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP); __hip_atomic_fetch_add(&h32[2*bin+1], (unsigned)q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP); }
      if (MODE==2) { float* hf=(float*)h; unsafeAtomicAdd(&hf[2*bin], (float)s[q]); unsafeAtomicAdd(&hf[2*bin+1], 1.0f); }
      if (MODE==3) { double* hd=(double*)h; unsafeAtomicAdd(&hd[2*bin], (double)s[q]); unsafeAtomicAdd(&hd[2*bin+1], 1.0); }
      if (MODE==4) { __hip_atomic_fetch_add(&h[2*bin], ((unsigned long long)q<<32) | s[q], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP); }
    }
  }
  __syncthreads();
  unsigned long long acc=0; for (int i=threadIdx.x;i<4*512;i+=256) acc+=h[i];
  atomicAdd(out, acc);
}
int main(){
  unsigned long long* d; CHECK(hipMalloc(&d, 8));
  int cu=0, clk=0; hipDeviceGetAttribute(&cu, hipDeviceAttributeMultiprocessorCount, 0); hipDeviceGetAttribute(&clk, hipDeviceAttributeClockRate, 0);
  hipEvent_t a,b; hipEventCreate(&a); hipEventCreate(&b);
  const int blocks = cu*8, iters=128;
  const char* names[]={"2x ds_add_u64","2x ds_add_u32","2x ds_add_f32 (native)","2x ds_add_f64 (native)","1x ds_add_u64 packed"};
  for (uint32_t mask : {255u, 15u}) for (int mode=0; mode<5; ++mode) for (int rep=0; rep<2; ++rep) {
    hipEventRecord(a);
    switch(mode){case 0: hipLaunchKernelGGL(k<0>,dim3(blocks),dim3(256),0,0,iters,d,mask);break;
                 case 1: hipLaunchKernelGGL(k<1>,dim3(blocks),dim3(256),0,0,iters,d,mask);break;
                 case 2: hipLaunchKernelGGL(k<2>,dim3(blocks),dim3(256),0,0,iters,d,mask);break;
                 case 3: hipLaunchKernelGGL(k<3>,dim3(blocks),dim3(256),0,0,iters,d,mask);break;
                 case 4: hipLaunchKernelGGL(k<4>,dim3(blocks),dim3(256),0,0,iters,d,mask);break;}
    hipEventRecord(b); CHECK(hipEventSynchronize(b));
    float ms; hipEventElapsedTime(&ms,a,b);
    if (rep==1) { double upd=(double)blocks*256*iters*8; printf("bins %3u %-24s %7.3f ms  %6.2f updates/clk/CU\n", mask+1, names[mode], ms, upd/(ms*1e-3)/(clk*1e3)/cu); }
  }
  return 0;
}
