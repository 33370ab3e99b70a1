#include <hip/hip_runtime.h>
#include <stdint.h>
__device__ __forceinline__ void load_lds16_async(const float* g, const float* lds) {
    const uint32_t a = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds);
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" :: "v"(g), "s"(a) : "memory", "m0");
}
__device__ __forceinline__ void wait_barrier() { asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
__global__ __launch_bounds__(256) void k(const float* g, float* out, int nk) {
    __shared__ __attribute__((aligned(16))) float lds[2][1024 * 4];
    const int w = threadIdx.x >> 6;
    float acc = 0;
    load_lds16_async(g + threadIdx.x * 4, &lds[0][w * 256]);
    for (int kt = 0; kt < nk; ++kt) {
        wait_barrier();
        if (kt + 1 < nk) load_lds16_async(g + ((kt + 1) * 1024 + threadIdx.x) * 4, &lds[(kt + 1) & 1][w * 256]);
        const float4 v = *reinterpret_cast<const float4*>(&lds[kt & 1][(threadIdx.x ^ 5) * 4]);
        acc += v.x * v.y + v.z * v.w;
    }
    out[threadIdx.x] = acc;
}
