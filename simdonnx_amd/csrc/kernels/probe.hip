// Throughput probes of the CU's LDS paths (measurement kernels; bench.py --only lds_peak). They bound
// what the LDS-fed kernels can reach: the fragment reads of the Gemm ring (ds_read_b128) and its
// global -> LDS slice loads (global_load_lds_dwordx4).
#include "sox_device.h"

#define LDS_PTR(p) ((__attribute__((address_space(3))) void*)(p))
typedef float f4v __attribute__((ext_vector_type(4)));

// 16 waves x 16 reads of 1 KiB in flight: each wave reads 16 KiB per round at consecutive 16-byte
// lane addresses (no bank conflicts), 8 rounds rotating through 64 KiB of LDS; the reads are inline
// ds_read_b128 so the compiler cannot narrow them, and the sum of one component keeps them live.
extern "C" __global__ void __launch_bounds__(1024) sox_probe_lds_read(sox_lds_probe_args p) {
    __shared__ __attribute__((aligned(1024))) unsigned char lds[65536];
    const int t = threadIdx.x, lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6);
    for (int i = t; i < 65536 / 16; i += blockDim.x) ((f4v*)lds)[i] = (f4v){(float)i, 1.0f, 2.0f, 3.0f};
    __syncthreads();
    const unsigned base = (unsigned)((wave & 7) * 8192 + lane * 16);
    float s = 0.0f;
    for (int it = 0; it < p.iters; it++) {
        f4v v[16];
#pragma unroll
        for (int u = 0; u < 16; u++) {
            const unsigned a = (unsigned)(uintptr_t)LDS_PTR(lds + ((base + (u + (it & 7)) * 1024) & 65535));
            asm volatile("ds_read_b128 %0, %1" : "=v"(v[u]) : "v"(a));
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
        for (int u = 0; u < 16; u++) s += v[u][0];
    }
    p.out[blockIdx.x * blockDim.x + t] = s;
}

// 16 waves x 8 global_load_lds_dwordx4 (1 KiB each) per round, from workgroup b's 64 KiB slice
// (b mod 64) of src into 64 KiB of LDS; one vmcnt(0) at the end.
extern "C" __global__ void __launch_bounds__(1024) sox_probe_lds_dma(sox_lds_probe_args p) {
    __shared__ __attribute__((aligned(1024))) unsigned char lds[65536];
    const int t = threadIdx.x, lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const unsigned char* src = (const unsigned char*)p.src + (long)(blockIdx.x % 64) * 65536;
    for (int it = 0; it < p.iters; it++) {
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int off = ((wave * 8 + u) * 1024) & 65535;
            __builtin_amdgcn_global_load_lds(src + off + lane * 16, LDS_PTR(lds + off), 16, 0, 0);
        }
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    p.out[blockIdx.x * blockDim.x + t] = ((const float*)lds)[t];
}
