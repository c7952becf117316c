// Dense fp16 Gemm instances of the LDS-DMA persistent ring (gemm_ring.h).
#include "gemm_ring.h"

// name: BMxBN tile, kBK slice depth, sSTAGES, wNW waves (4 when absent); SOX_GEMM_E: epilogue through LDS
SOX_GEMM(sox_gemm_f16_256x192_k32s5, half_t, 256, 192, 32, 128, 96, 5, 4, 1, 4)
SOX_GEMM(sox_gemm_f16_256x192_k32s4, half_t, 256, 192, 32, 128, 96, 4, 4, 1, 4)
SOX_GEMM_E(sox_gemm_f16_256x192_w8k64s2, half_t, 256, 192, 64, 64, 96, 2, 8, 1, 4)
SOX_GEMM_E(sox_gemm_f16_128x192_k32s3, half_t, 128, 192, 32, 64, 96, 3, 4, 2, 4)
SOX_GEMM(sox_gemm_f16_256x256_w8k32s4, half_t, 256, 256, 32, 128, 64, 4, 8, 1, 4)
SOX_GEMM(sox_gemm_f16_256x256_w8k64s2, half_t, 256, 256, 64, 128, 64, 2, 8, 1, 4)
SOX_GEMM(sox_gemm_f16_256x128_k32s3, half_t, 256, 128, 32, 128, 64, 3, 4, 2, 4)
SOX_GEMM(sox_gemm_f16_256x128_k32s5, half_t, 256, 128, 32, 128, 64, 5, 4, 1, 4)
SOX_GEMM_E(sox_gemm_f16_256x128_w8k64s2, half_t, 256, 128, 64, 64, 64, 2, 8, 1, 4)
SOX_GEMM(sox_gemm_f16_128x128_k64s2, half_t, 128, 128, 64, 64, 64, 2, 4, 2, 4)
SOX_GEMM(sox_gemm_f16_128x128_k32s4, half_t, 128, 128, 32, 64, 64, 4, 4, 2, 4)
SOX_GEMM(sox_gemm_f16_128x64_k64s2, half_t, 128, 64, 64, 64, 32, 2, 4, 3, 4)
SOX_GEMM(sox_gemm_f16_64x64_k64s2, half_t, 64, 64, 64, 32, 32, 2, 4, 4, 4)
// short K (a few slices): every slice of a tile in flight from the start
SOX_GEMM_E(sox_gemm_f16_64x64_k64s4, half_t, 64, 64, 64, 32, 32, 4, 4, 2, 4)
SOX_GEMM(sox_gemm_f16_128x64_k64s4, half_t, 128, 64, 64, 64, 32, 4, 4, 1, 4)
// A rows through a LayerNorm folded into the Gemm (the default tilings)
SOX_GEMM_LN(sox_gemm_ln_f16_256x128_w8k64s2, half_t, 256, 128, 64, 64, 64, 2, 8, 1, 4, true)
SOX_GEMM_LN(sox_gemm_ln_f16_128x128_k64s2, half_t, 128, 128, 64, 64, 64, 2, 4, 2, 4, false)
SOX_GEMM_LN(sox_gemm_ln_f16_128x64_k64s2, half_t, 128, 64, 64, 64, 32, 2, 4, 3, 4, false)
SOX_GEMM_LN(sox_gemm_ln_f16_64x64_k64s4, half_t, 64, 64, 64, 32, 32, 4, 4, 2, 4, true)

// Matrix-core rate probe (bench.py --only mfma_peak): every wave runs `iters` rounds of four
// independent v_mfma_f32_32x32x16_f16 chains on register operands, with operand bits from a per-lane
// hash (random data: the power the matrix pipe draws, and so its sustained clock, depends on operand
// toggling), and writes its accumulator sum so nothing is dead. No memory traffic in the loop.
extern "C" __global__ void __launch_bounds__(512) sox_probe_mfma_f16(sox_mfma_probe_args p) {
    const uint32_t gid = blockIdx.x * blockDim.x + threadIdx.x;
    half8 a, b;
#pragma unroll
    for (int e = 0; e < 8; e++) {
        uint32_t h = (gid * 8 + e) * 0x9E3779B1u ^ p.seed;
        h ^= h >> 15;
        h *= 0x2C1B3C6Du;
        h ^= h >> 12;
        a[e] = (half_t)((float)(h & 0xffff) * (1.0f / 32768.0f) - 1.0f);
        b[e] = (half_t)((float)(h >> 16) * (1.0f / 32768.0f) - 1.0f);
    }
    float16v c0 = {}, c1 = {}, c2 = {}, c3 = {};
    for (int i = 0; i < p.iters; i++) {
        c0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(b, a, c1, 0, 0, 0);
        c2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, a, c2, 0, 0, 0);
        c3 = __builtin_amdgcn_mfma_f32_32x32x16_f16(b, b, c3, 0, 0, 0);
    }
    float s = 0.0f;
#pragma unroll
    for (int e = 0; e < 16; e++) s += c0[e] + c1[e] + c2[e] + c3[e];
    p.out[gid] = s;
}
