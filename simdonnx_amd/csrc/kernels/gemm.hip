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
