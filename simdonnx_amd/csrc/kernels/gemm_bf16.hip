// bf16 instances of the dense Gemm ring (gemm_ring.h) for bf16 graphs: the default tilings of the
// fp16 table (gemm.hip), v_mfma_f32_32x32x16_bf16 with fp32 accumulation, bf16 storage.
#include "gemm_ring.h"

SOX_GEMM_E(sox_gemm_bf16_256x192_w8k64s2, bf16_t, 256, 192, 64, 64, 96, 2, 8, 1, 4)
SOX_GEMM_E(sox_gemm_bf16_256x128_w8k64s2, bf16_t, 256, 128, 64, 64, 64, 2, 8, 1, 4)
SOX_GEMM(sox_gemm_bf16_128x128_k64s2, bf16_t, 128, 128, 64, 64, 64, 2, 4, 2, 4)
SOX_GEMM(sox_gemm_bf16_128x64_k64s2, bf16_t, 128, 64, 64, 64, 32, 2, 4, 3, 4)
SOX_GEMM_E(sox_gemm_bf16_64x64_k64s4, bf16_t, 64, 64, 64, 32, 32, 4, 4, 2, 4)
SOX_GEMM_LN(sox_gemm_ln_bf16_256x128_w8k64s2, bf16_t, 256, 128, 64, 64, 64, 2, 8, 1, 4, true)
SOX_GEMM_LN(sox_gemm_ln_bf16_128x128_k64s2, bf16_t, 128, 128, 64, 64, 64, 2, 4, 2, 4, false)
SOX_GEMM_LN(sox_gemm_ln_bf16_128x64_k64s2, bf16_t, 128, 64, 64, 64, 32, 2, 4, 3, 4, false)
SOX_GEMM_LN(sox_gemm_ln_bf16_64x64_k64s4, bf16_t, 64, 64, 64, 32, 32, 4, 4, 2, 4, true)
