// bf16 instances of the implicit-GEMM Conv2d / ConvTranspose ring (gemm_ring.h) for bf16 graphs: the
// tilings of the fp16 table (conv_ring.hip), v_mfma_f32_32x32x16_bf16, bf16 storage.
#include "gemm_ring.h"

SOX_CONV(sox_conv_bf16_128x32_k32s4, bf16_t, 128, 32, 32, 32, 32, 4, 4, 2, 4)
SOX_CONV(sox_conv_bf16_64x64_k32s4, bf16_t, 64, 64, 32, 32, 32, 4, 4, 2, 4)
SOX_CONV(sox_conv_bf16_128x64_k32s4, bf16_t, 128, 64, 32, 64, 32, 4, 4, 2, 4)
SOX_CONV(sox_conv_bf16_128x128_k32s4, bf16_t, 128, 128, 32, 64, 64, 4, 4, 2, 4)
SOX_CONV(sox_conv_bf16_64x64_k64s4, bf16_t, 64, 64, 64, 32, 32, 4, 4, 2, 4)
SOX_CONV(sox_conv_bf16_128x64_k64s3, bf16_t, 128, 64, 64, 64, 32, 3, 4, 1, 4)
SOX_CONV(sox_conv_bf16_128x32_k64s6, bf16_t, 128, 32, 64, 32, 32, 6, 4, 1, 4)
SOX_CONV(sox_conv_bf16_64x64_k64s8, bf16_t, 64, 64, 64, 32, 32, 8, 4, 1, 4)
SOX_CONV(sox_conv_bf16_128x64_k64s5, bf16_t, 128, 64, 64, 64, 32, 5, 4, 1, 4)
// large convs (many output pixels, K >= 1024): the headline Gemm's 8-wave tilings, LDS-staged epilogue
SOX_CONV_E(sox_conv_bf16_256x128_w8k64s2, bf16_t, 256, 128, 64, 64, 64, 2, 8, 1, 4)
SOX_CONV_L(sox_conv_bf16_256x256_w8k64s2, bf16_t, 256, 256, 64, 128, 64, 2, 8, 1, 4, 2)
