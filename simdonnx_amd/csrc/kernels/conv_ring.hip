// Implicit-GEMM Conv2d / ConvTranspose instances of the LDS-DMA persistent ring (gemm_ring.h).
#include "gemm_ring.h"

// implicit-GEMM Conv2d on the same ring (fp16 NHWC, ic % 8 == 0, constant-0 or reflect padding)
SOX_CONV(sox_conv_f16_128x32_k32s4, half_t, 128, 32, 32, 32, 32, 4, 4, 2, 4)
SOX_CONV(sox_conv_f16_64x64_k32s4, half_t, 64, 64, 32, 32, 32, 4, 4, 2, 4)
SOX_CONV(sox_conv_f16_128x64_k32s4, half_t, 128, 64, 32, 64, 32, 4, 4, 2, 4)
SOX_CONV(sox_conv_f16_128x128_k32s4, half_t, 128, 128, 32, 64, 64, 4, 4, 2, 4)
SOX_CONV(sox_conv_f16_64x64_k64s4, half_t, 64, 64, 64, 32, 32, 4, 4, 2, 4)
SOX_CONV(sox_conv_f16_128x64_k64s3, half_t, 128, 64, 64, 64, 32, 3, 4, 1, 4)
// deep K (3x3 convs over many channels): more slices in flight per workgroup
SOX_CONV(sox_conv_f16_128x32_k64s6, half_t, 128, 32, 64, 32, 32, 6, 4, 1, 4)
SOX_CONV(sox_conv_f16_64x64_k64s8, half_t, 64, 64, 64, 32, 32, 8, 4, 1, 4)
SOX_CONV(sox_conv_f16_128x64_k64s5, half_t, 128, 64, 64, 64, 32, 5, 4, 1, 4)
// large convs (many output pixels, K >= 1024): the headline Gemm's 8-wave tilings, LDS-staged epilogue
SOX_CONV_E(sox_conv_f16_256x128_w8k64s2, half_t, 256, 128, 64, 64, 64, 2, 8, 1, 4)
// 256 output channels: the whole N in one tile (fewer DMA and LDS bytes per MFMA than 256 x 128); its
// LDS-staged epilogue would not fit beside the two 64 KiB stages, so it stores from registers. Each
// slice's DMA goes out in two parts (after the barrier and after the first k-step's MFMAs); its DMA
// rows hold 32-bit input offsets (the launcher routes inputs of fewer than 2^31 elements only)
SOX_CONV_L(sox_conv_f16_256x256_w8k64s2, half_t, 256, 256, 64, 128, 64, 2, 8, 1, 4, 2)
