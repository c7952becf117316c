// Dense 16-bit Gemm instances with the epilogue under the matrix-core work (gemm_pp.h): whole
// 256 x 128 tiles, K = 32 NK, bias + none / relu / GELU. Taken only when SIMDONNX_HIP_GEMMPP is set.
#include "gemm_pp.h"

// name: tile, K, activation
SOX_GEMM_PP(sox_gemmpp_f16_256x128_k768_gelu, half_t, 128, 24, SOX_ACT_GELU)
SOX_GEMM_PP(sox_gemmpp_f16_256x128_k768_relu, half_t, 128, 24, SOX_ACT_RELU)
SOX_GEMM_PP(sox_gemmpp_f16_256x128_k768_none, half_t, 128, 24, SOX_ACT_NONE)
SOX_GEMM_PP(sox_gemmpp_bf16_256x128_k768_gelu, bf16_t, 128, 24, SOX_ACT_GELU)
SOX_GEMM_PP(sox_gemmpp_bf16_256x128_k768_relu, bf16_t, 128, 24, SOX_ACT_RELU)
SOX_GEMM_PP(sox_gemmpp_bf16_256x128_k768_none, bf16_t, 128, 24, SOX_ACT_NONE)
