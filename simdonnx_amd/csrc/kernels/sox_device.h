// Device-side helpers shared by the gfx950 kernels: storage types, activation math.
//
// The activation math restates the reference's shared formulas so GPU and CPU agree to float
// rounding: exp by the Cephes-style 2^n * degree-5 polynomial with hi/lo ln2 split and clamp
// [-87.3, 88.7], erf by Abramowitz-Stegun 7.1.26, GELU = 0.5x(1 + erf(x/sqrt2))
// (Kernels/SimdMath.cs:121-168; the GPU shaders use the same A&S erf, Shaders/conv_cm.comp:104-111).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../../include/sox_abi.h"

typedef _Float16 half_t;
typedef half_t half8 __attribute__((ext_vector_type(8)));
typedef half_t half4 __attribute__((ext_vector_type(4)));
typedef half_t half2v __attribute__((ext_vector_type(2)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef float float16v __attribute__((ext_vector_type(16)));
// bfloat16 storage (the bf16 graph mode): conversions from fp32 round to nearest even
// (v_cvt_pk_bf16_f32), to fp32 are exact
typedef __bf16 bf16_t;
typedef bf16_t bf16x8 __attribute__((ext_vector_type(8)));
typedef bf16_t bf16x4 __attribute__((ext_vector_type(4)));
typedef bf16_t bf16x2 __attribute__((ext_vector_type(2)));

// N-element vector of a 16-bit storage type
template <typename T, int N> struct VecN {
    typedef T type __attribute__((ext_vector_type(N)));
};
template <typename T, int N> using vec_t = typename VecN<T, N>::type;

#define SOX_DEV static __device__ __forceinline__

SOX_DEV float sox_exp(float x) {
    x = fmaxf(x, -87.3f);
    x = fminf(x, 88.7f);
    float fx = __builtin_fmaf(x, 1.4426950408889634f, 0.5f);
    float nf = floorf(fx);
    float r = __builtin_fmaf(nf, -0.693359375f, x);
    r = __builtin_fmaf(nf, 0.00021219444005469058f, r);
    float p = 1.9875691500e-4f;
    p = __builtin_fmaf(p, r, 1.3981999507e-3f);
    p = __builtin_fmaf(p, r, 8.3334519073e-3f);
    p = __builtin_fmaf(p, r, 4.1665795894e-2f);
    p = __builtin_fmaf(p, r, 1.6666665459e-1f);
    p = __builtin_fmaf(p, r, 5.0000001201e-1f);
    float y = __builtin_fmaf(p, r * r, r) + 1.0f;
    int ni = (int)nf + 127;
    return y * __int_as_float(ni << 23);
}

// exp for results stored in 16 bits (softmax numerators of the attention kernels): the hardware exp2
// on x log2(e), about 1 ulp of fp32 plus the argument's rounding (|x| 2^-24), far below 16-bit rounding
SOX_DEV float exp16(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }

SOX_DEV float sox_sigmoid(float x) { return 1.0f / (1.0f + sox_exp(-x)); }

SOX_DEV float sox_erf(float x) {
    float ax = fabsf(x);
    float t = 1.0f / __builtin_fmaf(0.3275911f, ax, 1.0f);
    float p = 1.061405429f;
    p = __builtin_fmaf(p, t, -1.453152027f);
    p = __builtin_fmaf(p, t, 1.421413741f);
    p = __builtin_fmaf(p, t, -0.284496736f);
    p = __builtin_fmaf(p, t, 0.254829592f);
    float y = 1.0f - (p * t) * sox_exp(-(ax * ax));
    return copysignf(y, x);
}

SOX_DEV float sox_gelu(float x) { return (0.5f * x) * (1.0f + sox_erf(x * 0.70710678118654752f)); }

// ActivationKind epilogue (Kernels/Nhwc.cs:91-99).
SOX_DEV float sox_act(float v, int act) {
    switch (act) {
        case SOX_ACT_RELU: return fmaxf(v, 0.0f);
        case SOX_ACT_SIGMOID: return sox_sigmoid(v);
        case SOX_ACT_GELU: return sox_gelu(v);
        case SOX_ACT_HARDSWISH: return v * fminf(fmaxf(__builtin_fmaf(v, 1.0f / 6.0f, 0.5f), 0.0f), 1.0f);
        case SOX_ACT_SWISH: return v * sox_sigmoid(v);
        default: return v;
    }
}

// GELU for 16-bit outputs, with one transcendental per element:
//   gelu(x) = x Phi(x) = max(x, 0) - a Q(a),  a = |x|,  Q(a) = 1 - Phi(a),
//   Q(a) = 2^L(a), L a degree-6 polynomial in a on [0, 5.5] (a is capped at 5.5, where a Q(a) < 1.1e-7:
//   below every fp16 / bf16 output's resolution next to max(x, 0), so x = +-inf gives +inf / 0).
// L is the least-squares fit of log2(1 - Phi(a)) on [0, 5.5], reweighted toward the minimax error
// (max |error of L| 3.7e-5). Against the exact erf-GELU in float64 its float32 evaluation is off by at
// most 3.9e-6 absolute and 2.7e-5 relative (|gelu| >= 1e-3): every fp16 value in [-8, 8] rounds to
// within 0.55 ulp of the exact GELU, every bf16 value to within 0.51 ulp. The clamp and the ReLU are
// one v_med3_f32 each (no canonicalising max). Cost: 10 full-rate instructions and one exp2, against
// 15 and an exp2 plus a reciprocal for the A&S form of sox_gelu (v_rcp_f32 / v_exp_f32 issue at a
// quarter of the rate).
// In two halves of about five instructions each (gelu_fast_lo: the clamp and the polynomial's first
// three steps; gelu_fast_hi: the rest), for kernels that spread the work between matrix-core
// instructions; gelu_fast is the two in a row, so every kernel gets the same bits.
SOX_DEV void gelu_fast_lo(float x, float& a, float& l) {
    a = __builtin_amdgcn_fmed3f(fabsf(x), 0.0f, 5.5f);
    l = 2.614348522911314e-05f;
    l = __builtin_fmaf(l, a, -0.0006609178963117301f);
    l = __builtin_fmaf(l, a, 0.007488713134080172f);
    l = __builtin_fmaf(l, a, -0.05197449028491974f);
}
SOX_DEV float gelu_fast_hi(float x, float a, float l) {
    l = __builtin_fmaf(l, a, -0.4603187143802643f);
    l = __builtin_fmaf(l, a, -1.150593876838684f);
    l = __builtin_fmaf(l, a, -1.000033974647522f);
    return __builtin_fmaf(-a, __builtin_amdgcn_exp2f(l), __builtin_amdgcn_fmed3f(x, 0.0f, __builtin_inff()));
}
SOX_DEV float gelu_fast(float x) {
    float a, l;
    gelu_fast_lo(x, a, l);
    return gelu_fast_hi(x, a, l);
}

// Four fp32 results as rounded to fp32, before their conversion to 16 bits: without the empty asm the
// compiler may fold the last fma or add and the conversion into one mixed-precision op
// (v_fma_mixlo_f16) that rounds once, where the unfused kernels round to fp32 and then to 16 bits.
SOX_DEV void fp32_rounded(float4v& v) { asm volatile("" : "+v"(v)); }
SOX_DEV float fp32_value(float v) {  // the same for one value: (T)fp32_value(f) rounds f to fp32 first
    asm volatile("" : "+v"(v));
    return v;
}

// The split transformer MLP's outputs, four columns: act(b2 + part[0] + .. + part[parts - 1] (+ res)),
// summed in part order in fp32. sox_mlp_sum_* and the fused qkv-attention's row load both finish the
// MLP with it, so the two give the same bits. pv holds the parts' float4s, b4 the bias (or zeros), r the
// residual when has_r.
template <typename T>
SOX_DEV vec_t<T, 4> mlp_out4(const float4v (&pv)[4], int parts, float4v b4, vec_t<T, 4> r, bool has_r, int act) {
    float4v v = b4;
#pragma unroll
    for (int q = 0; q < 4; q++)
        if (q < parts) v += pv[q];
    float4v o;
#pragma unroll
    for (int e = 0; e < 4; e++) o[e] = sox_act(has_r ? v[e] + (float)r[e] : v[e], act);
    fp32_rounded(o);
    return __builtin_convertvector(o, vec_t<T, 4>);
}

// A LayerNorm folded into a Gemm (gamma-scaled weights W', c = column sums of W', b' = b + beta W):
// rstd from the row's sum of squares over K values, then rstd (acc - mean c) + b'. The fmas are spelled
// out so that every kernel folding a LayerNorm (the ring Gemm, the MLP, the fused qkv-attention) rounds
// the same way, whatever the compiler would contract in each.
SOX_DEV float ln_rstd(float mean, float s2, float inv_k, float eps) {
    return __builtin_amdgcn_rsqf(fmaxf(__builtin_fmaf(s2, inv_k, -(mean * mean)), 0.0f) + eps);
}
SOX_DEV float ln_out(float acc, float mean, float rstd, float c, float b) {
    return __builtin_fmaf(rstd, __builtin_fmaf(-mean, c, acc), b);
}

SOX_DEV float act_fast(float v, int act) { return act == SOX_ACT_GELU ? gelu_fast(v) : sox_act(v, act); }

// 32x32x16 matrix-core step for either 16-bit storage type, fp32 accumulation
SOX_DEV float16v mfma32x32x16(half8 a, half8 b, float16v c) { return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0); }
SOX_DEV float16v mfma32x32x16(bf16x8 a, bf16x8 b, float16v c) { return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0); }
SOX_DEV float4v mfma16x16x32(half8 a, half8 b, float4v c) { return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0); }
SOX_DEV float4v mfma16x16x32(bf16x8 a, bf16x8 b, float4v c) { return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0); }

SOX_DEV float sox_ew(float a, float b, int op) {
    switch (op) {
        case 0: return a + b;
        case 1: return a - b;
        case 2: return a * b;
        default: return a / b;
    }
}

template <typename T> SOX_DEV float to_f(T v) { return (float)v; }
template <typename T> SOX_DEV T from_f(float v) { return (T)v; }

// Reflect padding (no edge repeat): the index folds with period 2*dim - 2, in O(1) for any i.
SOX_DEV int sox_reflect(int i, int dim) {
    if (dim <= 1) return 0;
    const int period = 2 * dim - 2;
    i = abs(i) % period;
    return i < dim ? i : period - i;
}

// Source index along one axis, -1 for a constant-pad position (Kernels/Nhwc.cs:72-80).
SOX_DEV int sox_src_index(int s, int len, bool reflect) {
    if ((unsigned)s < (unsigned)len) return s;
    return reflect ? sox_reflect(s, len) : -1;
}
