// Transformer MLP in one dispatch: y = act2(GELU(LN(x) . W1 + b1) . W2 + b2 + r), the recognizer's
// ln2 -> fc1 (+GELU) -> fc2 (+ residual Add) chain (Ops.LayerNorm + two Gemm nodes of an SVTR mixer
// block, each the gemm.comp route of Backends/Vulkan/VkGraph.cs:731-793), fp16 storage, fp32 math.
//
// The LayerNorm arrives folded into W1 at graph creation (W1 = gamma-scaled weights, b1 = b + beta W,
// c1 = column sums of W1 as rounded to fp16): LN(x) . W1 + b1 = rstd (x . W1 - mean c1) + b1, with
// the row's mean and rstd from the single-pass sums (E[x^2] - mean^2, as layernorm.comp).
//
// One workgroup (8 waves) per 32 rows; the hidden tile [32][H] never leaves LDS:
//  phase 1: wave w computes hidden blocks w, w + 8, ... (32 columns each) on v_mfma_f32_32x32x16_f16
//           with W1 as the row operand (lane l: row l % 32, 16 hidden columns), every W1 fragment of
//           the wave's blocks loaded up front (weights packed in fragment order at graph creation, so
//           each fragment load is one contiguous KiB per wave); GELU (A&S erf, as the fused Gemm epilogue) and the fp16
//           rounding the unfused graph stores, into LDS.
//  phase 2: wave w < N2 / 32 computes output block w over the H-deep reduction (all W2 fragments of
//           its block loaded before the barrier, the hidden fragments read from LDS), then + b2 +
//           residual, act2, fp16.
// Rows past M re-read row M - 1 and are never stored.
#include <type_traits>

#include "sox_device.h"

template <typename T, int KS1, int HB, int KS2>  // storage type, K1 / 16, H / 32, H / 16
__device__ __forceinline__ void mlp_body(const sox_mlp_args& p) {
    typedef vec_t<T, 8> T8;
    typedef vec_t<T, 4> T4;
    typedef vec_t<T, 2> T2;
    constexpr int H = HB * 32;
    constexpr int HROW = H * 2 + 16;  // LDS bytes per hidden row (16 bytes of padding: conflict-free reads)
    constexpr int PB1 = (HB + 7) / 8;  // hidden blocks per wave
    __shared__ __attribute__((aligned(16))) unsigned char hs[32 * HROW];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6, l32 = lane & 31, hl = lane >> 5;
    const int m0 = blockIdx.x * 32;
    const int row = min(m0 + l32, p.m - 1);
    const T* __restrict__ X = (const T*)p.x;
    const T* __restrict__ W1 = (const T*)p.w1;
    const T* __restrict__ W2 = (const T*)p.w2;

    // ---- phase 1: hidden = GELU(rstd (x . W1 - mean c1) + b1) ----
    T8 a[KS1];
#pragma unroll
    for (int s = 0; s < KS1; s++) a[s] = *(const T8*)(X + (long)row * p.k1 + 16 * s + 8 * hl);
    T8 b[PB1][KS1];
#pragma unroll
    for (int i = 0; i < PB1; i++) {
        const int nb = min(wave + 8 * i, HB - 1);  // a wave past the last block re-reads it
#pragma unroll
        for (int s = 0; s < KS1; s++) b[i][s] = *(const T8*)(W1 + (((long)nb * KS1 + s) * 64 + lane) * 8);
    }
    // the row's sum and sum of squares: this lane's k-half by fp32 dot2, then the other half's lane
    float s1 = 0.0f, s2 = 0.0f;
    {
        const T2 one = {(T)1.0f, (T)1.0f};
#pragma unroll
        for (int s = 0; s < KS1; s++)
#pragma unroll
            for (int h = 0; h < 4; h++) {
                const T2 v = {a[s][2 * h], a[s][2 * h + 1]};
                if constexpr (std::is_same<T, half_t>::value) {
                    s1 = __builtin_amdgcn_fdot2(v, one, s1, false);
                    s2 = __builtin_amdgcn_fdot2(v, v, s2, false);
                } else {
                    s1 = __builtin_amdgcn_fdot2_f32_bf16(v, one, s1, false);
                    s2 = __builtin_amdgcn_fdot2_f32_bf16(v, v, s2, false);
                }
            }
        s1 += __shfl_xor(s1, 32);
        s2 += __shfl_xor(s2, 32);
    }
    const float inv_k = 1.0f / (float)p.k1;
    const float mean = s1 * inv_k;
    const float rstd = ln_rstd(mean, s2, inv_k, p.eps);
    // the wave's blocks interleaved k-step by k-step: independent accumulator chains
    float16v acc1[PB1];
#pragma unroll
    for (int i = 0; i < PB1; i++) acc1[i] = (float16v)0.0f;
#pragma unroll
    for (int s = 0; s < KS1; s++)
#pragma unroll
        for (int i = 0; i < PB1; i++) acc1[i] = mfma32x32x16(b[i][s], a[s], acc1[i]);
#pragma unroll
    for (int i = 0; i < PB1; i++) {
        const int jb = wave + 8 * i;
        if (jb >= HB) break;  // uniform
        const float16v& acc = acc1[i];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int n = jb * 32 + 8 * q + 4 * hl;
            const float4v c4 = *(const float4v*)(p.c1 + n);
            const float4v b4 = *(const float4v*)(p.b1 + n);
            T4 hv;
#pragma unroll
            for (int e = 0; e < 4; e++)
                hv[e] = (T)gelu_fast(ln_out(acc[4 * q + e], mean, rstd, c4[e], b4[e]));
            *(T4*)(hs + l32 * HROW + n * 2) = hv;
        }
    }

    // ---- phase 2: y = act2(hidden . W2 + b2 + r) ----
    const int ob = wave;  // output block of this wave (waves past N2 / 32 only help with phase 1)
    const bool out_wave = ob * 32 < p.n2;
    T8 w2f[KS2];
    if (out_wave) {
#pragma unroll
        for (int s = 0; s < KS2; s++) w2f[s] = *(const T8*)(W2 + (((long)ob * KS2 + s) * 64 + lane) * 8);
    }
    __syncthreads();  // every hidden column written
    if (!out_wave) return;
    // two accumulator chains (even / odd k-steps), added at the end
    float16v acc = (float16v)0.0f, acc_o = (float16v)0.0f;
    const unsigned char* hr = hs + l32 * HROW + 16 * hl;
#pragma unroll
    for (int s = 0; s < KS2; s += 2) {
        const T8 hv = *(const T8*)(hr + 32 * s);
        const T8 hv2 = *(const T8*)(hr + 32 * (s + 1));
        acc = mfma32x32x16(w2f[s], hv, acc);
        acc_o = mfma32x32x16(w2f[s + 1], hv2, acc_o);
    }
    acc += acc_o;
    const int m = m0 + l32;
    if (m >= p.m) return;
    const int act = (p.flags >> 4) & 15;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const int n = ob * 32 + 8 * q + 4 * hl;
        const float4v b4 = (p.flags & 1) ? *(const float4v*)(p.b2 + n) : (float4v)0.0f;
        T4 rv = {};
        if (p.flags & 2) rv = *(const T4*)((const T*)p.res + (long)m * p.n2 + n);
        T4 out;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            float v = acc[4 * q + e] + b4[e];
            if (p.flags & 2) v += (float)rv[e];
            out[e] = (T)sox_act(v, act);
        }
        *(T4*)((T*)p.y + (long)m * p.n2 + n) = out;
    }
}

// ------------------------------------------------------------------------------------------------
// Split form: workgroup (row block of 32, part q of Q) takes hidden blocks q HB/Q .. (q + 1) HB/Q - 1
// and fc2's k-steps over those hidden columns, so a grid of M/32 x Q workgroups shares the weights'
// traffic (each workgroup streams 1/Q of W1 and W2 through its CU) and fills the GPU where M/32 alone
// would not.
//  phase 0: the part's W1 fragments (one hidden block per wave), the wave's W2 fragments, the part's
//           c1 / b1 and the 32 x rows (both into LDS: each is read by several waves) all issued before
//           the first wait.
//  PROJ (sox_mlpqp_*): x itself is the preceding projection Gemm with its residual Add: phase 0 stages
//           the projection's input rows instead, with each wave's Wp fragments, bias and residual; then
//           wave w < K1 / 32 computes x's columns 32 w.. on v_mfma_f32_32x32x16 into LDS (part 0 also
//           stores them: the MLP's residual), and the W2 fragments load after it (registers).
//  phase 1: as sox_mlp_*: the LayerNorm from the row sums, one 32 x 32 hidden block per wave, GELU,
//           rounding to the storage type, into LDS.
//  phase 2: wave w < N2 / 32: output block w over the part's hidden k-steps (two accumulator chains),
//           stored as fp32 to part[q][m][n2]; sox_mlp_sum_* adds the parts, b2 and the residual.
// (The parts meet in a second dispatch: a last-arriver reduction inside this kernel needs agent-scope
// release / acquire fences, which write back and invalidate the XCD's L2 and cost several times the
// second dispatch.)
template <typename T, int KS1, int HB, int KS2, int Q, bool PROJ>  // storage, K1 / 16, H / 32, H / 16, parts
__device__ __forceinline__ void mlp_part_body(const sox_mlp_args& p) {
    typedef vec_t<T, 8> T8;
    typedef vec_t<T, 4> T4;
    typedef vec_t<T, 2> T2;
    constexpr int HBQ = HB / Q, KQ = KS2 / Q, K1 = KS1 * 16, HQ = HBQ * 32;
    static_assert(HB % Q == 0 && HBQ <= 8 && KQ % 2 == 0 && Q <= 4, "a part is at most one hidden block per wave");
    constexpr int HROW = HQ * 2 + 16;   // LDS bytes per hidden row (16 bytes of padding)
    constexpr int XP = K1 + 8;          // x row pitch in LDS, in elements
    constexpr int XC = 32 * K1 / 8;     // 16-byte chunks of the 32 x rows
    constexpr int XI = (XC + 511) / 512;
    __shared__ __attribute__((aligned(16))) unsigned char hs[32 * HROW];
    __shared__ __attribute__((aligned(16))) T xs[32 * XP];   // x rows (PROJ: the projection's input rows)
    __shared__ __attribute__((aligned(16))) T x2s[PROJ ? 32 * XP : 8];  // PROJ: the x rows computed here
    __shared__ __attribute__((aligned(16))) float cb[2][HQ];  // the part's c1 and b1
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6, l32 = lane & 31, hl = lane >> 5;
    const int q = blockIdx.x % Q, m0 = (blockIdx.x / Q) * 32;
    const T* __restrict__ X = (const T*)(PROJ ? p.po : p.x);
    const T* __restrict__ W1 = (const T*)p.w1;
    const T* __restrict__ W2 = (const T*)p.w2;
    const bool hid_wave = wave < HBQ, out_wave = wave * 32 < p.n2;
    const int jb = q * HBQ + wave;  // the wave's hidden block

    // ---- phase 0: every load of the workgroup in flight before the first wait ----
    T8 b[KS1], w2f[KQ];
    if (hid_wave) {
#pragma unroll
        for (int s = 0; s < KS1; s++) b[s] = *(const T8*)(W1 + (((long)jb * KS1 + s) * 64 + lane) * 8);
    }
    auto load_w2 = [&]() __attribute__((always_inline)) {
        if (out_wave) {
#pragma unroll
            for (int s = 0; s < KQ; s++) w2f[s] = *(const T8*)(W2 + (((long)wave * KS2 + q * KQ + s) * 64 + lane) * 8);
        }
    };
    if constexpr (!PROJ) load_w2();
    // PROJ: the projection's weight fragments (its 32 output columns per wave), bias and residual rows
    const bool proj_wave = PROJ && wave * 32 < K1;
    T8 pwf[PROJ ? KS1 : 1];
    float4v pbv[4];
    T4 pxv[4];
    if constexpr (PROJ) {
        if (proj_wave) {
            const int r = min(m0 + l32, p.m - 1);
#pragma unroll
            for (int s = 0; s < KS1; s++)
                pwf[s] = *(const T8*)((const T*)p.pw + (long)(wave * 32 + l32) * K1 + 16 * s + 8 * hl);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int n = wave * 32 + 8 * i + 4 * hl;
                pbv[i] = (p.pflags & 1) ? *(const float4v*)(p.pb + n) : (float4v)0.0f;
                pxv[i] = *(const T4*)((const T*)p.px + (long)r * K1 + n);
            }
        }
    }
    {
        T8 xv[XI];
        float4v cv;
        constexpr int CQ = HQ / 4;  // float4s of one of c1, b1 over the part
        const bool cl = t < 2 * CQ;
        if (cl) cv = *(const float4v*)((t < CQ ? p.c1 : p.b1) + q * HQ + 4 * (t % CQ));
#pragma unroll
        for (int u = 0; u < XI; u++) {
            const int i = t + 512 * u, r = i / (K1 / 8), c = i - r * (K1 / 8);
            if (i < XC) xv[u] = *(const T8*)(X + (long)min(m0 + r, p.m - 1) * p.k1 + 8 * c);
        }
        if (cl) *(float4v*)(&cb[t / CQ][4 * (t % CQ)]) = cv;
#pragma unroll
        for (int u = 0; u < XI; u++) {
            const int i = t + 512 * u, r = i / (K1 / 8), c = i - r * (K1 / 8);
            if (i < XC) *(T8*)(xs + r * XP + 8 * c) = xv[u];
        }
    }
    __syncthreads();

    // ---- PROJ: x = po . Wp^T + pb + px, the projection Gemm with its residual Add, for the 32 rows
    // (accumulators from the bias, k-steps ascending, rounded to fp32 and then to 16 bits) ----
    if constexpr (PROJ) {
        if (proj_wave) {
            float16v acc;
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int e = 0; e < 4; e++) acc[4 * i + e] = pbv[i][e];
            const T* ar = xs + l32 * XP + 8 * hl;
#pragma unroll
            for (int s = 0; s < KS1; s++) acc = mfma32x32x16(pwf[s], *(const T8*)(ar + 16 * s), acc);
            const int m = m0 + l32;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int n = wave * 32 + 8 * i + 4 * hl;
                float4v f;
#pragma unroll
                for (int e = 0; e < 4; e++) f[e] = acc[4 * i + e] + (float)pxv[i][e];
                fp32_rounded(f);
                const T4 h = __builtin_convertvector(f, T4);
                *(T4*)(x2s + l32 * XP + n) = h;
                if (q == 0 && m < p.m) *(T4*)((T*)p.xout + (long)m * K1 + n) = h;
            }
        }
        load_w2();
        __syncthreads();
    }

    // ---- phase 1: hidden = GELU(rstd (x . W1 - mean c1) + b1), the part's columns ----
    if (hid_wave) {
        const T* ar = (PROJ ? x2s : xs) + l32 * XP + 8 * hl;
        float s1 = 0.0f, s2 = 0.0f;
        float16v acc = (float16v)0.0f;
        const T2 one = {(T)1.0f, (T)1.0f};
#pragma unroll
        for (int s = 0; s < KS1; s++) {
            const T8 a = *(const T8*)(ar + 16 * s);
            acc = mfma32x32x16(b[s], a, acc);
#pragma unroll
            for (int h = 0; h < 4; h++) {
                const T2 v = {a[2 * h], a[2 * h + 1]};
                if constexpr (std::is_same<T, half_t>::value) {
                    s1 = __builtin_amdgcn_fdot2(v, one, s1, false);
                    s2 = __builtin_amdgcn_fdot2(v, v, s2, false);
                } else {
                    s1 = __builtin_amdgcn_fdot2_f32_bf16(v, one, s1, false);
                    s2 = __builtin_amdgcn_fdot2_f32_bf16(v, v, s2, false);
                }
            }
        }
        s1 += __shfl_xor(s1, 32);
        s2 += __shfl_xor(s2, 32);
        const float inv_k = 1.0f / (float)K1;
        const float mean = s1 * inv_k;
        const float rstd = ln_rstd(mean, s2, inv_k, p.eps);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int n = wave * 32 + 8 * i + 4 * hl;  // the part's hidden column
            const float4v c4 = *(const float4v*)(&cb[0][n]), b4 = *(const float4v*)(&cb[1][n]);
            T4 hv;
#pragma unroll
            for (int e = 0; e < 4; e++) hv[e] = (T)gelu_fast(ln_out(acc[4 * i + e], mean, rstd, c4[e], b4[e]));
            *(T4*)(hs + l32 * HROW + n * 2) = hv;
        }
    }
    __syncthreads();  // every hidden column of the part written

    // ---- phase 2: the part's share of hidden . W2, fp32 ----
    if (out_wave) {
        float16v acc = (float16v)0.0f, acc_o = (float16v)0.0f;
        const unsigned char* hr = hs + l32 * HROW + 16 * hl;
#pragma unroll
        for (int s = 0; s < KQ; s += 2) {
            acc = mfma32x32x16(w2f[s], *(const T8*)(hr + 32 * s), acc);
            acc_o = mfma32x32x16(w2f[s + 1], *(const T8*)(hr + 32 * (s + 1)), acc_o);
        }
        const int m = m0 + l32;
        if (m < p.m) {
            float* dst = p.part + ((long)q * p.m + m) * p.n2 + wave * 32 + 4 * hl;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                float4v v;
#pragma unroll
                for (int e = 0; e < 4; e++) v[e] = acc[4 * i + e] + acc_o[4 * i + e];
                *(float4v*)(dst + 8 * i) = v;
            }
        }
    }
}


// y = act2(b2 + part[0] + ... + part[parts - 1] + res), four consecutive outputs per thread
template <typename T>
__device__ __forceinline__ void mlp_sum_body(const sox_mlp_args& p) {
    typedef vec_t<T, 4> T4;
    const long i = ((long)blockIdx.x * blockDim.x + threadIdx.x) * 4, total = (long)p.m * p.n2;
    if (i >= total) return;
    const int n = (int)(i % p.n2);
    float4v pv[4];
#pragma unroll
    for (int q = 0; q < 4; q++)
        if (q < p.parts) pv[q] = *(const float4v*)(p.part + q * total + i);
    const float4v b4 = (p.flags & 1) ? *(const float4v*)(p.b2 + n) : (float4v)0.0f;
    T4 r = {};
    if (p.flags & 2) r = *(const T4*)((const T*)p.res + i);
    *(T4*)((T*)p.y + i) = mlp_out4<T>(pv, p.parts, b4, r, (p.flags & 2) != 0, (p.flags >> 4) & 15);
}

extern "C" __global__ void __launch_bounds__(256) sox_mlp_sum_f16(sox_mlp_args p) { mlp_sum_body<half_t>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_mlp_sum_bf16(sox_mlp_args p) { mlp_sum_body<bf16_t>(p); }

// name: K1 x H (inner dim x hidden width); N2 <= 256, a multiple of 32
#define SOX_MLP(K1, H)                                                                                           \
    extern "C" __global__ void __launch_bounds__(512) sox_mlp_f16_k##K1##_h##H(sox_mlp_args p) {                 \
        mlp_body<half_t, K1 / 16, H / 32, H / 16>(p);                                                            \
    }                                                                                                            \
    extern "C" __global__ void __launch_bounds__(512) sox_mlp_bf16_k##K1##_h##H(sox_mlp_args p) {                \
        mlp_body<bf16_t, K1 / 16, H / 32, H / 16>(p);                                                            \
    }
SOX_MLP(192, 768)
SOX_MLP(128, 512)
SOX_MLP(64, 256)

// name: K1 x H, Q parts of the hidden width (a part: at most 8 hidden blocks, an even number of k-steps)
#define SOX_MLPQ(K1, H, Q)                                                                                       \
    extern "C" __global__ void __launch_bounds__(512) sox_mlpq_f16_k##K1##_h##H##_q##Q(sox_mlp_args p) {         \
        mlp_part_body<half_t, K1 / 16, H / 32, H / 16, Q, false>(p);                                             \
    }                                                                                                            \
    extern "C" __global__ void __launch_bounds__(512) sox_mlpq_bf16_k##K1##_h##H##_q##Q(sox_mlp_args p) {        \
        mlp_part_body<bf16_t, K1 / 16, H / 32, H / 16, Q, false>(p);                                             \
    }                                                                                                            \
    extern "C" __global__ void __launch_bounds__(512) sox_mlpqp_f16_k##K1##_h##H##_q##Q(sox_mlp_args p) {        \
        mlp_part_body<half_t, K1 / 16, H / 32, H / 16, Q, true>(p);                                              \
    }                                                                                                            \
    extern "C" __global__ void __launch_bounds__(512) sox_mlpqp_bf16_k##K1##_h##H##_q##Q(sox_mlp_args p) {       \
        mlp_part_body<bf16_t, K1 / 16, H / 32, H / 16, Q, true>(p);                                              \
    }
SOX_MLPQ(192, 768, 3)
SOX_MLPQ(128, 512, 4)
SOX_MLPQ(64, 256, 2)
