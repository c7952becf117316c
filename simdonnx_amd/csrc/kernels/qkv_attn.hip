// LayerNorm -> qkv Gemm -> attention of a transformer block in one dispatch, one workgroup per (image, head)
// (the SVTR mixer's Ops.LayerNorm, qkv Gemm and attn.comp, Backends/Vulkan/VkGraph.cs:719-793 and 1029-1049;
// the LayerNorm arrives folded into the qkv weights at graph creation). 16-bit storage, fp32 math. The
// workgroup computes only its head's 96 qkv columns (its q, k and v), which never leave LDS, and writes
// the head's attention output; the proj Gemm and its residual Add stay a Gemm dispatch.
//
// Each phase does the arithmetic of the kernel it replaces, in the same order, and rounds where that
// kernel stores, so the output equals the two-dispatch path's bit for bit:
//  phase 0: the head's 96 rows of W' (its q, k and v columns, gamma-scaled), their column sums and
//           biases, and the image's x rows (t <= 96 tokens; rows past t zero) into LDS, all loads issued
//           before the first wait.
//  phase A: q, k, v = rstd (x . W' - mean c) + b' (sox_gemm_ln_*: v_mfma_f32_32x32x16, accumulators from
//           0, the row's sum and sum of squares from the A fragments by fp32 dot2, k-step by k-step),
//           rounded into LDS. Nine waves: wave w takes 32 rows (w / 3) of one of q, k, v (w % 3).
//  phase B: V^T staged from the v columns (keys past t zero), then per 16 queries the softmax attention
//           of sox_attn_*_mfma (v_mfma_f32_16x16x32, scores and softmax in registers, P as the A operand
//           at the key permutation V^T is read with).
// LDS: x rows, W' rows, the head's qkv rows and V^T, 102 KiB at dim 192; rows padded by 16 bytes.
#include <type_traits>

#include "sox_device.h"

template <typename T, int DIM>
__device__ __forceinline__ void qkv_attn_body(const sox_qkvattn_args& p) {
    // no contraction (as sox_attn_*_mfma): the softmax's scaled score and its distance to the row max
    // round separately; the LayerNorm epilogue's fmas are explicit (ln_out)
#pragma clang fp contract(off)
    typedef vec_t<T, 8> T8;
    typedef vec_t<T, 4> T4;
    typedef vec_t<T, 2> T2;
    constexpr int H = DIM / 32, XP = DIM + 8, QP = 96 + 8, TM = 96, VP = TM + 8, KS = DIM / 16;
    constexpr int NJ = TM / 16, NC = TM / 32, NT = 576;
    constexpr int XI = TM * (DIM / 8) / NT;  // x chunks per thread
    static_assert(TM * (DIM / 8) % NT == 0, "x rows split evenly over the threads");
    constexpr int WI = 96 * (DIM / 8) / NT;   // W' chunks per thread
    static_assert(96 * (DIM / 8) % NT == 0, "W' rows split evenly over the threads");
    __shared__ __attribute__((aligned(16))) T xs[TM * XP];  // x rows
    __shared__ __attribute__((aligned(16))) T ws[96 * XP];  // the head's W' rows: q, k, v columns
    __shared__ __attribute__((aligned(16))) T qs[TM * QP];  // the head's q | k | v per row
    __shared__ __attribute__((aligned(16))) T vt[32 * VP];  // V^T
    __shared__ __attribute__((aligned(16))) float cb[2][96];  // the head's column sums and biases
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, l32 = lane & 31, hl = lane >> 5;
    const int l16 = lane & 15, g = lane >> 4;
    const int b = blockIdx.x / H, h = blockIdx.x - b * H, t = p.t;
    const T* __restrict__ x = (const T*)p.x + (long)b * t * DIM;
    const T8 zero8 = (T8)(T)0.0f;
    // head column r (0..95: 32 of q, then k, then v) -> its qkv column
    auto qkv_col = [&](int r) { return (r >> 5) * DIM + h * 32 + (r & 31); };
    // wave roles in phase A: rows mb * 32.., columns of q (nb 0), k (1) or v (2)
    const int mb = wave / 3, nb = wave - 3 * mb;
    const bool active = mb * 32 < t;

    // ---- phase 0: the head's W' rows, column sums and biases, and the x rows, in one batch ----
    {
        T8 wv[WI];
        float4v cv = (float4v)0.0f;
#pragma unroll
        for (int u = 0; u < WI; u++) {
            const int i = tid + NT * u, r = i / (DIM / 8), c = i - r * (DIM / 8);
            wv[u] = *(const T8*)((const T*)p.wqkv + (long)qkv_col(r) * p.kpad + 8 * c);
        }
        const int cj = tid / 24, ck = tid - 24 * cj;  // threads 0..47: 4 columns of the sums (0) or biases (1)
        if (tid < 48 && (cj == 0 || (p.flags & 2)))
            cv = *(const float4v*)((cj == 0 ? p.cqkv : p.bqkv) + qkv_col(4 * ck));
        T8 xv[XI];
#pragma unroll
        for (int u = 0; u < XI; u++) {
            const int i = tid + NT * u, r = i / (DIM / 8), c = i - r * (DIM / 8);
            xv[u] = r < t ? *(const T8*)(x + (long)r * DIM + 8 * c) : zero8;
        }
#pragma unroll
        for (int u = 0; u < XI; u++) {
            const int i = tid + NT * u, r = i / (DIM / 8), c = i - r * (DIM / 8);
            *(T8*)(xs + r * XP + 8 * c) = xv[u];
        }
#pragma unroll
        for (int u = 0; u < WI; u++) {
            const int i = tid + NT * u, r = i / (DIM / 8), c = i - r * (DIM / 8);
            *(T8*)(ws + r * XP + 8 * c) = wv[u];
        }
        if (tid < 48) *(float4v*)(&cb[cj][4 * ck]) = cv;
    }
    __syncthreads();

    // ---- phase A: the wave's 32 x 32 block of the head's q, k or v, the LayerNorm folded in ----
    if (active) {
        const T* ar = xs + (mb * 32 + l32) * XP + 8 * hl;
        const T* wr = ws + (nb * 32 + l32) * XP + 8 * hl;
        float s1 = 0.0f, s2 = 0.0f;
        float16v acc = (float16v)0.0f;
        const T2 one = {(T)1.0f, (T)1.0f};
#pragma unroll
        for (int s = 0; s < KS; s++) {
            const T8 a = *(const T8*)(ar + 16 * s);
            acc = mfma32x32x16(*(const T8*)(wr + 16 * s), a, acc);
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const T2 v = {a[2 * e], a[2 * e + 1]};
                if constexpr (std::is_same<T, half_t>::value) {
                    s1 = __builtin_amdgcn_fdot2(v, one, s1, false);
                    s2 = __builtin_amdgcn_fdot2(v, v, s2, false);
                } else {
                    s1 = __builtin_amdgcn_fdot2_f32_bf16(v, one, s1, false);
                    s2 = __builtin_amdgcn_fdot2_f32_bf16(v, v, s2, false);
                }
            }
        }
        s1 += __shfl_xor(s1, 32);  // lanes l and l + 32 hold the two k-halves of a row
        s2 += __shfl_xor(s2, 32);
        const float inv_k = 1.0f / (float)DIM;
        const float mu = s1 * inv_k;
        const float rs = ln_rstd(mu, s2, inv_k, p.eps);
        T* qr = qs + (mb * 32 + l32) * QP + nb * 32 + 4 * hl;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const float4v cv = *(const float4v*)(&cb[0][nb * 32 + 8 * q + 4 * hl]);
            const float4v bv = *(const float4v*)(&cb[1][nb * 32 + 8 * q + 4 * hl]);
            float4v f;
#pragma unroll
            for (int e = 0; e < 4; e++) f[e] = ln_out(acc[4 * q + e], mu, rs, cv[e], bv[e]);
            fp32_rounded(f);
            *(T4*)(qr + 8 * q) = __builtin_convertvector(f, T4);
        }
    }
    __syncthreads();

    // ---- phase B: V^T (keys past t zero), then attention per 16 queries ----
    if (tid < TM * 4) {
        const int s = tid >> 2, c = tid & 3;
        const T8 v = s < t ? *(const T8*)(qs + s * QP + 64 + 8 * c) : zero8;
#pragma unroll
        for (int e = 0; e < 8; e++) vt[(8 * c + e) * VP + s] = v[e];
    }
    __syncthreads();
    const int tb = wave;
    if (tb * 16 >= t) return;
    const int tq = tb * 16 + l16;
    const T8 qf = tq < t ? *(const T8*)(qs + tq * QP + 8 * g) : zero8;
    float4v sc[NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        // key rows past the computed blocks are never written: their scores are masked below, and
        // their MFMA is skipped so no stale LDS bits enter the registers
        if (16 * j < t) {
            const T8 kf = *(const T8*)(qs + (16 * j + l16) * QP + 32 + 8 * g);
            sc[j] = mfma16x16x32(kf, qf, (float4v)0.0f);
        } else {
            sc[j] = (float4v)0.0f;
        }
    }
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < NJ; j++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int s = 16 * j + 4 * g + i;
            const float v = s < t ? sc[j][i] * p.scale : -INFINITY;
            sc[j][i] = v;
            m = fmaxf(m, v);
        }
    m = fmaxf(m, __shfl_xor(m, 16, 64));
    m = fmaxf(m, __shfl_xor(m, 32, 64));
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < NJ; j++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int s = 16 * j + 4 * g + i;
            const float e = s < t ? exp16(sc[j][i] - m) : 0.0f;
            sc[j][i] = e;
            sum += e;
        }
    sum += __shfl_xor(sum, 16, 64);
    sum += __shfl_xor(sum, 32, 64);
    float4v o[2] = {(float4v)0.0f, (float4v)0.0f};
#pragma unroll
    for (int c = 0; c < NC; c++) {
        T8 pa;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            pa[i] = (T)sc[2 * c][i];
            pa[4 + i] = (T)sc[2 * c + 1][i];
        }
#pragma unroll
        for (int jd = 0; jd < 2; jd++) {
            const T* row = vt + (16 * jd + l16) * VP + 32 * c + 4 * g;
            const T4 lo = *(const T4*)row, hi = *(const T4*)(row + 16);
            const T8 vb = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            o[jd] = mfma16x16x32(pa, vb, o[jd]);
        }
    }
    T* __restrict__ out = (T*)p.o + (long)b * t * DIM + h * 32;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int tt = tb * 16 + 4 * g + i;
        const float inv = 1.0f / __shfl(sum, 4 * g + i, 64);
        if (tt < t)
#pragma unroll
            for (int jd = 0; jd < 2; jd++) out[(long)tt * DIM + 16 * jd + l16] = (T)(o[jd][i] * inv);
    }
}

extern "C" __global__ void __launch_bounds__(576) sox_qkvattn_f16_d192(sox_qkvattn_args p) {
    qkv_attn_body<half_t, 192>(p);
}
extern "C" __global__ void __launch_bounds__(576) sox_qkvattn_bf16_d192(sox_qkvattn_args p) {
    qkv_attn_body<bf16_t, 192>(p);
}
