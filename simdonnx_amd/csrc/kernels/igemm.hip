// Implicit-GEMM Conv2d / Gemm on CDNA4 matrix cores, NHWC, fused bias + residual + activation.
//
// Replaces conv_cm.comp / conv_tile.comp / gemm.comp (Backends/Vulkan/Shaders) for the
// HIP backend. One kernel family covers dense k x k convs (any stride / pad / reflect) and
// Gemm (A as a plain [M][K] matrix): C[M,N] = A[M,K] . W[N,K]^T, with
//   M = n*oh*ow output pixels, N = oc, K = kh*kw*ic in tap-major order (channel fastest),
//   W packed [N][kpad] k-fastest (ConstKind.ConvWT / GemmNK, Engine/Extensions.cs:150-153).
// Epilogue per element: v = acc (+ bias[n]) (+ residual) -> act -> store (conv_cm.comp:326-367).
//
// Tiling: 256 threads = 4 waves (wave64). A workgroup owns a BM x BN output tile; each wave a
// WM x WN sub-tile made of 16x16 MFMA blocks: v_mfma_f32_16x16x32_f16 (fp16 storage, fp32
// accumulation) or v_mfma_f32_16x16x4_f32 (fp32 storage). K is staged through LDS in BK-deep
// slices, double-buffered: the global loads of slice k+1 are in flight while slice k is
// multiplied. LDS rows are padded by 16 bytes so the per-lane 16-byte fragment reads of one
// 16-lane group land in distinct banks.
//
// MFMA operand layout (both instructions): lane l supplies row (l % 16) of A and column (l % 16)
// of B, at the same KPL consecutive k of its group (l / 16); D lane l holds rows
// 4*(l/16) + 0..3 of column (l % 16).
#include "sox_device.h"

template <typename T> struct Mfma;

template <> struct Mfma<half_t> {
    static constexpr int KSTEP = 32;  // k per instruction
    static constexpr int KPL = 8;     // k per lane per instruction
    typedef half8 Frag;
    SOX_DEV static float4v mma(Frag a, Frag b, float4v c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    }
};

template <> struct Mfma<bf16_t> {
    static constexpr int KSTEP = 32;
    static constexpr int KPL = 8;
    typedef bf16x8 Frag;
    SOX_DEV static float4v mma(Frag a, Frag b, float4v c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
};

template <> struct Mfma<float> {
    static constexpr int KSTEP = 4;
    static constexpr int KPL = 1;
    typedef float Frag;
    SOX_DEV static float4v mma(Frag a, Frag b, float4v c) {
        return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
    }
};

// 16-byte global/LDS chunk of T.
template <typename T> struct Chunk {
    static constexpr int N = 16 / sizeof(T);
    typedef T Vec __attribute__((ext_vector_type(16 / sizeof(T))));
};

// A-operand addressing modes.
enum { A_IM2COL_VEC = 0, A_IM2COL_SCALAR = 1, A_DENSE = 2 };

template <typename T, int BM, int BN, int WM, int WN, int BK, int AMODE>
__device__ __forceinline__ void igemm_body(const sox_igemm_args& p) {
    typedef Mfma<T> MM;
    typedef typename Chunk<T>::Vec Vec;
    constexpr int LD = Chunk<T>::N;          // elements per 16-byte chunk
    constexpr int PAD = LD;                  // 16 bytes of row padding
    constexpr int ROW = BK + PAD;            // LDS row length (elements)
    constexpr int CPR = BK / LD;             // chunks per tile row
    constexpr int A_CHUNKS = BM * CPR, B_CHUNKS = BN * CPR;
    constexpr int A_IT = (A_CHUNKS + 255) / 256, B_IT = (B_CHUNKS + 255) / 256;
    constexpr int WAVES_N = BN / WN;
    constexpr int TM = WM / 16, TN = WN / 16;
    static_assert((BM / WM) * (BN / WN) == 4, "4 waves per workgroup");
    static_assert(BK % MM::KSTEP == 0 && BK % LD == 0, "BK");
    static_assert(A_CHUNKS % 256 == 0 || A_CHUNKS < 256, "A tile split");

    __shared__ __attribute__((aligned(16))) T As[2][BM * ROW];
    __shared__ __attribute__((aligned(16))) T Bs[2][BN * ROW];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int tiles_n = p.tiles_n;
    const int bm = (blockIdx.x / tiles_n) * BM;
    const int bn = (blockIdx.x % tiles_n) * BN;
    const int wm0 = (wave / WAVES_N) * WM, wn0 = (wave % WAVES_N) * WN;
    const int M = p.m, N = p.n, K = p.k, kpad = p.kpad;
    const bool reflect = (p.flags & SOX_F_REFLECT) != 0;
    const T* __restrict__ x = (const T*)p.x;
    const T* __restrict__ w = (const T*)p.w;

    // ---- per-thread A rows (fixed across the K loop) ----
    const int kc = tid % CPR;  // this thread's chunk column
    int a_row[A_IT];
    int a_iy0[A_IT], a_ix0[A_IT];
    long a_base[A_IT];
#pragma unroll
    for (int i = 0; i < A_IT; i++) {
        int chunk = tid + i * 256;
        int row = chunk / CPR;
        a_row[i] = row;
        int m = bm + row;
        a_iy0[i] = -(1 << 29);
        a_ix0[i] = 0;
        a_base[i] = 0;
        if (chunk < A_CHUNKS && m < M) {
            if (AMODE == A_DENSE) {
                a_base[i] = (long)m * p.lda;
                a_iy0[i] = 0;
            } else {
                int ohw = p.oh * p.ow;
                int b = m / ohw, r = m - b * ohw;
                int oy = r / p.ow, ox = r - oy * p.ow;
                a_iy0[i] = oy * p.sh - p.pt;
                a_ix0[i] = ox * p.sw - p.pl;
                a_base[i] = (long)b * p.ih * p.iw * p.ic;
            }
        }
    }

    Vec a_reg[A_IT], b_reg[B_IT];

    auto load_a = [&](int k0) {
        if (AMODE == A_IM2COL_SCALAR) {
            // generic gather: each element finds its own tap (cin % LD != 0, e.g. 3-channel stems)
#pragma unroll
            for (int i = 0; i < A_IT; i++) {
#pragma unroll
                for (int e = 0; e < LD; e++) {
                    int k = k0 + kc * LD + e;
                    float v = 0.0f;
                    if (a_iy0[i] > -(1 << 28) && k < K) {
                        int tap = k / p.ic, c = k - tap * p.ic;
                        int ky = tap / p.kw, kx = tap - ky * p.kw;
                        int iy = sox_src_index(a_iy0[i] + ky, p.ih, reflect);
                        int ix = sox_src_index(a_ix0[i] + kx, p.iw, reflect);
                        v = iy < 0 || ix < 0 ? p.pad_value
                                             : to_f(x[a_base[i] + ((long)iy * p.iw + ix) * p.ic + c]);
                    }
                    a_reg[i][e] = (T)v;
                }
            }
        } else {
            int k = k0 + kc * LD;
            int tap = 0, c = k, ky = 0, kx = 0;
            if (AMODE == A_IM2COL_VEC) {
                tap = k / p.ic;
                c = k - tap * p.ic;
                ky = tap / p.kw;
                kx = tap - ky * p.kw;
            }
            // every load is issued unconditionally (masked lanes read element 0 of x) and the mask
            // is applied afterwards, so all of a slice's loads are in flight together
            bool ok[A_IT], inside[A_IT];
#pragma unroll
            for (int i = 0; i < A_IT; i++) {
                ok[i] = a_iy0[i] > -(1 << 28) && k < K;
                long off = 0;
                inside[i] = true;
                if (AMODE == A_DENSE) {
                    off = a_base[i] + k;
                } else {
                    // rows past M carry a sentinel origin: give them pixel (0, 0) to fold
                    const bool row = a_iy0[i] > -(1 << 28);
                    const int iy = sox_src_index(row ? a_iy0[i] + ky : 0, p.ih, reflect);
                    const int ix = sox_src_index(row ? a_ix0[i] + kx : 0, p.iw, reflect);
                    inside[i] = iy >= 0 && ix >= 0;
                    off = a_base[i] + ((long)iy * p.iw + ix) * p.ic + c;
                }
                a_reg[i] = *(const Vec*)(x + (ok[i] && inside[i] ? off : 0));
            }
#pragma unroll
            for (int i = 0; i < A_IT; i++)
                a_reg[i] = ok[i] ? (inside[i] ? a_reg[i] : (Vec)(T)p.pad_value) : (Vec)(T)0;
        }
    };

    auto load_b = [&](int k0) {
        bool ok[B_IT];
#pragma unroll
        for (int i = 0; i < B_IT; i++) {
            int chunk = tid + i * 256;
            int row = chunk / CPR, n = bn + row, k = k0 + (chunk % CPR) * LD;
            ok[i] = chunk < B_CHUNKS && n < N && k < kpad;
            b_reg[i] = *(const Vec*)(w + (ok[i] ? (long)n * kpad + k : 0));
        }
#pragma unroll
        for (int i = 0; i < B_IT; i++)
            if (!ok[i]) b_reg[i] = (Vec)(T)0;
    };

    auto store_tiles = [&](int buf) {
#pragma unroll
        for (int i = 0; i < A_IT; i++) {
            int chunk = tid + i * 256;
            if (chunk < A_CHUNKS) *(Vec*)(&As[buf][a_row[i] * ROW + kc * LD]) = a_reg[i];
        }
#pragma unroll
        for (int i = 0; i < B_IT; i++) {
            int chunk = tid + i * 256;
            if (chunk < B_CHUNKS) *(Vec*)(&Bs[buf][(chunk / CPR) * ROW + (chunk % CPR) * LD]) = b_reg[i];
        }
    };

    float4v acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = (float4v)0.0f;

    const int nk = (K + BK - 1) / BK;
    load_a(0);
    load_b(0);
    store_tiles(0);
    __syncthreads();

    const int lrow = lane & 15, lk = (lane >> 4) * MM::KPL;
    for (int kt = 0; kt < nk; kt++) {
        const int cur = kt & 1;
        if (kt + 1 < nk) {
            load_a((kt + 1) * BK);
            load_b((kt + 1) * BK);
        }
        const T* as = As[cur];
        const T* bs = Bs[cur];
#pragma unroll
        for (int s = 0; s < BK / MM::KSTEP; s++) {
            typename MM::Frag af[TM], bf[TN];
#pragma unroll
            for (int i = 0; i < TM; i++)
                af[i] = *(const typename MM::Frag*)(as + (wm0 + i * 16 + lrow) * ROW + s * MM::KSTEP + lk);
#pragma unroll
            for (int j = 0; j < TN; j++)
                bf[j] = *(const typename MM::Frag*)(bs + (wn0 + j * 16 + lrow) * ROW + s * MM::KSTEP + lk);
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++) acc[i][j] = MM::mma(af[i], bf[j], acc[i][j]);
        }
        if (kt + 1 < nk) store_tiles(cur ^ 1);
        __syncthreads();
    }

    // ---- epilogue: bias, residual, activation, store ----
    const int act = (p.flags & SOX_F_ACT_MASK) >> SOX_F_ACT_SHIFT;
    const bool has_bias = (p.flags & SOX_F_BIAS) != 0, has_add = (p.flags & SOX_F_RESIDUAL) != 0;
    T* __restrict__ y = (T*)p.y;
    const T* __restrict__ add = (const T*)p.add;
    const int ldy = p.ldy;
#pragma unroll
    for (int j = 0; j < TN; j++) {
        int n = bn + wn0 + j * 16 + lrow;
        if (n >= N) continue;
        float bv = has_bias ? p.bias[n] : 0.0f;
#pragma unroll
        for (int i = 0; i < TM; i++) {
#pragma unroll
            for (int r = 0; r < 4; r++) {
                int m = bm + wm0 + i * 16 + (lane >> 4) * 4 + r;
                if (m >= M) continue;
                float v = acc[i][j][r] + bv;
                long o = (long)m * ldy + n;
                if (has_add) v = v + to_f(add[o]);
                y[o] = (T)sox_act(v, act);
            }
        }
    }
}

#define SOX_IGEMM(NAME, T, BM, BN, WM, WN, BK, AMODE)                                              \
    extern "C" __global__ void __launch_bounds__(256) NAME(sox_igemm_args p) {                     \
        igemm_body<T, BM, BN, WM, WN, BK, AMODE>(p);                                               \
    }

// fp32 storage (fp32 graphs, the 1e-4 parity path): small tiles, deep K slices (latency-bound shapes)
SOX_IGEMM(sox_igemm_f32_32x32_v, float, 32, 32, 16, 16, 64, A_IM2COL_VEC)
SOX_IGEMM(sox_igemm_f32_32x32_s, float, 32, 32, 16, 16, 64, A_IM2COL_SCALAR)
SOX_IGEMM(sox_igemm_f32_32x32_d, float, 32, 32, 16, 16, 64, A_DENSE)
SOX_IGEMM(sox_igemm_f32_64x64_v, float, 64, 64, 32, 32, 32, A_IM2COL_VEC)
SOX_IGEMM(sox_igemm_f32_64x64_s, float, 64, 64, 32, 32, 32, A_IM2COL_SCALAR)
SOX_IGEMM(sox_igemm_f32_64x64_d, float, 64, 64, 32, 32, 32, A_DENSE)

// fp16 storage, fp32 accumulation
SOX_IGEMM(sox_igemm_f16_128x128_v, half_t, 128, 128, 64, 64, 32, A_IM2COL_VEC)
SOX_IGEMM(sox_igemm_bf16_128x128_v, bf16_t, 128, 128, 64, 64, 32, A_IM2COL_VEC)
SOX_IGEMM(sox_igemm_f16_128x128_s, half_t, 128, 128, 64, 64, 32, A_IM2COL_SCALAR)
SOX_IGEMM(sox_igemm_bf16_128x128_s, bf16_t, 128, 128, 64, 64, 32, A_IM2COL_SCALAR)
SOX_IGEMM(sox_igemm_f16_128x128_d, half_t, 128, 128, 64, 64, 32, A_DENSE)
SOX_IGEMM(sox_igemm_bf16_128x128_d, bf16_t, 128, 128, 64, 64, 32, A_DENSE)
SOX_IGEMM(sox_igemm_f16_64x64_v, half_t, 64, 64, 32, 32, 32, A_IM2COL_VEC)
SOX_IGEMM(sox_igemm_bf16_64x64_v, bf16_t, 64, 64, 32, 32, 32, A_IM2COL_VEC)
SOX_IGEMM(sox_igemm_f16_64x64_s, half_t, 64, 64, 32, 32, 32, A_IM2COL_SCALAR)
SOX_IGEMM(sox_igemm_bf16_64x64_s, bf16_t, 64, 64, 32, 32, 32, A_IM2COL_SCALAR)
SOX_IGEMM(sox_igemm_f16_64x64_d, half_t, 64, 64, 32, 32, 32, A_DENSE)
SOX_IGEMM(sox_igemm_bf16_64x64_d, bf16_t, 64, 64, 32, 32, 32, A_DENSE)
SOX_IGEMM(sox_igemm_f16_64x32_v, half_t, 64, 32, 32, 16, 32, A_IM2COL_VEC)
SOX_IGEMM(sox_igemm_bf16_64x32_v, bf16_t, 64, 32, 32, 16, 32, A_IM2COL_VEC)
SOX_IGEMM(sox_igemm_f16_64x32_s, half_t, 64, 32, 32, 16, 32, A_IM2COL_SCALAR)
SOX_IGEMM(sox_igemm_bf16_64x32_s, bf16_t, 64, 32, 32, 16, 32, A_IM2COL_SCALAR)
SOX_IGEMM(sox_igemm_f16_64x32_d, half_t, 64, 32, 32, 16, 32, A_DENSE)
SOX_IGEMM(sox_igemm_bf16_64x32_d, bf16_t, 64, 32, 32, 16, 32, A_DENSE)
// long-K variants (K = kh*kw*ic >= 128, e.g. 3x3 convs over 96 channels): 128-deep slices, a quarter
// of the load round trips of the 32-deep ones
SOX_IGEMM(sox_igemm_f16_64x64_vk, half_t, 64, 64, 32, 32, 128, A_IM2COL_VEC)
SOX_IGEMM(sox_igemm_bf16_64x64_vk, bf16_t, 64, 64, 32, 32, 128, A_IM2COL_VEC)
SOX_IGEMM(sox_igemm_f16_64x64_dk, half_t, 64, 64, 32, 32, 128, A_DENSE)
SOX_IGEMM(sox_igemm_bf16_64x64_dk, bf16_t, 64, 64, 32, 32, 128, A_DENSE)
SOX_IGEMM(sox_igemm_f16_64x32_vk, half_t, 64, 32, 32, 16, 128, A_IM2COL_VEC)
SOX_IGEMM(sox_igemm_bf16_64x32_vk, bf16_t, 64, 32, 32, 16, 128, A_IM2COL_VEC)
SOX_IGEMM(sox_igemm_f16_64x32_dk, half_t, 64, 32, 32, 16, 128, A_DENSE)
SOX_IGEMM(sox_igemm_bf16_64x32_dk, bf16_t, 64, 32, 32, 16, 128, A_DENSE)
