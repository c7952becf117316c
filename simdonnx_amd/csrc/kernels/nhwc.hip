// Bandwidth-bound NHWC kernels of the detector / recognizer graphs: depthwise conv,
// stride==kernel ConvTranspose, squeeze-excitation (GAP partials + gate + channel broadcast),
// nearest upsample + add, channel-slice copies (concat), elementwise, staging conversions,
// LayerNorm, row softmax and fused attention.
//
// They replace depthwise(4).comp, convt.comp, gap_part/se_gate.comp, ew2(v).comp, unary(2).comp,
// nearest(4).comp, concat_ax.comp, f32to16/f16to32.comp, layernorm.comp, softmax.comp and
// attn.comp (Backends/Vulkan/Shaders). None of them is GEMM-shaped enough for MFMA: they read
// each input byte a small constant number of times, so they are written for coalesced 16-byte
// accesses along the contiguous channel axis and wavefront reductions.
#include "sox_device.h"

template <typename T> struct V16 {
    static constexpr int N = 16 / sizeof(T);
    typedef T Vec __attribute__((ext_vector_type(16 / sizeof(T))));
};

template <typename T, int CV> struct VecT {
    typedef T Vec __attribute__((ext_vector_type(CV)));
};

// Wave reductions (wave64).
SOX_DEV float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

SOX_DEV float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// f(i, x[i]) for i = start, start + step, ... < n, with U loads issued before the first is used.
// A loop with a runtime trip count otherwise waits on every load in turn (one memory round trip per
// element); here the U element numbers are clamped to the sequence's last element, so the loads
// carry no branch and stay in bounds, and the surplus results are dropped.
// The empty volatile asm after the loads keeps the compiler from sinking a load into the guarded
// use below (where it would be issued and waited on alone).
template <typename T> SOX_DEV void keep_in_vgprs(T& v) {
    typedef unsigned u2v __attribute__((ext_vector_type(2)));
    typedef unsigned u4v __attribute__((ext_vector_type(4)));
    if constexpr (sizeof(T) == 2) {
        unsigned u = __builtin_bit_cast(unsigned short, v);
        asm volatile("" : "+v"(u));
        v = __builtin_bit_cast(T, (unsigned short)u);
    } else if constexpr (sizeof(T) == 4) {
        unsigned u = __builtin_bit_cast(unsigned, v);
        asm volatile("" : "+v"(u));
        v = __builtin_bit_cast(T, u);
    } else if constexpr (sizeof(T) == 8) {
        u2v u = __builtin_bit_cast(u2v, v);
        asm volatile("" : "+v"(u));
        v = __builtin_bit_cast(T, u);
    } else if constexpr (sizeof(T) == 16) {
        u4v u = __builtin_bit_cast(u4v, v);
        asm volatile("" : "+v"(u));
        v = __builtin_bit_cast(T, u);
    } else {
        static_assert(sizeof(T) == 32, "2, 4, 8, 16 or 32-byte elements");
        typedef unsigned u8v __attribute__((ext_vector_type(8)));
        u8v u = __builtin_bit_cast(u8v, v);
        asm volatile("" : "+v"(u));
        v = __builtin_bit_cast(T, u);
    }
}

template <int U, typename T, typename L, typename F>
SOX_DEV void strided_foreach_ld(L&& load, long start, long n, long step, F&& f) {
    if (start >= n) return;
    const long cnt = (n - 1 - start) / step + 1;  // elements start, start + step, ... < n
    for (long j0 = 0; j0 < cnt; j0 += U) {
        T v[U];
#pragma unroll
        for (int u = 0; u < U; u++) v[u] = load(start + (j0 + u < cnt ? j0 + u : cnt - 1) * step);
#pragma unroll
        for (int u = 0; u < U; u++) keep_in_vgprs(v[u]);
#pragma unroll
        for (int u = 0; u < U; u++)
            if (j0 + u < cnt) f(start + (j0 + u) * step, v[u]);
    }
}
template <int U, typename T, typename F>
SOX_DEV void strided_foreach(const T* __restrict__ x, long start, long n, long step, F&& f) {
    strided_foreach_ld<U, T>([&](long i) { return x[i]; }, start, n, step, f);
}

// Data handed from workgroup to workgroup inside one launch (the fused SE gate) moves through
// agent-scope atomics: they are performed at the agent's coherence point, so no cache-wide
// write-back or invalidate (what an agent-scope fence costs on a multi-XCD part) is needed.
// store_coherent returns the old value, which the caller hands to wait_performed: once the wave has
// the old values, the stores are performed, before any later memory operation of the wave is issued.
SOX_DEV float store_coherent(float* p, float v) {
    return __hip_atomic_exchange(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
SOX_DEV void wait_performed(uint32_t dep) { asm volatile("" ::"v"(dep) : "memory"); }
SOX_DEV float load_coherent(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Dot of a contiguous fp32 row with a vector, lanes striding the row, 8 loads in flight per lane.
template <typename G>
SOX_DEV float row_dot(const float* __restrict__ w, int len, int lane, G&& vec) {
    float acc = 0.0f;
    strided_foreach<8>(w, lane, len, 64, [&](long k, float wv) { acc = __builtin_fmaf(wv, vec((int)k), acc); });
    return acc;
}

// ------------------------------------------------------------------------------------------
// Depthwise k x k (Kernels/Nhwc.cs:496-631): acc = bias[c] + sum over taps (row-major) x*w,
// + residual, act. One work item = CV channels of one output pixel; taps outside a
// constant-0 pad are skipped, a nonzero pad value contributes pad * w.
// ------------------------------------------------------------------------------------------
template <typename T, int CV>
__device__ __forceinline__ void dw_body(const sox_dw_args& p) {
    const int cvn = p.c / CV;
    const long total = (long)p.n * p.oh * p.ow * cvn;
    const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= total) return;
    const int cv = (int)(idx % cvn);
    long pix = idx / cvn;
    const int ox = (int)(pix % p.ow);
    pix /= p.ow;
    const int oy = (int)(pix % p.oh);
    const int b = (int)(pix / p.oh);
    const int c0 = cv * CV;
    const bool reflect = (p.flags & SOX_F_REFLECT) != 0;
    const T* __restrict__ x = (const T*)p.x + (long)b * p.ih * p.iw * p.c;
    const T* __restrict__ w = (const T*)p.w;
    float acc[CV];
#pragma unroll
    for (int e = 0; e < CV; e++) acc[e] = (p.flags & SOX_F_BIAS) ? p.bias[c0 + e] : 0.0f;
    typedef typename VecT<T, CV>::Vec Vec;
    for (int ky = 0; ky < p.kh; ky++) {
        int iy = sox_src_index(oy * p.sh + ky - p.pt, p.ih, reflect);
        if (iy < 0 && p.pad_value == 0.0f) continue;
        for (int kx = 0; kx < p.kw; kx++) {
            int ix = sox_src_index(ox * p.sw + kx - p.pl, p.iw, reflect);
            Vec wv = *(const Vec*)(w + (long)(ky * p.kw + kx) * p.c + c0);
            if (iy < 0 || ix < 0) {
                if (p.pad_value != 0.0f)
#pragma unroll
                    for (int e = 0; e < CV; e++) acc[e] = __builtin_fmaf(p.pad_value, to_f(wv[e]), acc[e]);
                continue;
            }
            Vec xv = *(const Vec*)(x + ((long)iy * p.iw + ix) * p.c + c0);
#pragma unroll
            for (int e = 0; e < CV; e++) acc[e] = __builtin_fmaf(to_f(xv[e]), to_f(wv[e]), acc[e]);
        }
    }
    const int act = (p.flags & SOX_F_ACT_MASK) >> SOX_F_ACT_SHIFT;
    long o = (((long)b * p.oh + oy) * p.ow + ox) * p.c + c0;
    Vec out;
    if (p.flags & SOX_F_RESIDUAL) {
        Vec av = *(const Vec*)((const T*)p.add + o);
#pragma unroll
        for (int e = 0; e < CV; e++) acc[e] = acc[e] + to_f(av[e]);
    }
#pragma unroll
    for (int e = 0; e < CV; e++) out[e] = (T)sox_act(acc[e], act);
    *(Vec*)((T*)p.y + o) = out;
}

// K x K specialisation (3x3, 5x5): the taps unroll, every tap's x and w load is issued up front
// (out-of-image taps read pixel 0 and are masked to the pad value), so a work item costs one memory
// round trip instead of one per tap.
template <typename T, int CV, int K>
__device__ __forceinline__ void dw_body_k(const sox_dw_args& p) {
    const int cvn = p.c / CV;
    const long total = (long)p.n * p.oh * p.ow * cvn;
    const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= total) return;
    const int cv = (int)(idx % cvn);
    long pix = idx / cvn;
    const int ox = (int)(pix % p.ow);
    pix /= p.ow;
    const int oy = (int)(pix % p.oh);
    const int b = (int)(pix / p.oh);
    const int c0 = cv * CV;
    const bool reflect = (p.flags & SOX_F_REFLECT) != 0;
    const T* __restrict__ x = (const T*)p.x + (long)b * p.ih * p.iw * p.c + c0;
    const T* __restrict__ w = (const T*)p.w + c0;
    typedef typename VecT<T, CV>::Vec Vec;
    Vec xv[K * K], wv[K * K];
    bool in[K * K];
#pragma unroll
    for (int ky = 0; ky < K; ky++) {
        const int iy = sox_src_index(oy * p.sh + ky - p.pt, p.ih, reflect);
#pragma unroll
        for (int kx = 0; kx < K; kx++) {
            const int ix = sox_src_index(ox * p.sw + kx - p.pl, p.iw, reflect);
            const int t = ky * K + kx;
            in[t] = iy >= 0 && ix >= 0;
            xv[t] = *(const Vec*)(x + (in[t] ? ((long)iy * p.iw + ix) * p.c : 0));
            wv[t] = *(const Vec*)(w + (long)t * p.c);
        }
    }
    float acc[CV];
#pragma unroll
    for (int e = 0; e < CV; e++) acc[e] = (p.flags & SOX_F_BIAS) ? p.bias[c0 + e] : 0.0f;
#pragma unroll
    for (int t = 0; t < K * K; t++)
#pragma unroll
        for (int e = 0; e < CV; e++)  // taps in row-major order, as the reference accumulates them
            acc[e] = __builtin_fmaf(in[t] ? to_f(xv[t][e]) : p.pad_value, to_f(wv[t][e]), acc[e]);
    const int act = (p.flags & SOX_F_ACT_MASK) >> SOX_F_ACT_SHIFT;
    const long o = (((long)b * p.oh + oy) * p.ow + ox) * p.c + c0;
    if (p.flags & SOX_F_RESIDUAL) {
        const Vec av = *(const Vec*)((const T*)p.add + o);
#pragma unroll
        for (int e = 0; e < CV; e++) acc[e] = acc[e] + to_f(av[e]);
    }
    Vec out;
#pragma unroll
    for (int e = 0; e < CV; e++) out[e] = (T)sox_act(acc[e], act);
    *(Vec*)((T*)p.y + o) = out;
}

extern "C" __global__ void __launch_bounds__(256) sox_dw_f16_v3(sox_dw_args p) { dw_body_k<half_t, 8, 3>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_dw_bf16_v3(sox_dw_args p) { dw_body_k<bf16_t, 8, 3>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_dw_f16_v5(sox_dw_args p) { dw_body_k<half_t, 8, 5>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_dw_bf16_v5(sox_dw_args p) { dw_body_k<bf16_t, 8, 5>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_dw_f32_v3(sox_dw_args p) { dw_body_k<float, 4, 3>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_dw_f32_v5(sox_dw_args p) { dw_body_k<float, 4, 5>(p); }
// Depthwise K x K, stride S, over LDS tiles (any storage type). A workgroup owns an output tile of
// TH x 8 pixels (TH = 8, or 4 for small maps) of 64 channels (8 vectors of 8): it stages the tile's
// input halo ((TH - 1) S + K rows x (8 - 1) S + K columns, 8-channel vectors, constant-0 or reflected
// padding, channels past c as zeros) and the 64 channels' K x K weights in LDS in one round trip,
// then each thread computes one channel vector of NP = TH / 4 horizontally adjacent pixels, tap row
// by tap row, keeping the row's input vectors in registers: every input byte is read from memory
// once per tile instead of once per tap (K^2 times), and the weights once per workgroup.
// Accumulation per pixel is bias, then the taps in row-major order (one fma each), as dw_body.
// Halo rows have a pitch of an odd number of 128-byte units so the two rows a 16-lane LDS pass reads
// hit different banks.
// GAP (p.gap): the channel sums of the tile's stored outputs (after rounding to T), over the
// thread's pixels and then the tile's 32 pixel lanes in a fixed order, to part[b][tile][c].
template <typename T, int K, int S, int TH_ = 8> struct DwtShape {
    // tile: TH_ (8 or 4) rows x 8 columns; the 32 pixel lanes take NP pixels of one row each
    static constexpr int TH = TH_, TW = 8, NP = TH * TW / 32;
    static constexpr int HH = (TH - 1) * S + K, HW = (TW - 1) * S + K;  // halo
    static constexpr int VB = 8 * sizeof(T), PB = 8 * VB;              // bytes of a channel vector, a pixel
    static constexpr int RP = ((HW * PB / 128) | 1) * 128;              // halo row pitch: an odd number of 128 B
    static constexpr int LDS = HH * RP + K * K * PB;                     // halo + weights
};

// The workgroup's (tile, channel group, image). Workgroups go to the 8 XCDs in turn, so consecutive
// ids land on different L2s; numbered XCD-major (when the grid divides by 8), one XCD runs a run of
// consecutive (tile, group) pairs, group fastest: the groups of a pixel (whose 128-byte slices share
// lines when c * 2 bytes is no multiple of 128) and neighbouring tiles (whose halos overlap) read the
// same L2.
struct DwtCoords {
    int tile, g, b;
};
__device__ __forceinline__ DwtCoords dwt_coords() {
    const int groups = gridDim.y, tiles = gridDim.x;
    const int total = tiles * groups * gridDim.z;
    const int lin = blockIdx.x + tiles * (blockIdx.y + groups * blockIdx.z);
    const int v = total % 8 == 0 ? (lin % 8) * (total / 8) + lin / 8 : lin;
    const int rest = v / groups;
    return DwtCoords{rest % tiles, v % groups, rest / tiles};
}

template <typename T, int K, int S, bool GAP, bool COH = false, int TH_ = 8>
__device__ __forceinline__ void dwt_body(const sox_dwt_args& p, unsigned char* lds) {
    typedef DwtShape<T, K, S, TH_> D;
    constexpr int TH = D::TH, TW = D::TW, NP = D::NP, HH = D::HH, HW = D::HW, VB = D::VB, PB = D::PB, RP = D::RP;
    constexpr int XR = (NP - 1) * S + K;  // input vectors of one tap row
    typedef vec_t<T, 8> T8;
    unsigned char* wl = lds + HH * RP;
    const int t = threadIdx.x, cv = t & 7, pl = t >> 3;
    const DwtCoords wc = dwt_coords();
    const int tile = wc.tile, b = wc.b;
    const int c0 = wc.g * 64 + cv * 8;  // this thread's channel vector
    const bool cok = c0 < p.c;                // p.c % 8 == 0
    const int ty0 = (tile / p.tiles_x) * TH, tx0 = (tile % p.tiles_x) * TW;
    const int iy0 = ty0 * S - p.pt, ix0 = tx0 * S - p.pl;
    const bool reflect = (p.flags & SOX_F_REFLECT) != 0;
    // every load that does not depend on the halo goes out first and stays in registers (else the
    // compiler issues each next to its use, one more memory round trip each)
    T8 wv[(K * K + 31) / 32];
#pragma unroll
    for (int i = 0; i < (K * K + 31) / 32; i++) {
        const int tap = min(pl + 32 * i, K * K - 1);
        wv[i] = cok ? *(const T8*)((const T*)p.w + (long)tap * p.c + c0) : (T8)(T)0.0f;
    }
    const bool hb = (p.flags & SOX_F_BIAS) && cok;
    float bv[8];
#pragma unroll
    for (int e = 0; e < 8; e++) bv[e] = hb ? p.bias[c0 + e] : 0.0f;
    const int orow = pl % TH, ocol = (pl / TH) * NP;  // thread pixel lanes: row, first of NP columns
    const int oy = ty0 + orow;
    T8 rv[NP];
#pragma unroll
    for (int q = 0; q < NP; q++) {
        const int ox = min(tx0 + ocol + q, p.ow - 1);
        const long o = (((long)b * p.oh + min(oy, p.oh - 1)) * p.ow + ox) * p.c + c0;
        rv[q] = (p.flags & SOX_F_RESIDUAL) && cok ? *(const T8*)((const T*)p.add + o) : (T8)(T)0.0f;
    }
    // the halo loads, issued with those before the first wait
    const T* __restrict__ x = (const T*)p.x + (long)b * p.ih * p.iw * p.c;
    constexpr int HL = (HH * HW + 31) / 32;
    T8 hv[HL];
#pragma unroll
    for (int i = 0; i < HL; i++) {
        const int h = pl + 32 * i;
        const int hr = h / HW, hc = h - hr * HW;
        const int iy = sox_src_index(iy0 + hr, p.ih, reflect), ix = sox_src_index(ix0 + hc, p.iw, reflect);
        const bool ok = h < HH * HW && cok && iy >= 0 && ix >= 0;
        hv[i] = *(const T8*)(x + (ok ? ((long)iy * p.iw + ix) * p.c + c0 : 0));
        if (!ok) hv[i] = (T8)(T)0.0f;
    }
#pragma unroll
    for (int i = 0; i < (K * K + 31) / 32; i++) keep_in_vgprs(wv[i]);
#pragma unroll
    for (int e = 0; e < 8; e++) keep_in_vgprs(bv[e]);
#pragma unroll
    for (int q = 0; q < NP; q++) keep_in_vgprs(rv[q]);
#pragma unroll
    for (int i = 0; i < HL; i++) {
        const int h = pl + 32 * i;
        if (h < HH * HW) {
            const int hr = h / HW, hc = h - hr * HW;
            *(T8*)(lds + hr * RP + hc * PB + cv * VB) = hv[i];
        }
    }
#pragma unroll
    for (int i = 0; i < (K * K + 31) / 32; i++)
        if (pl + 32 * i < K * K) *(T8*)(wl + (pl + 32 * i) * PB + cv * VB) = wv[i];
    __syncthreads();

    float acc[NP][8];
#pragma unroll
    for (int e = 0; e < 8; e++)
#pragma unroll
        for (int q = 0; q < NP; q++) acc[q][e] = bv[e];
#pragma unroll 1
    for (int ky = 0; ky < K; ky++) {
        const unsigned char* row = lds + (orow * S + ky) * RP + ocol * S * PB + cv * VB;
        T8 xr[XR], wr[K];
#pragma unroll
        for (int j = 0; j < XR; j++) xr[j] = *(const T8*)(row + j * PB);
#pragma unroll
        for (int kx = 0; kx < K; kx++) wr[kx] = *(const T8*)(wl + (ky * K + kx) * PB + cv * VB);
#pragma unroll
        for (int kx = 0; kx < K; kx++)
#pragma unroll
            for (int q = 0; q < NP; q++)
#pragma unroll
                for (int e = 0; e < 8; e++)
                    acc[q][e] = __builtin_fmaf(to_f(xr[q * S + kx][e]), to_f(wr[kx][e]), acc[q][e]);
    }
    const int act = (p.flags & SOX_F_ACT_MASK) >> SOX_F_ACT_SHIFT;
    float gs[8];
#pragma unroll
    for (int e = 0; e < 8; e++) gs[e] = 0.0f;
#pragma unroll
    for (int q = 0; q < NP; q++) {
        const int ox = tx0 + ocol + q;
        if (!cok || oy >= p.oh || ox >= p.ow) continue;
        const long o = (((long)b * p.oh + oy) * p.ow + ox) * p.c + c0;
        T8 out;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            float v = acc[q][e];
            if (p.flags & SOX_F_RESIDUAL) v = v + to_f(rv[q][e]);
            out[e] = (T)sox_act(v, act);
            if constexpr (GAP) gs[e] += to_f(out[e]);
        }
        *(T8*)((T*)p.y + o) = out;
    }
    if constexpr (GAP) {
        // 32 pixel lanes per channel vector fold in a fixed binary tree through LDS (the halo is done)
        __syncthreads();
        float* red = (float*)lds;  // [pl][64 channels]
#pragma unroll
        for (int e = 0; e < 8; e++) red[pl * 64 + cv * 8 + e] = gs[e];
        for (int st = 16; st > 0; st >>= 1) {
            __syncthreads();
            if (pl < st) {
#pragma unroll
                for (int e = 0; e < 8; e++) red[pl * 64 + cv * 8 + e] += red[(pl + st) * 64 + cv * 8 + e];
            }
        }
        __syncthreads();
        if (pl == 0 && cok) {
            float* dst = p.part + ((long)b * p.tiles_x * p.tiles_y + tile) * p.c + c0;
            if constexpr (COH) {  // read by the launch's last tile of the group (sox_dwt_*_se)
                uint32_t dep = 0;
#pragma unroll
                for (int e = 0; e < 8; e++) dep |= __float_as_uint(store_coherent(dst + e, red[cv * 8 + e]));
                wait_performed(dep);
            } else {
#pragma unroll
                for (int e = 0; e < 8; e++) dst[e] = red[cv * 8 + e];
            }
        }
    }
}

#define SOX_DWT(TY, T, K, S)                                                                                   \
    extern "C" __global__ void __launch_bounds__(256) sox_dwt_##TY##_k##K##s##S(sox_dwt_args p) {          \
        __shared__ __attribute__((aligned(16))) unsigned char lds[DwtShape<T, K, S>::LDS];                  \
        if (p.gap)                                                                                             \
            dwt_body<T, K, S, true>(p, lds);                                                                   \
        else                                                                                                   \
            dwt_body<T, K, S, false>(p, lds);                                                                  \
    }
SOX_DWT(f16, half_t, 3, 1)
SOX_DWT(f16, half_t, 3, 2)
SOX_DWT(f16, half_t, 5, 1)
SOX_DWT(f16, half_t, 5, 2)
SOX_DWT(bf16, bf16_t, 3, 1)
SOX_DWT(bf16, bf16_t, 3, 2)
SOX_DWT(bf16, bf16_t, 5, 1)
SOX_DWT(bf16, bf16_t, 5, 2)
SOX_DWT(f32, float, 3, 1)
SOX_DWT(f32, float, 3, 2)
SOX_DWT(f32, float, 5, 1)
SOX_DWT(f32, float, 5, 2)

// 4 x 8 tiles (one pixel per thread): twice the workgroups of the 8 x 8 form, for maps too small to
// fill the GPU with 8 x 8 tiles (the 40 x 40 / 20 x 20 levels of MobileNetV3-small at 640, the 60 x 60 /
// 30 x 30 ones of the detector)
#define SOX_DWT_H4(TY, T, K, S)                                                                                \
    extern "C" __global__ void __launch_bounds__(256) sox_dwt_##TY##_k##K##s##S##_h4(sox_dwt_args p) {     \
        __shared__ __attribute__((aligned(16))) unsigned char lds[DwtShape<T, K, S, 4>::LDS];               \
        if (p.gap)                                                                                             \
            dwt_body<T, K, S, true, false, 4>(p, lds);                                                         \
        else                                                                                                   \
            dwt_body<T, K, S, false, false, 4>(p, lds);                                                        \
    }
SOX_DWT_H4(f16, half_t, 3, 1)
SOX_DWT_H4(f16, half_t, 3, 2)
SOX_DWT_H4(f16, half_t, 5, 1)
SOX_DWT_H4(f16, half_t, 5, 2)
SOX_DWT_H4(bf16, bf16_t, 3, 1)
SOX_DWT_H4(bf16, bf16_t, 3, 2)
SOX_DWT_H4(bf16, bf16_t, 5, 1)
SOX_DWT_H4(bf16, bf16_t, 5, 2)
SOX_DWT_H4(f32, float, 3, 1)
SOX_DWT_H4(f32, float, 3, 2)
SOX_DWT_H4(f32, float, 5, 1)
SOX_DWT_H4(f32, float, 5, 2)


extern "C" __global__ void __launch_bounds__(256) sox_dw_f16_v(sox_dw_args p) { dw_body<half_t, 8>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_dw_bf16_v(sox_dw_args p) { dw_body<bf16_t, 8>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_dw_f16_s(sox_dw_args p) { dw_body<half_t, 1>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_dw_bf16_s(sox_dw_args p) { dw_body<bf16_t, 1>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_dw_f32_v(sox_dw_args p) { dw_body<float, 4>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_dw_f32_s(sox_dw_args p) { dw_body<float, 1>(p); }

// ------------------------------------------------------------------------------------------
// ConvTranspose, stride == kernel, no pad (Kernels/Nhwc.Det.cs:51-131): every input pixel owns
// a disjoint kh x kw output patch. One work item = one (input pixel, tap, oc) output element;
// w is [tap][ic][oc], so neighbouring items read neighbouring weights and the same x row.
// ------------------------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ void convt_body(const sox_convt_args& p) {
    const int taps = p.kh * p.kw;
    const long total = (long)p.n * p.ih * p.iw * taps * p.oc;
    const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= total) return;
    const int o = (int)(idx % p.oc);
    long r = idx / p.oc;
    const int tap = (int)(r % taps);
    long pix = r / taps;  // (b, y, x) of the input
    const int x = (int)(pix % p.iw);
    long q = pix / p.iw;
    const int y = (int)(q % p.ih);
    const int b = (int)(q / p.ih);
    const T* __restrict__ xp = (const T*)p.x + pix * p.ic;
    const T* __restrict__ w = (const T*)p.w + (long)tap * p.ic * p.oc + o;
    float s = (p.flags & SOX_F_BIAS) ? p.bias[o] : 0.0f;
    for (int c = 0; c < p.ic; c++) s = __builtin_fmaf(to_f(xp[c]), to_f(w[(long)c * p.oc]), s);
    const int act = (p.flags & SOX_F_ACT_MASK) >> SOX_F_ACT_SHIFT;
    const int dy = tap / p.kw, dx = tap - dy * p.kw;
    const int ow = p.iw * p.kw, oh = p.ih * p.kh;
    long out = (((long)b * oh + (y * p.kh + dy)) * ow + (x * p.kw + dx)) * p.oc + o;
    ((T*)p.y)[out] = (T)sox_act(s, act);
}

extern "C" __global__ void __launch_bounds__(256) sox_convt_f16(sox_convt_args p) { convt_body<half_t>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_convt_bf16(sox_convt_args p) { convt_body<bf16_t>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_convt_f32(sox_convt_args p) { convt_body<float>(p); }

// Pixel-major ConvTranspose for kh*kw <= 4 taps (the 2x2 stride-2 DBNet head): one work item = one
// input pixel x 8 output channels for ALL taps, so the pixel's ic channels are loaded once and reused
// for every tap; the packed weights [tap][ic][oc] sit in LDS as fp32 (host guarantees
// taps*ic*oc <= 16384) and are read as broadcasts. When ic is a multiple of the 16-byte vector and
// at most 8 vectors, the pixel's loads (and its bias) are all issued before the weights are staged,
// so the kernel waits on memory once. Output channels of one tap are contiguous: 16-byte stores
// when oc % 8 == 0.
template <typename T>
__device__ __forceinline__ void convt_pix_body(const sox_convt_args& p) {
    extern __shared__ float wl[];  // [tap][ic][oc]
    typedef typename V16<T>::Vec Vec;
    constexpr int VE = V16<T>::N;
    const int taps = p.kh * p.kw, nw = taps * p.ic * p.oc;
    const int og_n = (p.oc + 7) / 8;
    const long items = (long)p.n * p.ih * p.iw * og_n;
    const long item_raw = (long)blockIdx.x * blockDim.x + threadIdx.x;
    const long item = min(item_raw, items - 1);  // threads past the end still stage weights
    const int og = (int)(item % og_n);
    const long pix = item / og_n;
    const int o0 = og * 8, on = min(8, p.oc - o0);
    const int nv = p.ic / VE;
    const bool vec = p.ic % VE == 0 && nv <= 8;  // uniform
    Vec xv[8];
    if (vec) {
        const Vec* __restrict__ xp = (const Vec*)((const T*)p.x + pix * p.ic);
#pragma unroll
        for (int u = 0; u < 8; u++) xv[u] = xp[min(u, nv - 1)];
#pragma unroll
        for (int u = 0; u < 8; u++) keep_in_vgprs(xv[u]);
    }
    float acc[4][8];
#pragma unroll
    for (int o = 0; o < 8; o++) {
        const float bv = (p.flags & SOX_F_BIAS) ? p.bias[o0 + min(o, on - 1)] : 0.0f;
#pragma unroll
        for (int t = 0; t < 4; t++) acc[t][o] = o < on ? bv : 0.0f;
    }
    strided_foreach<8>((const T*)p.w, (long)threadIdx.x, (long)nw, (long)blockDim.x,
                       [&](long i, T v) { wl[i] = to_f(v); });
    __syncthreads();
    if (item_raw >= items) return;
    if (vec) {
#pragma unroll
        for (int u = 0; u < 8; u++) {
            if (u >= nv) break;
#pragma unroll
            for (int e = 0; e < VE; e++) {
                const float xe = to_f(xv[u][e]);
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    if (t >= taps) break;
                    const float* wr = wl + ((long)t * p.ic + u * VE + e) * p.oc + o0;
#pragma unroll
                    for (int o = 0; o < 8; o++) acc[t][o] = __builtin_fmaf(xe, wr[o < on ? o : 0], acc[t][o]);
                }
            }
        }
    } else {
        const T* __restrict__ xp = (const T*)p.x + pix * p.ic;
        for (int c0 = 0; c0 < p.ic; c0 += 8) {
            float xs[8];
#pragma unroll
            for (int e = 0; e < 8; e++) xs[e] = to_f(xp[min(c0 + e, p.ic - 1)]);
#pragma unroll
            for (int e = 0; e < 8; e++) {
                if (c0 + e >= p.ic) break;
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    if (t >= taps) break;
                    const float* wr = wl + ((long)t * p.ic + c0 + e) * p.oc + o0;
#pragma unroll
                    for (int o = 0; o < 8; o++) acc[t][o] = __builtin_fmaf(xs[e], wr[o < on ? o : 0], acc[t][o]);
                }
            }
        }
    }
    const int act = (p.flags & SOX_F_ACT_MASK) >> SOX_F_ACT_SHIFT;
    const int x = (int)(pix % p.iw);
    const long q = pix / p.iw;
    const int y = (int)(q % p.ih), b = (int)(q / p.ih);
    const int ow = p.iw * p.kw, oh = p.ih * p.kh;
#pragma unroll
    for (int t = 0; t < 4; t++) {
        if (t >= taps) break;
        const int dy = t / p.kw, dx = t - dy * p.kw;
        T* out = (T*)p.y + (((long)b * oh + (y * p.kh + dy)) * ow + (x * p.kw + dx)) * p.oc + o0;
        if (on == 8 && (p.oc & 7) == 0) {
            typedef typename VecT<T, 8>::Vec Vec8;
            Vec8 v;
#pragma unroll
            for (int o = 0; o < 8; o++) v[o] = (T)sox_act(acc[t][o], act);
            if (sizeof(T) == 2) {
                *(Vec8*)out = v;
            } else {
#pragma unroll
                for (int o = 0; o < 8; o++) out[o] = v[o];
            }
        } else {
#pragma unroll
            for (int o = 0; o < 8; o++)
                if (o < on) out[o] = (T)sox_act(acc[t][o], act);
        }
    }
}

// ConvTranspose to one output channel (the DB head's probability map, 24 -> 1 with a 2x2 kernel):
// one input pixel per thread, its channels in 16-byte loads, the kh*kw taps' dot products against
// the [tap][ic] weights staged in LDS (every lane reads the same word: broadcasts), and each output
// row's kw values written by one store. Route: oc == 1, kh*kw <= 4, kw <= 2, ic % (16 / sizeof(T)) == 0.
template <typename T>
__device__ __forceinline__ void convt_one_body(const sox_convt_args& p) {
    extern __shared__ float wl[];  // [tap][ic] (the [tap][ic][oc] packing with oc = 1)
    typedef typename V16<T>::Vec Vec;
    constexpr int VE = V16<T>::N;
    const int taps = p.kh * p.kw, nw = taps * p.ic;
    for (int i = threadIdx.x; i < nw; i += blockDim.x) wl[i] = to_f(((const T*)p.w)[i]);
    __syncthreads();
    const long pixels = (long)p.n * p.ih * p.iw;
    const long pix = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (pix >= pixels) return;
    const float bv = (p.flags & SOX_F_BIAS) ? p.bias[0] : 0.0f;
    float acc[4] = {bv, bv, bv, bv};
    const T* __restrict__ xp = (const T*)p.x + pix * p.ic;
    for (int c0 = 0; c0 < p.ic; c0 += VE) {
        const Vec xv = *(const Vec*)(xp + c0);
#pragma unroll
        for (int e = 0; e < VE; e++) {
            const float xe = to_f(xv[e]);
#pragma unroll
            for (int t = 0; t < 4; t++)
                if (t < taps) acc[t] = __builtin_fmaf(xe, wl[t * p.ic + c0 + e], acc[t]);
        }
    }
    const int act = (p.flags & SOX_F_ACT_MASK) >> SOX_F_ACT_SHIFT;
    const int x = (int)(pix % p.iw);
    const long q = pix / p.iw;
    const int y = (int)(q % p.ih), b = (int)(q / p.ih);
    const int ow = p.iw * p.kw, oh = p.ih * p.kh;
    for (int dy = 0; dy < p.kh; dy++) {
        T* out = (T*)p.y + ((long)b * oh + (y * p.kh + dy)) * ow + (long)x * p.kw;
        if (p.kw == 2) {
            typedef typename VecT<T, 2>::Vec Vec2;
            Vec2 v;
            v[0] = (T)fp32_value(sox_act(acc[2 * dy], act));
            v[1] = (T)fp32_value(sox_act(acc[2 * dy + 1], act));
            *(Vec2*)out = v;
        } else {
            for (int dx = 0; dx < p.kw; dx++) out[dx] = (T)fp32_value(sox_act(acc[dy * p.kw + dx], act));
        }
    }
}

extern "C" __global__ void __launch_bounds__(256) sox_convt_pix_f16(sox_convt_args p) { convt_pix_body<half_t>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_convt_pix_bf16(sox_convt_args p) { convt_pix_body<bf16_t>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_convt_one_f16(sox_convt_args p) { convt_one_body<half_t>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_convt_one_bf16(sox_convt_args p) { convt_one_body<bf16_t>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_convt_one_f32(sox_convt_args p) { convt_one_body<float>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_convt_pix_f32(sox_convt_args p) { convt_pix_body<float>(p); }

// ------------------------------------------------------------------------------------------
// Global-average-pool partials (gap_part.comp): part[b][chunk][c] = sum over the chunk's pixels.
// Grid (chunks, n); the 256 threads are (c / CV) channel vectors x P pixel phases, each thread
// accumulating CV channels of every P-th pixel of the chunk (16-byte loads, many in flight),
// then the P phases are reduced in LDS in a fixed order.
// ------------------------------------------------------------------------------------------
template <typename T, int CV>
__device__ __forceinline__ void gap_body(const sox_gap_args& p) {
    __shared__ float red[256 * CV];
    const int cg = p.c / CV;
    const int P = max(1, 256 / cg);
    const int t = threadIdx.x;
    const int g = t % cg, ph = t / cg;
    const int chunk = blockIdx.x, b = blockIdx.y;
    const long p0 = (long)chunk * p.hw / p.chunks, p1 = (long)(chunk + 1) * p.hw / p.chunks;
    typedef typename VecT<T, CV>::Vec Vec;
    if (cg > 256) {  // more channel vectors than threads: each thread owns whole channel vectors
        const T* __restrict__ xb = (const T*)p.x + (long)b * p.hw * p.c;
        for (int gg = t; gg < cg; gg += 256) {
            float a2[CV];
#pragma unroll
            for (int e = 0; e < CV; e++) a2[e] = 0.0f;
            for (long px = p0; px < p1; px++) {
                Vec v = *(const Vec*)(xb + px * p.c + gg * CV);
#pragma unroll
                for (int e = 0; e < CV; e++) a2[e] += to_f(v[e]);
            }
#pragma unroll
            for (int e = 0; e < CV; e++) p.part[((long)b * p.chunks + chunk) * p.c + gg * CV + e] = a2[e];
        }
        return;
    }
    float acc[CV];
#pragma unroll
    for (int e = 0; e < CV; e++) acc[e] = 0.0f;
    if (ph < P && t < cg * P && p0 + ph < p1) {
        // pixel px of this channel vector is Vec element px * (c / CV)
        const Vec* __restrict__ x = (const Vec*)((const T*)p.x + (long)b * p.hw * p.c + g * CV);
        const long stride = p.c / CV;
        strided_foreach<4>(x, (p0 + ph) * stride, p1 * stride, P * stride, [&](long, Vec v) {
#pragma unroll
            for (int e = 0; e < CV; e++) acc[e] += to_f(v[e]);
        });
    }
#pragma unroll
    for (int e = 0; e < CV; e++) red[t * CV + e] = acc[e];
    // the P phases of each channel vector fold in a fixed binary tree (log2 P steps; a serial loop
    // over P = 256 / cg phases is long for few channels)
    for (int st = 1; st < P; st *= 2) {
        __syncthreads();
        if (t < cg * P && ph % (2 * st) == 0 && ph + st < P) {
#pragma unroll
            for (int e = 0; e < CV; e++) red[t * CV + e] += red[(t + st * cg) * CV + e];
        }
    }
    __syncthreads();
    for (int ch = t; ch < p.c; ch += 256) p.part[((long)b * p.chunks + chunk) * p.c + ch] = red[ch];
}

extern "C" __global__ void __launch_bounds__(256) sox_gap_f16_v(sox_gap_args p) { gap_body<half_t, 8>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_gap_bf16_v(sox_gap_args p) { gap_body<bf16_t, 8>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_gap_f16_s(sox_gap_args p) { gap_body<half_t, 1>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_gap_bf16_s(sox_gap_args p) { gap_body<bf16_t, 1>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_gap_f32_v(sox_gap_args p) { gap_body<float, 4>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_gap_f32_s(sox_gap_args p) { gap_body<float, 1>(p); }

// ------------------------------------------------------------------------------------------
// SE gate (se_gate.comp; Kernels/Nhwc.Det.cs:287-314) as two passes over many workgroups.
// ------------------------------------------------------------------------------------------
// The SE weights are read once per inference, so what costs is the number of dependent memory
// round trips, not bytes. fc1 is split by channel groups so every GAP partial is read once: group g
// reduces its 64 channels' partials (4 chunk phases per channel, one batch of loads each), then
// 16 lanes x 4 channels cover the group's slice of four W1 rows per wave instruction, and a 16-lane
// shuffle reduces each row.
constexpr int SE_CG = 64;
constexpr int SE_FC1_U = 16;  // W1 rows prefetched per lane: r <= 16 * SE_FC1_U takes the one-round-trip path
// Channel group g of image b (256 threads; red: 256 floats, mean: SE_CG floats of LDS).
// COH: the partials come from other workgroups of the same launch, and hid goes to one (coherent
// loads and stores).
template <bool COH = false>
__device__ __forceinline__ void se_fc1_group(const sox_se_args& p, int g, int b, float* red, float* mean) {
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int c0 = g * SE_CG, cn = min(SE_CG, p.c - c0);
    const int sub = lane & 15, rq = lane >> 4;  // channel quad, row within the wave's four
    const bool vec = (p.c & 3) == 0;            // rows and groups start 16-byte aligned, cn % 4 == 0
    const bool pre = vec && p.r <= 16 * SE_FC1_U;
    // the group's W1 slice does not depend on the mean: its loads go out first, with the partials'
    // (rows wave*4 + rq + 16u, clamped; this lane's quad of channels)
    float4v wv[SE_FC1_U];
    if (pre) {
#pragma unroll
        for (int u = 0; u < SE_FC1_U; u++) {
            const int j = min(wave * 4 + rq + 16 * u, p.r - 1);
            wv[u] = *(const float4v*)(p.w1 + (long)j * p.c + c0 + min(4 * sub, cn - 4));
        }
    }
    // cw channel lanes x nph chunk phases: a group of few channels takes more phases, so a depthwise
    // conv of many tiles can hand over its per-tile partials (up to 64 per thread)
    const int cw = cn <= 16 ? 16 : cn <= 32 ? 32 : SE_CG, nph = 256 / cw;
    {
        const int ch = t % cw, ph = t / cw;
        float acc = 0.0f;
        if (ch < cn)
            strided_foreach_ld<16, float>(
                [&](long i) {
                    const float* q = p.part + (long)b * p.chunks * p.c + c0 + ch + i;
                    return COH ? load_coherent(q) : *q;
                },
                (long)ph * p.c, (long)p.chunks * p.c, (long)nph * p.c, [&](long, float v) { acc += v; });
        red[t] = acc;
    }
    // the W1 loads stay ahead of the barrier (issued with the first partials, one wait for both)
    if (pre) {
#pragma unroll
        for (int u = 0; u < SE_FC1_U; u++) keep_in_vgprs(wv[u]);
    }
    // the phases fold in a fixed binary tree, adjacent phases first ((0+1) + (2+3) for four)
    for (int st = 1; st < nph; st *= 2) {
        __syncthreads();
        const int ph = t / cw;
        if (ph % (2 * st) == 0 && ph + st < nph) red[t] += red[t + st * cw];
    }
    __syncthreads();
    if (t < cw) mean[t] = red[t] * (1.0f / p.hw);
    __syncthreads();
    float m4[4];
#pragma unroll
    for (int e = 0; e < 4; e++) m4[e] = 4 * sub + e < cn ? mean[4 * sub + e] : 0.0f;  // 0: lane past the group
    float* hid = p.hid + ((long)b * p.groups + g) * p.r;
    uint32_t dep = 0;
    auto put = [&](int j, float v) {
        if constexpr (COH)
            dep |= __float_as_uint(store_coherent(hid + j, v));
        else
            hid[j] = v;
    };
    if (pre) {
#pragma unroll
        for (int u = 0; u < SE_FC1_U; u++) {
            const int j = wave * 4 + rq + 16 * u;
            if (wave * 4 + 16 * u >= p.r) break;  // uniform
            float s = wv[u][0] * m4[0] + wv[u][1] * m4[1] + wv[u][2] * m4[2] + wv[u][3] * m4[3];
#pragma unroll
            for (int o = 8; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
            if (sub == 0 && j < p.r) put(j, s);
        }
        if constexpr (COH) wait_performed(dep);
        return;
    }
    // four rows per wave instruction, four instructions' loads in flight (clamped, branch-free)
    for (int j0 = wave * 4; j0 < p.r; j0 += 64) {
        float s[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int j = min(j0 + 16 * u + rq, p.r - 1);
            const float* w = p.w1 + (long)j * p.c + c0;
            if (vec) {
                const float4v v = *(const float4v*)(w + min(4 * sub, cn - 4));
                s[u] = v[0] * m4[0] + v[1] * m4[1] + v[2] * m4[2] + v[3] * m4[3];
            } else {
                s[u] = 0.0f;
#pragma unroll
                for (int e = 0; e < 4; e++) s[u] += w[min(4 * sub + e, cn - 1)] * m4[e];
            }
        }
#pragma unroll
        for (int u = 0; u < 4; u++) {
#pragma unroll
            for (int o = 8; o > 0; o >>= 1) s[u] += __shfl_xor(s[u], o, 64);
            const int j = j0 + 16 * u + rq;
            if (sub == 0 && j < p.r) put(j, s[u]);
        }
    }
    if constexpr (COH) wait_performed(dep);
}

extern "C" __global__ void __launch_bounds__(256) sox_se_fc1(sox_se_args p) {
    __shared__ float red[256];
    __shared__ float mean[SE_CG];
    se_fc1_group(p, blockIdx.x, blockIdx.y, red, mean);
}

// A folded weight: w * gate rounded to fp32, then to T. The product is pinned in a register first:
// the compiler otherwise may or may not fuse the multiply with the conversion into one
// mixed-precision instruction that rounds once, depending on the surrounding code, and the separate
// fc2 pass and the fused depthwise launch would differ in the last bit.
template <typename T> __device__ __forceinline__ T se_scaled(T w, float gate) {
    float prod = to_f(w) * gate;
    keep_in_vgprs(prod);
    return (T)prod;
}

// The gate of channel ch from its fc2 dot product z (before b2).
__device__ __forceinline__ float se_gate_value(const sox_se_args& p, int ch, float z) {
    z += (p.flags & 2) ? p.b2[ch] : 0.0f;
    return ((p.flags & 8) ? fminf(fmaxf(z * p.alpha + p.beta, 0.0f), 1.0f) : sox_sigmoid(z)) + p.offset;
}

// fc2: the workgroup rebuilds h from the groups' partials in LDS (fixed summation order), then one
// wave per output channel. The wave's W2 row and, when folding, its column of the consumer's weights
// (r, wn <= 256: four per lane) are loaded before h is gathered, so the kernel waits on memory once.
template <typename T>
__device__ __forceinline__ void se_fc2_body(const sox_se_args& p) {
    extern __shared__ float h[];  // [r]
    const int b = blockIdx.y, t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int ch = blockIdx.x * (blockDim.x >> 6) + wave, chc = min(ch, p.c - 1);
    const bool fold = (p.flags & SOX_SE_FOLD) != 0;
    const bool pre = p.r <= 256 && (!fold || p.wn <= 256);
    const T* __restrict__ ws = (const T*)p.wsrc;
    float w2v[4];
    // the consumer's weights as zero-extended 32-bit words: 16-bit values would be packed in pairs,
    // which waits for their loads right away
    typedef std::conditional_t<sizeof(T) == 2, unsigned short, unsigned> WU;
    unsigned wsv[4];
    if (pre) {
#pragma unroll
        for (int u = 0; u < 4; u++) w2v[u] = p.w2[(long)chc * p.r + min(lane + 64 * u, p.r - 1)];
        if (fold) {
#pragma unroll
            for (int u = 0; u < 4; u++) wsv[u] = ((const WU*)ws)[(long)min(lane + 64 * u, p.wn - 1) * p.wk + chc];
        }
    }
    const float* part = p.hid + (long)b * p.groups * p.r;
    if (pre && p.groups <= 16 && p.r <= (int)blockDim.x) {
        // one hidden unit per thread, its <= 16 group partials in one batch with the weights: no loop,
        // so nothing makes the compiler wait for the weight loads before it (a loop preheader would)
        const int k = min(t, p.r - 1);
        float pv[16];
#pragma unroll
        for (int gi = 0; gi < 16; gi++) pv[gi] = part[(long)min(gi, p.groups - 1) * p.r + k];
        float s = (p.flags & 1) ? p.b1[k] : 0.0f;
#pragma unroll
        for (int gi = 0; gi < 16; gi++)
            if (gi < p.groups) s += pv[gi];
        if (t < p.r) h[k] = (p.flags & 4) ? fmaxf(s, 0.0f) : s;
    } else {
        for (int k = t; k < p.r; k += blockDim.x) {
            float s = (p.flags & 1) ? p.b1[k] : 0.0f;
            strided_foreach<16>(part + k, 0, (long)p.groups * p.r, p.r, [&](long, float v) { s += v; });
            h[k] = (p.flags & 4) ? fmaxf(s, 0.0f) : s;
        }
    }
    // the weight loads stay ahead of the barrier (issued with the first partials, one wait for all)
    if (pre) {
        if (fold) {
#pragma unroll
            for (int u = 0; u < 4; u++) keep_in_vgprs(wsv[u]);
        }
#pragma unroll
        for (int u = 0; u < 4; u++) keep_in_vgprs(w2v[u]);
    }
    __syncthreads();
    if (ch >= p.c) return;
    float z;
    if (pre) {
        z = 0.0f;
#pragma unroll
        for (int u = 0; u < 4; u++)
            if (lane + 64 * u < p.r) z = __builtin_fmaf(w2v[u], h[lane + 64 * u], z);
        z = wave_sum(z);
    } else {
        z = wave_sum(row_dot(p.w2 + (long)ch * p.r, p.r, lane, [&](int k) { return h[k]; }));
    }
    const float gate = se_gate_value(p, ch, z);
    if (fold) {
        T* __restrict__ wd = (T*)p.wdst;
        if (pre) {
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int n = lane + 64 * u;
                if (n < p.wn) wd[(long)n * p.wk + ch] = se_scaled(__builtin_bit_cast(T, (WU)wsv[u]), gate);
            }
        } else {
            strided_foreach<4>(ws + ch, (long)lane * p.wk, (long)p.wn * p.wk, 64L * p.wk,
                               [&](long i, T v) { wd[ch + i] = se_scaled(v, gate); });
        }
    } else if (lane == 0) {
        ((T*)p.s)[(long)b * p.c + ch] = (T)gate;
    }
}

extern "C" __global__ void __launch_bounds__(256) sox_se_fc2_f16(sox_se_args p) { se_fc2_body<half_t>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_se_fc2_bf16(sox_se_args p) { se_fc2_body<bf16_t>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_se_fc2_f32(sox_se_args p) { se_fc2_body<float>(p); }

// ------------------------------------------------------------------------------------------
// Depthwise tiles + their SE gate in one launch (sox_dwt_se_args). After its tile, a workgroup counts
// itself; the last tile of a channel group runs that group's fc1 (se_fc1_group), the last group's
// workgroup runs fc2 for all of the image's channels. The arithmetic is sox_se_fc1's and sox_se_fc2's,
// in the same order, so the gates and the folded weights equal the separate passes' bit for bit.
// ------------------------------------------------------------------------------------------
// Whether this workgroup is the last of `total` to arrive at `counter` (an agent-scope atomic
// increment that wraps back to 0 at the last arrival). What the arrivers hand over went out with
// store_coherent and wait_performed before the call, so it is performed before the count is; the last
// arriver reads it with load_coherent after.
__device__ __forceinline__ bool arrive_last(uint32_t* counter, uint32_t total, uint32_t* flag) {
    __syncthreads();
    if (threadIdx.x == 0) *flag = atomicInc(counter, total - 1) == total - 1;
    __syncthreads();
    const bool last = *flag != 0;
    asm volatile("" ::: "memory");
    return last;
}

// fc2 of image b in one workgroup: h into LDS, then a wave per channel (NB channels' W2 rows in flight
// per wave) into gate[] in LDS, then the folded weights (16-byte vectors along the channels) or s.
// lds: >= 4 (align64(r) + c) bytes; r <= 256; c % 8 == 0.
template <typename T>
__device__ __forceinline__ void se_fc2_image(const sox_se_args& p, int b, float* lds) {
    constexpr int NB = 8;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6, nw = blockDim.x >> 6;
    float* h = lds;
    float* gate = lds + ((p.r + 63) & ~63);
    const float* part = p.hid + (long)b * p.groups * p.r;
    for (int k = t; k < p.r; k += blockDim.x) {
        float s = (p.flags & 1) ? p.b1[k] : 0.0f;
        strided_foreach_ld<16, float>([&](long i) { return load_coherent(part + k + i); }, 0, (long)p.groups * p.r,
                                      p.r, [&](long, float v) { s += v; });
        h[k] = (p.flags & 4) ? fmaxf(s, 0.0f) : s;
    }
    __syncthreads();
    for (int c0 = wave * NB; c0 < p.c; c0 += nw * NB) {
        float w2v[NB][4];
#pragma unroll
        for (int j = 0; j < NB; j++) {
            const int ch = min(c0 + j, p.c - 1);
#pragma unroll
            for (int u = 0; u < 4; u++) w2v[j][u] = p.w2[(long)ch * p.r + min(lane + 64 * u, p.r - 1)];
        }
#pragma unroll
        for (int j = 0; j < NB; j++) {
            float z = 0.0f;
#pragma unroll
            for (int u = 0; u < 4; u++)
                if (lane + 64 * u < p.r) z = __builtin_fmaf(w2v[j][u], h[lane + 64 * u], z);
            z = wave_sum(z);
            if (lane == 0 && c0 + j < p.c) gate[c0 + j] = se_gate_value(p, c0 + j, z);
        }
    }
    __syncthreads();
    if (p.flags & SOX_SE_FOLD) {
        typedef vec_t<T, 8> T8;
        const int cv = p.c / 8;  // wk == c
        strided_foreach<8>((const T8*)p.wsrc, t, (long)p.wn * cv, blockDim.x, [&](long i, T8 v) {
            const float* gt = gate + (int)(i % cv) * 8;
            T8 o;
#pragma unroll
            for (int e = 0; e < 8; e++) o[e] = se_scaled(v[e], gt[e]);
            ((T8*)p.wdst)[i] = o;
        });
    } else {
        for (int ch = t; ch < p.c; ch += blockDim.x) ((T*)p.s)[(long)b * p.c + ch] = (T)gate[ch];
    }
}

#define SOX_DWT_SE(TY, T, K, S)                                                                                \
    extern "C" __global__ void __launch_bounds__(256) sox_dwt_##TY##_k##K##s##S##_se(sox_dwt_se_args p) {  \
        __shared__ __attribute__((aligned(16))) unsigned char lds[DwtShape<T, K, S>::LDS];                  \
        __shared__ uint32_t flag;                                                                              \
        dwt_body<T, K, S, true, true>(p.dw, lds);                                                              \
        const DwtCoords wc = dwt_coords();                                                                     \
        const int g = wc.g, b = wc.b, groups = p.se.groups;                                                    \
        uint32_t* sync = p.sync + (long)b * (groups + 1);                                                      \
        if (!arrive_last(sync + g, p.dw.tiles_x * p.dw.tiles_y, &flag)) return;                               \
        se_fc1_group<true>(p.se, g, b, (float*)lds, (float*)lds + 256);                                        \
        if (!arrive_last(sync + groups, groups, &flag)) return;                                                \
        se_fc2_image<T>(p.se, b, (float*)lds);                                                                 \
    }
SOX_DWT_SE(f16, half_t, 3, 1)
SOX_DWT_SE(f16, half_t, 3, 2)
SOX_DWT_SE(f16, half_t, 5, 1)
SOX_DWT_SE(f16, half_t, 5, 2)
SOX_DWT_SE(bf16, bf16_t, 3, 1)
SOX_DWT_SE(bf16, bf16_t, 3, 2)
SOX_DWT_SE(bf16, bf16_t, 5, 1)
SOX_DWT_SE(bf16, bf16_t, 5, 2)
SOX_DWT_SE(f32, float, 3, 1)
SOX_DWT_SE(f32, float, 3, 2)
SOX_DWT_SE(f32, float, 5, 1)
SOX_DWT_SE(f32, float, 5, 2)

// ------------------------------------------------------------------------------------------
// Per-channel broadcast y[p, c] = act(x[p, c] op v[img, c]) (ChannelBroadcast, Nhwc.Det.cs:317-351).
// ------------------------------------------------------------------------------------------
template <typename T, int CV>
__device__ __forceinline__ void chan_body(const sox_chan_args& p) {
    const int cvn = p.c / CV;
    const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= p.rows * cvn) return;
    const long row = idx / cvn;
    const int c0 = (int)(idx % cvn) * CV;
    const long img = (p.flags & 2) ? 0 : row / p.hw;
    typedef typename VecT<T, CV>::Vec Vec;
    Vec xv = *(const Vec*)((const T*)p.x + row * p.c + c0);
    Vec vv = *(const Vec*)((const T*)p.v + img * p.c + c0);
    const int act = (p.flags & SOX_F_ACT_MASK) >> SOX_F_ACT_SHIFT;
    const bool rev = p.flags & 1;
    Vec out;
#pragma unroll
    for (int e = 0; e < CV; e++) {
        float a = to_f(xv[e]), b = to_f(vv[e]);
        out[e] = (T)sox_act(rev ? sox_ew(b, a, p.op) : sox_ew(a, b, p.op), act);
    }
    *(Vec*)((T*)p.y + row * p.c + c0) = out;
}

extern "C" __global__ void __launch_bounds__(256) sox_chan_f16_v(sox_chan_args p) { chan_body<half_t, 8>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_chan_bf16_v(sox_chan_args p) { chan_body<bf16_t, 8>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_chan_f16_s(sox_chan_args p) { chan_body<half_t, 1>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_chan_bf16_s(sox_chan_args p) { chan_body<bf16_t, 1>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_chan_f32_v(sox_chan_args p) { chan_body<float, 4>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_chan_f32_s(sox_chan_args p) { chan_body<float, 1>(p); }

// ------------------------------------------------------------------------------------------
// Same-shape elementwise binary op + act (ew2v.comp), 16-byte vectors, scalar tail.
// ------------------------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ void ew_body(const sox_ew_args& p) {
    constexpr int CV = V16<T>::N;
    typedef typename V16<T>::Vec Vec;
    const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
    const long base = idx * CV;
    const int act = (p.flags & SOX_F_ACT_MASK) >> SOX_F_ACT_SHIFT;
    const T* a = (const T*)p.a;
    const T* b = (const T*)p.b;
    T* y = (T*)p.y;
    if (base + CV <= p.count) {
        Vec av = *(const Vec*)(a + base), bv = *(const Vec*)(b + base), out;
#pragma unroll
        for (int e = 0; e < CV; e++) out[e] = (T)sox_act(sox_ew(to_f(av[e]), to_f(bv[e]), p.op), act);
        *(Vec*)(y + base) = out;
    } else {
        for (long i = base; i < p.count; i++) y[i] = (T)sox_act(sox_ew(to_f(a[i]), to_f(b[i]), p.op), act);
    }
}

extern "C" __global__ void __launch_bounds__(256) sox_ew_f16(sox_ew_args p) { ew_body<half_t>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_ew_bf16(sox_ew_args p) { ew_body<bf16_t>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_ew_f32(sox_ew_args p) { ew_body<float>(p); }

// ------------------------------------------------------------------------------------------
// Unary: act / affine / hard-sigmoid / copy (unary.comp, unary2.comp, hsig.comp).
// ------------------------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ float unary_op(float v, const sox_unary_args& p) {
    switch (p.mode) {
        case 0: return sox_act(v, p.act);
        case 1: return v * p.alpha + p.beta;
        case 2: return fminf(fmaxf(v * p.alpha + p.beta, 0.0f), 1.0f);
        default: return v;
    }
}

template <typename T>
__device__ __forceinline__ void unary_body(const sox_unary_args& p) {
    constexpr int CV = V16<T>::N;
    typedef typename V16<T>::Vec Vec;
    const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
    const long base = idx * CV;
    const T* x = (const T*)p.x;
    T* y = (T*)p.y;
    if (base + CV <= p.count) {
        Vec xv = *(const Vec*)(x + base), out;
#pragma unroll
        for (int e = 0; e < CV; e++) out[e] = (T)unary_op<T>(to_f(xv[e]), p);
        *(Vec*)(y + base) = out;
    } else {
        for (long i = base; i < p.count; i++) y[i] = (T)unary_op<T>(to_f(x[i]), p);
    }
}

extern "C" __global__ void __launch_bounds__(256) sox_unary_f16(sox_unary_args p) { unary_body<half_t>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_unary_bf16(sox_unary_args p) { unary_body<bf16_t>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_unary_f32(sox_unary_args p) { unary_body<float>(p); }

// ------------------------------------------------------------------------------------------
// Nearest resize, asymmetric / floor (Nhwc.Det.cs:167-204) + optional [relu] addend; writes a
// channel slice [y_off, y_off + c) of a ldy-channel output (so FPN concats need no copy).
// ------------------------------------------------------------------------------------------
template <typename T, int CV>
__device__ __forceinline__ void nearest_body(const sox_nearest_args& p) {
    const int cvn = p.c / CV;
    // workgroups numbered XCD-major (when the grid divides by 8): the output rows that read the same
    // input row, a few workgroups apart, then run on one XCD and find that row in its L2
    const int G = gridDim.x;
    const int bid = G % 8 == 0 ? (int)(blockIdx.x % 8) * (G / 8) + (int)(blockIdx.x / 8) : (int)blockIdx.x;
    const long idx = (long)bid * blockDim.x + threadIdx.x;
    const long total = (long)p.n * p.oh * p.ow * cvn;
    if (idx >= total) return;
    const int c0 = (int)(idx % cvn) * CV;
    long pix = idx / cvn;
    const int ox = (int)(pix % p.ow);
    long q = pix / p.ow;
    const int oy = (int)(q % p.oh);
    const int b = (int)(q / p.oh);
    const int ys = min((int)floorf(oy / p.sy), p.ih - 1);
    const int xs = min((int)floorf(ox / p.sx), p.iw - 1);
    typedef typename VecT<T, CV>::Vec Vec;
    Vec v = *(const Vec*)((const T*)p.x + (((long)b * p.ih + ys) * p.iw + xs) * p.c + c0);
    if (p.flags & 1) {
        Vec av = *(const Vec*)((const T*)p.add + pix * p.c + c0);
#pragma unroll
        for (int e = 0; e < CV; e++) {
            float a = to_f(av[e]);
            v[e] = (T)(to_f(v[e]) + ((p.flags & 2) ? fmaxf(a, 0.0f) : a));
        }
    }
    *(Vec*)((T*)p.y + pix * p.ldy + p.y_off + c0) = v;
}

extern "C" __global__ void __launch_bounds__(256) sox_nearest_f16_v(sox_nearest_args p) { nearest_body<half_t, 8>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_nearest_bf16_v(sox_nearest_args p) { nearest_body<bf16_t, 8>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_nearest_f16_s(sox_nearest_args p) { nearest_body<half_t, 1>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_nearest_bf16_s(sox_nearest_args p) { nearest_body<bf16_t, 1>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_nearest_f32_v(sox_nearest_args p) { nearest_body<float, 4>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_nearest_f32_s(sox_nearest_args p) { nearest_body<float, 1>(p); }

// ------------------------------------------------------------------------------------------
// Channel-slice copy (NHWC concat along C, concat_ax.comp).
// ------------------------------------------------------------------------------------------
template <typename T, int CV>
__device__ __forceinline__ void slice_body(const sox_slice_copy_args& p) {
    const int cvn = p.c / CV;
    const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= p.rows * cvn) return;
    const long row = idx / cvn;
    const int c0 = (int)(idx % cvn) * CV;
    typedef typename VecT<T, CV>::Vec Vec;
    *(Vec*)((T*)p.y + row * p.ldy + p.y_off + c0) = *(const Vec*)((const T*)p.x + row * p.c + c0);
}

extern "C" __global__ void __launch_bounds__(256) sox_slice_f16_v(sox_slice_copy_args p) { slice_body<half_t, 8>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_slice_bf16_v(sox_slice_copy_args p) { slice_body<bf16_t, 8>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_slice_f16_s(sox_slice_copy_args p) { slice_body<half_t, 1>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_slice_bf16_s(sox_slice_copy_args p) { slice_body<bf16_t, 1>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_slice_f32_v(sox_slice_copy_args p) { slice_body<float, 4>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_slice_f32_s(sox_slice_copy_args p) { slice_body<float, 1>(p); }

// ------------------------------------------------------------------------------------------
// Staging conversions (f32to16.comp / f16to32.comp): fp16 / bf16 round to nearest even, as the
// (Half) cast.
// ------------------------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ void f32_to_body(const sox_cvt_args& p) {
    typedef vec_t<T, 4> T4;
    const long i = ((long)blockIdx.x * blockDim.x + threadIdx.x) * 4;
    const float* x = (const float*)p.x;
    T* y = (T*)p.y;
    if (i + 4 <= p.count) {
        const float4v v = *(const float4v*)(x + i);
        *(T4*)(y + i) = __builtin_convertvector(v, T4);  // round to nearest even
    } else {
        for (long j = i; j < p.count; j++) y[j] = (T)x[j];
    }
}

template <typename T>
__device__ __forceinline__ void to_f32_body(const sox_cvt_args& p) {
    typedef vec_t<T, 4> T4;
    const long i = ((long)blockIdx.x * blockDim.x + threadIdx.x) * 4;
    const T* x = (const T*)p.x;
    float* y = (float*)p.y;
    if (i + 4 <= p.count) {
        const T4 h = *(const T4*)(x + i);
        *(float4v*)(y + i) = __builtin_convertvector(h, float4v);
    } else {
        for (long j = i; j < p.count; j++) y[j] = (float)x[j];
    }
}

extern "C" __global__ void __launch_bounds__(256) sox_f32_to_f16(sox_cvt_args p) { f32_to_body<half_t>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_f32_to_bf16(sox_cvt_args p) { f32_to_body<bf16_t>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_f16_to_f32(sox_cvt_args p) { to_f32_body<half_t>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_bf16_to_f32(sox_cvt_args p) { to_f32_body<bf16_t>(p); }


// ------------------------------------------------------------------------------------------
// LayerNorm (Kernels/Ops.cs:544-574, Avx2Kernels.cs:562-600): one wave per row; single pass
// mean and E[x^2] - mean^2 (clamped at 0), inv = 1/sqrt(var + eps), y = (x - mean) * (inv*g) + b.
// ------------------------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ void ln_body(const sox_ln_args& p) {
    const long row = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= p.rows) return;
    const T* x = (const T*)p.x + row * p.len;
    T* y = (T*)p.y + row * p.len;
    // rows up to 512 stay in registers (8 per lane, loaded together); longer rows are re-read
    constexpr int R = 8;
    float xr[R];
    float s = 0.0f, ss = 0.0f;
    if (p.len <= 64 * R) {
#pragma unroll
        for (int u = 0; u < R; u++) xr[u] = to_f(x[min(lane + 64 * u, p.len - 1)]);
#pragma unroll
        for (int u = 0; u < R; u++)
            if (lane + 64 * u < p.len) {
                s += xr[u];
                ss = __builtin_fmaf(xr[u], xr[u], ss);
            }
    } else {
        strided_foreach<8>(x, lane, p.len, 64, [&](long, T v) {
            const float f = to_f(v);
            s += f;
            ss = __builtin_fmaf(f, f, ss);
        });
    }
    s = wave_sum(s);
    ss = wave_sum(ss);
    const float mean = s / p.len;
    const float inv = 1.0f / sqrtf(fmaxf(ss / p.len - mean * mean, 0.0f) + p.eps);
    if (p.len <= 64 * R) {
        float g[R], bt[R];
#pragma unroll
        for (int u = 0; u < R; u++) {
            const int i = min(lane + 64 * u, p.len - 1);
            g[u] = p.gamma[i];
            bt[u] = p.beta[i];
        }
#pragma unroll
        for (int u = 0; u < R; u++)
            if (lane + 64 * u < p.len) y[lane + 64 * u] = (T)__builtin_fmaf(xr[u] - mean, inv * g[u], bt[u]);
    } else {
        strided_foreach<8>(x, lane, p.len, 64, [&](long i, T v) {
            y[i] = (T)__builtin_fmaf(to_f(v) - mean, inv * p.gamma[i], p.beta[i]);
        });
    }
}

extern "C" __global__ void __launch_bounds__(256) sox_ln_f16(sox_ln_args p) { ln_body<half_t>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_ln_bf16(sox_ln_args p) { ln_body<bf16_t>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_ln_f32(sox_ln_args p) { ln_body<float>(p); }

// ------------------------------------------------------------------------------------------
// Row softmax (Kernels/Ops.Seq.cs:28-72): max, exp(x - max) by the shared exp core, 1/sum.
// One 256-thread workgroup per row.
// ------------------------------------------------------------------------------------------
// 16-bit rows of at most 8192 values read from a stride that is a multiple of 8: the thread's four
// 16-byte vectors stay in registers (one read of the row, the exps computed once), and the output,
// staged in LDS as 16-bit values, leaves in 16-byte stores aligned to the output (dense rows of any
// length start at any element), a scalar head and tail around them.
template <typename T>
__device__ __forceinline__ void softmax_regs(const sox_softmax_args& p, T* ob, float* red) {
    typedef vec_t<T, 8> T8;
    const long row = blockIdx.x;
    const int len = p.len, t = threadIdx.x, lane = t & 63, wv = t >> 6, nv = (len + 7) / 8;
    const T* x = (const T*)p.x + row * p.ldx;
    T8 v[4];
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const int j = t + 256 * u;
        if (j < nv) v[u] = *(const T8*)(x + 8 * j);
    }
    float f[4][8];
    float m = -INFINITY;
#pragma unroll
    for (int u = 0; u < 4; u++)
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const int i = 8 * (t + 256 * u) + e;
            f[u][e] = i < len ? (float)v[u][e] : -INFINITY;
            m = fmaxf(m, f[u][e]);
        }
    m = wave_max(m);
    if (lane == 0) red[wv] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    float s = 0.0f;
#pragma unroll
    for (int u = 0; u < 4; u++)
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const float ev = f[u][e] == -INFINITY ? 0.0f : exp16(f[u][e] - m);
            f[u][e] = ev;
            s += ev;
        }
    s = wave_sum(s);
    if (lane == 0) red[wv] = s;
    __syncthreads();
    const float inv = 1.0f / ((red[0] + red[1]) + (red[2] + red[3]));
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const int j = t + 256 * u;
        if (j < nv) {
            T8 o;
#pragma unroll
            for (int e = 0; e < 8; e++) o[e] = (T)(f[u][e] * inv);
            *(T8*)(ob + 8 * j) = o;
        }
    }
    __syncthreads();
    T* y = (T*)p.y + row * len;
    const int head = min(len, (int)(((16 - ((uintptr_t)y & 15)) & 15) / sizeof(T)));  // to a 16-byte boundary
    const int groups = (len - head) / 8, tail0 = head + 8 * groups;
    if (t < head) y[t] = ob[t];
    for (int g = t; g < groups; g += 256) {
        T8 o;
#pragma unroll
        for (int e = 0; e < 8; e++) o[e] = ob[head + 8 * g + e];
        *(T8*)(y + head + 8 * g) = o;
    }
    if (tail0 + t < len) y[tail0 + t] = ob[tail0 + t];
}

template <typename T>
__device__ __forceinline__ void softmax_body(const sox_softmax_args& p) {
    // the row is read once (16 loads in flight per thread) into LDS as fp32 when it fits (dynamic
    // LDS of len floats, granted by the host), then max, sum and the output come from LDS
    extern __shared__ __attribute__((aligned(16))) float rowbuf[];
    __shared__ float red[4];
    if constexpr (sizeof(T) == 2) {
        if (p.staged && p.ldx % 8 == 0 && p.len <= 8192 && p.len >= 8) {
            softmax_regs<T>(p, (T*)rowbuf, red);
            return;
        }
    }
    const long row = blockIdx.x;
    const T* x = (const T*)p.x + row * p.ldx;
    T* y = (T*)p.y + row * p.len;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const bool staged = p.staged != 0;
    float m = -INFINITY;
    typedef typename V16<T>::Vec Vec;
    constexpr int VE = V16<T>::N;
    if (staged && p.ldx % VE == 0) {
        // 16-byte aligned rows (a padded stride): vector loads, the last vector clipped at len
        const int nv = (p.len + VE - 1) / VE;
        strided_foreach<8>((const Vec*)x, threadIdx.x, nv, 256, [&](long j, Vec v) {
#pragma unroll
            for (int e = 0; e < VE; e++) {
                if (j * VE + e < p.len) {
                    const float f = to_f(v[e]);
                    m = fmaxf(m, f);
                    rowbuf[j * VE + e] = f;
                }
            }
        });
    } else {
        strided_foreach<16>(x, threadIdx.x, p.len, 256, [&](long i, T v) {
            const float f = to_f(v);
            m = fmaxf(m, f);
            if (staged) rowbuf[i] = f;
        });
    }
    m = wave_max(m);
    if (lane == 0) red[wv] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    // fp16 outputs take the hardware exp2 (~1 ulp of fp32, far below the fp16 rounding); fp32
    // outputs keep the shared Cephes-style exp core
    auto ex = [](float v) { return sizeof(T) == 2 ? __builtin_amdgcn_exp2f(v * 1.4426950408889634f) : sox_exp(v); };
    float s = 0.0f;
    if (staged) {  // each exp once: kept in the row buffer for the output pass
        for (int i = threadIdx.x; i < p.len; i += 256) {
            const float e = ex(rowbuf[i] - m);
            rowbuf[i] = e;
            s += e;
        }
    } else {
        strided_foreach<16>(x, threadIdx.x, p.len, 256, [&](long, T v) { s += sox_exp(to_f(v) - m); });
    }
    s = wave_sum(s);
    if (lane == 0) red[wv] = s;
    __syncthreads();
    const float inv = 1.0f / ((red[0] + red[1]) + (red[2] + red[3]));
    if (staged) {
        for (int i = threadIdx.x; i < p.len; i += 256) y[i] = (T)(rowbuf[i] * inv);
    } else {
        strided_foreach<16>(x, threadIdx.x, p.len, 256, [&](long i, T v) { y[i] = (T)(sox_exp(to_f(v) - m) * inv); });
    }
}

extern "C" __global__ void __launch_bounds__(256) sox_softmax_f16(sox_softmax_args p) { softmax_body<half_t>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_softmax_bf16(sox_softmax_args p) { softmax_body<bf16_t>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_softmax_f32(sox_softmax_args p) { softmax_body<float>(p); }

// ------------------------------------------------------------------------------------------
// Fused attention (attn.comp): one workgroup per (batch, head); K and V staged in LDS as fp32;
// one thread per query row with an online softmax (running max / sum rescaling). D <= 64.
// ------------------------------------------------------------------------------------------
template <typename T, int D>
__device__ __forceinline__ void attn_body(const sox_attn_args& p) {
    extern __shared__ float kv[];  // [s][D] keys then [s][D] values
    const int bh = blockIdx.x, b = bh / p.heads, h = bh - b * p.heads;
    const T* kp = (const T*)p.k + b * p.k_sb + h * p.k_sh;
    const T* vp = (const T*)p.v + b * p.v_sb + h * p.v_sh;
    float* ks = kv;
    float* vs = kv + p.s * D;
    for (int i = threadIdx.x; i < p.s * D; i += blockDim.x) {
        int j = i / D, e = i - j * D;
        ks[i] = e < p.d ? to_f(kp[j * p.k_st + e]) : 0.0f;
        vs[i] = e < p.d ? to_f(vp[j * p.v_st + e]) : 0.0f;
    }
    __syncthreads();
    for (int t = blockIdx.y * blockDim.x + threadIdx.x; t < p.t; t += gridDim.y * blockDim.x) {
        const T* qp = (const T*)p.q + b * p.q_sb + h * p.q_sh + t * p.q_st;
        float q[D], acc[D];
#pragma unroll
        for (int e = 0; e < D; e++) {
            q[e] = e < p.d ? to_f(qp[e]) : 0.0f;
            acc[e] = 0.0f;
        }
        float mx = -INFINITY, sum = 0.0f;
        for (int j = 0; j < p.s; j++) {
            float sc = 0.0f;
#pragma unroll
            for (int e = 0; e < D; e++) sc = __builtin_fmaf(q[e], ks[j * D + e], sc);
            sc *= p.scale;
            float nm = fmaxf(mx, sc);
            float corr = sox_exp(mx - nm), pj = sox_exp(sc - nm);
            sum = sum * corr + pj;
#pragma unroll
            for (int e = 0; e < D; e++) acc[e] = __builtin_fmaf(pj, vs[j * D + e], acc[e] * corr);
            mx = nm;
        }
        const float inv = 1.0f / sum;
        T* op = (T*)p.o + b * p.o_sb + h * p.o_sh + t * p.o_st;
#pragma unroll
        for (int e = 0; e < D; e++)
            if (e < p.d) op[e] = (T)(acc[e] * inv);
    }
}

extern "C" __global__ void __launch_bounds__(128) sox_attn_f16_d32(sox_attn_args p) { attn_body<half_t, 32>(p); }
extern "C" __global__ void __launch_bounds__(128) sox_attn_bf16_d32(sox_attn_args p) { attn_body<bf16_t, 32>(p); }
extern "C" __global__ void __launch_bounds__(128) sox_attn_f16_d64(sox_attn_args p) { attn_body<half_t, 64>(p); }
extern "C" __global__ void __launch_bounds__(128) sox_attn_bf16_d64(sox_attn_args p) { attn_body<bf16_t, 64>(p); }
extern "C" __global__ void __launch_bounds__(128) sox_attn_f32_d32(sox_attn_args p) { attn_body<float, 32>(p); }
extern "C" __global__ void __launch_bounds__(128) sox_attn_f32_d64(sox_attn_args p) { attn_body<float, 64>(p); }

// ------------------------------------------------------------------------------------------
// Max pool (+relu) over NHWC, constant padding ignored (maxpool.comp).
// ------------------------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ void pool_body(const sox_pool_args& p) {
    const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
    const long total = (long)p.n * p.oh * p.ow * p.c;
    if (idx >= total) return;
    const int c = (int)(idx % p.c);
    long pix = idx / p.c;
    const int ox = (int)(pix % p.ow);
    long q = pix / p.ow;
    const int oy = (int)(q % p.oh);
    const int b = (int)(q / p.oh);
    const T* x = (const T*)p.x + (long)b * p.ih * p.iw * p.c;
    float m = -INFINITY;
    bool any = false;
    for (int ky = 0; ky < p.kh; ky++) {
        int iy = oy * p.sh + ky - p.pt;
        if ((unsigned)iy >= (unsigned)p.ih) continue;
        for (int kx = 0; kx < p.kw; kx++) {
            int ix = ox * p.sw + kx - p.pl;
            if ((unsigned)ix >= (unsigned)p.iw) continue;
            m = fmaxf(m, to_f(x[((long)iy * p.iw + ix) * p.c + c]));
            any = true;
        }
    }
    if (!any) m = 0.0f;
    if (p.flags & 1) m = fmaxf(m, 0.0f);
    ((T*)p.y)[idx] = (T)m;
}

extern "C" __global__ void __launch_bounds__(256) sox_pool_f16(sox_pool_args p) { pool_body<half_t>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_pool_bf16(sox_pool_args p) { pool_body<bf16_t>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_pool_f32(sox_pool_args p) { pool_body<float>(p); }

// ------------------------------------------------------------------------------------------
// Attention on matrix cores (attn.comp's SDPA, D = 32 or 64, S <= 128), fp16 storage.
// One workgroup per (batch, head); its waves take 16 queries at a time. K ([s][d], rows padded by
// 16 bytes) and V^T ([d][s]) are staged in LDS once per workgroup with 16-byte loads, and each wave's
// first Q fragments load in the same round trip.
// S^T = K Q^T is built with v_mfma_f32_16x16x32_f16 (lane l: K row s = 16j + l%16, Q row t = l%16,
// 8 consecutive d), so lane l ends up holding the scores of query t = l%16 for keys
// s = 16j + 4(l/16) + i. The softmax over s is an in-register max/sum plus two cross-lane steps
// (lanes l, l^16, l^32, l^48), its numerators from the hardware exp2 (exp16). O = P V reuses that register layout directly as the MFMA A operand:
// within each 32-key step the lane's 8 keys are {32c + 4g + i, 32c + 16 + 4g + i} (g = l/16), and
// the B operand (V) is read at the same key permutation (two 8-byte runs of V^T), which leaves the
// sum over keys unchanged. Keys past S hold P = 0 and V = 0.
// ------------------------------------------------------------------------------------------
template <typename T, int NJ, int KD>
__device__ __forceinline__ void attn_mfma_body(const sox_attn_args& p) {
    // no contraction: the scaled score and its distance to the row max round separately, here and in the
    // fused qkv-attention kernel alike, so the two give the same bits
#pragma clang fp contract(off)
    typedef vec_t<T, 8> T8;
    typedef vec_t<T, 4> T4;
    constexpr int S = 16 * NJ, D = 32 * KD, NC = (NJ + 1) / 2, SP = 32 * NC, JD = 2 * KD;
    constexpr int KP = D + 8, VP = SP + 8;  // LDS row pitches in halves
    __shared__ __attribute__((aligned(16))) T ks[S * KP];
    __shared__ __attribute__((aligned(16))) T vt[D * VP];
    const int tid = threadIdx.x, nthr = blockDim.x, lane = tid & 63, wave = tid >> 6, nwaves = nthr >> 6;
    const int l16 = lane & 15, g = lane >> 4;
    const int bh = blockIdx.x;
    const int b = bh / p.heads, h = bh - b * p.heads;
    const T* __restrict__ q = (const T*)p.q + b * p.q_sb + h * p.q_sh;
    const T* __restrict__ k = (const T*)p.k + b * p.k_sb + h * p.k_sh;
    const T* __restrict__ v = (const T*)p.v + b * p.v_sb + h * p.v_sh;
    const int tblocks = (p.t + 15) / 16;
    auto load_q = [&](int tb, T8 (&qf)[KD]) {
        const int t = tb * 16 + l16;
#pragma unroll
        for (int kd = 0; kd < KD; kd++)
            qf[kd] = t < p.t ? *(const T8*)(q + (long)t * p.q_st + 32 * kd + 8 * g) : (T8)(T)0;
    };
    T8 qf[KD];
    if (wave < tblocks) load_q(wave, qf);
    for (int i = tid; i < SP * (D / 8); i += nthr) {
        const int s = i / (D / 8), c = i - s * (D / 8);
        const T8 zero = (T8)(T)0;
        const T8 vv = s < p.s ? *(const T8*)(v + (long)s * p.v_st + 8 * c) : zero;
        if (s < S) *(T8*)(ks + s * KP + 8 * c) = s < p.s ? *(const T8*)(k + (long)s * p.k_st + 8 * c) : zero;
#pragma unroll
        for (int e = 0; e < 8; e++) vt[(8 * c + e) * VP + s] = vv[e];
    }
    __syncthreads();
    for (int tb = wave; tb < tblocks; tb += nwaves) {
        if (tb != wave) load_q(tb, qf);
        float4v sc[NJ];
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            float4v acc = (float4v)0.0f;
#pragma unroll
            for (int kd = 0; kd < KD; kd++) {
                const T8 kf = *(const T8*)(ks + (16 * j + l16) * KP + 32 * kd + 8 * g);
                acc = mfma16x16x32(kf, qf[kd], acc);
            }
            sc[j] = acc;
        }
        float m = -INFINITY;
#pragma unroll
        for (int j = 0; j < NJ; j++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int s = 16 * j + 4 * g + i;
                const float x = s < p.s ? sc[j][i] * p.scale : -INFINITY;
                sc[j][i] = x;
                m = fmaxf(m, x);
            }
        m = fmaxf(m, __shfl_xor(m, 16, 64));
        m = fmaxf(m, __shfl_xor(m, 32, 64));
        float sum = 0.0f;
#pragma unroll
        for (int j = 0; j < NJ; j++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int s = 16 * j + 4 * g + i;
                const float e = s < p.s ? exp16(sc[j][i] - m) : 0.0f;
                sc[j][i] = e;
                sum += e;
            }
        sum += __shfl_xor(sum, 16, 64);
        sum += __shfl_xor(sum, 32, 64);
        float4v o[JD];
#pragma unroll
        for (int jd = 0; jd < JD; jd++) o[jd] = (float4v)0.0f;
#pragma unroll
        for (int c = 0; c < NC; c++) {
            T8 pa;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                pa[i] = (T)sc[2 * c][i];
                pa[4 + i] = 2 * c + 1 < NJ ? (T)sc[2 * c + 1][i] : (T)0;
            }
#pragma unroll
            for (int jd = 0; jd < JD; jd++) {
                const T* row = vt + (16 * jd + l16) * VP + 32 * c + 4 * g;
                const T4 lo = *(const T4*)row, hi = *(const T4*)(row + 16);
                const T8 vb = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                o[jd] = mfma16x16x32(pa, vb, o[jd]);
            }
        }
        T* __restrict__ out = (T*)p.o + b * p.o_sb + h * p.o_sh;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int tt = tb * 16 + 4 * g + i;
            const float inv = 1.0f / __shfl(sum, 4 * g + i, 64);
            if (tt < p.t)
#pragma unroll
                for (int jd = 0; jd < JD; jd++) out[(long)tt * p.o_st + 16 * jd + l16] = (T)(o[jd][i] * inv);
        }
    }
}

#define SOX_ATTN_MFMA(S, D)                                                                                  \
    extern "C" __global__ void __launch_bounds__(512) sox_attn_f16_mfma_s##S##_d##D(sox_attn_args p) {        \
        attn_mfma_body<half_t, S / 16, D / 32>(p);                                                           \
    }                                                                                                        \
    extern "C" __global__ void __launch_bounds__(512) sox_attn_bf16_mfma_s##S##_d##D(sox_attn_args p) {       \
        attn_mfma_body<bf16_t, S / 16, D / 32>(p);                                                           \
    }
SOX_ATTN_MFMA(32, 32)
SOX_ATTN_MFMA(64, 32)
SOX_ATTN_MFMA(80, 32)
SOX_ATTN_MFMA(128, 32)
SOX_ATTN_MFMA(32, 64)
SOX_ATTN_MFMA(64, 64)
SOX_ATTN_MFMA(80, 64)
SOX_ATTN_MFMA(128, 64)

// ------------------------------------------------------------------------------------------
// Direct conv for few input channels (3-channel stems; convpool.comp / conv_tile.comp's role):
// one work item = one output pixel x OCV output channels; the packed [oc][kpad] weights are
// staged once per workgroup in LDS as fp32. acc = bias + sum over taps, channels (FMA), then
// residual and activation, one 16-byte store.
// POOL (SOX_F_POOL, ConvP.Pool of a small-ic stem, Kernels/Nhwc.cs:661-727 / convpool.comp): the work
// item is one pixel of the 2x2/2 max pool over the conv output instead. It computes the four conv
// pixels of its quad (top-left, top-right, bottom-left, bottom-right, each with its bias and
// activation, as the separate Conv node would), folds them with max in that order (PoolBand), then
// the pool's relu, and stores only the pooled pixel: the full-resolution conv is never written.
// p.m counts output (pooled) pixels, p.oh / p.ow stay the conv output's size (twice the pooled one).
// ------------------------------------------------------------------------------------------
template <typename T, int OCV, bool POOL>
__device__ __forceinline__ void conv_direct_body(const sox_igemm_args& p) {
    extern __shared__ float wl[];  // [oc][K]
    const int K = p.k;
    for (int i = threadIdx.x; i < p.n * K; i += blockDim.x) {
        int o = i / K, kk = i - o * K;
        wl[i] = to_f(((const T*)p.w)[(long)o * p.kpad + kk]);
    }
    __syncthreads();
    const int ocg = p.n / OCV;
    const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (long)p.m * ocg) return;
    const int og = (int)(idx % ocg);
    const long m = idx / ocg;
    const int yh = POOL ? p.oh / 2 : p.oh, yw = POOL ? p.ow / 2 : p.ow;  // output grid
    const int ohw = yh * yw;
    const int b = (int)(m / ohw), r = (int)(m - (long)b * ohw);
    const int py = r / yw, px = r - py * yw;
    const bool reflect = (p.flags & SOX_F_REFLECT) != 0;
    const int act = (p.flags & SOX_F_ACT_MASK) >> SOX_F_ACT_SHIFT;
    const T* __restrict__ x = (const T*)p.x + (long)b * p.ih * p.iw * p.ic;
    const float* w0 = wl + (long)og * OCV * K;
    // bias + taps of conv pixel (oy, ox)
    auto conv_at = [&](int oy, int ox, float (&acc)[OCV]) __attribute__((always_inline)) {
#pragma unroll
        for (int e = 0; e < OCV; e++) acc[e] = (p.flags & SOX_F_BIAS) ? p.bias[og * OCV + e] : 0.0f;
        for (int ky = 0; ky < p.kh; ky++) {
            int iy = sox_src_index(oy * p.sh + ky - p.pt, p.ih, reflect);
            for (int kx = 0; kx < p.kw; kx++) {
                int ix = sox_src_index(ox * p.sw + kx - p.pl, p.iw, reflect);
                const int k0 = (ky * p.kw + kx) * p.ic;
                for (int c = 0; c < p.ic; c++) {
                    float xv = iy < 0 || ix < 0 ? p.pad_value : to_f(x[((long)iy * p.iw + ix) * p.ic + c]);
#pragma unroll
                    for (int e = 0; e < OCV; e++) acc[e] = __builtin_fmaf(xv, w0[e * K + k0 + c], acc[e]);
                }
            }
        }
    };
    typedef typename VecT<T, OCV>::Vec Vec;
    const long o = m * p.ldy + og * OCV;
    Vec out;
    if constexpr (POOL) {
        float best[OCV];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            float acc[OCV];
            conv_at(2 * py + (q >> 1), 2 * px + (q & 1), acc);
#pragma unroll
            for (int e = 0; e < OCV; e++) {
                const float v = sox_act(acc[e], act);
                best[e] = q == 0 ? v : fmaxf(best[e], v);
            }
        }
#pragma unroll
        for (int e = 0; e < OCV; e++) out[e] = (T)((p.flags & SOX_F_POOL_RELU) ? fmaxf(best[e], 0.0f) : best[e]);
    } else {
        float acc[OCV];
        conv_at(py, px, acc);
        if (p.flags & SOX_F_RESIDUAL) {
            Vec av = *(const Vec*)((const T*)p.add + o);
#pragma unroll
            for (int e = 0; e < OCV; e++) acc[e] = acc[e] + to_f(av[e]);
        }
#pragma unroll
        for (int e = 0; e < OCV; e++) out[e] = (T)sox_act(acc[e], act);
    }
    *(Vec*)((T*)p.y + o) = out;
}

// 3x3 taps over 3 channels (the RGB stems): all 27 input values of a pixel are loaded up front
// (out-of-image taps read pixel 0 and take the pad value) instead of one dependent load per term.
// The weights are staged k-major ([K][oc]), so a thread's OCV weights of one term are OCV / 4
// 16-byte LDS reads. POOL as conv_direct_body.
template <typename T, int OCV, bool POOL>
__device__ __forceinline__ void conv_direct_333_body(const sox_igemm_args& p) {
    constexpr int KH = 3, KW = 3, IC = 3, K = KH * KW * IC;
    extern __shared__ float wl[];  // [K][oc]
    for (int i = threadIdx.x; i < p.n * K; i += blockDim.x) {
        const int o = i / K, kk = i - o * K;
        wl[kk * p.n + o] = to_f(((const T*)p.w)[(long)o * p.kpad + kk]);
    }
    __syncthreads();
    const int ocg = p.n / OCV;
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;  // m * ocg < 2^31 (the launcher checks)
    if (idx >= p.m * ocg) return;
    const int m = idx / ocg, og = idx - m * ocg;
    const int yh = POOL ? p.oh / 2 : p.oh, yw = POOL ? p.ow / 2 : p.ow;
    const int ohw = yh * yw;
    const int b = m / ohw, r = m - b * ohw;
    const int py = r / yw, px = r - py * yw;
    const bool reflect = (p.flags & SOX_F_REFLECT) != 0;
    const int act = (p.flags & SOX_F_ACT_MASK) >> SOX_F_ACT_SHIFT;
    const T* __restrict__ x = (const T*)p.x + (long)b * p.ih * p.iw * IC;
    const float* w0 = wl + og * OCV;  // oc % 4 == 0: 16-byte aligned rows
    auto conv_at = [&](int oy, int ox, float (&acc)[OCV]) __attribute__((always_inline)) {
        float xv[K];
#pragma unroll
        for (int ky = 0; ky < KH; ky++) {
            const int iy = sox_src_index(oy * p.sh + ky - p.pt, p.ih, reflect);
#pragma unroll
            for (int kx = 0; kx < KW; kx++) {
                const int ix = sox_src_index(ox * p.sw + kx - p.pl, p.iw, reflect);
                const bool in = iy >= 0 && ix >= 0;
                const T* px_ = x + (in ? ((long)iy * p.iw + ix) * IC : 0);
#pragma unroll
                for (int c = 0; c < IC; c++) {
                    const float v = to_f(px_[c]);  // always a valid address: issued with the others
                    xv[(ky * KW + kx) * IC + c] = in ? v : p.pad_value;
                }
            }
        }
#pragma unroll
        for (int e = 0; e < OCV; e++) acc[e] = (p.flags & SOX_F_BIAS) ? p.bias[og * OCV + e] : 0.0f;
#pragma unroll
        for (int kk = 0; kk < K; kk++) {
            float4v wv[OCV / 4];
#pragma unroll
            for (int v = 0; v < OCV / 4; v++) wv[v] = *(const float4v*)(w0 + kk * p.n + 4 * v);
#pragma unroll
            for (int e = 0; e < OCV; e++) acc[e] = __builtin_fmaf(xv[kk], wv[e / 4][e % 4], acc[e]);
        }
    };
    auto fin = [&](float v) __attribute__((always_inline)) {
        return sizeof(T) == 2 ? act_fast(v, act) : sox_act(v, act);
    };
    typedef typename VecT<T, OCV>::Vec Vec;
    const long o = (long)m * p.ldy + og * OCV;
    Vec out;
    if constexpr (POOL) {
        float best[OCV];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            float acc[OCV];
            conv_at(2 * py + (q >> 1), 2 * px + (q & 1), acc);
#pragma unroll
            for (int e = 0; e < OCV; e++) best[e] = q == 0 ? fin(acc[e]) : fmaxf(best[e], fin(acc[e]));
        }
#pragma unroll
        for (int e = 0; e < OCV; e++) out[e] = (T)((p.flags & SOX_F_POOL_RELU) ? fmaxf(best[e], 0.0f) : best[e]);
    } else {
        float acc[OCV];
        conv_at(py, px, acc);
        if (p.flags & SOX_F_RESIDUAL) {
            const Vec av = *(const Vec*)((const T*)p.add + o);
#pragma unroll
            for (int e = 0; e < OCV; e++) acc[e] = acc[e] + to_f(av[e]);
        }
#pragma unroll
        for (int e = 0; e < OCV; e++) out[e] = (T)fin(acc[e]);
    }
    *(Vec*)((T*)p.y + o) = out;
}

// 3x3 over 3 channels (the RGB stems), stride S = 1 or 2, 16-bit storage: one workgroup per 16 x 16 output
// pixels of one image, as a K = 27 matrix product on the matrix cores. The tile's input window
// ((16 - 1) S + 3 square, the reflection or pad value already applied) is staged in LDS once, every
// load of it issued before the first use; each wave then gathers the A fragments of 2 x 32 pixels from
// the window (k = (ky * 3 + kx) * 3 + c, zero past 27: the packed weights are zero there too) and runs
// two v_mfma_f32_32x32x16 steps per 32-channel block from accumulators holding the bias. The per-pixel
// kernel (conv_direct_333) spends 27 fp32 FMAs and two broadcast LDS reads per output and term.
template <typename T, int S>
__device__ __forceinline__ void conv_stem_body(const sox_igemm_args& p) {
    typedef vec_t<T, 8> T8;
    typedef vec_t<T, 4> T4;
    constexpr int IC = 3, K = 27, TO = 16, TH = (TO - 1) * S + 3, NEL = TH * TH * IC, NI = (NEL + 255) / 256;
    __shared__ T xt[NEL];  // [TH][TH][IC]
    const int oc = p.n, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, l32 = lane & 31, hl = lane >> 5;
    const int tiles_x = (p.ow + TO - 1) / TO;
    const int ty0 = (blockIdx.x / tiles_x) * TO, tx0 = (blockIdx.x % tiles_x) * TO, b = blockIdx.y;
    const bool reflect = (p.flags & SOX_F_REFLECT) != 0;
    const T* __restrict__ x = (const T*)p.x + (long)b * p.ih * p.iw * IC;
    const int iy0 = ty0 * S - p.pt, ix0 = tx0 * S - p.pl;
    {
        T xv[NI];
#pragma unroll
        for (int u = 0; u < NI; u++) {
            const int i = tid + 256 * u, r = i / (TH * IC), rem = i - r * (TH * IC), cx = rem / IC, c = rem - cx * IC;
            const int iy = sox_src_index(iy0 + r, p.ih, reflect), ix = sox_src_index(ix0 + cx, p.iw, reflect);
            const bool in = i < NEL && iy >= 0 && ix >= 0;
            const T v = x[in ? ((long)iy * p.iw + ix) * IC + c : 0];  // a valid address either way
            xv[u] = in ? v : (T)p.pad_value;
        }
#pragma unroll
        for (int u = 0; u < NI; u++)
            if (tid + 256 * u < NEL) xt[tid + 256 * u] = xv[u];
    }
    // the wave's W fragments and bias (oc <= 32: one 32-channel block; rows past oc are zero)
    const T* __restrict__ W = (const T*)p.w;
    T8 bw[2];
#pragma unroll
    for (int s2 = 0; s2 < 2; s2++)
        bw[s2] = l32 < oc ? *(const T8*)(W + (long)l32 * p.kpad + 16 * s2 + 8 * hl) : (T8)(T)0.0f;
    float4v bv[4];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const int n = 8 * q + 4 * hl;
        bv[q] = ((p.flags & SOX_F_BIAS) && n < oc) ? *(const float4v*)(p.bias + n) : (float4v)0.0f;
    }
    __syncthreads();
    const int act = (p.flags & SOX_F_ACT_MASK) >> SOX_F_ACT_SHIFT;
#pragma unroll
    for (int g2 = 0; g2 < 2; g2++) {
        const int pg = wave * 2 + g2;               // 32 pixels: tile rows 2 pg, 2 pg + 1
        const int ty = 2 * pg + (l32 >> 4), tx = l32 & 15;
        const T* base = xt + ((ty * S) * TH + tx * S) * IC;
        T8 a[2];
#pragma unroll
        for (int s2 = 0; s2 < 2; s2++)
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const int k = 16 * s2 + 8 * hl + e, ky = k / 9, r9 = k - 9 * ky;
                a[s2][e] = k < K ? base[ky * TH * IC + r9] : (T)0.0f;  // (kx, c) = r9 / 3, r9 % 3: contiguous
            }
        float16v acc;
#pragma unroll
        for (int q = 0; q < 4; q++)
#pragma unroll
            for (int e = 0; e < 4; e++) acc[4 * q + e] = bv[q][e];
        acc = mfma32x32x16(bw[0], a[0], acc);
        acc = mfma32x32x16(bw[1], a[1], acc);
        const int oy = ty0 + ty, ox = tx0 + tx;
        if (oy >= p.oh || ox >= p.ow) continue;
        const long m = ((long)b * p.oh + oy) * p.ow + ox;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int n = 8 * q + 4 * hl;
            if (n >= oc) continue;  // oc % 8 == 0: a group of 4 is whole or absent
            const long o = m * p.ldy + n;
            T4 rv = {};
            if (p.flags & SOX_F_RESIDUAL) rv = *(const T4*)((const T*)p.add + o);
            T4 h;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                float v = acc[4 * q + e];
                if (p.flags & SOX_F_RESIDUAL) v += (float)rv[e];
                h[e] = (T)act_fast(v, act);
            }
            *(T4*)((T*)p.y + o) = h;
        }
    }
}

#define SOX_STEM(S)                                                                                             \
    extern "C" __global__ void __launch_bounds__(256) sox_conv_stem_s##S##_f16(sox_igemm_args p) {              \
        conv_stem_body<half_t, S>(p);                                                                           \
    }                                                                                                           \
    extern "C" __global__ void __launch_bounds__(256) sox_conv_stem_s##S##_bf16(sox_igemm_args p) {             \
        conv_stem_body<bf16_t, S>(p);                                                                           \
    }
SOX_STEM(1)
SOX_STEM(2)

// Direct conv for few OUTPUT channels (oc < 8: a final 3x3 conv to an image or a probability map),
// fp16 with ic % 8 == 0: a 32-channel matrix tile would leave most of its columns empty. One work
// item = one output pixel x all OC channels (one instance per OC, so no FMA is spent on padding);
// the weights are staged once per workgroup in LDS as fp32, k-major and padded to 8 channels
// ([K][8], zeros past OC), so each input value meets its weights in one or two broadcast 16-byte
// LDS reads; the input comes in 16-byte runs of 8 channels.
template <typename T, int OC>
__device__ __forceinline__ void conv_narrow_body(const sox_igemm_args& p) {
    typedef vec_t<T, 8> T8;
    extern __shared__ float wl[];  // [K][8]
    const int K = p.k;
    for (int i = threadIdx.x; i < K * 8; i += blockDim.x) {
        const int kk = i >> 3, o = i & 7;
        wl[i] = o < OC ? (float)((const T*)p.w)[(long)o * p.kpad + kk] : 0.0f;
    }
    __syncthreads();
    const long m = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (m >= p.m) return;
    const int ohw = p.oh * p.ow;
    const int b = (int)(m / ohw), r = (int)(m - (long)b * ohw);
    const int oy = r / p.ow, ox = r - oy * p.ow;
    const bool reflect = (p.flags & SOX_F_REFLECT) != 0;
    const T* __restrict__ x = (const T*)p.x + (long)b * p.ih * p.iw * p.ic;
    float acc[OC];
#pragma unroll
    for (int e = 0; e < OC; e++) acc[e] = (p.flags & SOX_F_BIAS) ? p.bias[e] : 0.0f;
    for (int ky = 0; ky < p.kh; ky++) {
        const int iy = sox_src_index(oy * p.sh + ky - p.pt, p.ih, reflect);
        for (int kx = 0; kx < p.kw; kx++) {
            const int ix = sox_src_index(ox * p.sw + kx - p.pl, p.iw, reflect);
            const bool in = iy >= 0 && ix >= 0;
            const T* xr = x + ((long)(in ? iy : 0) * p.iw + (in ? ix : 0)) * p.ic;
            const float* wk = wl + (ky * p.kw + kx) * p.ic * 8;
            for (int c = 0; c < p.ic; c += 8) {
                const T8 xv = *(const T8*)(xr + c);  // pixel 0 for a padding tap (not used)
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const float xf = in ? (float)xv[j] : p.pad_value;  // the pad value stays fp32
                    const float4v w0 = *(const float4v*)(wk + (c + j) * 8);
#pragma unroll
                    for (int e = 0; e < (OC < 4 ? OC : 4); e++) acc[e] = __builtin_fmaf(xf, w0[e], acc[e]);
                    if constexpr (OC > 4) {
                        const float4v w1 = *(const float4v*)(wk + (c + j) * 8 + 4);
#pragma unroll
                        for (int e = 4; e < OC; e++) acc[e] = __builtin_fmaf(xf, w1[e - 4], acc[e]);
                    }
                }
            }
        }
    }
    const int act = (p.flags & SOX_F_ACT_MASK) >> SOX_F_ACT_SHIFT;
    const long o = m * p.ldy;
#pragma unroll
    for (int e = 0; e < OC; e++) {
        float v = acc[e];
        if (p.flags & SOX_F_RESIDUAL) v += (float)((const T*)p.add)[o + e];
        ((T*)p.y)[o + e] = (T)act_fast(v, act);
    }
}

#define SOX_CONV_NARROW(OC)                                                                                   \
    extern "C" __global__ void __launch_bounds__(256) sox_conv_narrow_f16_o##OC(sox_igemm_args p) { conv_narrow_body<half_t, OC>(p); } \
    extern "C" __global__ void __launch_bounds__(256) sox_conv_narrow_bf16_o##OC(sox_igemm_args p) { conv_narrow_body<bf16_t, OC>(p); }
SOX_CONV_NARROW(1) SOX_CONV_NARROW(2) SOX_CONV_NARROW(3) SOX_CONV_NARROW(4)
SOX_CONV_NARROW(5) SOX_CONV_NARROW(6) SOX_CONV_NARROW(7)

extern "C" __global__ void __launch_bounds__(256) sox_conv_direct_333_f16(sox_igemm_args p) { conv_direct_333_body<half_t, 8, false>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_conv_direct_333_bf16(sox_igemm_args p) { conv_direct_333_body<bf16_t, 8, false>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_conv_direct_333_f32(sox_igemm_args p) { conv_direct_333_body<float, 4, false>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_conv_direct_f16(sox_igemm_args p) { conv_direct_body<half_t, 8, false>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_conv_direct_bf16(sox_igemm_args p) { conv_direct_body<bf16_t, 8, false>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_conv_direct_f32(sox_igemm_args p) { conv_direct_body<float, 4, false>(p); }
// with the fused 2x2/2 max pool (SOX_F_POOL)
extern "C" __global__ void __launch_bounds__(256) sox_conv_direct_333_pool_f16(sox_igemm_args p) { conv_direct_333_body<half_t, 8, true>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_conv_direct_333_pool_bf16(sox_igemm_args p) { conv_direct_333_body<bf16_t, 8, true>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_conv_direct_333_pool_f32(sox_igemm_args p) { conv_direct_333_body<float, 4, true>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_conv_direct_pool_f16(sox_igemm_args p) { conv_direct_body<half_t, 8, true>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_conv_direct_pool_bf16(sox_igemm_args p) { conv_direct_body<bf16_t, 8, true>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_conv_direct_pool_f32(sox_igemm_args p) { conv_direct_body<float, 4, true>(p); }
