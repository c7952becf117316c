// Large 3x3 stride-1 zero-padded Conv2d over multiples of 256 output channels from LDS input halos on
// CDNA4 matrix cores: the fp16 / bf16 Conv2d route (conv_cm.comp, Backends/Vulkan/VkGraph.cs:555-703)
// for ic % 64 == 0, whose implicit-GEMM form moves every input pixel through the CU once per tap.
//  * A workgroup (8 waves) owns TH x TW = 8 x 32 output pixels x 256 output channels; wave w takes
//    tile rows 4 (w / 4) .. +3 (four 32-pixel blocks) x channels 64 (w % 4) .. +63 (two 32-channel
//    blocks): 8 v_mfma_f32_32x32x16 per 16-channel k-step, W as the row operand and pixels as the
//    column operand, so lane l ends with pixel l % 32 and channels 8q + 4(l / 32) + e in accumulator
//    4q + e, as in the Gemm ring (whose epilogue, store_tile, this kernel shares).
//  * The K loop walks 64-channel blocks x 9 taps; each (block, tap) is one K slice. The block's input
//    halo, (TH + 2) x (TW + 2) pixels x 64 channels (42.5 KiB), sits in one of two LDS halo buffers for
//    the block's nine slices, and each slice's [256 n][64 c] weights (32 KiB) run through a two-stage
//    ring. The next block's halo (or the next tile's first) loads in six parts during the first six
//    slices of the current block, into the other halo buffer. Per slice the CU moves 32 KiB of weights
//    and ~5 KiB of halo, where the implicit GEMM moves 32 + 32 KiB.
//  * Every LDS row (a pixel's or an output channel's 64 channels, 128 bytes) stores its 16-byte chunks
//    XOR-swizzled by swz<8>(row), applied on the DMA source side, so the 16 lanes one ds_read_b128 cycle
//    serves (16 consecutive pixels or channels, one chunk) hit 16 distinct bank groups.
//  * One wait (vmcnt 0) and one barrier per slice, at its start: the slice's weights and the halo part
//    issued with them have landed, and every wave is done with the stage the next issue refills. Each
//    k-step then reads its six fragments and runs its eight MFMAs; the other wave on the SIMD covers the
//    read latency. (Reading k-step s + 1's fragments during k-step s's MFMAs, with the barrier moved
//    into the last k-step as in the Gemm ring, measured slower: 148.0-150.6 against 145.8-148.3 us.)
//  * Persistent: grid.x workgroups walk the tiles with stride grid.x, numbered XCD-major, so the tiles
//    in flight on one XCD are neighbours that share halo rows in its L2; grid.y picks the 256-channel
//    block. The accumulators start from the bias (LDS, loaded once).
// The per-output sum order is the bias, then channel blocks, taps and 16-channel k-steps in the ring
// conv's order (channel blocks outermost), so the result equals the implicit-GEMM ring's bit for bit.
#include "gemm_ring.h"

template <typename T>
__device__ __forceinline__ void conv_h256_body(const sox_igemm_args& p) {
    typedef vec_t<T, 8> T8;
    constexpr int TH = 8, TW = 32, HWD = TW + 2, HP = (TH + 2) * HWD;  // 340 halo pixels
    constexpr int HSLOTS = HP * 8;                                    // 16-byte slots of a halo
    constexpr int H_IT = (HSLOTS + 511) / 512;                        // DMA rounds of 512 lanes: 6
    constexpr int H_LASTW = (HSLOTS - (H_IT - 1) * 512 + 63) / 64;    // waves with slots in the last: 3
    constexpr int HBUF = ((H_IT - 1) * 512 + H_LASTW * 64) * 16;      // 44032 bytes
    constexpr int WBUF = 256 * 128, W_IT = WBUF / (512 * 16);         // 32 KiB, 4 rounds
    constexpr int OFF_W = 2 * HBUF, OFF_B = OFF_W + 2 * WBUF, SMEM = OFF_B + 1024;
    static_assert(SMEM <= 160 * 1024 && HBUF % 1024 == 0 && H_IT <= 9, "LDS plan");
    __shared__ __attribute__((aligned(1024))) unsigned char smem[SMEM];

    const int t = threadIdx.x, lane = t & 63, l32 = lane & 31, hl = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int ph = wave >> 2, oq = wave & 3;

    const int N = p.n, ic = p.ic, ih = p.ih, iw = p.iw, oh = p.oh, ow = p.ow;
    const int n0 = blockIdx.y * 256;
    const int tiles_x = (ow + TW - 1) / TW, tiles_y = (oh + TH - 1) / TH, per_img = tiles_x * tiles_y;
    const int ntiles = (p.m / (oh * ow)) * per_img;
    const int ncb = ic / 64, nk = ncb * 9;
    const T* __restrict__ X = (const T*)p.x;
    const T* __restrict__ W = (const T*)p.w;
    const T* __restrict__ Z = (const T*)p.zeros;

    const int G = gridDim.x;
    const int b0 = G % 8 == 0 ? (blockIdx.x % 8) * (G / 8) + blockIdx.x / 8 : blockIdx.x;
    const int my_tiles = b0 < ntiles ? (ntiles - 1 - b0) / G + 1 : 0;
    const int S = my_tiles * nk;

    auto origin = [&](int k, int& b, int& oy0, int& ox0) __attribute__((always_inline)) {
        const int tl = b0 + k * G;
        b = tl / per_img;
        const int r = tl - b * per_img, ty = r / tiles_x;
        oy0 = ty * TH;
        ox0 = (r - ty * tiles_x) * TW;
    };
    // the weights of global slice gs (its block and tap) into ring stage gs & 1. Round i of the DMA
    // fills rows t / 8 + 64 i at slot t % 8, whose chunk (slot ^ swz<8>(row)) does not depend on i, so
    // one source pointer per lane serves every round (N % 256 == 0: every row exists)
    const int wrow = t >> 3;
    const T* __restrict__ wlane = W + (long)(n0 + wrow) * p.kpad + (((t & 7) ^ swz<8>(wrow)) << 3);
    auto issue_w = [&](int gs) __attribute__((always_inline)) {
        const int s = gs % nk, cb = s / 9, tap = s - cb * 9;
        unsigned char* dst = smem + OFF_W + (gs & 1) * WBUF + wave * 64 * 16;
        const T* src = wlane + tap * ic + cb * 64;
#pragma unroll
        for (int i = 0; i < W_IT; i++)
            __builtin_amdgcn_global_load_lds(src + (long)i * 64 * p.kpad, LDS_PTR(dst + i * 512 * 16), 16, 0, 0);
    };
    // part i of the halo of (the workgroup's tile k, channel block cb) into halo buffer hb
    auto issue_halo = [&](int k, int cb, int hb, int i) __attribute__((always_inline)) {
        if (i == H_IT - 1 && wave >= H_LASTW) return;  // past the halo's slots (wave-uniform)
        int b, oy0, ox0;
        origin(k, b, oy0, ox0);
        const int q = i * 512 + t, hp = q >> 3, c = (q & 7) ^ swz<8>(hp);  // c: the same for every i
        const int hy = hp / HWD, hx = hp - hy * HWD, iy = oy0 - 1 + hy, ix = ox0 - 1 + hx;
        const T* src = Z;
        if (hp < HP && (unsigned)iy < (unsigned)ih && (unsigned)ix < (unsigned)iw)
            src = X + (((long)b * ih + iy) * iw + ix) * ic + cb * 64 + c * 8;
        __builtin_amdgcn_global_load_lds(src, LDS_PTR(smem + hb * HBUF + (i * 512 + wave * 64) * 16), 16, 0, 0);
    };

    const int act = (p.flags & SOX_F_ACT_MASK) >> SOX_F_ACT_SHIFT;
    const T* __restrict__ R = (p.flags & SOX_F_RESIDUAL) ? (const T*)p.add : nullptr;
    T* __restrict__ Y = (T*)p.y;
    const float* bl = (const float*)(smem + OFF_B);
    float16v acc[4][2][1];
    T8 wf[2], pf[4];  // a k-step's fragments

    // the part of the next channel block's halo (or the next tile's first) that slice gs issues
    auto issue_next_halo = [&](int gs) __attribute__((always_inline)) {
        const int k = gs / nk, s = gs - k * nk, cb = s / 9, tap = s - cb * 9;
        if (tap >= H_IT) return;
        const int hb = (k * ncb + cb + 1) & 1;
        if (cb + 1 < ncb) issue_halo(k, cb + 1, hb, tap);
        else if (k + 1 < my_tiles) issue_halo(k + 1, 0, hb, tap);
    };
    // k-step ks's fragments of slice gs: the wave's two 32-channel weight rows and its four 32-pixel
    // rows of the halo, shifted by the slice's tap
    auto read_step = [&](int gs, int ks) __attribute__((always_inline)) {
        const int k = gs / nk, s = gs - k * nk, cb = s / 9, tap = s - cb * 9;
        const unsigned char* ws = smem + OFF_W + (gs & 1) * WBUF;
        const unsigned char* hs = smem + ((k * ncb + cb) & 1) * HBUF;
        const int dy = tap / 3, dx = tap - dy * 3, c = 2 * ks + hl;
        static_for<0, 2>([&](auto oo) {
            constexpr int ob = decltype(oo)::value;
            const int row = oq * 64 + ob * 32 + l32;
            wf[ob] = *(const T8*)(ws + row * 128 + ((c ^ swz<8>(row)) << 4));
        });
        static_for<0, 4>([&](auto rr) {
            constexpr int pr = decltype(rr)::value;
            const int hp = (4 * ph + pr + dy) * HWD + l32 + dx;
            pf[pr] = *(const T8*)(hs + hp * 128 + ((c ^ swz<8>(hp)) << 4));
        });
    };
    auto init_acc = [&]() __attribute__((always_inline)) {
        static_for<0, 8>([&](auto po) {
            constexpr int pr = decltype(po)::value / 2, ob = decltype(po)::value % 2;
            static_for<0, 4>([&](auto qq) {
                constexpr int q = decltype(qq)::value;
                const float4v b4 = *(const float4v*)(bl + oq * 64 + ob * 32 + 8 * q + 4 * hl);
                static_for<0, 4>([&](auto ee) {
                    constexpr int e = decltype(ee)::value;
                    acc[pr][ob][0][4 * q + e] = b4[e];
                });
            });
        });
    };

    // tile k's outputs: activation (+ residual) and stores from the accumulators; rows past oh are
    // skipped, and in the last column tile of a row whose width is not a multiple of 32 the pixels past
    // ow (lanes l32 >= ow - ox0: their m would run into the next row) by a row-local bound on m
    auto epilogue = [&](int k) __attribute__((always_inline)) {
        int b, oy0, ox0;
        origin(k, b, oy0, ox0);
        const int valid = min(TW, ow - ox0);
        static_for<0, 4>([&](auto rr) {
            constexpr int pr = decltype(rr)::value;
            const int oy = oy0 + 4 * ph + pr;
            if (oy < oh) {
                const int m0 = (b * oh + oy) * ow + ox0, mb = m0 + valid, nw = n0 + oq * 64;
                switch (act) {
                    case SOX_ACT_NONE: store_tile<T, SOX_ACT_NONE, 2, 1, false, true>(Y, R, p.ldy, mb, N, m0, nw, acc[pr]); break;
                    case SOX_ACT_RELU: store_tile<T, SOX_ACT_RELU, 2, 1, false, true>(Y, R, p.ldy, mb, N, m0, nw, acc[pr]); break;
                    case SOX_ACT_GELU: store_tile<T, SOX_ACT_GELU, 2, 1, false, true>(Y, R, p.ldy, mb, N, m0, nw, acc[pr]); break;
                    default: store_tile<T, -1, 2, 1, false, true>(Y, R, p.ldy, mb, N, m0, nw, acc[pr], act); break;
                }
            }
        });
    };

    if (S == 0) return;  // uniform: no tile for this workgroup
    if (wave == 0) {     // the 256 bias floats, once (zeros without a bias)
        const float* src = (p.flags & SOX_F_BIAS) ? p.bias + n0 + lane * 4 : (const float*)Z;
        __builtin_amdgcn_global_load_lds(src, LDS_PTR(smem + OFF_B), 16, 0, 0);
    }
    for (int i = 0; i < H_IT; i++) issue_halo(0, 0, 0, i);
    issue_w(0);
    for (int gs = 0; gs < S; gs++) {
        const int k = gs / nk, s = gs - k * nk;
        wait_vmcnt<0>();
        __builtin_amdgcn_s_barrier();
        if (gs + 1 < S) issue_w(gs + 1);
        issue_next_halo(gs);
        if (s == 0) init_acc();
        static_for<0, 4>([&](auto kk) {
            constexpr int ks = decltype(kk)::value;
            read_step(gs, ks);
            static_for<0, 8>([&](auto po) {
                constexpr int pr = decltype(po)::value / 2, ob = decltype(po)::value % 2;
                acc[pr][ob][0] = mfma32x32x16(wf[ob], pf[pr], acc[pr][ob][0]);
            });
        });
        wait_lgkmcnt0();
        if (s == nk - 1) epilogue(k);
    }
    wait_vmcnt<0>();
}

extern "C" __global__ void __launch_bounds__(512, 1) sox_conv_f16_h256(sox_igemm_args p) { conv_h256_body<half_t>(p); }
extern "C" __global__ void __launch_bounds__(512, 1) sox_conv_bf16_h256(sox_igemm_args p) { conv_h256_body<bf16_t>(p); }
