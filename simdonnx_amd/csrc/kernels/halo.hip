// Direct KH x KW convolution (stride SH x SW, zero padding) from an LDS halo tile on CDNA4 matrix
// cores: the fp16 Conv2d route (conv_cm.comp, Backends/Vulkan/VkGraph.cs:555-703) for convs with few
// output channels, whose implicit-GEMM form would fetch every input pixel kh*kw times.
//  * A workgroup owns a TH x TW tile of output pixels x 32 output channels. Per block of CB input
//    channels it copies the tile's input halo ((TH-1)SH+KH x (TW-1)SW+KW pixels) and the block's
//    weights [tap][32 n] into LDS with global_load_lds (padding pixels, channel tails and absent
//    output channels read p.zeros), double-buffered: block c+1 loads while block c multiplies.
//  * Halo pixels and weight rows are PITCH = 5 sixteen-byte slots apart (4 channel chunks + 1 pad
//    slot): 8 consecutive pixels then fall on 8 distinct 16-byte bank groups with no swizzle, so a
//    tap's fragment is the lane's base address + a compile-time offset.
//  * Each wave takes 2 output rows (32 pixels) x 32 channels: per tap and 16-channel k-step one
//    v_mfma_f32_32x32x16_f16 (weights as the row operand, pixels as the column operand: lane l ends
//    with pixel l % 32 and channels 8q + 4(l/32) + e in accumulator 4q + e, as in the Gemm ring).
//  * Epilogue: bias (in the accumulators from the start), residual, activation, 8-byte stores with
//    row stride ldy (a concat slice works).
// Every DMA lane writes a slot (the regions are padded to whole instructions), so every wave issues
// the same number of loads per block and one static vmcnt covers them.
// UPC (sox_conv_halo_*_upcat): the input is a channel concat of nearest upsamples by powers of two
// (the DB FPN's fuse = concat(up8(p5), up4(p4), up2(p3), p2), Backends/Vulkan/VkGraph.cs:486-510 and
// concat_ax.comp), never stored: each 8-channel chunk's DMA reads its source at (iy >> s, ix >> s).
// The gathered bytes are the concat's, so the result is the same bits.
#include "gemm_ring.h"

template <typename T, int KH, int KW, int SH, int SW, bool UPC>
__device__ __forceinline__ void halo_body(const sox_igemm_args& p) {
    typedef vec_t<T, 8> T8;
    typedef vec_t<T, 4> T4;
    constexpr int TW = 16, TH = 8, CB = 32, PITCH = 5;
    constexpr int HW = (TW - 1) * SW + KW, HH = (TH - 1) * SH + KH, HP = HH * HW, TAPS = KH * KW;
    constexpr int HALO_IT = (HP * PITCH + 255) / 256, W_IT = (TAPS * 32 * PITCH + 255) / 256;
    constexpr int HALO_SLOTS = HALO_IT * 256, W_SLOTS = W_IT * 256, STAGE = HALO_SLOTS + W_SLOTS;
    constexpr int LOADS = HALO_IT + W_IT;
    static_assert(2 * STAGE * 16 <= 160 * 1024, "two stages fit the LDS");
    static_assert(LOADS < 32, "vmcnt range");
    __shared__ __attribute__((aligned(1024))) unsigned char smem[2 * STAGE * 16];

    const int t = threadIdx.x, lane = t & 63, wave = t >> 6, l32 = lane & 31, hl = lane >> 5;
    const int M = p.m, N = p.n;
    const int tiles_x = (p.ow + TW - 1) / TW, tiles_y = (p.oh + TH - 1) / TH;
    const int tx = blockIdx.x % tiles_x, tyb = blockIdx.x / tiles_x;
    const int ty = tyb % tiles_y, b = tyb / tiles_y;
    const int n0 = blockIdx.y * 32;
    const int oy0 = ty * TH, ox0 = tx * TW;
    const int iy0 = oy0 * SH - p.pt, ix0 = ox0 * SW - p.pl;
    const T* __restrict__ X = (const T*)p.x + (long)b * p.ih * p.iw * p.ic;
    const T* __restrict__ W = (const T*)p.w;
    const T* __restrict__ Z = (const T*)p.zeros;
    const int ncb = (p.ic + CB - 1) / CB;

    // this thread's DMA sources in channel block 0 (nullptr: the slot is padding and reads zeros);
    // block c adds c * CB channels, and a chunk past ic reads zeros too
    const T* hsrc[HALO_IT];
    int hch[HALO_IT], hpy[UPC ? HALO_IT : 1], hpx[UPC ? HALO_IT : 1];
#pragma unroll
    for (int i = 0; i < HALO_IT; i++) {
        const int q = i * 256 + t, hp = q / PITCH, sub = q - hp * PITCH;
        const int hy = hp / HW, hx = hp - hy * HW, iy = iy0 + hy, ix = ix0 + hx;
        const bool ok = q < HP * PITCH && sub < 4 && (unsigned)iy < (unsigned)p.ih && (unsigned)ix < (unsigned)p.iw;
        if constexpr (UPC) {  // hsrc only flags the pixel in the image; the source is picked per block
            hsrc[i] = ok ? Z : nullptr;
            hpy[i] = iy;
            hpx[i] = ix;
        } else {
            hsrc[i] = ok ? X + ((long)iy * p.iw + ix) * p.ic + sub * 8 : nullptr;
        }
        hch[i] = sub * 8;
    }
    const T* wsrc[W_IT];
    int wch[W_IT];
#pragma unroll
    for (int i = 0; i < W_IT; i++) {
        const int q = i * 256 + t, row = q / PITCH, sub = q - row * PITCH;
        const int tap = row / 32, n = row - tap * 32;
        const bool ok = q < TAPS * 32 * PITCH && sub < 4 && n0 + n < N;
        wsrc[i] = ok ? W + (long)(n0 + n) * p.kpad + tap * p.ic + sub * 8 : nullptr;
        wch[i] = sub * 8;
    }
    auto issue = [&](int cb, int stage) __attribute__((always_inline)) {
        unsigned char* st = smem + stage * STAGE * 16 + wave * 64 * 16;
        const int c0 = cb * CB;
#pragma unroll
        for (int i = 0; i < HALO_IT; i++) {
            const T* src = Z;
            if constexpr (UPC) {
                const int c = c0 + hch[i];
                if (hsrc[i] && c < p.ic) {
                    const int s = c / p.up_c, cl = c - s * p.up_c;
                    const int sh = s == 0 ? p.up_shift[0] : s == 1 ? p.up_shift[1] : s == 2 ? p.up_shift[2] : p.up_shift[3];
                    const void* up = s == 0 ? p.up[0] : s == 1 ? p.up[1] : s == 2 ? p.up[2] : p.up[3];
                    const int sw = p.iw >> sh;
                    src = (const T*)up + (((long)b * (p.ih >> sh) + (hpy[i] >> sh)) * sw + (hpx[i] >> sh)) * p.up_c + cl;
                }
            } else {
                if (hsrc[i] && c0 + hch[i] < p.ic) src = hsrc[i] + c0;
            }
            __builtin_amdgcn_global_load_lds(src, LDS_PTR(st + i * 256 * 16), 16, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < W_IT; i++) {
            const T* src = wsrc[i] && c0 + wch[i] < p.ic ? wsrc[i] + c0 : Z;
            __builtin_amdgcn_global_load_lds(src, LDS_PTR(st + (HALO_SLOTS + i * 256) * 16), 16, 0, 0);
        }
    };

    // lane's output pixel (row 2 wave + l32 / 16, column l32 % 16 of the tile) and fragment bases
    const int py = 2 * wave + (l32 >> 4), px = l32 & 15;
    const int a_base = ((py * SH * HW + px * SW) * PITCH + hl) * 16;
    const int b_base = (HALO_SLOTS + l32 * PITCH + hl) * 16;

    float16v acc;
    const bool has_bias = (p.flags & SOX_F_BIAS) != 0;
    static_for<0, 16>([&](auto qe) {
        constexpr int q = decltype(qe)::value / 4, e = decltype(qe)::value % 4;
        const int n = n0 + 8 * q + 4 * hl + e;
        acc[decltype(qe)::value] = has_bias && n < N ? p.bias[n] : 0.0f;
    });

    issue(0, 0);
    for (int cb = 0; cb < ncb; cb++) {
        issue(cb + 1, (cb + 1) & 1);  // past the last block: zeros into the idle stage, never read
        wait_vmcnt<LOADS>();          // this wave's block cb landed
        __builtin_amdgcn_s_barrier();  // ... and every wave's
        const unsigned char* st = smem + (cb & 1) * STAGE * 16;
        static_for<0, TAPS * 2>([&](auto ts) {
            constexpr int tap = decltype(ts)::value / 2, s = decltype(ts)::value % 2;
            constexpr int a_off = (((tap / KW) * HW + tap % KW) * PITCH + 2 * s) * 16;
            constexpr int b_off = (tap * 32 * PITCH + 2 * s) * 16;
            const T8 wf = *(const T8*)(st + b_base + b_off);
            const T8 af = *(const T8*)(st + a_base + a_off);
            acc = mfma32x32x16(wf, af, acc);
        });
        wait_lgkmcnt0();
        __builtin_amdgcn_s_barrier();  // stage cb & 1 is refilled by the next iteration's issue
    }
    wait_vmcnt<0>();

    const int oy = oy0 + py, ox = ox0 + px;
    if (oy >= p.oh || ox >= p.ow) return;
    const long m = ((long)b * p.oh + oy) * p.ow + ox;
    if (m >= M) return;
    const int act = (p.flags & SOX_F_ACT_MASK) >> SOX_F_ACT_SHIFT;
    const T* __restrict__ R = (p.flags & SOX_F_RESIDUAL) ? (const T*)p.add : nullptr;
    T* __restrict__ Y = (T*)p.y + m * p.ldy;
    const bool aligned = ((p.ldy | N) & 3) == 0;
    static_for<0, 4>([&](auto qq) {
        constexpr int q = decltype(qq)::value;
        const int n = n0 + 8 * q + 4 * hl;
        if (n >= N) return;
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            v[e] = acc[4 * q + e];
            if (R && n + e < N) v[e] += (float)R[m * p.ldy + n + e];
            v[e] = act_fast(v[e], act);
        }
        if (aligned) {
            T4 h;
#pragma unroll
            for (int e = 0; e < 4; e++) h[e] = (T)v[e];
            *(T4*)(Y + n) = h;
        } else {
#pragma unroll
            for (int e = 0; e < 4; e++)
                if (n + e < N) Y[n + e] = (T)v[e];
        }
    });
}

#define SOX_HALO(NAME, T, KH, KW, SH, SW, OCC, UPC)                                               \
    extern "C" __global__ void __launch_bounds__(256, OCC) NAME(sox_igemm_args p) {            \
        halo_body<T, KH, KW, SH, SW, UPC>(p);                                                  \
    }

SOX_HALO(sox_conv_halo_f16_3x3s1, half_t, 3, 3, 1, 1, 2, false)
SOX_HALO(sox_conv_halo_bf16_3x3s1, bf16_t, 3, 3, 1, 1, 2, false)
SOX_HALO(sox_conv_halo_f16_3x3s1_upcat, half_t, 3, 3, 1, 1, 2, true)
SOX_HALO(sox_conv_halo_bf16_3x3s1_upcat, bf16_t, 3, 3, 1, 1, 2, true)
