// Two chained stride-2 2x2 ConvTransposes in one kernel (sox_convt2_*): the DB head's
// ConvT(ic -> oc1) + bias + act1 followed by ConvT(oc1 -> 1) + bias + act2 (convt.comp dispatched for
// each by the reference, Backends/Vulkan/VkGraph.cs:918-926; on the CPU Kernels/Nhwc.Det.cs:51-131).
// Every output pixel of the second depends on one input pixel of the first, so a workgroup takes 128
// input pixels through both and only the 16 final values per pixel reach memory: the first one's
// 4 x oc1 outputs per pixel (an 11 MB map at the detector's 240 x 240 x 24) are neither written nor
// read back.
//  phase 1: the first ConvT as the same matrix product the LDS-DMA ring runs for it unfused
//           ([pixels][ic] x [ic][tap * oc1]): accumulators from zero, v_mfma_f32_32x32x16 over
//           k 0..15 then 16..31 (channels past ic are zero), then + bias[o], act1 and rounding to the
//           storage type, as the ring's ConvTranspose epilogue does: the staged values equal the
//           unfused first output bit for bit. Wave w takes pixels 32 w .. 32 w + 31, all 4 oc1
//           columns, into LDS.
//  phase 2: the second ConvT as sox_convt_one_* computes it: per (pixel, first-ConvT tap) item,
//           bias + the oc1 channels in order (fused multiply-adds against the [tap][oc1] weights
//           in fp32), act2, then two 2-value stores (one per output row).
#include "sox_device.h"

template <typename T, int NB>  // NB = 4 * oc1 / 32 column blocks of the first ConvT
__device__ __forceinline__ void convt2_body(const sox_convt2_args& p) {
    typedef vec_t<T, 8> T8;
    typedef vec_t<T, 4> T4;
    typedef vec_t<T, 2> T2;
    constexpr int NC = NB * 32, OC1 = NB * 8, PITCH = NC + 8;  // LDS row: 16 bytes of padding
    __shared__ __attribute__((aligned(16))) T hs[128 * PITCH];
    __shared__ float w2s[4 * OC1];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6, l32 = lane & 31, hl = lane >> 5;
    const long M = (long)p.n * p.ih * p.iw, pix0 = (long)blockIdx.x * 128;
    const T* __restrict__ X = (const T*)p.x;
    const T* __restrict__ W1 = (const T*)p.w1;
    if (t < 4 * OC1) w2s[t] = to_f(((const T*)p.w2)[t]);

    // ---- phase 1: the first ConvT on matrix cores ----
    const long m = pix0 + wave * 32 + l32;
    const T8 zero = {};
    // k-step s of lane l covers channels 16 s + 8 (l / 32) .. + 7 of its row (zero past ic)
    const T8 a0 = (m < M && 8 * hl < p.ic) ? *(const T8*)(X + m * p.ic + 8 * hl) : zero;
    const T8 a1 = (m < M && 16 + 8 * hl < p.ic) ? *(const T8*)(X + m * p.ic + 16 + 8 * hl) : zero;
    T* hrow = hs + (wave * 32 + l32) * PITCH;
#pragma unroll
    for (int j = 0; j < NB; j++) {
        const int n = 32 * j + l32;  // the column this lane feeds: tap n / oc1, channel n % oc1
        const T8 b0 = 8 * hl < p.ic ? *(const T8*)(W1 + (long)n * p.kpad + 8 * hl) : zero;
        const T8 b1 = 16 + 8 * hl < p.ic ? *(const T8*)(W1 + (long)n * p.kpad + 16 + 8 * hl) : zero;
        float16v acc = {};
        acc = mfma32x32x16(b0, a0, acc);
        acc = mfma32x32x16(b1, a1, acc);
        // lane l holds columns 32 j + 8 q + 4 (l / 32) + r, r = 0..3, of pixel l % 32
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int c0 = 32 * j + 8 * q + 4 * hl;
            T4 h;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int o = (c0 + r) % OC1;
                h[r] = (T)fp32_value(sox_act(acc[4 * q + r] + (p.b1 ? p.b1[o] : 0.0f), p.act1));
            }
            *(T4*)(hrow + c0) = h;
        }
    }
    __syncthreads();

    // ---- phase 2: the second ConvT, item (pixel, dy1, dx1); dx1 fastest, so a wave's stores of one
    // output row are contiguous ----
    const float bv = p.b2 ? p.b2[0] : 0.0f;
    const int OH = 4 * p.ih, OW = 4 * p.iw;
#pragma unroll
    for (int dy1 = 0; dy1 < 2; dy1++) {
        const int pl = t >> 1, dx1 = t & 1, t1 = dy1 * 2 + dx1;
        const long mm = pix0 + pl;
        if (mm >= M) continue;
        const T* hp = hs + pl * PITCH + t1 * OC1;
        float acc[4] = {bv, bv, bv, bv};
#pragma unroll
        for (int c0 = 0; c0 < OC1; c0 += 8) {
            const T8 hv = *(const T8*)(hp + c0);
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float he = to_f(hv[e]);
#pragma unroll
                for (int t2 = 0; t2 < 4; t2++) acc[t2] = __builtin_fmaf(he, w2s[t2 * OC1 + c0 + e], acc[t2]);
            }
        }
        const int x = (int)(mm % p.iw);
        const long q = mm / p.iw;
        const int y = (int)(q % p.ih), b = (int)(q / p.ih);
        const int Y = 2 * (2 * y + dy1), X0 = 2 * (2 * x + dx1);
#pragma unroll
        for (int dy2 = 0; dy2 < 2; dy2++) {
            T2 v;
            v[0] = (T)fp32_value(sox_act(acc[2 * dy2], p.act2));
            v[1] = (T)fp32_value(sox_act(acc[2 * dy2 + 1], p.act2));
            *(T2*)((T*)p.y + ((long)b * OH + Y + dy2) * OW + X0) = v;
        }
    }
}

#define SOX_CONVT2(NB)                                                                                   \
    extern "C" __global__ void __launch_bounds__(256) sox_convt2_f16_n##NB(sox_convt2_args p) {          \
        convt2_body<half_t, NB>(p);                                                                      \
    }                                                                                                    \
    extern "C" __global__ void __launch_bounds__(256) sox_convt2_bf16_n##NB(sox_convt2_args p) {         \
        convt2_body<bf16_t, NB>(p);                                                                      \
    }
SOX_CONVT2(1)
SOX_CONVT2(2)
SOX_CONVT2(3)
SOX_CONVT2(4)
