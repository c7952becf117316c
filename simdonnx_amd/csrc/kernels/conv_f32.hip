// fp32 implicit-GEMM Conv2d for short K (kh*kw*ic <= 576, a multiple of 64) on CDNA4 fp32 matrix
// cores: the Conv2d route of fp32 graphs where the whole reduction fits in LDS (conv_cm.comp's role
// for fp32 storage, Backends/Vulkan/VkGraph.cs:555-703; the CPU oracle is Nhwc.Dense,
// Kernels/Nhwc.cs:235-323).
//  * A workgroup owns 32 output pixels x 32 output channels. It copies the tile's whole im2col A
//    (32 x K) and W (32 x K) into LDS with global_load_lds (144 KiB at K = 576), in groups of 16 k
//    (64 contiguous bytes of a pixel per DMA lane quad); padding taps and rows / channels past M / N
//    read p.zeros or the last row.
//  * Each of its 4 waves multiplies a quarter of K for the whole tile with v_mfma_f32_16x16x4_f32
//    (2 x 2 blocks), and loads exactly that quarter of A and W itself, group by group in k order: no
//    barrier before the products, and group j's products wait only for the wave's loads up to group
//    j (loads complete in order), so they run while the later groups land. In group G lane group
//    g = l / 16 takes the 4 consecutive k 16 G + 4 g .. +3 (one 16-byte LDS read per operand), one
//    per MFMA step.
//  * The four partial tiles are summed through LDS in a fixed order; epilogue bias, residual,
//    activation (v = acc + bias + residual -> act), 16-byte stores with row stride ldy.
// Requirements (checked by the launcher): ic % 16 == 0, N % 4 == 0, constant-0 padding.
#include "gemm_ring.h"

template <int K>
__device__ __forceinline__ void conv_f32_short_body(const sox_igemm_args& p) {
    constexpr int BM = 32, BN = 32, CPR = K / 4;  // 16-byte k-chunks per row (a multiple of 16)
    constexpr int A_BYTES = CPR * BM * 16, BYTES = CPR * (BM + BN) * 16;
    constexpr int IT = BYTES / 1024 / 4;  // DMA instructions per wave (4 per 16-k group of its quarter)
    static_assert(K % 64 == 0 && BYTES <= 160 * 1024 && A_BYTES % 1024 == 0 && IT < 64 && IT == K / 16, "short-K tile");
    static_assert(4 * BM * BN * 4 <= BYTES, "partial tiles fit the operand space");
    // LDS: A then W, each [k / 16][row][4 chunks of 16 bytes] (a chunk = 4 consecutive k of one pixel /
    // channel row); within a row's 64 bytes chunk c % 4 sits at slot (c % 4) ^ ((row / 2) % 4), so the 16
    // lanes that read 16 consecutive rows of one chunk hit 8 distinct 16-byte bank groups
    __shared__ __attribute__((aligned(1024))) unsigned char smem[BYTES];

    const int t = threadIdx.x, lane = t & 63, wave = t >> 6, l16 = lane & 15, g = lane >> 4;
    const int M = p.m, N = p.n;
    const int m0 = blockIdx.x * BM, n0 = blockIdx.y * BN;

    // ---- the tile into LDS: the A (W) DMA instruction of chunk group gi and half h fills rows
    // 16 h + 0..15 of the group; lane l takes row 16 h + l / 4, slot l % 4. A chunk group is 16 k of one
    // tap (ic % 16 == 0), so its tap and first channel are wave-uniform and walk forward group by group;
    // a lane only adds its window origin, checks the image bounds and picks the address ----
    const int wv = __builtin_amdgcn_readfirstlane(wave);
    const int slot_c = (lane & 3) ^ ((lane >> 3) & 3);  // the chunk (mod 4) this lane's slot holds (row / 2 = lane / 8 mod 4)
    const int ohw = p.oh * p.ow;
    int iy0[2], ix0[2];
    const float* xo[2];  // the window origin of the lane's pixel (outside the image where the window starts there)
    const float* wr[2];
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const int row = 16 * h + (lane >> 2);
        const int m = min(m0 + row, M - 1), b = m / ohw, rem = m - b * ohw;
        const int oy = rem / p.ow, ox = rem - oy * p.ow;
        iy0[h] = oy * p.sh - p.pt;
        ix0[h] = ox * p.sw - p.pl;
        xo[h] = (const float*)p.x + (((long)b * p.ih + iy0[h]) * p.iw + ix0[h]) * p.ic + 4 * slot_c;
        wr[h] = (const float*)p.w + (long)min(n0 + row, N - 1) * p.kpad + 4 * slot_c;
    }
    const float* __restrict__ Z = (const float*)p.zeros;
    constexpr int GW = K / 64;  // 16-k chunk groups per wave: its quarter of K
    int ch, kx, ky;             // uniform: the tap and first channel of the wave's first group
    {
        const int k0 = 16 * GW * wv, tap = k0 / p.ic;
        ch = k0 - tap * p.ic;
        ky = tap / p.kw;
        kx = tap - ky * p.kw;
    }
    // group gi = GW wv + j: A rows 0-15 and 16-31, then W rows 0-15 and 16-31 (4 DMA instructions)
#pragma unroll
    for (int j = 0; j < GW; j++) {
        const int gi = GW * wv + j;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int iy = iy0[h] + ky, ix = ix0[h] + kx;
            const bool in = (unsigned)iy < (unsigned)p.ih && (unsigned)ix < (unsigned)p.iw;
            const float* src = in ? xo[h] + ((long)ky * p.iw + kx) * p.ic + ch : Z;
            __builtin_amdgcn_global_load_lds(src, LDS_PTR(smem + (2 * gi + h) * 1024), 16, 0, 0);
        }
#pragma unroll
        for (int h = 0; h < 2; h++)
            __builtin_amdgcn_global_load_lds(wr[h] + 16 * gi, LDS_PTR(smem + A_BYTES + (2 * gi + h) * 1024), 16, 0, 0);
        ch += 16;  // next group
        if (ch == p.ic) {
            ch = 0;
            if (++kx == p.kw) {
                kx = 0;
                ++ky;
            }
        }
    }

    // ---- this wave's quarter of K for the whole 32 x 32 tile ----
    float4v acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = (float4v)0.0f;
    static_for<0, GW>([&](auto jj) {
        constexpr int j = decltype(jj)::value;
        wait_vmcnt<4 * (GW - 1 - j)>();  // this wave's group j landed
        const int c = 4 * (GW * wv + j) + g;  // this lane's chunk (k / 4)
        float4v a[2], w[2];
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int r = 16 * i + l16, off = (c >> 2) * (BM * 64) + r * 64 + (((c & 3) ^ ((r >> 1) & 3)) << 4);
            a[i] = *(const float4v*)(smem + off);
            w[i] = *(const float4v*)(smem + A_BYTES + off);
        }
#pragma unroll
        for (int e = 0; e < 4; e++)
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int jn = 0; jn < 2; jn++) acc[i][jn] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i][e], w[jn][e], acc[i][jn], 0, 0, 0);
    });
    __syncthreads();  // every wave is done with the operands: their space takes the partial tiles

    // ---- partial tiles [wave][pixel][channel]; lane l of block (i, j) holds pixels 16 i + 4 g + q,
    // channel 16 j + l16 ----
    float* part = (float*)smem;
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int q = 0; q < 4; q++) part[(wave * BM + 16 * i + 4 * g + q) * BN + 16 * j + l16] = acc[i][j][q];
    __syncthreads();

    const int px = t >> 3, c4 = (t & 7) * 4;  // one pixel x 4 channels per thread
    const int mo = m0 + px, n = n0 + c4;
    if (mo >= M || n >= N) return;
    float4v v = (*(const float4v*)(part + (0 * BM + px) * BN + c4) + *(const float4v*)(part + (1 * BM + px) * BN + c4)) +
                (*(const float4v*)(part + (2 * BM + px) * BN + c4) + *(const float4v*)(part + (3 * BM + px) * BN + c4));
    if (p.flags & SOX_F_BIAS) v += *(const float4v*)(p.bias + n);
    const long o = (long)mo * p.ldy + n;
    if (p.flags & SOX_F_RESIDUAL) v += *(const float4v*)((const float*)p.add + o);
    const int act = (p.flags & SOX_F_ACT_MASK) >> SOX_F_ACT_SHIFT;
#pragma unroll
    for (int e = 0; e < 4; e++) v[e] = sox_act(v[e], act);
    *(float4v*)((float*)p.y + o) = v;
}

#define SOX_CONV_F32_SHORT(K)                                                                        \
    extern "C" __global__ void __launch_bounds__(256, 1) sox_conv_f32_short_k##K(sox_igemm_args p) { \
        conv_f32_short_body<K>(p);                                                                   \
    }
SOX_CONV_F32_SHORT(64)
SOX_CONV_F32_SHORT(128)
SOX_CONV_F32_SHORT(192)
SOX_CONV_F32_SHORT(256)
SOX_CONV_F32_SHORT(320)
SOX_CONV_F32_SHORT(384)
SOX_CONV_F32_SHORT(448)
SOX_CONV_F32_SHORT(512)
SOX_CONV_F32_SHORT(576)
