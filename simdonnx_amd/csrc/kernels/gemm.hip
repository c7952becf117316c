// Large fp16 Gemm with fused bias + activation on CDNA4 matrix cores (the conv_cm.comp Gemm route,
// Backends/Vulkan/VkGraph.cs:760-773, rebuilt for gfx950):
//   Y[M,N] = act(A[M,K] . W[N,K]^T + bias[N]),  A dense rows (lda), W packed [N][kpad] k-fastest,
//   fp16 storage, fp32 accumulation, fp16 output.
//
// Structure (256 threads = 4 waves, BM x BN tile, BK-deep K slices):
//  * K slices move global -> LDS with global_load_lds_dwordx4 (no register staging), STAGES deep:
//    slice k+STAGES-1 is in flight while slice k is multiplied. Completion is tracked with an
//    explicit s_waitcnt vmcnt + s_barrier per slice.
//  * LDS rows are BK fp16 (128 B for BK = 64) of 16-byte chunks stored XOR-swizzled
//    (slot = chunk ^ f(row), f(r) = (r & 7) ^ ((r >> 3) & 1)), so the 16 lanes of an MFMA
//    fragment read (16 rows, same chunk) hit 16 distinct 16-byte bank groups. The swizzle is applied
//    on the load side: each lane of a DMA instruction fetches the chunk that belongs at its slot.
//  * v_mfma_f32_16x16x32_f16 with W as the row operand and A as the column operand: lane l then
//    holds Y^T[n = 4(l/16) + q][m = l%16], i.e. 4 consecutive output channels of one row, so the
//    epilogue applies bias / activation on float4s and writes 8-byte packets to an LDS staging tile,
//    from which the workgroup stores full 16-byte row segments (coalesced, no partial lines).
//  * Tile order is XCD-aware: the hardware deals workgroups round-robin to the 8 XCDs, so block b
//    is remapped to tile (b % 8) * (tiles / 8) + b / 8, and tiles are walked in groups of GM
//    M-tiles, so the workgroups resident on one XCD share A rows and W columns in its L2.
#include "sox_device.h"

#define LDS_PTR(p) ((__attribute__((address_space(3))) void*)(p))

// s_waitcnt with only vmcnt constrained (gfx9 encoding: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt_hi[15:14]).
template <int N> SOX_DEV void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

SOX_DEV int swz(int r) { return (r & 7) ^ ((r >> 3) & 1); }

// erf-GELU with the A&S 7.1.26 polynomial evaluated with the hardware reciprocal and exp2 (fp16
// outputs: the approximations' ~1e-7 relative error is far below the fp16 output rounding).
SOX_DEV float gelu_fast(float x) {
    float z = x * 0.70710678118654752f;
    float az = fabsf(z);
    float t = __builtin_amdgcn_rcpf(__builtin_fmaf(0.3275911f, az, 1.0f));
    float p = 1.061405429f;
    p = __builtin_fmaf(p, t, -1.453152027f);
    p = __builtin_fmaf(p, t, 1.421413741f);
    p = __builtin_fmaf(p, t, -0.284496736f);
    p = __builtin_fmaf(p, t, 0.254829592f);
    float e = __builtin_amdgcn_exp2f(-(az * az) * 1.4426950408889634f);
    float erf = copysignf(1.0f - (p * t) * e, z);
    return (0.5f * x) * (1.0f + erf);
}

SOX_DEV float act_fast(float v, int act) { return act == SOX_ACT_GELU ? gelu_fast(v) : sox_act(v, act); }

template <int BM, int BN, int BK, int WM, int WN, int STAGES, int GM>
__device__ __forceinline__ void gemm_body(const sox_igemm_args& p) {
    constexpr int CPR = BK / 8;                 // 16-byte chunks per LDS row
    constexpr int ROWB = BK * 2;                // LDS row bytes
    constexpr int A_BYTES = BM * ROWB, B_BYTES = BN * ROWB;
    constexpr int A_IT = A_BYTES / 1024 / 4;    // DMA instructions per wave per slice (1 KiB each)
    constexpr int B_IT = B_BYTES / 1024 / 4;
    constexpr int LOADS = A_IT + B_IT;
    constexpr int TJ = WN / 16, TI = WM / 16;   // MFMA blocks: n (rows) x m (cols)
    constexpr int WAVES_N = BN / WN;
    constexpr int STAGE_BYTES = A_BYTES + B_BYTES;
    constexpr int EPI_ROW = BN + 8;             // epilogue staging row (fp16), 16 B pad
    constexpr int LDS_BYTES = STAGE_BYTES * STAGES > BM * EPI_ROW * 2 ? STAGE_BYTES * STAGES : BM * EPI_ROW * 2;
    static_assert(CPR == 8, "the swizzle assumes 8 chunks per row (BK = 64)");
    static_assert((BM / WM) * (BN / WN) == 4 && A_IT >= 1 && B_IT >= 1, "tiling");
    static_assert((STAGES - 2) * LOADS < 64, "vmcnt range");

    __shared__ __attribute__((aligned(1024))) unsigned char smem[LDS_BYTES];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l16 = lane & 15, g = lane >> 4;
    const int M = p.m, N = p.n, K = p.k;
    const int tiles_n = p.tiles_n, tiles_m = (M + BM - 1) / BM, ntiles = tiles_m * tiles_n;

    // ---- XCD-aware, grouped tile order ----
    int bid = blockIdx.x;
    if (ntiles % 8 == 0) bid = (bid % 8) * (ntiles / 8) + bid / 8;
    const int group = bid / (GM * tiles_n), first_m = group * GM;
    const int gsize = min(tiles_m - first_m, GM);
    const int in_group = bid - group * GM * tiles_n;
    const int bm = (first_m + in_group % gsize) * BM;
    const int bn = (in_group / gsize) * BN;

    const int wm0 = (wave / WAVES_N) * WM, wn0 = (wave % WAVES_N) * WN;
    const half_t* __restrict__ A = (const half_t*)p.x;
    const half_t* __restrict__ W = (const half_t*)p.w;

    // ---- DMA source addresses: lane l of instruction i of this wave fills LDS slot l of the
    //      1 KiB block (wave * IT + i); that slot is (row, slot) -> global chunk slot ^ swz(row)
    const half_t* a_src[A_IT];
    const half_t* b_src[B_IT];
#pragma unroll
    for (int i = 0; i < A_IT; i++) {
        int r = (wave * A_IT + i) * 8 + lane / 8;
        int c = (lane % 8) ^ swz(r);
        int m = min(bm + r, M - 1);
        a_src[i] = A + (long)m * p.lda + c * 8;
    }
#pragma unroll
    for (int i = 0; i < B_IT; i++) {
        int r = (wave * B_IT + i) * 8 + lane / 8;
        int c = (lane % 8) ^ swz(r);
        int n = min(bn + r, N - 1);
        b_src[i] = W + (long)n * p.kpad + c * 8;
    }

    auto issue = [&](int slice) {
        unsigned char* st = smem + (slice % STAGES) * STAGE_BYTES;
        const int k0 = slice * BK;
#pragma unroll
        for (int i = 0; i < A_IT; i++)
            __builtin_amdgcn_global_load_lds(a_src[i] + k0, LDS_PTR(st + (wave * A_IT + i) * 1024), 16, 0, 0);
#pragma unroll
        for (int i = 0; i < B_IT; i++)
            __builtin_amdgcn_global_load_lds(b_src[i] + k0, LDS_PTR(st + A_BYTES + (wave * B_IT + i) * 1024), 16, 0, 0);
    };

    float4v acc[TJ][TI];
#pragma unroll
    for (int j = 0; j < TJ; j++)
#pragma unroll
        for (int i = 0; i < TI; i++) acc[j][i] = (float4v)0.0f;

    const int nk = K / BK;
#pragma unroll
    for (int s = 0; s < STAGES - 1; s++)
        if (s < nk) issue(s);

    // fragment read offsets (bytes within a stage): row * ROWB + ((chunk ^ swz(row)) * 16)
    int a_row[TI], b_row[TJ];
#pragma unroll
    for (int i = 0; i < TI; i++) a_row[i] = wm0 + i * 16 + l16;
#pragma unroll
    for (int j = 0; j < TJ; j++) b_row[j] = wn0 + j * 16 + l16;

    for (int kt = 0; kt < nk; kt++) {
        // slice kt complete for this wave (later slices may stay in flight), then for all waves
        if (kt + STAGES - 2 < nk) wait_vmcnt<(STAGES - 2) * LOADS>();
        else wait_vmcnt<0>();
        __builtin_amdgcn_s_barrier();
        if (kt + STAGES - 1 < nk) issue(kt + STAGES - 1);
        const unsigned char* st = smem + (kt % STAGES) * STAGE_BYTES;
#pragma unroll
        for (int s = 0; s < BK / 32; s++) {
            const int chunk = s * 4 + g;
            half8 af[TI], bf[TJ];
#pragma unroll
            for (int j = 0; j < TJ; j++)
                bf[j] = *(const half8*)(st + A_BYTES + b_row[j] * ROWB + ((chunk ^ swz(b_row[j])) << 4));
#pragma unroll
            for (int i = 0; i < TI; i++)
                af[i] = *(const half8*)(st + a_row[i] * ROWB + ((chunk ^ swz(a_row[i])) << 4));
#pragma unroll
            for (int j = 0; j < TJ; j++)
#pragma unroll
                for (int i = 0; i < TI; i++)
                    acc[j][i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bf[j], af[i], acc[j][i], 0, 0, 0);
        }
    }

    // ---- epilogue: bias + act on float4s (4 consecutive n), fp16 into the LDS staging tile ----
    __syncthreads();  // every wave is done with the stage buffers
    const int act = (p.flags & SOX_F_ACT_MASK) >> SOX_F_ACT_SHIFT;
    const bool has_bias = (p.flags & SOX_F_BIAS) != 0;
    half_t* epi = (half_t*)smem;
#pragma unroll
    for (int j = 0; j < TJ; j++) {
        const int nl = wn0 + j * 16 + 4 * g;  // local n of q = 0
        float4v bias = (float4v)0.0f;
        if (has_bias && bn + nl + 3 < N) bias = *(const float4v*)(p.bias + bn + nl);
        else if (has_bias)
            for (int q = 0; q < 4; q++) bias[q] = bn + nl + q < N ? p.bias[bn + nl + q] : 0.0f;
#pragma unroll
        for (int i = 0; i < TI; i++) {
            const int ml = wm0 + i * 16 + l16;
            half4 h;
#pragma unroll
            for (int q = 0; q < 4; q++) h[q] = (half_t)act_fast(acc[j][i][q] + bias[q], act);
            *(half4*)(epi + ml * EPI_ROW + nl) = h;
        }
    }
    __syncthreads();
    // ---- coalesced stores: 16 B per thread, consecutive threads along a row ----
    constexpr int CH = BN / 8;  // 16-byte chunks per output row
    half_t* __restrict__ Y = (half_t*)p.y;
#pragma unroll 4
    for (int idx = tid; idx < BM * CH; idx += 256) {
        const int r = idx / CH, c = idx - r * CH;
        const int m = bm + r, n = bn + c * 8;
        if (m < M && n < N) *(half8*)(Y + (long)m * p.ldy + n) = *(const half8*)(epi + r * EPI_ROW + c * 8);
    }
}

#define SOX_GEMM(NAME, BM, BN, BK, WM, WN, ST, GM)                                                  \
    extern "C" __global__ void __launch_bounds__(256) NAME(sox_igemm_args p) {                    \
        gemm_body<BM, BN, BK, WM, WN, ST, GM>(p);                                                 \
    }

SOX_GEMM(sox_gemm_f16_256x128_s2, 256, 128, 64, 128, 64, 2, 4)
SOX_GEMM(sox_gemm_f16_256x128_s3, 256, 128, 64, 128, 64, 3, 4)
SOX_GEMM(sox_gemm_f16_128x128_s2, 128, 128, 64, 64, 64, 2, 4)
SOX_GEMM(sox_gemm_f16_128x128_s3, 128, 128, 64, 64, 64, 3, 4)
SOX_GEMM(sox_gemm_f16_128x256_s2, 128, 256, 64, 64, 128, 2, 4)
SOX_GEMM(sox_gemm_f16_128x64_s3, 128, 64, 64, 64, 32, 3, 4)
SOX_GEMM(sox_gemm_f16_64x64_s3, 64, 64, 64, 32, 32, 3, 4)
