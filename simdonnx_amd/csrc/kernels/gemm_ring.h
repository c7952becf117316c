// The LDS-DMA persistent ring (instantiated by gemm.hip / gemm_bf16.hip for dense Gemm and
// conv_ring.hip / conv_ring_bf16.hip for Conv2d / ConvTranspose): 16-bit Gemm with fused bias +
// activation on CDNA4 matrix cores (the conv_cm.comp Gemm route, Backends/Vulkan/VkGraph.cs:760-773,
// rebuilt for gfx950):
//   Y[M,N] = act(A[M,K] . W[N,K]^T + bias[N] (+ R[M,N])),  A dense rows (lda), W packed [N][kpad]
//   k-fastest, R an optional same-shape residual, fp16 or bf16 storage (T), fp32 accumulation.
//
// Structure (NW waves, BM x BN output tile, BK-deep K slices):
//  * v_mfma_f32_32x32x16_f16 / _bf16 (the gfx950 instruction that sustains the dense rate with one wave
//    per SIMD; the 16x16x32 form needs two waves per SIMD and still tops out lower). W is the row
//    operand and A the column operand, so lane l holds Y^T[n = 8(q/4) + 4(l/32) + q%4][m = l%32]:
//    4 runs of 4 consecutive output channels of one row, i.e. float4 bias/activation and 8-byte stores
//    straight from the accumulators, or (EPI_LDS instances) staged through LDS into 16-byte stores of
//    whole 128-byte row segments.
//  * K slices move global -> LDS with global_load_lds_dwordx4 (no register staging), STAGES deep.
//    LDS rows are BK fp16 (CPR 16-byte chunks) stored XOR-swizzled (slot = chunk ^ f(row),
//    f(r) = (r / (16 / CPR)) % CPR), so the 16 lanes that one ds_read_b128 cycle serves (16 consecutive
//    rows, same chunk) hit 16 distinct 16-byte bank groups. The swizzle is applied on the load side.
//  * Register pipeline: k-step s+1's fragments are read while k-step s multiplies; the last k-step of
//    a slice reads the NEXT slice's first step. One s_barrier per slice, placed there: it publishes
//    slice g+1 (explicit vmcnt, loads complete in order) and retires slice g's stage, which is
//    refilled at once with slice g+STAGES.
//  * The bias never passes through vector registers on its own: each stage carries the tile's BN bias
//    floats (loaded by the same DMA), and a tile's accumulators start from them, so the epilogue is
//    activation + store only and no global load result is waited on outside the slice protocol.
//  * Persistent: each workgroup walks its tiles as ONE ring of K-slices, so the next tile's slices load
//    while the current tile's epilogue runs. Workgroups are numbered XCD-major (consecutive dispatch
//    ids land on different XCDs), so the tiles in flight on one XCD are a compact group of GM M-tiles
//    x some N-tiles and share A rows and W columns in that XCD's L2.
#pragma once
#include <type_traits>

#include "sox_device.h"

#define LDS_PTR(p) ((__attribute__((address_space(3))) void*)(p))

// s_waitcnt with only vmcnt constrained (gfx9 encoding: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt_hi[15:14]).
template <int N> SOX_DEV void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}
SOX_DEV void wait_lgkmcnt0() { __builtin_amdgcn_s_waitcnt(0xc07f); }

template <int I, int N, class F> SOX_DEV void static_for(F&& f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for<I + 1, N>(f);
    }
}

// LDS chunk swizzle for rows of CPR 16-byte chunks: rows sharing a 256-byte bank window get distinct
// slots, so 16 consecutive rows read at one chunk hit 16 distinct 16-byte bank groups.
template <int CPR> SOX_DEV int swz(int r) { return (r / (16 / CPR)) % CPR; }


// Epilogue of one wave's WM x WN block: lane l (l32 = l % 32, hl = l / 32) of 32x32 block (j, i) holds
// output row m0 + 32 i + l32 and, for q = 0..3, channels n0 + 32 j + 8 q + 4 hl .. +3 in accumulator
// elements 4q .. 4q+3 (the bias is already in the accumulators): activation on a float4, one 8-byte
// store each.
// ConvTranspose scatter (SOX_F_CONVT): output row m = (b, y, x) of the ih x iw input and column
// n = tap * oc + o land at pixel (y * kh + dy, x * kw + dx) of the output, tap = dy * kw + dx; the
// per-channel bias (bias[o], the same for every tap) is added here, before the activation.
struct ConvtOut {
    int ih, iw, kh, kw, oc;
    const float* bias;
};
// A conv's residual read as the nearest upsample by 2^shift of a map of (oh >> shift) x (ow >> shift)
// pixels (shift 0: the residual has the output's rows).
struct ResUp {
    int shift, oh, ow;
};

// RU: ru may upsample the residual; WIDE: 16-byte stores where the rows allow (the large-conv tile; on
// the smaller conv tiles of the detector it measured 0.6% slower)
template <typename T, int ACT, int TJ, int TI, bool RU = false, bool WIDE = true>
SOX_DEV void store_tile(T* __restrict__ Y, const T* __restrict__ R, int ldy, int M, int N, int m0, int n0,
                        const float16v (&acc)[TJ][TI], int act = 0, bool convt = false, ConvtOut ctv = {},
                        bool pad_rows = false, ResUp ru = {}) {
    typedef vec_t<T, 4> T4;
    const int lane = threadIdx.x & 63, l32 = lane & 31, hl = lane >> 5;
    // whole 4-element groups: rows of a multiple of 4 elements, or rows padded past the N tail
    const bool aligned = pad_rows ? (ldy & 3) == 0 : ((ldy | N) & 3) == 0;
    if (convt) {  // uniform: ConvTranspose output, no residual
        const ConvtOut* ct = &ctv;
        auto fin = [&](float a) { return ACT == SOX_ACT_GELU ? gelu_fast(a) : ACT >= 0 ? sox_act(a, ACT) : act_fast(a, act); };
        static_for<0, TJ * TI>([&](auto ji) {
            constexpr int j = decltype(ji)::value / TI, i = decltype(ji)::value % TI;
            const int m = m0 + i * 32 + l32;
            const int x = m % ct->iw, yb = m / ct->iw, y = yb % ct->ih, b = yb / ct->ih;
            const long ow = (long)ct->iw * ct->kw, base = ((long)b * ct->ih * ct->kh + (long)y * ct->kh) * ow + (long)x * ct->kw;
            static_for<0, 4>([&](auto qq) {
                constexpr int q = decltype(qq)::value;
                const int n = n0 + j * 32 + 8 * q + 4 * hl;
                if (m < M) {
                    if (ct->oc % 4 == 0) {  // the group's four channels share one tap
                        if (n < N) {
                            const int t = n / ct->oc, o = n - t * ct->oc, dy = t / ct->kw, dx = t - dy * ct->kw;
                            T4 h;
                            static_for<0, 4>([&](auto ee) {
                                constexpr int e = decltype(ee)::value;
                                h[e] = (T)fp32_value(fin(acc[j][i][4 * q + e] + (ct->bias ? ct->bias[o + e] : 0.0f)));
                            });
                            *(T4*)(Y + (base + (long)dy * ow + dx) * ct->oc + o) = h;
                        }
                    } else {
                        static_for<0, 4>([&](auto ee) {
                            constexpr int e = decltype(ee)::value;
                            if (n + e < N) {
                                const int t = (n + e) / ct->oc, o = n + e - t * ct->oc, dy = t / ct->kw, dx = t - dy * ct->kw;
                                Y[(base + (long)dy * ow + dx) * ct->oc + o] =
                                    (T)fp32_value(fin(acc[j][i][4 * q + e] + (ct->bias ? ct->bias[o] : 0.0f)));
                            }
                        });
                    }
                }
            });
            __builtin_amdgcn_sched_barrier(0);
        });
        return;
    }
    // No residual, rows on 16-byte boundaries and every column of the wave's blocks inside N (uniform):
    // lanes l and l + 32 hold channels 8q .. 8q+3 and 8q+4 .. 8q+7 of one row, so after converting q
    // pairs (2p, 2p+1) to 16-bit, one v_permlane32_swap per dword gives lane l all 8 channels of group
    // 2p and lane l + 32 all 8 of group 2p+1: one 16-byte store each instead of two 8-byte ones
    if (WIDE && !R && (ldy & 7) == 0 && n0 + TJ * 32 <= N) {
        typedef vec_t<unsigned, 2> U2;
        typedef vec_t<unsigned, 4> U4;
        auto fin = [&](float a) { return ACT == SOX_ACT_GELU ? gelu_fast(a) : ACT >= 0 ? sox_act(a, ACT) : act_fast(a, act); };
        static_for<0, TJ * TI>([&](auto ji) {
            constexpr int j = decltype(ji)::value / TI, i = decltype(ji)::value % TI;
            const int m = m0 + i * 32 + l32;
            static_for<0, 2>([&](auto pp) {
                constexpr int q0 = 2 * decltype(pp)::value, q1 = q0 + 1;
                T4 h0, h1;
                static_for<0, 4>([&](auto ee) {
                    constexpr int e = decltype(ee)::value;
                    h0[e] = (T)fp32_value(fin(acc[j][i][4 * q0 + e]));
                    h1[e] = (T)fp32_value(fin(acc[j][i][4 * q1 + e]));
                });
                const U2 d0 = __builtin_bit_cast(U2, h0), d1 = __builtin_bit_cast(U2, h1);
                // lanes 0-31 keep their dword of group q0 and receive lane + 32's; lanes 32-63 receive
                // lane - 32's dword of group q1 and keep their own
                const auto sx = __builtin_amdgcn_permlane32_swap(d0[0], d1[0], false, false);
                const auto sy = __builtin_amdgcn_permlane32_swap(d0[1], d1[1], false, false);
                const U4 out = {sx[0], sy[0], sx[1], sy[1]};
                if (m < M) *(U4*)(Y + (long)m * ldy + n0 + j * 32 + 8 * (hl ? q1 : q0)) = out;
                __builtin_amdgcn_sched_barrier(0);  // one pair at a time: bounded register pressure
            });
        });
        return;
    }
    // static_for, not #pragma unroll: the accumulators must only ever be indexed by constants, or they
    // leave registers
    static_for<0, TJ * TI>([&](auto ji) {
        constexpr int j = decltype(ji)::value / TI, i = decltype(ji)::value % TI;
        const int m = m0 + i * 32 + l32;
        // residual (the next node's Add, fused): the block's four 8-byte groups load together
        T4 rv[4];
        if (R) {
            long rm = m;  // the residual's row
            if constexpr (RU) {
                if (ru.shift > 0) {
                    const int q = m / ru.ow, x = m - q * ru.ow, y = q % ru.oh, b = q / ru.oh;
                    rm = ((long)b * (ru.oh >> ru.shift) + (y >> ru.shift)) * (ru.ow >> ru.shift) + (x >> ru.shift);
                }
            }
            static_for<0, 4>([&](auto qq) {
                constexpr int q = decltype(qq)::value;
                const int n = n0 + j * 32 + 8 * q + 4 * hl;
                const long o = (m < M && n < N) ? (RU ? rm : (long)m) * ldy + n : 0;
                if (aligned) {
                    rv[q] = *(const T4*)(R + o);
                } else {
#pragma unroll
                    for (int e = 0; e < 4; e++) rv[q][e] = R[o + (n + e < N ? e : 0)];
                }
            });
            // vmcnt counts in order, so these wait behind every DMA in flight anyway; waiting here, on
            // every path that loaded, keeps the compiler from carrying them into the K loop as pending
            // writes (which costs a full vmcnt(0) drain per slice)
            wait_vmcnt<0>();
        }
        static_for<0, 4>([&](auto qq) {
            constexpr int q = decltype(qq)::value;
            const int n = n0 + j * 32 + 8 * q + 4 * hl;
            T4 h;
            static_for<0, 4>([&](auto ee) {
                constexpr int e = decltype(ee)::value;
                float v = acc[j][i][4 * q + e];
                if (R) v += (float)rv[q][e];
                h[e] = (T)fp32_value(ACT == SOX_ACT_GELU ? gelu_fast(v) : ACT >= 0 ? sox_act(v, ACT) : act_fast(v, act));
            });
            if (m < M && n < N) {
                T* yp = Y + (long)m * ldy + n;
                if (aligned) {
                    *(T4*)yp = h;  // 8-byte aligned rows, whole groups of 4
                } else {
#pragma unroll
                    for (int e = 0; e < 4; e++)
                        if (n + e < N) yp[e] = h[e];
                }
            }
        });
        __builtin_amdgcn_sched_barrier(0);  // one block at a time: bounded register pressure
    });
}

// Epilogue through LDS (no residual, no scatter, rows of whole 8-element groups): each wave stages
// 32 rows x 64 channels (two 32x32 blocks; 32 when it has one) of fp16 results in its own 4 KiB
// (2 KiB) of LDS and stores them back as 16-byte chunks, 8 (4) lanes per row, so every store
// instruction writes 8 whole 128-byte row segments (16 of 64 bytes) instead of 32 scattered 16-byte
// pieces. The staged rows hold 16-byte chunks XOR-swizzled
// by row (slot = chunk ^ row % chunks), which spreads both the 8-byte writes (one row per lane) and
// the 16-byte reads (one row per 8 lanes) evenly over the banks.
template <typename T, int ACT, int TJ, int TI>
SOX_DEV void store_tile_lds(T* __restrict__ Y, int ldy, int M, int N, int m0, int n0,
                            const float16v (&acc)[TJ][TI], int act, unsigned char* stg) {
    typedef vec_t<T, 4> T4;
    typedef vec_t<T, 8> T8;
    const int lane = threadIdx.x & 63, l32 = lane & 31, hl = lane >> 5;
    auto fin = [&](float a) { return ACT == SOX_ACT_GELU ? gelu_fast(a) : ACT >= 0 ? sox_act(a, ACT) : act_fast(a, act); };
    static_for<0, TI * ((TJ + 1) / 2)>([&](auto ip) {
        constexpr int i = decltype(ip)::value / ((TJ + 1) / 2), j0 = 2 * (decltype(ip)::value % ((TJ + 1) / 2));
        constexpr int JG = j0 + 1 < TJ ? 2 : 1, CH = JG * 4;  // blocks staged together, 16-byte chunks per row
        static_for<0, CH>([&](auto cc) {
            constexpr int c = decltype(cc)::value, j = j0 + c / 4, q = c % 4;
            float4v f;
            static_for<0, 4>([&](auto ee) { f[decltype(ee)::value] = fin(acc[j][i][4 * q + decltype(ee)::value]); });
            // a vector conversion: two v_cvt_pk_f16_f32 / v_cvt_pk_bf16_f32 (round to nearest even)
            // instead of four conversions and the packing moves, from the values rounded to fp32
            fp32_rounded(f);
            const T4 h = __builtin_convertvector(f, T4);
            *(T4*)(stg + l32 * CH * 16 + ((c ^ (l32 % CH)) << 4) + hl * 8) = h;
        });
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");  // other lanes' rows are read back
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        static_for<0, CH / 2>([&](auto tt) {
            const int idx = decltype(tt)::value * 64 + lane, r = idx / CH, c = idx % CH;
            const T8 v = *(const T8*)(stg + r * CH * 16 + ((c ^ (r % CH)) << 4));
            const int m = m0 + i * 32 + r, n = n0 + j0 * 32 + c * 8;
            // streaming (nontemporal) stores: the output is not read again by this kernel, so its lines
            // do not displace the A rows and W columns the other workgroups of the XCD re-read from L2
            if (m < M && n < N) __builtin_nontemporal_store(v, (T8*)(Y + (long)m * ldy + n));
        });
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");  // the next group overwrites the stage
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        __builtin_amdgcn_sched_barrier(0);
    });
}

// Bytes one wave's DMA instruction fills: its whole share when that is at most 1 KiB (64 lanes x 16 B),
// else the largest of 1024 / 768 / 512 / 256 that divides the share (e.g. 1.5 KiB -> 2 x 768).
constexpr int dma_chunk(int share) {
    return share <= 1024 ? share : share % 1024 == 0 ? 1024 : share % 768 == 0 ? 768 : share % 512 == 0 ? 512 : 256;
}

// CONV = false: A is a dense [M][lda] matrix (Gemm). CONV = true: A is the implicit im2col matrix of
// an NHWC image, A[m][k] = x[b][oy*sh - pt + ky][ox*sw - pl + kx][c] for m = (b, oy, ox) and
// k = (ky*kw + kx)*ic + c (tap-major, the packed weights' order). The K loop walks channel blocks of
// BK x taps (taps innermost; any order of the slices gives the same sum set, and this one keeps a
// block's rows in L2 across its taps), so a slice never straddles a tap: its tap is uniform (scalar
// math) and a lane's source is its row's offset + the tap's offset + its channel. Channels past ic (the last block of a tap
// when BK does not divide ic) and zero-padding taps are fetched from p.zeros; ic % 8 == 0. Rows past
// M re-read row M - 1 (never stored).
template <typename T, int BM, int BN, int BK, int WM, int WN, int STAGES, int NW, int GM, bool CONV = false,
          bool EPI_LDS = false, bool LN = false, int CPARTS = 0, bool LARGE = false>
__device__ __forceinline__ void gemm_body(const sox_igemm_args& p) {
    typedef vec_t<T, 8> T8;
    typedef vec_t<T, 2> T2;
    constexpr int CPR = BK / 8;                 // 16-byte chunks per LDS row
    constexpr int ROWB = BK * 2;                // LDS row bytes
    constexpr int KS = BK / 16;                 // MFMA k-steps per slice
    constexpr int A_BYTES = BM * ROWB, B_BYTES = BN * ROWB, BIAS_BYTES = BN * 4;
    constexpr int STAGE_BYTES = A_BYTES + B_BYTES + BIAS_BYTES;
    constexpr int BIAS_LANES = BIAS_BYTES / 16 / NW;  // lanes of each wave's bias DMA (16 B each)
    // DMA instructions per wave per slice; each fills CH contiguous LDS bytes (<= 1 KiB: lanes past
    // CH / 16 are idle when a wave's share is smaller)
    constexpr int CH_A = dma_chunk(A_BYTES / NW), A_IT = A_BYTES / NW / CH_A;
    constexpr int CH_B = dma_chunk(B_BYTES / NW), B_IT = B_BYTES / NW / CH_B;
    constexpr int LOADS = A_IT + B_IT + 1;      // + the bias DMA
    // two stages: the K loop waits for every load in flight (vmcnt 0), so slices need not carry the
    // same number of loads and the bias DMA goes out with a tile's first slice only
    constexpr bool BIAS_ONCE = STAGES == 2;
    constexpr int TI = WM / 32, TJ = WN / 32;   // 32x32 MFMA blocks: m (columns) x n (rows)
    constexpr int WAVES_N = BN / WN;
    static_assert(CPR == 4 || CPR == 8, "BK = 32 or 64");
    static_assert(KS % 2 == 0, "fragment sets alternate per k-step and must realign per slice");
    static_assert((BM / WM) * (BN / WN) == NW && WM % 32 == 0 && WN % 32 == 0, "tiling");
    static_assert(A_IT * CH_A * NW == A_BYTES && B_IT * CH_B * NW == B_BYTES && CH_A % 16 == 0 && CH_B % 16 == 0,
                  "DMA split");
    static_assert(BIAS_LANES * 16 * NW == BIAS_BYTES && BIAS_LANES <= 64 && STAGE_BYTES % 16 == 0, "bias DMA split");
    static_assert(STAGES >= 2 && (STAGES - 1) * LOADS < 64, "vmcnt range");

    constexpr int EPI_WAVE = 32 * 32 * (TJ < 2 ? TJ : 2) * 2;  // store_tile_lds staging per wave (2 or 4 KiB)
    constexpr int EPI_BYTES = EPI_LDS ? NW * EPI_WAVE : 0;
    __shared__ __attribute__((aligned(1024))) unsigned char smem[STAGE_BYTES * STAGES + EPI_BYTES];

    // the wave number in a scalar register: the LDS addresses derived from it (the DMA destinations in
    // M0) are computed by the scalar unit
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l32 = lane & 31, hl = lane >> 5;
    const int M = p.m, N = p.n, K = p.k;
    const int tiles_n = p.tiles_n, tiles_m = (M + BM - 1) / BM, ntiles = tiles_m * tiles_n;
    const int wm0 = (wave / WAVES_N) * WM, wn0 = (wave % WAVES_N) * WN;
    const T* __restrict__ A = (const T*)p.x;
    const T* __restrict__ W = (const T*)p.w;
    const T* __restrict__ Z = (const T*)p.zeros;
    T* __restrict__ Y = (T*)p.y;
    const T* __restrict__ R = (p.flags & SOX_F_RESIDUAL) ? (const T*)p.add : nullptr;  // [M][ldy]
    const int act = (p.flags & SOX_F_ACT_MASK) >> SOX_F_ACT_SHIFT;
    static_assert(!LN || !CONV, "LayerNorm-folded A: dense Gemm only");
    // a ConvTranspose's bias is per output channel, added in its scatter epilogue, not per column;
    // with LN the bias is added after the normalisation, so the accumulators start from zero
    const bool has_bias = (p.flags & SOX_F_BIAS) != 0 && !(CONV && (p.flags & SOX_F_CONVT)) && !LN;
    const int cblocks = CONV ? (p.ic + BK - 1) / BK : 1;  // channel blocks per tap
    const int nk = CONV ? p.kh * p.kw * cblocks : K / BK;
    const long img_elems = CONV ? (long)p.ih * p.iw * p.ic : 0;  // conv: elements of one input image
    const bool reflect = (p.flags & SOX_F_REFLECT) != 0;

    // XCD-major workgroup number: dispatch id b runs on XCD b % 8, so XCD x gets the contiguous
    // numbers [x G/8, (x+1) G/8) and with them consecutive tiles of every round
    const int G = gridDim.x;
    const int vid = (G % 8 == 0) ? (blockIdx.x % 8) * (G / 8) + blockIdx.x / 8 : blockIdx.x;
    const int my_tiles = vid < ntiles ? (ntiles - 1 - vid) / G + 1 : 0;
    const int total = my_tiles * nk;  // this workgroup's ring of K-slices
    auto tile_origin = [&](int t, int& bm, int& bn) __attribute__((always_inline)) {  // M-tiles walked in groups of GM
        const int group = t / (GM * tiles_n), first_m = group * GM;
        const int gsize = min(tiles_m - first_m, GM);
        const int in_group = t - group * GM * tiles_n;
        bm = (first_m + in_group % gsize) * BM;
        bn = (in_group / gsize) * BN;
    };

    // DMA sources of the tile being issued: lane l of instruction i of this wave fills the 16 LDS bytes
    // at (wave * IT + i) * CH + 16 l, i.e. row r = that offset / ROWB, slot (offset % ROWB) / 16, which
    // holds global chunk slot ^ swz(r). Rows past M / N re-read the last row (never stored).
    const bool a_lane = lane * 16 < CH_A, b_lane = lane * 16 < CH_B;
    // global chunk (k / 8 within the slice) of DMA instruction i, recomputed where it is used (a few
    // VALU per slice in conv mode; held across the K loop it would take a register per instruction)
    auto a_chunk = [&](int i) __attribute__((always_inline)) {
        const int off = (wave * A_IT + i) * CH_A + lane * 16, r = off / ROWB;
        return ((off % ROWB) / 16) ^ swz<CPR>(r);
    };
    auto b_chunk = [&](int i) __attribute__((always_inline)) {
        const int off = (wave * B_IT + i) * CH_B + lane * 16, r = off / ROWB;
        return ((off % ROWB) / 16) ^ swz<CPR>(r);
    };
    const T* a_src[A_IT];              // dense A: row base + chunk
    const T* a_img[A_IT];              // conv, !LARGE: the base of the row's image in the batch
    unsigned a_yx[A_IT];               // conv: the row's receptive-field origin, (iy0, ix0) + 2^15 in 16 bits each
    int a_off0[A_IT];                  // conv: (iy0 * iw + ix0) * ic, the origin's offset in its image
                                       // (LARGE: in the whole input, which has < 2^31 elements)
    const T* b_src[B_IT];              // dense: W row base + chunk
    int b_o[B_IT];                     // conv: the same as an element offset from W
    const float* c_src;  // this lane's 4 bias floats (a duplicate A chunk when there is no bias)
    auto set_sources = [&](int t) __attribute__((always_inline)) {
        int bm, bn;
        tile_origin(t, bm, bn);
        // the bias const is zero-padded to a multiple of 4 floats: the clamped float4 stays inside it
        c_src = has_bias ? p.bias + min(bn + (wave * BIAS_LANES + lane) * 4, ((N + 3) & ~3) - 4) : (const float*)A;
#pragma unroll
        for (int i = 0; i < A_IT; i++) {
            const int r = ((wave * A_IT + i) * CH_A + lane * 16) / ROWB;
            if constexpr (CONV) {
                const int m = min(bm + r, M - 1);
                const int ohw = p.oh * p.ow, b = m / ohw, rem = m - b * ohw;
                const int oy = rem / p.ow, ox = rem - oy * p.ow;
                const int iy0 = oy * p.sh - p.pt, ix0 = ox * p.sw - p.pl;  // |.| < 2^15 (the launcher checks)
                a_yx[i] = ((unsigned)(iy0 + 32768) << 16) | (unsigned)(ix0 + 32768);
                a_off0[i] = (iy0 * p.iw + ix0) * p.ic;
                if constexpr (LARGE)
                    a_off0[i] += b * (int)img_elems;
                else
                    a_img[i] = A + (long)b * img_elems;
            } else {
                a_src[i] = A + (long)min(bm + r, M - 1) * p.lda + a_chunk(i) * 8;
            }
        }
#pragma unroll
        for (int i = 0; i < B_IT; i++) {
            const int r = ((wave * B_IT + i) * CH_B + lane * 16) / ROWB;
            if constexpr (CONV)
                b_o[i] = min(bn + r, N - 1) * p.kpad + b_chunk(i) * 8;  // W < 2^31 elements (the launcher checks)
            else
                b_src[i] = W + (long)min(bn + r, N - 1) * p.kpad + b_chunk(i) * 8;
        }
    };
    // ring slice gs = (index in this workgroup's tile list) * nk + k-slice. Slices past the end are
    // still issued (re-reading the last tile's rows into a stage nobody reads again), so every slice
    // has the same number of loads in flight and one static vmcnt covers them all.
    // prep computes a slice's DMA sources (calling set_sources at a tile's first slice), fire issues
    // the DMAs.
    struct Src {
        const T* a[A_IT];
        const T* b[B_IT];
        const float* c;
    };
    // conv: the slice's tap (ky, kx), its offset in an image and the first channel c0 (uniform). The
    // K loop walks channel blocks outermost and taps innermost: a tile's kh * kw consecutive slices
    // read shifted windows of the same BK channels of the same input rows, which stay in L2 between
    // them (taps outermost, every tile re-read all ic channels of its rows once per tap, and the rows
    // of an XCD's tiles in flight outgrew its L2)
    struct Tap {
        int tap, c0, ky, kx, off;
    };
    auto slice_tap = [&](int gs) __attribute__((always_inline)) {
        Tap t;
        const int kt = gs % nk, taps = p.kh * p.kw, cb = kt / taps;
        t.tap = kt - cb * taps;
        t.c0 = cb * BK;
        t.ky = t.tap / p.kw;
        t.kx = t.tap - t.ky * p.kw;
        t.off = (t.ky * p.iw + t.kx) * p.ic;
        return t;
    };
    // conv DMA source of A instruction i / B instruction i for a slice
    auto conv_a = [&](int i, const Tap& t) __attribute__((always_inline)) {
        const int ch = t.c0 + a_chunk(i) * 8;
        const int iy = (int)(a_yx[i] >> 16) - 32768 + t.ky, ix = (int)(a_yx[i] & 0xffffu) - 32768 + t.kx;
        bool ok = (unsigned)iy < (unsigned)p.ih && (unsigned)ix < (unsigned)p.iw;
        int off = a_off0[i] + t.off + ch;
        if (reflect) {  // uniform; folds once: the launcher only routes pads < the image size here
            const int ry = iy < 0 ? -iy : iy >= p.ih ? 2 * p.ih - 2 - iy : iy;
            const int rx = ix < 0 ? -ix : ix >= p.iw ? 2 * p.iw - 2 - ix : ix;
            // LARGE: the image's base is the origin's offset less the origin's place in its image
            const int img0 = LARGE ? a_off0[i] - ((iy - t.ky) * p.iw + (ix - t.kx)) * p.ic : 0;
            off = img0 + (ry * p.iw + rx) * p.ic + ch;
            ok = true;
        }
        ok = ok && ch < p.ic;
        if constexpr (LARGE) return ok ? A + off : Z;
        return ok ? a_img[i] + off : Z;  // one image < 2^31 elements
    };
    auto conv_b = [&](int i, const Tap& t) __attribute__((always_inline)) {
        const int ch = t.c0 + b_chunk(i) * 8;
        return ch < p.ic ? W + b_o[i] + t.tap * p.ic + t.c0 : Z;  // b_o includes the chunk
    };
    auto prep = [&](int gs, Src& q) __attribute__((always_inline)) {
        const int kt = gs % nk;
        if (kt == 0 && gs < total) set_sources(vid + (gs / nk) * G);
        if constexpr (CONV) {
            const Tap t = slice_tap(gs);
#pragma unroll
            for (int i = 0; i < A_IT; i++) q.a[i] = conv_a(i, t);
#pragma unroll
            for (int i = 0; i < B_IT; i++) q.b[i] = conv_b(i, t);
        } else {
            const int k0 = kt * BK;
#pragma unroll
            for (int i = 0; i < A_IT; i++) q.a[i] = a_src[i] + k0;
#pragma unroll
            for (int i = 0; i < B_IT; i++) q.b[i] = b_src[i] + k0;
        }
        q.c = c_src;
    };
    auto fire = [&](int gs, const Src& q) __attribute__((always_inline)) {
        unsigned char* st = smem + (gs % STAGES) * STAGE_BYTES;
#pragma unroll
        for (int i = 0; i < A_IT; i++)
            if (a_lane) __builtin_amdgcn_global_load_lds(q.a[i], LDS_PTR(st + (wave * A_IT + i) * CH_A), 16, 0, 0);
#pragma unroll
        for (int i = 0; i < B_IT; i++)
            if (b_lane)
                __builtin_amdgcn_global_load_lds(q.b[i], LDS_PTR(st + A_BYTES + (wave * B_IT + i) * CH_B), 16, 0, 0);
        // the tile's bias rides along with its first slice (with every slice when the in-loop waits
        // count loads: more than two stages); the accumulators of a new tile start from it
        if (lane < BIAS_LANES && (!BIAS_ONCE || gs % nk == 0))
            __builtin_amdgcn_global_load_lds(q.c, LDS_PTR(st + A_BYTES + B_BYTES + wave * BIAS_LANES * 16), 16, 0, 0);
    };
    auto issue = [&](int gs) __attribute__((always_inline)) {
        Src q;
        prep(gs, q);
        fire(gs, q);
    };
    // Dense A: a slice's DMA instructions go out in two parts: part 0 right after the slice barrier,
    // part 1 after the next k-step's MFMAs. A wave that issues global -> LDS DMA stalls at issue while
    // the CU's ~64 B/cycle path drains; in two parts the stall falls while its MFMAs (and the other
    // wave's) keep the matrix pipe busy, and the loads still go out early enough to land before the
    // slice's vmcnt wait (one part per k-step over all four k-steps left the last part too little time).
    // Every part of slice g + STAGES - 1 is out before the vmcnt wait of slice g, so the waits count the
    // same loads as before.
    constexpr bool SPREAD = (!CONV || CPARTS > 1) && KS >= 2;
    constexpr int NPARTS = !SPREAD ? 1 : CONV ? (CPARTS < KS ? CPARTS : KS) : 2;
    constexpr int PER = (LOADS + NPARTS - 1) / NPARTS;  // DMA instructions per part
    auto fire_part = [&](int gs, auto pp) __attribute__((always_inline)) {
        constexpr int p0 = decltype(pp)::value * PER;
        if constexpr (p0 == 0) {
            if (gs % nk == 0 && gs < total) set_sources(vid + (gs / nk) * G);
        }
        const int k0 = (gs % nk) * BK;
        Tap t{};
        if constexpr (CONV) t = slice_tap(gs);  // recomputed per part: scalar work, no registers held
        unsigned char* st = smem + (gs % STAGES) * STAGE_BYTES;
        static_for<p0, (p0 + PER < LOADS ? p0 + PER : LOADS)>([&](auto xx) {
            constexpr int x = decltype(xx)::value;
            if constexpr (x < A_IT) {
                const T* src = CONV ? conv_a(x, t) : a_src[x] + k0;
                if (a_lane) __builtin_amdgcn_global_load_lds(src, LDS_PTR(st + (wave * A_IT + x) * CH_A), 16, 0, 0);
            } else if constexpr (x < A_IT + B_IT) {
                const T* src = CONV ? conv_b(x - A_IT, t) : b_src[x - A_IT] + k0;
                if (b_lane)
                    __builtin_amdgcn_global_load_lds(src, LDS_PTR(st + A_BYTES + (wave * B_IT + x - A_IT) * CH_B), 16, 0, 0);
            } else {
                if (lane < BIAS_LANES && (!BIAS_ONCE || gs % nk == 0))
                    __builtin_amdgcn_global_load_lds(c_src, LDS_PTR(st + A_BYTES + B_BYTES + wave * BIAS_LANES * 16), 16, 0, 0);
            }
        });
    };

    // fragment offsets: k-step s of a lane covers chunk 2s + l/32 of rows (row0 + l%32), stored at slot
    // (2s + l/32) ^ swz(row) = 2s ^ (l/32 ^ swz(row)): the offset of step 0 with bit 5 flipped by s
    // (the row's byte offset has no bits below ROWB >= 64)
    int a_off[TI], b_off[TJ];
#pragma unroll
    for (int i = 0; i < TI; i++) {
        const int r = wm0 + i * 32 + l32;
        a_off[i] = r * ROWB + ((hl ^ swz<CPR>(r)) << 4);
    }
#pragma unroll
    for (int j = 0; j < TJ; j++) {
        const int r = wn0 + j * 32 + l32;
        b_off[j] = A_BYTES + r * ROWB + ((hl ^ swz<CPR>(r)) << 4);
    }

    if (total == 0) return;
    int bm_cur, bn_cur;  // origin of the tile being multiplied
    tile_origin(vid, bm_cur, bn_cur);

    float16v acc[TJ][TI];
    T8 fa0[TI], fb0[TJ], fa1[TI], fb1[TJ];
    float ls1[TI], ls2[TI];  // LN: this lane's share of its rows' sum and sum of squares
    auto read_step = [&](int gs, int s, T8 (&fa)[TI], T8 (&fb)[TJ]) __attribute__((always_inline)) {
        const unsigned char* st = smem + (gs % STAGES) * STAGE_BYTES;
#pragma unroll
        for (int j = 0; j < TJ; j++) fb[j] = *(const T8*)(st + (b_off[j] ^ (s << 5)));
#pragma unroll
        for (int i = 0; i < TI; i++) fa[i] = *(const T8*)(st + (a_off[i] ^ (s << 5)));
    };
    // accumulators of a new tile = its bias (from the LDS stage of the tile's first slice)
    auto init_acc = [&](int gs) __attribute__((always_inline)) {
        const float* bl = (const float*)(smem + (gs % STAGES) * STAGE_BYTES + A_BYTES + B_BYTES);
        static_for<0, TJ>([&](auto jj) {
            constexpr int j = decltype(jj)::value;
            float4v b4[4];
#pragma unroll
            for (int q = 0; q < 4; q++)
                b4[q] = has_bias ? *(const float4v*)(bl + wn0 + j * 32 + 8 * q + 4 * hl) : (float4v)0.0f;
            float16v v;
            static_for<0, 16>([&](auto qe) { v[decltype(qe)::value] = b4[decltype(qe)::value / 4][decltype(qe)::value % 4]; });
            static_for<0, TI>([&](auto ii) { acc[j][decltype(ii)::value] = v; });
        });
        if constexpr (LN) {
#pragma unroll
            for (int i = 0; i < TI; i++) ls1[i] = ls2[i] = 0.0f;
        }
    };
    // LN (the Gemm's A rows are the input of a LayerNorm folded into it at graph creation: W holds
    // gamma-scaled weights, bias = b + beta W, p.ln_c[n] = sum_k W[n][k]): the accumulators hold
    // sum_k x[m][k] W[n][k]; with the row's mean and rsqrt(var + eps) from the sums that the k-steps
    // gathered, y = rstd (acc - mean c[n]) + bias[n], i.e. LN(x) . W^T + b up to rounding.
    auto ln_apply = [&]() __attribute__((always_inline)) {
        float mu[TI], rs[TI];
        const float inv_k = 1.0f / (float)K;
#pragma unroll
        for (int i = 0; i < TI; i++) {  // lanes l and l + 32 hold the two k-halves of a row
            const float s1 = ls1[i] + __shfl_xor(ls1[i], 32), s2 = ls2[i] + __shfl_xor(ls2[i], 32);
            mu[i] = s1 * inv_k;
            rs[i] = ln_rstd(mu[i], s2, inv_k, p.ln_eps);
        }
        const bool hb = (p.flags & SOX_F_BIAS) != 0;
        static_for<0, TJ>([&](auto jj) {
            constexpr int j = decltype(jj)::value;
            float4v cv[4], bv[4];
#pragma unroll
            for (int q = 0; q < 4; q++) {  // both consts are zero-padded to a multiple of 4 floats
                const int n = min(bn_cur + wn0 + j * 32 + 8 * q + 4 * hl, ((N + 3) & ~3) - 4);
                cv[q] = *(const float4v*)(p.ln_c + n);
                bv[q] = hb ? *(const float4v*)(p.bias + n) : (float4v)0.0f;
            }
            wait_vmcnt<0>();  // as for the residual: no loads carried into the K loop
            static_for<0, TI * 16>([&](auto ie) {
                constexpr int i = decltype(ie)::value / 16, e = decltype(ie)::value % 16;
                acc[j][i][e] = ln_out(acc[j][i][e], mu[i], rs[i], cv[e / 4][e % 4], bv[e / 4][e % 4]);
            });
        });
    };

    const ConvtOut cto{p.ih, p.iw, p.ct_kh, p.ct_kw, p.ct_oc, (p.flags & SOX_F_BIAS) ? p.bias : nullptr};
    const bool ctp = CONV && (p.flags & SOX_F_CONVT);
    const bool pad_rows = (p.flags & SOX_F_PAD_ROWS) != 0;
    const ResUp ru = CONV ? ResUp{p.res_shift, p.oh, p.ow} : ResUp{};
    // whole 16-byte chunks of every stored row (pad_rows: the row pitch covers N rounded up to 8)
    const bool lds_ok = EPI_LDS && !R && !ctp && (p.ldy & 7) == 0 && (pad_rows || (N & 7) == 0);
    auto epilogue = [&](int gs) __attribute__((always_inline)) {
        // ---- epilogue from registers (the next tile's first slices are already loading) ----
        if constexpr (LN) ln_apply();
        if constexpr (EPI_LDS) {
            if (lds_ok) {
                unsigned char* stg = smem + STAGE_BYTES * STAGES + wave * EPI_WAVE;
                switch (act) {
                case SOX_ACT_NONE: store_tile_lds<T, SOX_ACT_NONE>(Y, p.ldy, M, N, bm_cur + wm0, bn_cur + wn0, acc, 0, stg); break;
                case SOX_ACT_GELU: store_tile_lds<T, SOX_ACT_GELU>(Y, p.ldy, M, N, bm_cur + wm0, bn_cur + wn0, acc, 0, stg); break;
                default: store_tile_lds<T, -1>(Y, p.ldy, M, N, bm_cur + wm0, bn_cur + wn0, acc, act, stg); break;
                }
                if (gs + 1 < total) {
                    tile_origin(vid + (gs + 1) / nk * G, bm_cur, bn_cur);
                    init_acc(gs + 1);
                }
                return;
            }
        }
        switch (act) {
        case SOX_ACT_NONE: store_tile<T, SOX_ACT_NONE, TJ, TI, CONV, LARGE>(Y, R, p.ldy, M, N, bm_cur + wm0, bn_cur + wn0, acc, 0, ctp, cto, pad_rows, ru); break;
        case SOX_ACT_RELU: store_tile<T, SOX_ACT_RELU, TJ, TI, CONV, LARGE>(Y, R, p.ldy, M, N, bm_cur + wm0, bn_cur + wn0, acc, 0, ctp, cto, pad_rows, ru); break;
        case SOX_ACT_GELU: store_tile<T, SOX_ACT_GELU, TJ, TI, CONV, LARGE>(Y, R, p.ldy, M, N, bm_cur + wm0, bn_cur + wn0, acc, 0, ctp, cto, pad_rows, ru); break;
        default: store_tile<T, -1, TJ, TI, CONV, LARGE>(Y, R, p.ldy, M, N, bm_cur + wm0, bn_cur + wn0, acc, act, ctp, cto, pad_rows, ru); break;
        }
        if (gs + 1 < total) {
            tile_origin(vid + (gs + 1) / nk * G, bm_cur, bn_cur);
            init_acc(gs + 1);  // published by this slice's barrier
        }
    };

#pragma unroll
    for (int s = 0; s < STAGES; s++) issue(s);
    // slice 0 (loads complete in order; slice 1 carries LOADS - 1 of them when it does not start a tile)
    wait_vmcnt<(STAGES - 1) * LOADS - (BIAS_ONCE ? 1 : 0)>();
    __builtin_amdgcn_s_barrier();
    init_acc(0);
    read_step(0, 0, fa0, fb0);
    for (int gs = 0; gs < total; gs++) {
        static_for<0, KS>([&](auto step) {
            constexpr int s = decltype(step)::value;
            T8(&ca)[TI] = (s & 1) ? fa1 : fa0;
            T8(&cb)[TJ] = (s & 1) ? fb1 : fb0;
            T8(&na)[TI] = (s & 1) ? fa0 : fa1;
            T8(&nb)[TJ] = (s & 1) ? fb0 : fb1;
            if constexpr (s == KS - 1) {
                // slice gs+1 landed (this wave's loads; later slices may stay in flight) and every read
                // of slice gs done; after the barrier both hold for all waves
                wait_vmcnt<(STAGES - 2) * LOADS>();
                wait_lgkmcnt0();
                __builtin_amdgcn_s_barrier();
                // into stage gs % STAGES; may already be a later tile's slice
                if constexpr (SPREAD)
                    fire_part(gs + STAGES, std::integral_constant<int, 0>{});
                else
                    issue(gs + STAGES);
                read_step(gs + 1, 0, na, nb);
            } else {
                read_step(gs, s + 1, na, nb);
            }
            static_for<0, TJ * TI>([&](auto ji) {
                constexpr int j = decltype(ji)::value / TI, i = decltype(ji)::value % TI;
                acc[j][i] = mfma32x32x16(cb[j], ca[i], acc[j][i]);
            });
            if constexpr (SPREAD && s + 1 < NPARTS && (s + 1) * PER < LOADS) {
                // part s + 1 of the slice whose part 0 went out after the last barrier (the prologue
                // issued slices 0 .. STAGES - 1 whole)
                if (gs >= 1) fire_part(gs - 1 + STAGES, std::integral_constant<int, s + 1>{});
            }
            if constexpr (LN) {  // the step's 8 values of each of the lane's rows, by fp32 dot2
                const T2 one = {(T)1.0f, (T)1.0f};
                static_for<0, TI * 4>([&](auto ih) {
                    constexpr int i = decltype(ih)::value / 4, h = decltype(ih)::value % 4;
                    const T2 v = {ca[i][2 * h], ca[i][2 * h + 1]};
                    if constexpr (std::is_same<T, half_t>::value) {
                        ls1[i] = __builtin_amdgcn_fdot2(v, one, ls1[i], false);
                        ls2[i] = __builtin_amdgcn_fdot2(v, v, ls2[i], false);
                    } else {
                        ls1[i] = __builtin_amdgcn_fdot2_f32_bf16(v, one, ls1[i], false);
                        ls2[i] = __builtin_amdgcn_fdot2_f32_bf16(v, v, ls2[i], false);
                    }
                });
            }
            // MFMA, read, MFMA, read, ...: this step's operands were read one step earlier, and the
            // next step's reads issue while the matrix pipe works through this step
            constexpr int RD = TI + TJ, MF = TI * TJ;
            if constexpr (!CONV) {
                // dense Gemm: the DMA instructions this step issues (a part after the barrier or after a
                // k-step) go one after each MFMA, so a wave that stalls on DMA issue has MFMAs of its own
                // queued between (headline: 46.9 against 47.4 us on one box, 45.4 against 45.6 on
                // another; the conv ring measured 0.5% slower with it and keeps MFMA / read pairs only)
                constexpr int PART = s == KS - 1 ? 0 : s + 1;
                constexpr int DM = !SPREAD ? (s == KS - 1 ? LOADS : 0)
                                   : (PART < NPARTS && PART * PER < LOADS)
                                         ? (LOADS - PART * PER < PER ? LOADS - PART * PER : PER)
                                         : 0;
                static_for<0, MF>([&](auto ii) {
                    constexpr int i = decltype(ii)::value;
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    if constexpr (i < DM) __builtin_amdgcn_sched_group_barrier(0x010, 1, 0);
                    if constexpr (i < RD) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                });
                if constexpr (DM > MF) __builtin_amdgcn_sched_group_barrier(0x010, DM - MF, 0);
                if constexpr (RD > MF) __builtin_amdgcn_sched_group_barrier(0x100, RD - MF, 0);
            } else {
                static_for<0, (RD < MF ? RD : MF)>([&](auto) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                });
                if constexpr (MF > RD) __builtin_amdgcn_sched_group_barrier(0x008, MF - RD, 0);
                if constexpr (RD > MF) __builtin_amdgcn_sched_group_barrier(0x100, RD - MF, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
        });
        wait_lgkmcnt0();  // next slice's first fragments (read before this slice's last MFMAs)
        if (gs % nk == nk - 1) epilogue(gs);
    }
    wait_vmcnt<0>();  // the trailing (unused) slices land before the workgroup's LDS is released
}

// T: the 16-bit storage type (half_t or bf16_t)
#define SOX_GEMM(NAME, T, BM, BN, BK, WM, WN, ST, NW, OCC, GM)                                      \
    extern "C" __global__ void __launch_bounds__(64 * NW, OCC) NAME(sox_igemm_args p) {           \
        gemm_body<T, BM, BN, BK, WM, WN, ST, NW, GM>(p);                                          \
    }
// epilogue staged through LDS (store_tile_lds)
#define SOX_GEMM_E(NAME, T, BM, BN, BK, WM, WN, ST, NW, OCC, GM)                                    \
    extern "C" __global__ void __launch_bounds__(64 * NW, OCC) NAME(sox_igemm_args p) {           \
        gemm_body<T, BM, BN, BK, WM, WN, ST, NW, GM, false, true>(p);                             \
    }
// A rows LayerNorm'ed on the fly (the LayerNorm folded into the Gemm); E = epilogue through LDS
#define SOX_GEMM_LN(NAME, T, BM, BN, BK, WM, WN, ST, NW, OCC, GM, E)                               \
    extern "C" __global__ void __launch_bounds__(64 * NW, OCC) NAME(sox_igemm_args p) {           \
        gemm_body<T, BM, BN, BK, WM, WN, ST, NW, GM, false, E, true>(p);                          \
    }
#define SOX_CONV(NAME, T, BM, BN, BK, WM, WN, ST, NW, OCC, GM)                                      \
    extern "C" __global__ void __launch_bounds__(64 * NW, OCC) NAME(sox_igemm_args p) {           \
        gemm_body<T, BM, BN, BK, WM, WN, ST, NW, GM, true>(p);                                    \
    }
// conv mode with the epilogue staged through LDS (large convs: whole 128-byte row segments per store)
#define SOX_CONV_E(NAME, T, BM, BN, BK, WM, WN, ST, NW, OCC, GM)                                    \
    extern "C" __global__ void __launch_bounds__(64 * NW, OCC) NAME(sox_igemm_args p) {           \
        gemm_body<T, BM, BN, BK, WM, WN, ST, NW, GM, true, true>(p);                              \
    }
// large convs: the slice's DMA issued in PARTS parts (as the dense Gemm issues it in two), 32-bit
// input offsets (the launcher routes inputs of fewer than 2^31 elements only) and 16-byte stores
#define SOX_CONV_L(NAME, T, BM, BN, BK, WM, WN, ST, NW, OCC, GM, PARTS)                             \
    extern "C" __global__ void __launch_bounds__(64 * NW, OCC) NAME(sox_igemm_args p) {           \
        gemm_body<T, BM, BN, BK, WM, WN, ST, NW, GM, true, false, false, PARTS, true>(p);         \
    }
