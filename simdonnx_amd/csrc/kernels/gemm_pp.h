// Dense 16-bit Gemm + bias + activation with the epilogue under the matrix-core work (instantiated by
// gemm_pp.hip): Y[M,N] = act(A[M,K] . W[N,K]^T + bias[N]), the conv_cm.comp / gemm.comp Gemm route
// (Backends/Vulkan/VkGraph.cs:760-773) for whole 256 x BN tiles and a compile-time K.
//
// Why a second dense kernel. On the LDS-DMA ring (gemm_ring.h: 8 waves, two per SIMD, barrier per
// slice) every wave reaches a tile's epilogue at the same time, so the GELU epilogue (~11 full-rate
// instructions per output) runs while the matrix cores idle. A wave's VALU work can issue while its
// own MFMAs execute (measured on gfx950: up to ~6 independent VALU instructions per
// v_mfma_f32_32x32x16 are free), so here each wave holds two accumulator sets and runs tile t's
// epilogue, in pieces, between tile t+1's MFMAs.
//
// Measured on MI355X for A[8192,768] x W[768,3072] + GELU: about 48.5 us against the ring's 46 us. At
// one wave per SIMD the 256 x 128 tile's DMA (more bytes per flop than the ring's 256 x 192; the CU's
// global -> LDS path takes ~14 us of the loop) and the epilogue pieces do not hide under the MFMAs, so
// the ring stays the default Gemm and this route is taken only when SIMDONNX_HIP_GEMMPP is set.
//
// Structure (4 waves, one per SIMD; 256 x BN tile; each wave 128 x BN/2 = 4 x BN/64 blocks of 32 x 32):
//  * K moves in 32-deep slices through a 4-stage LDS ring, global -> LDS with global_load_lds_dwordx4
//    (rows of 64 bytes, 16-byte chunks XOR-swizzled by row as in the ring, so fragment reads are free
//    of bank conflicts). Per slice a wave issues 4 + BN/64 DMA instructions (A, then W), spread one per
//    two MFMAs over both k-steps; the tile's bias rides once per tile with its first slice, into an LDS
//    copy per tile that is triple-buffered by tile (the next tile's bias lands while the previous
//    tile's epilogue may still run). One s_barrier per slice, at its second k-step; the slice three
//    ahead refills the stage the barrier retired.
//  * The whole tile's K loop is unrolled (NK slices) and every k-step is laid out by hand as micro-steps
//    fenced with sched_barrier: one MFMA, then that step's share of the next fragment reads, of the DMA
//    and of the epilogue piece. A single wave per SIMD has no second wave to cover a stall, so the DMA
//    (whose issue stalls when the CU's ~64 B/cycle global -> LDS path backs up) and the VALU work must
//    be spread evenly between the MFMAs rather than left to cluster.
//  * Accumulators: accc (the tile being multiplied) starts from the tile's bias at its first k-step, so
//    the epilogue is activation + store only; the last k-step writes accp (the finished tile). The
//    k-steps run in the ring's order on the same instruction, so the outputs equal the ring's bit for bit.
//  * Epilogue of tile t during tile t+1: one piece per half block (8 outputs per lane), at most one per
//    slice and none in the last (whose final k-step overwrites accp). Each output's activation is split
//    in two halves of ~5 instructions (gelu_fast_lo / _hi), one per micro-step, so every MFMA carries
//    about as much VALU work as it can hide; each run of 4 outputs is converted and staged in the wave's
//    4 KiB of LDS. When a piece completes two blocks (one for an odd last block), the next slice reads
//    them back in its first k-step and stores whole 128-byte (64-byte) row segments with streaming
//    stores in its second. The last tile's epilogue runs after its K loop.
//  * Persistent grid of one workgroup per CU, XCD-major numbering and GM-grouped tile order as the ring.
#pragma once
#include "gemm_ring.h"

template <typename T, int BN, int NK, int ACT>
__device__ __forceinline__ void gemm_pp_body(const sox_igemm_args& p) {
    typedef vec_t<T, 8> T8;
    typedef vec_t<T, 4> T4;
    constexpr int BM = 256, NW = 4, WM = 128, WN = BN / 2, STAGES = 4, GM = 4;
    constexpr int ROWB = 64;                   // 32 16-bit values per LDS row: 4 chunks of 16 bytes
    constexpr int TI = WM / 32, TJ = WN / 32;  // blocks of 32 x 32 per wave
    constexpr int MF = TI * TJ;                // MFMAs per k-step
    constexpr int RD = TI + TJ;                // fragment reads per k-step
    constexpr int A_ST = BM * ROWB, B_ST = BN * ROWB;
    constexpr int B_OFF = STAGES * A_ST;                 // every A stage first: A fragment offsets < 64 KiB
    constexpr int BIAS_OFF = B_OFF + STAGES * B_ST;      // 3 tiles x 4 waves x 1 KiB
    constexpr int EPI_OFF = BIAS_OFF + 3 * NW * 1024;    // 4 waves x 4 KiB of epilogue staging
    constexpr int LDS_BYTES = EPI_OFF + NW * 4096;
    constexpr int PIECES = TI * TJ * 2;                  // half blocks
    constexpr int B_IT = BN / 64;                        // W DMA instructions per wave per slice
    constexpr int LOADS = 4 + B_IT;                      // DMA instructions per wave per slice (+1 bias)
    constexpr int H1 = LOADS / 2;                        // of them issued in the first k-step
    static_assert(NK % STAGES == 0 && NK >= PIECES, "stage of every slice compile-time; pieces fit");
    static_assert(BN % 64 == 0 && BN <= 256, "tiling");
    static_assert(RD <= MF && 2 * H1 <= MF && 2 * (LOADS - H1 + 1) <= MF, "one read / DMA per micro-step");
    static_assert(LDS_BYTES <= 160 * 1024, "LDS");
    __shared__ __attribute__((aligned(1024))) unsigned char smem[LDS_BYTES];

    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l32 = lane & 31, hl = lane >> 5;
    const int wm0 = (wave >> 1) * WM, wn0 = (wave & 1) * WN;
    const int tiles_n = p.tiles_n, tiles_m = p.m / BM, ntiles = tiles_m * tiles_n;
    const char* __restrict__ Ab = (const char*)p.x;
    const char* __restrict__ Wb = (const char*)p.w;
    T* __restrict__ Y = (T*)p.y;
    const int ldy = p.ldy;
    const bool has_bias = (p.flags & SOX_F_BIAS) != 0;

    const int G = gridDim.x;
    const int vid = (G % 8 == 0) ? (blockIdx.x % 8) * (G / 8) + blockIdx.x / 8 : blockIdx.x;
    const int my_tiles = vid < ntiles ? (ntiles - 1 - vid) / G + 1 : 0;
    if (my_tiles == 0) return;
    auto tile_origin = [&](int t, int& bm, int& bn) __attribute__((always_inline)) {
        const int tt = vid + t * G;
        const int group = tt / (GM * tiles_n), first_m = group * GM;
        const int gsize = min(tiles_m - first_m, GM);
        const int in_group = tt - group * GM * tiles_n;
        bm = __builtin_amdgcn_readfirstlane((first_m + in_group % gsize) * BM);
        bn = __builtin_amdgcn_readfirstlane((in_group / gsize) * BN);
    };

    // DMA: lane l of A instruction i fills 16 bytes of LDS row r = (wave * 4 + i) * 16 + l / 4, slot
    // l % 4, which holds global chunk (l % 4) ^ swz(r); W likewise with B_IT instructions per wave. The
    // per-lane byte offsets from the tile's first row are fixed; the uniform base moves per tile and slice.
    uint32_t a_voff[4], b_voff[B_IT];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int r = (wave * 4 + i) * 16 + (lane >> 2);
        a_voff[i] = (uint32_t)r * (uint32_t)p.lda * 2u + (uint32_t)(((lane & 3) ^ swz<4>(r)) * 16);
    }
#pragma unroll
    for (int i = 0; i < B_IT; i++) {
        const int r = (wave * B_IT + i) * 16 + (lane >> 2);
        b_voff[i] = (uint32_t)r * (uint32_t)p.kpad * 2u + (uint32_t)(((lane & 3) ^ swz<4>(r)) * 16);
    }
    // the bias DMA: every lane loads 16 bytes, lanes past BN / 4 repeat the first ones; without a bias,
    // 16 zero bytes of p.zeros per lane
    const uint32_t c_voff = has_bias ? (uint32_t)(lane % (BN / 4)) * 16u : (uint32_t)(lane & 15) * 16u;
    const char* a_base = nullptr;
    const char* b_base = nullptr;
    const char* c_base = nullptr;
    auto set_sources = [&](int t) __attribute__((always_inline)) {
        int bm, bn;
        tile_origin(t, bm, bn);
        a_base = Ab + (long)bm * p.lda * 2;
        b_base = Wb + (long)bn * p.kpad * 2;
        c_base = has_bias ? (const char*)(p.bias + bn) : (const char*)p.zeros;
    };
    // DMA instruction x of slice `ks` of the tile whose sources are set, into `stage` (x = LOADS: the
    // tile's bias, into bias slot `bslot`)
    auto dma = [&](int ks, auto stage_c, auto x_c, int bslot) __attribute__((always_inline)) {
        constexpr int st = decltype(stage_c)::value, x = decltype(x_c)::value;
        if constexpr (x < 4) {
            __builtin_amdgcn_global_load_lds((const void*)(a_base + ks * 64 + a_voff[x]),
                                             LDS_PTR(smem + st * A_ST + (wave * 4 + x) * 1024), 16, 0, 0);
        } else if constexpr (x < LOADS) {
            __builtin_amdgcn_global_load_lds((const void*)(b_base + ks * 64 + b_voff[x - 4]),
                                             LDS_PTR(smem + B_OFF + st * B_ST + (wave * B_IT + x - 4) * 1024), 16, 0, 0);
        } else {
            __builtin_amdgcn_global_load_lds((const void*)(c_base + c_voff),
                                             LDS_PTR(smem + BIAS_OFF + bslot * (NW * 1024) + wave * 1024), 16, 0, 0);
        }
    };

    // fragment reads: k-step kk of a lane covers chunk 2 kk + l / 32 of its rows, stored at slot
    // (2 kk + l / 32) ^ swz(row): step 0's offset with bit 5 flipped for step 1
    int a_off[2][TI], b_off[2][TJ];
#pragma unroll
    for (int i = 0; i < TI; i++) {
        const int r = wm0 + i * 32 + l32;
        a_off[0][i] = r * ROWB + ((hl ^ swz<4>(r)) << 4);
        a_off[1][i] = a_off[0][i] ^ 32;
    }
#pragma unroll
    for (int j = 0; j < TJ; j++) {
        const int r = wn0 + j * 32 + l32;
        b_off[0][j] = B_OFF + r * ROWB + ((hl ^ swz<4>(r)) << 4);
        b_off[1][j] = b_off[0][j] ^ 32;
    }
    T8 fa[2][TI], fb[2][TJ];
    // fragment read r (B fragments first) of k-step kk of the slice in `stage`, into buffer b
    auto read_frag = [&](auto stage_c, auto kk_c, auto buf_c, auto r_c) __attribute__((always_inline)) {
        constexpr int st = decltype(stage_c)::value, kk = decltype(kk_c)::value, b = decltype(buf_c)::value;
        constexpr int r = decltype(r_c)::value;
        if constexpr (r < TJ)
            fb[b][r] = *(const T8*)(smem + b_off[kk][r] + st * B_ST);
        else
            fa[b][r - TJ] = *(const T8*)(smem + a_off[kk][r - TJ] + st * A_ST);
    };
    // this wave's share of the bias of the tile in bias slot `slot`, as MFMA accumulator vectors
    float16v cb[TJ];
    auto read_bias = [&](int slot) __attribute__((always_inline)) {
        const float* bl = (const float*)(smem + BIAS_OFF + slot * (NW * 1024) + wave * 1024);
        static_for<0, TJ>([&](auto jj) {
            constexpr int j = decltype(jj)::value;
            static_for<0, 4>([&](auto qq) {
                constexpr int q = decltype(qq)::value;
                const float4v b4 = *(const float4v*)(bl + wn0 + 32 * j + 8 * q + 4 * hl);
                static_for<0, 4>([&](auto ee) { cb[j][4 * q + decltype(ee)::value] = b4[decltype(ee)::value]; });
            });
        });
    };

    float16v accc[TJ][TI], accp[TJ][TI];
    int bm_p = 0, bn_p = 0;  // origin of the previous tile (its epilogue runs now)
    unsigned char* stg = smem + EPI_OFF + wave * 4096;

    // Epilogue piece P of the previous tile (accp): pieces of row block i in column-block order, block
    // (j, i), outputs 8 h .. 8 h + 7 of each lane (runs q = 2 h, 2 h + 1 of 4 channels); blocks staged
    // two at a time (an odd last one alone): CH 16-byte chunks per staged row, the group done at `last`.
    struct Geom {
        int i, j, h, j0, ch;
        bool last;
    };
    constexpr auto geom = [](int P) constexpr {
        const int r = P % (2 * TJ), j = r / 2, h = r % 2, j0 = j & ~1;
        return Geom{P / (2 * TJ), j, h, j0, j0 + 1 < TJ ? 8 : 4, h == 1 && (j == j0 + 1 || j0 + 1 == TJ)};
    };
    float4v pv, px, pa, pl;
    // half `hf` of output e (0..7) of piece P (the activation in two halves of ~5 instructions); after
    // each run of 4 outputs, their conversion and staging write
    auto piece_out = [&](auto P_c, auto e_c, auto hf_c) __attribute__((always_inline)) {
        constexpr int P = decltype(P_c)::value, e = decltype(e_c)::value, hf = decltype(hf_c)::value;
        constexpr Geom g = geom(P);
        constexpr int q = 2 * g.h + e / 4, c = (g.j - g.j0) * 4 + q;
        if constexpr (hf == 0) {
            px[e % 4] = accp[g.j][g.i][4 * q + e % 4];
            if constexpr (ACT == SOX_ACT_GELU) {
                float a, l;
                gelu_fast_lo(px[e % 4], a, l);
                pa[e % 4] = a;
                pl[e % 4] = l;
            }
        } else {
            const float x = px[e % 4];
            pv[e % 4] = ACT == SOX_ACT_GELU ? gelu_fast_hi(x, pa[e % 4], pl[e % 4])
                        : ACT == SOX_ACT_RELU ? __builtin_amdgcn_fmed3f(x, 0.0f, __builtin_inff()) : x;
            if constexpr (e % 4 == 3) {
                fp32_rounded(pv);
                const T4 hv = __builtin_convertvector(pv, T4);
                *(T4*)(stg + l32 * g.ch * 16 + ((c ^ (l32 % g.ch)) << 4) + hl * 8) = hv;
            }
        }
    };
    // the store of a completed group (piece P its last): part u < CH / 2 reads staged chunk row u (into
    // registers), part CH / 2 + u stores it as whole row segments
    T8 sv[4];
    auto group_store = [&](auto P_c, auto u_c) __attribute__((always_inline)) {
        constexpr int P = decltype(P_c)::value, u = decltype(u_c)::value;
        constexpr Geom g = geom(P);
        constexpr int CH = g.ch;
        if constexpr (u < CH / 2) {
            const int idx = u * 64 + lane, row = idx / CH, c = idx % CH;
            sv[u] = *(const T8*)(stg + row * CH * 16 + ((c ^ (row % CH)) << 4));
        } else if constexpr (u < CH) {
            constexpr int v = u - CH / 2;
            const int idx = v * 64 + lane, row = idx / CH, c = idx % CH;
            T* yp = Y + (long)(bm_p + wm0 + 32 * g.i + row) * ldy + bn_p + wn0 + 32 * g.j0 + 8 * c;
            __builtin_nontemporal_store(sv[v], (T8*)yp);
        }
    };
    static_assert(PIECES <= NK - 1, "at most one piece per slice, none in the last");

    // slice S of tile t (stream slice t NK + S). fa[0] / fb[0] hold its first k-step's fragments.
    // DMA of the slice three ahead (this tile's S + 3, or the next tile's S + 3 - NK with the sources
    // switched at S = NK - 3; that slice 0 also carries the next tile's bias) into the stage the
    // previous slice's barrier retired.
    auto slice = [&](auto S_c, auto first_c, int t) __attribute__((always_inline)) {
        constexpr int S = decltype(S_c)::value;
        constexpr bool FIRST = decltype(first_c)::value;  // tile 0: no previous tile to store
        constexpr int st = S % STAGES, st_next = (S + 1) % STAGES, st_dma = (S + 3) % STAGES;
        constexpr int ks_dma = (S + 3) % NK;
        constexpr bool dma_bias = ks_dma == 0;  // the DMA'd slice is a tile's first: its bias too
        // loads issued after slice S + 1's by the wait in k-step 1: slice S + 2's (with its bias when it is
        // a tile's first) and the first H1 of slice S + 3's
        constexpr int WAIT = LOADS + ((S + 2) % NK == 0 ? 1 : 0) + H1;
        if constexpr (S == NK - 3) set_sources(min(t + 1, my_tiles - 1));
        const int bslot_dma = (t + 1) % 3;
        // the piece of this slice (piece P runs in slice P (NK - 1) / PIECES: outputs 0..3 over k-step 0,
        // 4..7 over k-step 1, two micro-steps each), and the group its predecessor completed (read back in
        // k-step 0, stored in k-step 1)
        constexpr int P0 = (S * PIECES + NK - 2) / (NK - 1);  // the first P with P (NK - 1) / PIECES >= S
        constexpr bool has_piece = !FIRST && P0 < PIECES && P0 * (NK - 1) / PIECES == S;
        constexpr int Pprev = S > 0 ? ((S - 1) * PIECES + NK - 2) / (NK - 1) : 0;
        constexpr bool store_prev = !FIRST && S > 0 && Pprev < PIECES && Pprev * (NK - 1) / PIECES == S - 1 &&
                                    geom(Pprev).last;
        static_assert(MF == 8, "two micro-steps per output of a 4-output run");
        // ---- k-step 0: MFMA, the next k-step's fragment reads, half the DMA, the piece's outputs ----
        static_for<0, MF>([&](auto m_c) {
            constexpr int m = decltype(m_c)::value, i = m / TJ, j = m % TJ;
            if constexpr (S == 0)
                accc[j][i] = mfma32x32x16(fb[0][j], fa[0][i], cb[j]);
            else
                accc[j][i] = mfma32x32x16(fb[0][j], fa[0][i], accc[j][i]);
            if constexpr (m < RD)
                read_frag(std::integral_constant<int, st>{}, std::integral_constant<int, 1>{},
                          std::integral_constant<int, 1>{}, m_c);
            if constexpr (m % 2 == 1 && m / 2 < H1)
                dma(ks_dma, std::integral_constant<int, st_dma>{}, std::integral_constant<int, m / 2>{}, bslot_dma);
            if constexpr (store_prev) group_store(std::integral_constant<int, Pprev>{}, m_c);
            if constexpr (has_piece)
                piece_out(std::integral_constant<int, P0>{}, std::integral_constant<int, m / 2>{},
                          std::integral_constant<int, m % 2>{});
            __builtin_amdgcn_sched_barrier(0);
        });
        // ---- k-step 1: slice S + 1 landed (this wave's loads; WAIT newer ones may stay in flight) and
        // every read of slice S done (and the piece's staging writes); after the barrier both hold for
        // all waves ----
        wait_vmcnt<WAIT>();
        wait_lgkmcnt0();
        __builtin_amdgcn_s_barrier();
        if constexpr (S == NK - 1) read_bias((t + 1) % 3);  // the next tile starts from its bias
        static_for<0, MF>([&](auto m_c) {
            constexpr int m = decltype(m_c)::value, i = m / TJ, j = m % TJ;
            if constexpr (S == NK - 1)
                accp[j][i] = mfma32x32x16(fb[1][j], fa[1][i], accc[j][i]);
            else
                accc[j][i] = mfma32x32x16(fb[1][j], fa[1][i], accc[j][i]);
            if constexpr (m < RD)
                read_frag(std::integral_constant<int, st_next>{}, std::integral_constant<int, 0>{},
                          std::integral_constant<int, 0>{}, m_c);
            if constexpr (m % 2 == 1 && H1 + m / 2 < LOADS)
                dma(ks_dma, std::integral_constant<int, st_dma>{}, std::integral_constant<int, H1 + m / 2>{}, bslot_dma);
            if constexpr (m % 2 == 1 && H1 + m / 2 == LOADS && dma_bias)
                dma(ks_dma, std::integral_constant<int, st_dma>{}, std::integral_constant<int, LOADS>{}, bslot_dma);
            if constexpr (store_prev)
                group_store(std::integral_constant<int, Pprev>{}, std::integral_constant<int, geom(Pprev).ch / 2 + m>{});
            if constexpr (has_piece)
                piece_out(std::integral_constant<int, P0>{}, std::integral_constant<int, 4 + m / 2>{},
                          std::integral_constant<int, m % 2>{});
            __builtin_amdgcn_sched_barrier(0);
        });
    };

    // prologue: slices 0..2 of the first tile in flight (slice 0 with its bias), slice 0 landed, its
    // first fragments and the bias read
    set_sources(0);
    static_for<0, 3>([&](auto s) {
        static_for<0, LOADS>([&](auto x) { dma(decltype(s)::value, s, x, 0); });
        if constexpr (decltype(s)::value == 0) dma(0, s, std::integral_constant<int, LOADS>{}, 0);
    });
    wait_vmcnt<2 * LOADS>();
    __builtin_amdgcn_s_barrier();
    static_for<0, RD>([&](auto r) {
        read_frag(std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{}, r);
    });
    read_bias(0);

    static_for<0, NK>([&](auto S) { slice(S, std::true_type{}, 0); });
    tile_origin(0, bm_p, bn_p);
    for (int t = 1; t < my_tiles; t++) {
        static_for<0, NK>([&](auto S) { slice(S, std::false_type{}, t); });
        tile_origin(t, bm_p, bn_p);
    }
    // the last tile's epilogue (nothing left to hide it under)
    static_for<0, PIECES>([&](auto P) {
        static_for<0, 8>([&](auto e) {
            piece_out(P, e, std::integral_constant<int, 0>{});
            piece_out(P, e, std::integral_constant<int, 1>{});
        });
        if constexpr (geom(decltype(P)::value).last) {
            wait_lgkmcnt0();
            static_for<0, 8>([&](auto u) { group_store(P, u); });
            wait_lgkmcnt0();
        }
    });
    wait_vmcnt<0>();  // the trailing (unused) slices land before the workgroup's LDS is released
}

#define SOX_GEMM_PP(NAME, T, BN, NK, ACT)                                                      \
    extern "C" __global__ void __launch_bounds__(256, 1) NAME(sox_igemm_args p) {                 \
        gemm_pp_body<T, BN, NK, ACT>(p);                                                      \
    }
