// CTC recognizer head on gfx950: the class projection logits = features . W + bias fused with the
// per-row argmax and the winner's softmax probability (Decoding/CtcProjection.cs:5-58,
// Decoding/Kernels/MatMul.ArgMax.cs:29-299), so the [rows, classes] logits are never stored.
//
// Pass 1 (sox_ctc_part_k*): grid (ceil(rows / 256), splits). An 8-wave workgroup owns 256 feature
// rows (32 per wave, its fragments held in registers for the whole pass) and one contiguous range
// of W columns (with their bias, at most 128 KiB), which it DMAs into LDS at once (global_load_lds,
// one wait), then walks in tiles of 32 columns with no further barrier or global load. Per tile each wave issues inner / 16
// v_mfma_f32_32x32x16_f16 with W as the row operand, so lane l holds row (l % 32) and 16 of the
// tile's columns in increasing order. The lane folds them into its running (max, sum, argmax) the
// way UpdateArgMax does (a larger maximum rescales the sum by exp(old max - new max); ties keep the
// earlier column; exp by the hardware exp2), then lanes l and l + 32 (the same row, the other 16 columns) merge, and the row's
// (max, sum, argmax) of this column range goes to part[split][row].
// Pass 2 (sox_ctc_merge): per row (one wave) the splits merge in a butterfly (ties keep the lower column);
// probability = min(1, 1 / sum). A non-finite logit anywhere sets *status (the reference throws
// "Recognizer output is invalid."), which pass 1 cleared.
#include "sox_device.h"

SOX_DEV void ctc_fold(float& m, float& s, int& idx, float m2, float s2, int i2) {
    // merge a (max, sum relative to that max, argmax) triple; equal maxima keep the lower column
    if (m2 > m || (m2 == m && i2 < idx)) {
        s = s * __expf(m - m2) + s2;
        m = m2;
        idx = i2;
    } else {
        s += s2 * __expf(m2 - m);
    }
}

#define LDS_PTR(p) ((__attribute__((address_space(3))) void*)(p))

// bytes of LDS for one workgroup's W columns and their bias (the launcher sizes the column range
// so that 32-column tiles x (inner fp16 + 1 fp32) fit)
#define SOX_CTC_LDS 131072

template <int KS>
__device__ __forceinline__ void ctc_part_body(const sox_ctc_args& p) {
    constexpr int ROWB = KS * 32;                      // LDS bytes per column: inner fp16, no padding
    constexpr int CPR = 2 * KS;                        // 16-byte chunks per column
    constexpr int SWZ = CPR % 8 == 0 ? 8 : CPR % 4 == 0 ? 4 : 2;  // chunk slot = chunk ^ (column % SWZ)
    __shared__ __attribute__((aligned(1024))) unsigned char wt[SOX_CTC_LDS];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6, l32 = lane & 31, hl = lane >> 5;
    const int row = blockIdx.x * 256 + wave * 32 + l32;
    const int c_beg = blockIdx.y * p.cols_per_split, c_end = min(c_beg + p.cols_per_split, p.columns);
    const int ncols = c_end - c_beg;
    const half_t* __restrict__ X = (const half_t*)p.x;
    const half_t* __restrict__ W = (const half_t*)p.w;
    if (blockIdx.x == 0 && blockIdx.y == 0 && t == 0) *p.status = 0;  // pass 2 runs after every pass-1 store

    // every W column of the range global -> LDS at once: 1 KiB DMA instructions dealt round-robin to
    // the 8 waves; lane l of instruction i fills bytes i * 1024 + 16 l = column n, slot j, which
    // holds chunk j ^ (n % SWZ) of that column
    const int bytes = ((ncols + 31) & ~31) * ROWB;
    for (int i = wave; i * 1024 < bytes; i += 8) {
        const int off = i * 1024 + lane * 16;
        if (off < bytes) {
            const int n = off / ROWB, slot = (off - n * ROWB) / 16;
            const half_t* src = W + (long)(c_beg + min(n, ncols - 1)) * p.ldw + 8 * (slot ^ (n % SWZ));
            __builtin_amdgcn_global_load_lds(src, LDS_PTR(wt + i * 1024), 16, 0, 0);
        }
    }
    // the range's bias (0 without one, or past the last column) after the W columns
    float* lb = (float*)(wt + bytes);
    for (int c = t; c < ((ncols + 31) & ~31); c += 512)
        lb[c] = (p.has_bias && c < ncols) ? p.bias[c_beg + c] : 0.0f;
    half8 a[KS];
    {
        const half_t* xr = X + (long)min(row, p.rows - 1) * p.inner + 8 * hl;
#pragma unroll
        for (int s = 0; s < KS; s++) a[s] = *(const half8*)(xr + 16 * s);
    }
    __builtin_amdgcn_s_waitcnt(0);  // this wave's DMAs and fragment loads landed
    __syncthreads();                 // ... and every other wave's

    // non-finite features are the only way to a non-finite logit: the weights and bias were checked
    // finite when the head was created, and fp16 products summed over <= 256 terms cannot overflow
    bool bad = false;
#pragma unroll
    for (int s = 0; s < KS; s++)
#pragma unroll
        for (int e = 0; e < 8; e++) bad = bad || !__builtin_isfinite((float)a[s][e]);

    float m = -INFINITY, sum = 0.0f;
    int idx = 0x7fffffff;
    constexpr float L2E = 1.4426950408889634f;
    // lane: row l32, columns c0 + 8 (q / 4) + 4 hl + q % 4 for q = 0..15 (increasing); the
    // accumulators start from those columns' bias
    auto bias_acc = [&](int c0) __attribute__((always_inline)) {
        float16v acc;
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const float4v b4 = *(const float4v*)(lb + c0 + 8 * g + 4 * hl);
#pragma unroll
            for (int e = 0; e < 4; e++) acc[4 * g + e] = b4[e];
        }
        return acc;
    };
    // UpdateArgMax over a tile: the tile maximum, the running sum rescaled once to the new maximum
    // plus the tile's exp(v - new max); the first column of the tile maximum only when it raises the
    // running maximum (ties keep the earlier column)
    auto fold_tile = [&](float16v v, int c0) __attribute__((always_inline)) {
        if (c0 + 32 > ncols) {  // uniform: the range's last, partial tile
#pragma unroll
            for (int q = 0; q < 16; q++)
                if (c0 + 8 * (q / 4) + 4 * hl + q % 4 >= ncols) v[q] = -INFINITY;
        }
        float tm = v[0];
#pragma unroll
        for (int q = 1; q < 16; q++) tm = fmaxf(tm, v[q]);
        const float mn = fmaxf(m, tm);
        const float ml = -mn * L2E;
        float ts = 0.0f;
#pragma unroll
        for (int q = 0; q < 16; q++) ts += __builtin_amdgcn_exp2f(__builtin_fmaf(v[q], L2E, ml));
        if (tm > m) {
            int ti = 0;
#pragma unroll
            for (int q = 15; q >= 0; q--)
                if (v[q] == tm) ti = c0 + 8 * (q / 4) + 4 * hl + q % 4;
            sum = (m == -INFINITY ? 0.0f : sum * __builtin_amdgcn_exp2f((m - mn) * L2E)) + ts;
            m = mn;
            idx = c_beg + ti;
        } else {
            sum += ts;
        }
    };
    // two 32-column tiles per step: their MFMA chains interleave (each MFMA depends only on the
    // previous one of its own tile)
    for (int c0 = 0; c0 < ncols; c0 += 64) {
        const bool two = c0 + 32 < ncols;  // uniform
        float16v acc0 = bias_acc(c0), acc1 = two ? bias_acc(c0 + 32) : acc0;
        const int n0 = c0 + l32, n1 = c0 + 32 + l32;  // the tile columns this lane feeds
        const unsigned char* wb0 = wt + n0 * ROWB;
        const unsigned char* wb1 = wt + n1 * ROWB;
#pragma unroll
        for (int s = 0; s < KS; s++) {
            const half8 b0 = *(const half8*)(wb0 + 16 * ((2 * s + hl) ^ (n0 % SWZ)));
            acc0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(b0, a[s], acc0, 0, 0, 0);
            if (two) {
                const half8 b1 = *(const half8*)(wb1 + 16 * ((2 * s + hl) ^ (n1 % SWZ)));
                acc1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(b1, a[s], acc1, 0, 0, 0);
            }
        }
        fold_tile(acc0, c0);
        if (two) fold_tile(acc1, c0 + 32);
    }
    // lanes l and l + 32 hold the same row
    const float m2 = __shfl_xor(m, 32), s2 = __shfl_xor(sum, 32);
    const int i2 = __shfl_xor(idx, 32);
    const bool bad2 = __shfl_xor((int)bad, 32) != 0;
    if (hl == 0 && row < p.rows) {
        if (m2 > -INFINITY) {
            if (m > -INFINITY) ctc_fold(m, sum, idx, m2, s2, i2);
            else { m = m2; sum = s2; idx = i2; }
        }
        float* o = p.part + ((long)blockIdx.y * p.rows + row) * 3;
        o[0] = m;
        o[1] = (bad || bad2) ? __builtin_nanf("") : sum;
        o[2] = __int_as_float(idx);
    }
}

// one instance per inner / 16 (inner = 64 .. 256, a multiple of 16)
#define SOX_CTC_PART(KS) \
    extern "C" __global__ void __launch_bounds__(512) sox_ctc_part_k##KS(sox_ctc_args p) { ctc_part_body<KS>(p); }
SOX_CTC_PART(4) SOX_CTC_PART(5) SOX_CTC_PART(6) SOX_CTC_PART(7) SOX_CTC_PART(8) SOX_CTC_PART(9) SOX_CTC_PART(10)
SOX_CTC_PART(11) SOX_CTC_PART(12) SOX_CTC_PART(13) SOX_CTC_PART(14) SOX_CTC_PART(15) SOX_CTC_PART(16)

// one wave per row: lane k holds split k (k < splits <= 64); the triples fold in a fixed butterfly
// (equal maxima keep the lower column, so the argmax is the first one whatever the order)
extern "C" __global__ void __launch_bounds__(256) sox_ctc_merge(sox_ctc_merge_args p) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= p.rows) return;  // wave-uniform
    float m = -INFINITY, s = 0.0f;
    int idx = 0x7fffffff;
    bool bad = false;
    if (lane < p.splits) {
        const float* q = p.part + ((long)lane * p.rows + row) * 3;
        m = q[0];
        s = q[1];
        idx = __float_as_int(q[2]);
        bad = s != s;
        if (m == -INFINITY) { s = 0.0f; idx = 0x7fffffff; }  // an empty split
    }
#pragma unroll
    for (int d = 1; d < 64; d *= 2) {
        const float m2 = __shfl_xor(m, d), s2 = __shfl_xor(s, d);
        const int i2 = __shfl_xor(idx, d);
        bad = (__shfl_xor((int)bad, d) != 0) || bad;
        if (m2 > -INFINITY) {
            if (m > -INFINITY) ctc_fold(m, s, idx, m2, s2, i2);
            else { m = m2; s = s2; idx = i2; }
        }
    }
    if (lane == 0) {
        if (bad || !(s > 0.0f) || __builtin_isinf(s)) {
            *p.status = 1;
            s = 1.0f;
        }
        p.indices[row] = idx;
        p.probs[row] = fminf(1.0f, 1.0f / s);
    }
}
