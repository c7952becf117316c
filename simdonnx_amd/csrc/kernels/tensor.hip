// The rest of the ExecOp surface on gfx950 (the cases of Backends/Vulkan/VkGraph.cs:795-1068):
// bilinear resize, pad, transpose / slice (one strided gather), LeakyRelu / Tanh / Clip / Erf,
// DepthToSpace / SpaceToDepth, average pool, global average pool and batched MatMul.
//
// All of them move bytes rather than multiply: one work item per output element or per 16-byte
// channel vector of an NHWC pixel (when the channel count allows), fp32 math, fp16 or fp32 storage.
// Index arithmetic is 32-bit; the launchers reject tensors past 2^31 elements.
#include "sox_device.h"

template <typename T, int CV> struct Vt {
    typedef T V __attribute__((ext_vector_type(CV)));
};

// The global thread index of a 1-D grid, workgroups numbered XCD-major when the grid divides by 8:
// consecutive workgroups go to the 8 XCDs in turn, so renumbered, each XCD runs one contiguous range
// and the output rows that read the same input rows (resize, pooling) find them in its L2.
SOX_DEV long xcd_block() {
    const int G = gridDim.x;
    return G % 8 == 0 ? (long)(blockIdx.x % 8) * (G / 8) + blockIdx.x / 8 : (long)blockIdx.x;
}
SOX_DEV long gid() { return xcd_block() * blockDim.x + threadIdx.x; }

// ------------------------------------------------------------------------------------------
// Bilinear resize (Kernels/Nhwc.cs:773-870): per axis f = (o + 0.5) / scale - 0.5, taps floor(f)
// and floor(f) + 1 clamped to the image, weight f - floor(f); v = top + (bot - top) wy with
// top/bot = a + (b - a) wx; [relu]; + [relu](addend). No contraction, so the per-element operations
// are the CPU's.
// ------------------------------------------------------------------------------------------
template <typename T, int CV>
__device__ __forceinline__ void bilinear_body(const sox_bilinear_args& p) {
#pragma clang fp contract(off)
    typedef typename Vt<T, CV>::V Vec;
    const int cvn = p.c / CV;
    const long idx = gid();
    if (idx >= (long)p.n * p.oh * p.ow * cvn) return;
    const int c0 = (int)(idx % cvn) * CV;
    const long pix = idx / cvn;
    const int ox = (int)(pix % p.ow);
    const int q = (int)(pix / p.ow), oy = q % p.oh, b = q / p.oh;
    const float fy = ((float)oy + 0.5f) / p.sy - 0.5f, fx = ((float)ox + 0.5f) / p.sx - 0.5f;
    const float fly = floorf(fy), flx = floorf(fx);
    const int y0 = min(max((int)fly, 0), p.ih - 1), y1 = min(max((int)fly + 1, 0), p.ih - 1);
    const int x0 = min(max((int)flx, 0), p.iw - 1), x1 = min(max((int)flx + 1, 0), p.iw - 1);
    const float wy = fy - fly, wx = fx - flx;
    const T* img = (const T*)p.x + (long)b * p.ih * p.iw * p.c + c0;
    const Vec va = *(const Vec*)(img + ((long)y0 * p.iw + x0) * p.c);
    const Vec vb = *(const Vec*)(img + ((long)y0 * p.iw + x1) * p.c);
    const Vec ve = *(const Vec*)(img + ((long)y1 * p.iw + x0) * p.c);
    const Vec vf = *(const Vec*)(img + ((long)y1 * p.iw + x1) * p.c);
    Vec vadd;
    if (p.flags & 2) vadd = *(const Vec*)((const T*)p.add + pix * p.c + c0);
    Vec out;
#pragma unroll
    for (int e = 0; e < CV; e++) {
        const float a = to_f(va[e]), bb = to_f(vb[e]), ee = to_f(ve[e]), ff = to_f(vf[e]);
        const float top = a + (bb - a) * wx;
        const float bot = ee + (ff - ee) * wx;
        float v = top + (bot - top) * wy;
        if (p.flags & 1) v = fmaxf(v, 0.0f);
        if (p.flags & 2) {
            const float s = to_f(vadd[e]);
            v += (p.flags & 4) ? fmaxf(s, 0.0f) : s;
        }
        out[e] = (T)v;
    }
    *(Vec*)((T*)p.y + pix * p.c + c0) = out;
}

extern "C" __global__ void __launch_bounds__(256) sox_bilinear_f16_v(sox_bilinear_args p) { bilinear_body<half_t, 8>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_bilinear_bf16_v(sox_bilinear_args p) { bilinear_body<bf16_t, 8>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_bilinear_f16_s(sox_bilinear_args p) { bilinear_body<half_t, 1>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_bilinear_bf16_s(sox_bilinear_args p) { bilinear_body<bf16_t, 1>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_bilinear_f32_v(sox_bilinear_args p) { bilinear_body<float, 4>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_bilinear_f32_s(sox_bilinear_args p) { bilinear_body<float, 1>(p); }

// ------------------------------------------------------------------------------------------
// Rank-4 pad in storage order (Kernels/Nhwc.cs:877-900 for the NHWC spatial case): source index
// o - pb per dim; outside -> the constant, or the reflected index (Nhwc.Reflect, no edge repeat).
// CV > 1 only when the innermost dim is unpadded and a multiple of CV (the launcher checks).
// ------------------------------------------------------------------------------------------
template <typename T, int CV>
__device__ __forceinline__ void pad_body(const sox_pad_args& p) {
    typedef typename Vt<T, CV>::V Vec;
    const int d3v = p.od[3] / CV;
    const long idx = gid();
    if (idx >= (long)p.od[0] * p.od[1] * p.od[2] * d3v) return;
    int s3 = (int)(idx % d3v) * CV;
    int r = (int)(idx / d3v);
    int s2 = r % p.od[2];
    r /= p.od[2];
    int s1 = r % p.od[1], s0 = r / p.od[1];
    int s[4] = {s0 - p.pb[0], s1 - p.pb[1], s2 - p.pb[2], s3 - p.pb[3]};
    bool inside = true;
#pragma unroll
    for (int d = 0; d < 4; d++)
        if ((unsigned)s[d] >= (unsigned)p.id[d]) {
            if (p.reflect) s[d] = sox_reflect(s[d], p.id[d]);
            else inside = false;
        }
    Vec v;
    if (inside) {
        v = *(const Vec*)((const T*)p.x + (((long)s[0] * p.id[1] + s[1]) * p.id[2] + s[2]) * p.id[3] + s[3]);
    } else {
#pragma unroll
        for (int e = 0; e < CV; e++) v[e] = (T)p.value;
    }
    *(Vec*)((T*)p.y + idx * CV) = v;
}

extern "C" __global__ void __launch_bounds__(256) sox_pad_f16_v(sox_pad_args p) { pad_body<half_t, 8>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_pad_bf16_v(sox_pad_args p) { pad_body<bf16_t, 8>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_pad_f16_s(sox_pad_args p) { pad_body<half_t, 1>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_pad_bf16_s(sox_pad_args p) { pad_body<bf16_t, 1>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_pad_f32_v(sox_pad_args p) { pad_body<float, 4>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_pad_f32_s(sox_pad_args p) { pad_body<float, 1>(p); }

// ------------------------------------------------------------------------------------------
// Strided gather (Transpose, Slice; Kernels/Ops.cs:798-883): the output index's digits over od[]
// (innermost last) times the per-dim source strides, from base. The launcher checks that every
// source offset stays inside the input.
// ------------------------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ void gather_body(const sox_gather_args& p) {
    const long idx = gid();
    if (idx >= p.count) return;
    unsigned r = (unsigned)idx;
    long off = p.base;
#pragma unroll
    for (int k = 5; k >= 0; k--) {
        const unsigned d = (unsigned)p.od[k];
        const unsigned o = r % d;
        r /= d;
        off += (long)o * p.str[k];
    }
    ((T*)p.y)[idx] = ((const T*)p.x)[off];
}

extern "C" __global__ void __launch_bounds__(256) sox_gather_f16(sox_gather_args p) { gather_body<half_t>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_gather_bf16(sox_gather_args p) { gather_body<bf16_t>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_gather_f32(sox_gather_args p) { gather_body<float>(p); }

// ------------------------------------------------------------------------------------------
// Batched 2D transpose through LDS, the permutations that swap two contiguous groups of dims
// (NHWC <-> NCHW, the last-two-dims swap; the reference's fast paths, Kernels/Ops.cs:802-868):
// x [batch][R][C] -> y [batch][C][R]. A 256-thread workgroup moves one 64 x 64 tile: reads 64
// consecutive columns of 16 rows per pass, writes 64 consecutive rows of 16 columns per pass. The
// tile rows are padded by one 4-byte word, so the column reads hit 64 distinct banks.
// Grid (ceil(C / 64), ceil(R / 64), batch).
// ------------------------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ void transpose2d_body(const sox_transpose2d_args& p) {
    constexpr int PADE = 4 / sizeof(T);  // one 4-byte word of padding per tile row
    __shared__ T tile[64][64 + PADE];
    const int tx = threadIdx.x % 64, ty = threadIdx.x / 64;
    const int c0 = blockIdx.x * 64, r0 = blockIdx.y * 64;
    const T* __restrict__ x = (const T*)p.x + (long)blockIdx.z * p.rows * p.cols;
    T* __restrict__ y = (T*)p.y + (long)blockIdx.z * p.rows * p.cols;
#pragma unroll
    for (int k = 0; k < 16; k++) {
        const int r = r0 + ty + 4 * k, c = c0 + tx;
        if (r < p.rows && c < p.cols) tile[ty + 4 * k][tx] = x[(long)r * p.cols + c];
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 16; k++) {
        const int c = c0 + ty + 4 * k, r = r0 + tx;
        if (r < p.rows && c < p.cols) y[(long)c * p.rows + r] = tile[tx][ty + 4 * k];
    }
}

extern "C" __global__ void __launch_bounds__(256) sox_transpose2d_f16(sox_transpose2d_args p) { transpose2d_body<half_t>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_transpose2d_bf16(sox_transpose2d_args p) { transpose2d_body<bf16_t>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_transpose2d_f32(sox_transpose2d_args p) { transpose2d_body<float>(p); }

// ------------------------------------------------------------------------------------------
// LeakyRelu / Tanh / Clip / Erf (Kernels/Act.cs:83-147, the vector forms): leaky = max(x, a x)
// for a <= 1 else min(x, a x); o tanh(i x) = 2o sigmoid(2i x) - o with the Cephes sigmoid;
// clip = min(max(x, lo), hi); erf = A&S 7.1.26.
// ------------------------------------------------------------------------------------------
SOX_DEV float unary2_op(float x, int mode, float a, float b) {
#pragma clang fp contract(off)
    switch (mode) {
        case 0: return a <= 1.0f ? fmaxf(x, x * a) : fminf(x, x * a);
        case 1: return sox_sigmoid(x * (2.0f * a)) * (2.0f * b) - b;
        case 2: return fminf(fmaxf(x, a), b);
        default: return sox_erf(x);
    }
}

template <typename T>
__device__ __forceinline__ void unary2_body(const sox_unary2_args& p) {
    constexpr int CV = 16 / sizeof(T);
    typedef typename Vt<T, CV>::V Vec;
    const long base = gid() * CV;
    const T* x = (const T*)p.x;
    T* y = (T*)p.y;
    if (base + CV <= p.count) {
        const Vec xv = *(const Vec*)(x + base);
        Vec out;
#pragma unroll
        for (int e = 0; e < CV; e++) out[e] = (T)unary2_op(to_f(xv[e]), p.mode, p.a, p.b);
        *(Vec*)(y + base) = out;
    } else {
        for (long i = base; i < p.count; i++) y[i] = (T)unary2_op(to_f(x[i]), p.mode, p.a, p.b);
    }
}

extern "C" __global__ void __launch_bounds__(256) sox_unary2_f16(sox_unary2_args p) { unary2_body<half_t>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_unary2_bf16(sox_unary2_args p) { unary2_body<bf16_t>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_unary2_f32(sox_unary2_args p) { unary2_body<float>(p); }

// ------------------------------------------------------------------------------------------
// DepthToSpace / SpaceToDepth, NHWC (Kernels/Nhwc.Det.cs:210-282). Depth-to-space: output (y, x, c)
// reads input (y / b, x / b) channel c b^2 + sub (CRD) or sub oc + c (DCR), sub = (y % b) b + x % b.
// Space-to-depth is the inverse: output channel c' = c b^2 + sub (CRD) or sub ic + c (DCR) reads
// input (y b + sub / b, x b + sub % b) channel c. One work item per output element; consecutive
// items are consecutive output channels (coalesced stores).
// ------------------------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ void d2s_body(const sox_d2s_args& p) {
    const long idx = gid();
    if (idx >= p.count) return;
    const int bk = p.block, bb = bk * bk;
    const int ch = (int)(idx % p.oc);
    const int pix = (int)(idx / p.oc);
    const int ox = pix % p.ow, q = pix / p.ow, oy = q % p.oh, b = q / p.oh;
    int sy, sx, sc;
    if (!p.s2d) {
        const int sub = (oy % bk) * bk + ox % bk;
        sy = oy / bk;
        sx = ox / bk;
        sc = p.crd ? ch * bb + sub : sub * p.oc + ch;
    } else {
        const int sub = p.crd ? ch % bb : ch / p.ic;
        sc = p.crd ? ch / bb : ch % p.ic;
        sy = oy * bk + sub / bk;
        sx = ox * bk + sub % bk;
    }
    ((T*)p.y)[idx] = ((const T*)p.x)[(((long)b * p.ih + sy) * p.iw + sx) * p.ic + sc];
}

extern "C" __global__ void __launch_bounds__(256) sox_d2s_f16(sox_d2s_args p) { d2s_body<half_t>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_d2s_bf16(sox_d2s_args p) { d2s_body<bf16_t>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_d2s_f32(sox_d2s_args p) { d2s_body<float>(p); }

// DCR order with whole 16-byte channel vectors: the CV consecutive output channels of a work item
// are CV consecutive input channels (depth-to-space: sub oc + c; space-to-depth: output channel
// sub ic + c), so each item is one 16-byte load and store. The launcher routes here when oc
// (depth-to-space) or ic (space-to-depth) is a multiple of CV.
template <typename T, int CV>
__device__ __forceinline__ void d2s_dcr_body(const sox_d2s_args& p) {
    typedef typename Vt<T, CV>::V Vec;
    const long idx = gid();
    if (idx * CV >= p.count) return;
    const int bk = p.block;
    const int ch = (int)((idx * CV) % p.oc);
    const int pix = (int)((idx * CV) / p.oc);
    const int ox = pix % p.ow, q = pix / p.ow, oy = q % p.oh, b = q / p.oh;
    int sy, sx, sc;
    if (!p.s2d) {
        const int sub = (oy % bk) * bk + ox % bk;
        sy = oy / bk;
        sx = ox / bk;
        sc = sub * p.oc + ch;
    } else {
        const int sub = ch / p.ic;
        sc = ch % p.ic;
        sy = oy * bk + sub / bk;
        sx = ox * bk + sub % bk;
    }
    *(Vec*)((T*)p.y + idx * CV) = *(const Vec*)((const T*)p.x + (((long)b * p.ih + sy) * p.iw + sx) * p.ic + sc);
}

extern "C" __global__ void __launch_bounds__(256) sox_d2s_dcr_f16(sox_d2s_args p) { d2s_dcr_body<half_t, 8>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_d2s_dcr_bf16(sox_d2s_args p) { d2s_dcr_body<bf16_t, 8>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_d2s_dcr_f32(sox_d2s_args p) { d2s_dcr_body<float, 4>(p); }

// ------------------------------------------------------------------------------------------
// Average pool, NHWC (Kernels/Ops.Seq.cs:180-215): taps summed in (ky, kx) order from zero, then
// one multiply by 1 / count, count = kh kw (count_include_pad) or the in-bounds taps.
// ------------------------------------------------------------------------------------------
template <typename T, int CV>
__device__ __forceinline__ void avgpool_body(const sox_avgpool_args& p) {
    typedef typename Vt<T, CV>::V Vec;
    const int cvn = p.c / CV;
    const long idx = gid();
    if (idx >= (long)p.n * p.oh * p.ow * cvn) return;
    const int c0 = (int)(idx % cvn) * CV;
    const int pix = (int)(idx / cvn);
    const int ox = pix % p.ow, q = pix / p.ow, oy = q % p.oh, b = q / p.oh;
    const T* img = (const T*)p.x + (long)b * p.ih * p.iw * p.c + c0;
    float acc[CV];
#pragma unroll
    for (int e = 0; e < CV; e++) acc[e] = 0.0f;
    int cnt = 0;
    for (int ky = 0; ky < p.kh; ky++) {
        const int iy = oy * p.sh + ky - p.pt;
        if ((unsigned)iy >= (unsigned)p.ih) continue;
        for (int kx = 0; kx < p.kw; kx++) {
            const int ix = ox * p.sw + kx - p.pl;
            if ((unsigned)ix >= (unsigned)p.iw) continue;
            const Vec v = *(const Vec*)(img + ((long)iy * p.iw + ix) * p.c);
#pragma unroll
            for (int e = 0; e < CV; e++) acc[e] += to_f(v[e]);
            cnt++;
        }
    }
    const float inv = 1.0f / (float)(p.count_include_pad ? p.kh * p.kw : max(cnt, 1));
    Vec out;
#pragma unroll
    for (int e = 0; e < CV; e++) out[e] = (T)(acc[e] * inv);
    *(Vec*)((T*)p.y + (long)pix * p.c + c0) = out;
}

extern "C" __global__ void __launch_bounds__(256) sox_avgpool_f16_v(sox_avgpool_args p) { avgpool_body<half_t, 8>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_avgpool_bf16_v(sox_avgpool_args p) { avgpool_body<bf16_t, 8>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_avgpool_f16_s(sox_avgpool_args p) { avgpool_body<half_t, 1>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_avgpool_bf16_s(sox_avgpool_args p) { avgpool_body<bf16_t, 1>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_avgpool_f32_v(sox_avgpool_args p) { avgpool_body<float, 4>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_avgpool_f32_s(sox_avgpool_args p) { avgpool_body<float, 1>(p); }

// ------------------------------------------------------------------------------------------
// GlobalAvgPool finish (gap_sum.comp): the GAP partial kernel's per-chunk channel sums times
// 1 / hw. Grid (ceil(c / 64), n): thread (phase f = t / 64, channel t % 64) adds chunks f, f + 4,
// f + 8, ... with 8 loads in flight, then the 4 phase sums are added in phase order.
// ------------------------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ void gap_mean_body(const sox_gap_mean_args& p) {
    __shared__ float red[4][64];
    const int t = threadIdx.x, f = t / 64, cl = t % 64;
    const int ch = blockIdx.x * 64 + cl, b = blockIdx.y;
    float s = 0.0f;
    if (ch < p.c) {
        const float* part = p.part + (long)b * p.chunks * p.c + ch;
        for (int k0 = f; k0 < p.chunks; k0 += 32) {
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int k = k0 + 4 * u;
                v[u] = k < p.chunks ? part[(long)k * p.c] : 0.0f;
            }
#pragma unroll
            for (int u = 0; u < 8; u++) s += v[u];
        }
    }
    red[f][cl] = s;
    __syncthreads();
    if (f == 0 && ch < p.c)
        ((T*)p.y)[(long)b * p.c + ch] = (T)((((red[0][cl] + red[1][cl]) + red[2][cl]) + red[3][cl]) * p.inv_hw);
}

extern "C" __global__ void __launch_bounds__(256) sox_gap_mean_f16(sox_gap_mean_args p) { gap_mean_body<half_t>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_gap_mean_bf16(sox_gap_mean_args p) { gap_mean_body<bf16_t>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_gap_mean_f32(sox_gap_mean_args p) { gap_mean_body<float>(p); }

// ------------------------------------------------------------------------------------------
// Batched MatMul of two activations (Kernels/Ops.Seq.cs:92-116): y[b] = a[b] . b[b or 0], fp32
// accumulation in ascending k, one fma each. 64 x 64 output tile per 256-thread workgroup (4 x 4
// per thread), 16-deep k slices staged in LDS as fp32 ([k][m] and [k][n], so each thread reads
// its 4 rows / 4 columns as one 16-byte LDS read). Grid (ceil(n / 64), ceil(m / 64), batch).
// ------------------------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ void matmul_body(const sox_matmul_args& p) {
    __shared__ __attribute__((aligned(16))) float As[16][64];
    __shared__ __attribute__((aligned(16))) float Bs[16][64];
    const int t = threadIdx.x, tm = t / 16, tn = t % 16;
    const int m0 = blockIdx.y * 64, n0 = blockIdx.x * 64, bz = blockIdx.z;
    const T* __restrict__ A = (const T*)p.a + bz * p.a_stride;
    const T* __restrict__ B = (const T*)p.b + bz * p.b_stride;
    T* __restrict__ Y = (T*)p.y + bz * p.y_stride;
    float acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = 0.0f;
    for (int k0 = 0; k0 < p.k; k0 += 16) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int e = t + 256 * i;
            const int ar = e / 16, ak = e % 16;  // A: 64 rows x 16 k, k fastest (row-contiguous reads)
            const int gm = m0 + ar, gk = k0 + ak;
            As[ak][ar] = (gm < p.m && gk < p.k) ? to_f(A[(long)gm * p.k + gk]) : 0.0f;
            const int bk = e / 64, bn = e % 64;  // B: 16 k x 64 columns, columns fastest
            const int gk2 = k0 + bk, gn = n0 + bn;
            Bs[bk][bn] = (gk2 < p.k && gn < p.n) ? to_f(B[(long)gk2 * p.n + gn]) : 0.0f;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < 16; kk++) {
            const float4v a4 = *(const float4v*)&As[kk][tm * 4];
            const float4v b4 = *(const float4v*)&Bs[kk][tn * 4];
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) acc[i][j] = __builtin_fmaf(a4[i], b4[j], acc[i][j]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int gm = m0 + tm * 4 + i;
        if (gm >= p.m) continue;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int gn = n0 + tn * 4 + j;
            if (gn < p.n) Y[(long)gm * p.n + gn] = (T)acc[i][j];
        }
    }
}

extern "C" __global__ void __launch_bounds__(256) sox_matmul_f16(sox_matmul_args p) { matmul_body<half_t>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_matmul_bf16(sox_matmul_args p) { matmul_body<bf16_t>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_matmul_f32(sox_matmul_args p) { matmul_body<float>(p); }

// ------------------------------------------------------------------------------------------
// SafeDiv (Engine/Fusions/SafeDivOp.cs, Kernels/FusedKernels.cs:35-57): y = clamp(a / max(b, eps),
// lo, hi), fp32 math whatever the storage (the eps floor survives fp16 storage).
// ------------------------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ void safediv_body(const sox_safediv_args& p) {
    constexpr int CV = 16 / sizeof(T);
    typedef typename Vt<T, CV>::V Vec;
    const long base = gid() * CV;
    const T* a = (const T*)p.a;
    const T* b = (const T*)p.b;
    T* y = (T*)p.y;
    auto f = [&](float av, float bv) { return fminf(fmaxf(av / fmaxf(bv, p.eps), p.lo), p.hi); };
    if (base + CV <= p.count) {
        const Vec av = *(const Vec*)(a + base), bv = *(const Vec*)(b + base);
        Vec out;
#pragma unroll
        for (int e = 0; e < CV; e++) out[e] = (T)f(to_f(av[e]), to_f(bv[e]));
        *(Vec*)(y + base) = out;
    } else {
        for (long i = base; i < p.count; i++) y[i] = (T)f(to_f(a[i]), to_f(b[i]));
    }
}

extern "C" __global__ void __launch_bounds__(256) sox_safediv_f16(sox_safediv_args p) { safediv_body<half_t>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_safediv_bf16(sox_safediv_args p) { safediv_body<bf16_t>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_safediv_f32(sox_safediv_args p) { safediv_body<float>(p); }

// ------------------------------------------------------------------------------------------
// ChannelShift (Engine/Fusions/ChannelShiftOp.cs, Kernels/FusedKernels.cs:195-222), NHWC: one work
// item per CV channels of an output pixel (CV > 1 only when every group end is a multiple of CV).
// ------------------------------------------------------------------------------------------
template <typename T, int CV>
__device__ __forceinline__ void shift_body(const sox_shift_args& p) {
    typedef typename Vt<T, CV>::V Vec;
    const int cvn = p.c / CV;
    const long idx = gid();
    if (idx >= (long)p.n * p.h * p.w * cvn) return;
    const int c0 = (int)(idx % cvn) * CV;
    const int pix = (int)(idx / cvn);
    const int x = pix % p.w, q = pix / p.w, yy = q % p.h, b = q / p.h;
    int off = 0;
    bool shifted = false;
#pragma unroll
    for (int g = 4; g >= 0; g--)  // the group holding c0: the first g with c0 < ends[g]
        if (g < p.ngroups && c0 < p.ends[g]) {
            off = p.offs[g];
            shifted = true;
        }
    int sy = yy, sx = x;
    if (shifted) {
        if (p.axis == 2) sy += off;
        else sx += off;
    }
    Vec v;
    if ((unsigned)sy < (unsigned)p.h && (unsigned)sx < (unsigned)p.w) {
        v = *(const Vec*)((const T*)p.x + (((long)b * p.h + sy) * p.w + sx) * p.c + c0);
    } else {
#pragma unroll
        for (int e = 0; e < CV; e++) v[e] = (T)0.0f;
    }
    *(Vec*)((T*)p.y + (long)pix * p.c + c0) = v;
}

extern "C" __global__ void __launch_bounds__(256) sox_shift_f16_v(sox_shift_args p) { shift_body<half_t, 8>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_shift_bf16_v(sox_shift_args p) { shift_body<bf16_t, 8>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_shift_f16_s(sox_shift_args p) { shift_body<half_t, 1>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_shift_bf16_s(sox_shift_args p) { shift_body<bf16_t, 1>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_shift_f32_v(sox_shift_args p) { shift_body<float, 4>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_shift_f32_s(sox_shift_args p) { shift_body<float, 1>(p); }

// ------------------------------------------------------------------------------------------
// UpHead (Engine/Fusions/UpHeadOp.cs, Kernels/FusedKernels.cs:62-192): one thread per output pixel,
// CV channels per load (c is a multiple of 4: 16-byte loads for fp32 and c % 8 == 0 fp16, else 8).
// s[c] = [relu](bilinear(x)) + [relu](skip) (Nhwc.ResizePixel's operations, no contraction), then
// out[o] = act(bias[o] + sum_c s[c] w[o][c]) in ascending c. The head weights (oc x c <= 1024) and
// the skip conv's weights (<= 4096) sit in LDS as fp32. With the skip conv the skip channel is
// recomputed here: bias + sum over taps (ky, kx) and input channels of x w, [relu] (the stem conv's
// direct order, Nhwc.cs:343-373), constant or reflect padding.
// ------------------------------------------------------------------------------------------
template <typename T, int CV>
__device__ __forceinline__ void uphead_body(const sox_uphead_args& p) {
#pragma clang fp contract(off)
    typedef typename Vt<T, CV>::V Vec;
    __shared__ float ws[1024];
    __shared__ float wsc[4096];
    const bool has_sc = (p.flags & 8) != 0;
    const int nsc = has_sc ? p.c * p.skc * p.kh * p.kw : 0;
    for (int i = threadIdx.x; i < p.oc * p.c; i += blockDim.x) ws[i] = to_f(((const T*)p.w)[i]);
    for (int i = threadIdx.x; i < nsc; i += blockDim.x) wsc[i] = to_f(((const T*)p.w_sc)[i]);
    __syncthreads();
    const long idx = gid();
    if (idx >= (long)p.n * p.oh * p.ow) return;
    const int ox = (int)(idx % p.ow);
    const int q = (int)(idx / p.ow), oy = q % p.oh, b = q / p.oh;
    const float fy = ((float)oy + 0.5f) / p.sy - 0.5f, fx = ((float)ox + 0.5f) / p.sx - 0.5f;
    const float fly = floorf(fy), flx = floorf(fx);
    const int y0 = min(max((int)fly, 0), p.ih - 1), y1 = min(max((int)fly + 1, 0), p.ih - 1);
    const int x0 = min(max((int)flx, 0), p.iw - 1), x1 = min(max((int)flx + 1, 0), p.iw - 1);
    const float wy = fy - fly, wx = fx - flx;
    const T* img = (const T*)p.x + (long)b * p.ih * p.iw * p.c;
    const T* pa = img + ((long)y0 * p.iw + x0) * p.c;
    const T* pb = img + ((long)y0 * p.iw + x1) * p.c;
    const T* pe = img + ((long)y1 * p.iw + x0) * p.c;
    const T* pf = img + ((long)y1 * p.iw + x1) * p.c;
    float acc[8];
#pragma unroll
    for (int o = 0; o < 8; o++) acc[o] = (o < p.oc && (p.flags & 4)) ? p.bias[o] : 0.0f;
    // CV channels at a time: one 16-byte load per tap (and per skip pixel) when c allows
    for (int c0 = 0; c0 < p.c; c0 += CV) {
        const Vec va = *(const Vec*)(pa + c0), vb = *(const Vec*)(pb + c0);
        const Vec ve = *(const Vec*)(pe + c0), vf = *(const Vec*)(pf + c0);
        Vec vs;
        if (!has_sc) vs = *(const Vec*)((const T*)p.skip + idx * p.c + c0);
#pragma unroll
        for (int u = 0; u < CV; u++) {
            const int ch = c0 + u;
            const float a = to_f(va[u]), bb = to_f(vb[u]), e = to_f(ve[u]), f = to_f(vf[u]);
            const float top = a + (bb - a) * wx;
            const float bot = e + (f - e) * wx;
            float v = top + (bot - top) * wy;
            if (p.flags & 1) v = fmaxf(v, 0.0f);
            float sk;
            if (has_sc) {
                sk = (p.sc_flags & 1) ? p.b_sc[ch] : 0.0f;
                const T* sx0 = (const T*)p.skip + (long)b * p.oh * p.ow * p.skc;
                for (int ky = 0; ky < p.kh; ky++) {
                    int iy = oy + ky - p.pt;
                    bool rin = (unsigned)iy < (unsigned)p.oh;
                    if (!rin && (p.sc_flags & 2)) { iy = sox_reflect(iy, p.oh); rin = true; }
                    for (int kx = 0; kx < p.kw; kx++) {
                        int ix = ox + kx - p.pl;
                        bool cin = (unsigned)ix < (unsigned)p.ow;
                        if (!cin && (p.sc_flags & 2)) { ix = sox_reflect(ix, p.ow); cin = true; }
                        const float* wk = wsc + ((long)ch * p.skc * p.kh + ky) * p.kw + kx;
                        for (int ci = 0; ci < p.skc; ci++) {
                            const float xv = (rin && cin) ? to_f(sx0[((long)iy * p.ow + ix) * p.skc + ci]) : p.sc_pad_value;
                            sk = __builtin_fmaf(xv, wk[(long)ci * p.kh * p.kw], sk);
                        }
                    }
                }
                if (p.sc_flags & 4) sk = fmaxf(sk, 0.0f);
            } else {
                sk = to_f(vs[u]);
            }
            v += (p.flags & 2) ? fmaxf(sk, 0.0f) : sk;
#pragma unroll
            for (int o = 0; o < 8; o++)
                if (o < p.oc) acc[o] = acc[o] + v * ws[o * p.c + ch];
        }
    }
    const int act = (p.flags >> 4) & 15;
    T* yo = (T*)p.y + idx * p.oc;
#pragma unroll
    for (int o = 0; o < 8; o++)
        if (o < p.oc) yo[o] = (T)sox_act(acc[o], act);
}

extern "C" __global__ void __launch_bounds__(256) sox_uphead_f16_v(sox_uphead_args p) { uphead_body<half_t, 8>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_uphead_bf16_v(sox_uphead_args p) { uphead_body<bf16_t, 8>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_uphead_f16_s(sox_uphead_args p) { uphead_body<half_t, 4>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_uphead_bf16_s(sox_uphead_args p) { uphead_body<bf16_t, 4>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_uphead_f32_v(sox_uphead_args p) { uphead_body<float, 4>(p); }

// ------------------------------------------------------------------------------------------
// Image session pixel conversions (Backends/Vulkan/VkImageSession.cs:160-210). img2nhwc: one thread
// per tensor pixel, the three bytes of its (clamped) image pixel through the normalization table.
// nhwc2img: one thread per output 4-byte word.
// ------------------------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ void img2nhwc_body(const sox_img2nhwc_args& p) {
    // flat tensor pixels 2t and 2t + 1 per thread: their 6 values leave as 3 aligned 2-element words
    // (element offset 6t) instead of 6 separate stores; an odd last pixel alone
    const long total = (long)p.oh * p.ow;
    const long p0 = 2 * gid();
    if (p0 >= total) return;
    const int ob = p.swap * 2;
    T v[6];
#pragma unroll
    for (int k = 0; k < 2; k++) {
        const long pi = min(p0 + k, total - 1);
        const int oy = (int)(pi / p.ow), ox = (int)(pi - (long)oy * p.ow);
        const int sy = min(max(oy - p.pt, 0), p.ih - 1), sx = min(max(ox - p.pl, 0), p.iw - 1);
        const uint8_t* px = p.src + (long)sy * p.stride + (long)sx * p.bpp;
        v[3 * k] = (T)p.lut[px[ob]];
        v[3 * k + 1] = (T)p.lut[256 + px[1]];
        v[3 * k + 2] = (T)p.lut[512 + px[2 - ob]];
    }
    T* o = (T*)p.y + p0 * 3;
    if (p0 + 1 < total) {
        typedef T T2 __attribute__((ext_vector_type(2)));
#pragma unroll
        for (int k = 0; k < 3; k++) ((T2*)o)[k] = T2{v[2 * k], v[2 * k + 1]};
    } else {
#pragma unroll
        for (int k = 0; k < 3; k++) o[k] = v[k];
    }
}

extern "C" __global__ void __launch_bounds__(256) sox_img2nhwc_f16(sox_img2nhwc_args p) { img2nhwc_body<half_t>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_img2nhwc_bf16(sox_img2nhwc_args p) { img2nhwc_body<bf16_t>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_img2nhwc_f32(sox_img2nhwc_args p) { img2nhwc_body<float>(p); }

template <typename T>
__device__ __forceinline__ void nhwc2img_body(const sox_nhwc2img_args& p) {
#pragma clang fp contract(off)
    const int w4 = blockIdx.x * blockDim.x + threadIdx.x;
    if (w4 >= p.nwords) return;
    const T* x = (const T*)p.x;
    auto u8 = [&](long i) { return (uint32_t)fminf(fmaxf(to_f(x[i]) * p.scale + 0.5f, 0.0f), 255.0f); };
    const int ob = p.swap * 2;
    if (p.bpp == 4) {
        const int dy = w4 / p.iw, dx = w4 - dy * p.iw;
        const long i = ((long)(dy + p.pt) * p.w + dx + p.pl) * 3;
        p.dst[w4] = u8(i + ob) | (u8(i + 1) << 8) | (u8(i + 2 - ob) << 16) | (p.alpha[w4] & 0xff000000u);
        return;
    }
    long byte = (long)w4 * 4;
    const long total = (long)p.ih * p.iw * 3;
    long px = byte / 3;
    int c = (int)(byte - px * 3);
    int dy = (int)(px / p.iw), dx = (int)(px - (long)dy * p.iw);
    uint32_t packed = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        uint32_t v = 0;
        if (byte < total) {
            const int ch = c == 1 ? 1 : (c == 0 ? ob : 2 - ob);
            v = u8(((long)(dy + p.pt) * p.w + dx + p.pl) * 3 + ch);
        }
        packed |= v << (8 * j);
        byte++;
        if (++c == 3) {
            c = 0;
            if (++dx == p.iw) { dx = 0; dy++; }
        }
    }
    p.dst[w4] = packed;
}

extern "C" __global__ void __launch_bounds__(256) sox_nhwc2img_f16(sox_nhwc2img_args p) { nhwc2img_body<half_t>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_nhwc2img_bf16(sox_nhwc2img_args p) { nhwc2img_body<bf16_t>(p); }
extern "C" __global__ void __launch_bounds__(256) sox_nhwc2img_f32(sox_nhwc2img_args p) { nhwc2img_body<float>(p); }

