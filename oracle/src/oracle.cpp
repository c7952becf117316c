// CPU oracle: C++ restatement of SimdOnnx's NHWC CPU kernels (see oracle/oracle.h).
// TEST INFRASTRUCTURE ONLY - the product never links or loads this file.
//
// Built with -ffp-contract=off: a multiply followed by an add stays two roundings unless the
// reference itself uses a fused multiply-add, which is then written as fmaf / _mm*_fmadd_ps.
#include "../oracle.h"

#include <immintrin.h>
#include <math.h>
#include <omp.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <vector>

namespace {

int g_threads = 0;

int threads() { return g_threads > 0 ? g_threads : omp_get_num_procs(); }

// ---------------------------------------------------------------------------------------------
// SimdMath vector cores written per lane (Kernels/SimdMath.cs:121-168). Same operations and
// fusions as the Vector256 code, so a lane of the AVX2 epilogue and this function agree.
// ---------------------------------------------------------------------------------------------
inline float exp_core(float x) {
    x = fmaxf(x, -87.3f);
    x = fminf(x, 88.7f);
    float fx = fmaf(x, 1.4426950408889634f, 0.5f);
    float nf = floorf(fx);
    float r = fmaf(nf, -0.693359375f, x);
    r = fmaf(nf, 0.00021219444005469058f, r);
    float p = 1.9875691500e-4f;
    p = fmaf(p, r, 1.3981999507e-3f);
    p = fmaf(p, r, 8.3334519073e-3f);
    p = fmaf(p, r, 4.1665795894e-2f);
    p = fmaf(p, r, 1.6666665459e-1f);
    p = fmaf(p, r, 5.0000001201e-1f);
    float y = fmaf(p, r * r, r) + 1.0f;
    int ni = (int)nf + 127;
    uint32_t bits = (uint32_t)ni << 23;
    float pow2n;
    memcpy(&pow2n, &bits, 4);
    return y * pow2n;
}

inline float sigmoid_core(float x) { return 1.0f / (1.0f + exp_core(-x)); }

inline float erf_core(float x) {
    float sign = x < 0.0f || (x == 0.0f && signbit(x)) ? -1.0f : 1.0f;
    float ax = fabsf(x);
    float t = 1.0f / (1.0f + 0.3275911f * ax);
    float p = 1.061405429f;
    p = fmaf(p, t, -1.453152027f);
    p = fmaf(p, t, 1.421413741f);
    p = fmaf(p, t, -0.284496736f);
    p = fmaf(p, t, 0.254829592f);
    float y = 1.0f - (p * t) * exp_core(-(ax * ax));
    return y * sign;
}

inline float gelu_core(float x) { return (0.5f * x) * (1.0f + erf_core(x * 0.70710678118654752f)); }

// Act8 (Kernels/Nhwc.cs:91-99).
inline float act8(float v, int act) {
    switch (act) {
        case ORA_ACT_RELU: return fmaxf(v, 0.0f);
        case ORA_ACT_SIGMOID: return sigmoid_core(v);
        case ORA_ACT_GELU: return gelu_core(v);
        case ORA_ACT_HARDSWISH: return v * fminf(fmaxf(fmaf(v, 1.0f / 6.0f, 0.5f), 0.0f), 1.0f);
        case ORA_ACT_SWISH: return v * sigmoid_core(v);
        default: return v;
    }
}

// Nhwc.Reflect / Map (Kernels/Nhwc.cs:57-80): source index per (output, tap), -1 = constant pad.
int reflect_idx(int i, int dim) {
    if (dim <= 1) return 0;
    while (i < 0 || i >= dim) i = i < 0 ? -i : 2 * dim - 2 - i;
    return i;
}

std::vector<int> make_map(int out_len, int k, int stride, int pad, int in_len, int mode) {
    std::vector<int> m((size_t)out_len * k);
    for (int o = 0; o < out_len; o++)
        for (int kk = 0; kk < k; kk++) {
            int s = o * stride + kk - pad;
            m[(size_t)o * k + kk] = (unsigned)s < (unsigned)in_len ? s : mode == 1 ? reflect_idx(s, in_len) : -1;
        }
    return m;
}

constexpr int Ob = 16;

// ---------------------------------------------------------------------------------------------
// Micro-kernels. ptrs is [taps][R] (R rows of one tile), each pointing at `run` contiguous
// floats; weights wb are [taps][run][16] for block 0 and wb + wstep for block 1. part is
// [R][32]: part[r*32 + 0..15] block 0, part[r*32 + 16..31] block 1.
// acc = bias; for tap: for c: acc = fma(x, w, acc)  (Nhwc.cs:343-373, Nhwc.Avx512.cs:33-79).
// ---------------------------------------------------------------------------------------------
void tile_scalar(const float* const* ptrs, int R, int taps, int run, const float* wb, long wstep, int nblk,
                 const float* bias, float* part) {
    for (int r = 0; r < R; r++)
        for (int h = 0; h < nblk; h++)
            for (int l = 0; l < Ob; l++) {
                float acc = bias[h * Ob + l];
                for (int tap = 0; tap < taps; tap++) {
                    const float* p = ptrs[tap * R + r];
                    const float* w = wb + h * wstep + (long)tap * run * Ob + l;
                    for (int c = 0; c < run; c++) acc = fmaf(p[c], w[(long)c * Ob], acc);
                }
                part[r * 32 + h * Ob + l] = acc;
            }
}

__attribute__((target("avx2,fma"))) void tile_avx2(const float* const* ptrs, int taps, int run, const float* wb,
                                                   const float* bias, float* part /* stride 32 */) {
    // TileAvxK: 6 rows x 16 oc (Kernels/Nhwc.cs:343-373)
    __m256 a0 = _mm256_loadu_ps(bias), b0 = _mm256_loadu_ps(bias + 8);
    __m256 a1 = a0, a2 = a0, a3 = a0, a4 = a0, a5 = a0;
    __m256 b1 = b0, b2 = b0, b3 = b0, b4 = b0, b5 = b0;
    for (int tap = 0; tap < taps; tap++) {
        const float* const* pp = ptrs + tap * 6;
        const float *p0 = pp[0], *p1 = pp[1], *p2 = pp[2], *p3 = pp[3], *p4 = pp[4], *p5 = pp[5];
        const float* w = wb + (long)tap * run * Ob;
        for (int c = 0; c < run; c++, w += Ob) {
            __m256 w0 = _mm256_loadu_ps(w), w1 = _mm256_loadu_ps(w + 8);
            __m256 v0 = _mm256_broadcast_ss(p0 + c), v1 = _mm256_broadcast_ss(p1 + c);
            a0 = _mm256_fmadd_ps(v0, w0, a0); b0 = _mm256_fmadd_ps(v0, w1, b0);
            a1 = _mm256_fmadd_ps(v1, w0, a1); b1 = _mm256_fmadd_ps(v1, w1, b1);
            __m256 v2 = _mm256_broadcast_ss(p2 + c), v3 = _mm256_broadcast_ss(p3 + c);
            a2 = _mm256_fmadd_ps(v2, w0, a2); b2 = _mm256_fmadd_ps(v2, w1, b2);
            a3 = _mm256_fmadd_ps(v3, w0, a3); b3 = _mm256_fmadd_ps(v3, w1, b3);
            __m256 v4 = _mm256_broadcast_ss(p4 + c), v5 = _mm256_broadcast_ss(p5 + c);
            a4 = _mm256_fmadd_ps(v4, w0, a4); b4 = _mm256_fmadd_ps(v4, w1, b4);
            a5 = _mm256_fmadd_ps(v5, w0, a5); b5 = _mm256_fmadd_ps(v5, w1, b5);
        }
    }
    float* d = part;
    _mm256_storeu_ps(d, a0); _mm256_storeu_ps(d + 8, b0); d += 32;
    _mm256_storeu_ps(d, a1); _mm256_storeu_ps(d + 8, b1); d += 32;
    _mm256_storeu_ps(d, a2); _mm256_storeu_ps(d + 8, b2); d += 32;
    _mm256_storeu_ps(d, a3); _mm256_storeu_ps(d + 8, b3); d += 32;
    _mm256_storeu_ps(d, a4); _mm256_storeu_ps(d + 8, b4); d += 32;
    _mm256_storeu_ps(d, a5); _mm256_storeu_ps(d + 8, b5);
}

__attribute__((target("avx512f"))) void tile_avx512(const float* const* ptrs, int taps, int run, const float* wb,
                                                    long wstep, int nblk, const float* bias, float* part) {
    // Tile512x32 / Tile512x16: 10 rows x 32 (or 16) oc (Kernels/Nhwc.Avx512.cs:33-117)
    if (nblk == 2) {
        __m512 a[10], b[10];
        a[0] = _mm512_loadu_ps(bias);
        b[0] = _mm512_loadu_ps(bias + Ob);
        for (int i = 1; i < 10; i++) { a[i] = a[0]; b[i] = b[0]; }
        for (int tap = 0; tap < taps; tap++) {
            const float* const* pp = ptrs + tap * 10;
            const float* w = wb + (long)tap * run * Ob;
            const float* x = w + wstep;
            for (int c = 0; c < run; c++, w += Ob, x += Ob) {
                __m512 wa = _mm512_loadu_ps(w), wx = _mm512_loadu_ps(x);
#pragma GCC unroll 10
                for (int i = 0; i < 10; i++) {
                    __m512 v = _mm512_set1_ps(pp[i][c]);
                    a[i] = _mm512_fmadd_ps(v, wa, a[i]);
                    b[i] = _mm512_fmadd_ps(v, wx, b[i]);
                }
            }
        }
        for (int i = 0; i < 10; i++) {
            _mm512_storeu_ps(part + i * 32, a[i]);
            _mm512_storeu_ps(part + i * 32 + Ob, b[i]);
        }
    } else {
        __m512 a[10];
        a[0] = _mm512_loadu_ps(bias);
        for (int i = 1; i < 10; i++) a[i] = a[0];
        for (int tap = 0; tap < taps; tap++) {
            const float* const* pp = ptrs + tap * 10;
            const float* w = wb + (long)tap * run * Ob;
            for (int c = 0; c < run; c++, w += Ob) {
                __m512 wa = _mm512_loadu_ps(w);
#pragma GCC unroll 10
                for (int i = 0; i < 10; i++) a[i] = _mm512_fmadd_ps(_mm512_set1_ps(pp[i][c]), wa, a[i]);
            }
        }
        for (int i = 0; i < 10; i++) _mm512_storeu_ps(part + i * 32, a[i]);
    }
}

bool has_avx2() { return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma"); }
bool has_avx512() { return __builtin_cpu_supports("avx512f"); }

int resolve_tier(int tier) {
    if (tier == ORA_TIER_AUTO) return has_avx512() ? ORA_TIER_AVX512 : has_avx2() ? ORA_TIER_AVX2 : ORA_TIER_SCALAR;
    if (tier == ORA_TIER_AVX512 && !has_avx512()) return -1;
    if (tier == ORA_TIER_AVX2 && !has_avx2()) return -1;
    return tier;
}

// Rows per tile and oc blocks per tile for a tier (Tile = 6 / Tile5 = 10, Nhwc.cs:37, Nhwc.Avx512.cs:22).
int tier_rows(int tier) { return tier == ORA_TIER_AVX512 ? 10 : tier == ORA_TIER_AVX2 ? 6 : 4; }
int tier_blocks(int tier) { return tier == ORA_TIER_AVX512 ? 2 : 1; }

// Runs one tile: R rows (the tier's tile height), nblk blocks.
void run_tile(int tier, const float* const* ptrs, int taps, int run, const float* wb, long wstep, int nblk,
              const float* bias, float* part) {
    if (tier == ORA_TIER_AVX512) {
        tile_avx512(ptrs, taps, run, wb, wstep, nblk, bias, part);
    } else if (tier == ORA_TIER_AVX2) {
        for (int h = 0; h < nblk; h++) {
            // TileAvxK writes rows at stride 32 into part + h*16
            float tmp[6 * 32];
            tile_avx2(ptrs, taps, run, wb + h * wstep, bias + h * Ob, tmp);
            for (int r = 0; r < 6; r++) memcpy(part + r * 32 + h * Ob, tmp + r * 32, Ob * 4);
        }
    } else {
        tile_scalar(ptrs, tier_rows(tier), taps, run, wb, wstep, nblk, bias, part);
    }
}

// Store16 / Epilogue512 (Kernels/Nhwc.cs:376-398, Nhwc.Avx512.cs:129-152): + residual, activation.
inline void epilogue(const float* part, int rows, int lanes0, int lanes1, float* outp, const float* addp, long ostride,
                     int act) {
    for (int r = 0; r < rows; r++) {
        float* o = outp + r * ostride;
        const float* ad = addp ? addp + r * ostride : nullptr;
        for (int l = 0; l < lanes0 + lanes1; l++) {
            int src = l < lanes0 ? l : Ob + (l - lanes0);
            float v = part[r * 32 + src];
            if (ad) v = v + ad[l];
            o[l] = act8(v, act);
        }
    }
}

// Nhwc.Pack dense (Kernels/Nhwc.cs:102-125): [oc][ic][kh][kw] -> [nb][tap][ic][16], oc zero-padded.
// An extra zero block keeps block-pair tiles in bounds when nb is odd.
void pack_dense(const float* w, int oc, int ic, int taps, const float* bias, std::vector<float>& pw,
                std::vector<float>& pb, int& nb) {
    nb = (oc + Ob - 1) / Ob;
    pw.assign((size_t)(nb + 1) * taps * ic * Ob, 0.0f);
    pb.assign((size_t)(nb + 1) * Ob, 0.0f);
    for (int o = 0; o < oc; o++)
        for (int c = 0; c < ic; c++)
            for (int t = 0; t < taps; t++)
                pw[((size_t)((o / Ob) * taps + t) * ic + c) * Ob + o % Ob] = w[((size_t)o * ic + c) * taps + t];
    if (bias) memcpy(pb.data(), bias, sizeof(float) * oc);
}

// ---------------------------------------------------------------------------------------------
// Direct dense conv (Nhwc.Dense / Dense512, Kernels/Nhwc.cs:235-323, Nhwc.Avx512.cs:154-239).
// ---------------------------------------------------------------------------------------------
struct DenseCtx {
    const float* src;
    int ih, iw, ic, oh, ow, oc, kh, kw, nb;
    const int *rm, *cm;
    const float* padvec;
    const float *pw, *pb;
    int act, tier;
};

void dense_row(const DenseCtx& a, const float* src, int y, int blk, int nblk, float* orow, const float* arow) {
    int taps = a.kh * a.kw, R = tier_rows(a.tier), ic = a.ic;
    long wstep = (long)taps * ic * Ob;
    std::vector<const float*> ptrs((size_t)taps * R);
    float part[10 * 32];
    const float* wb = a.pw + blk * wstep;
    const float* bb = a.pb + blk * Ob;
    int lanes0 = std::min(Ob, a.oc - blk * Ob);
    int lanes1 = nblk == 2 ? std::max(0, std::min(Ob, a.oc - (blk + 1) * Ob)) : 0;
    for (int x0 = 0; x0 < a.ow; x0 += R) {
        int rows = std::min(R, a.ow - x0);
        for (int tap = 0; tap < taps; tap++) {
            int r = a.rm[y * a.kh + tap / a.kw];
            for (int i = 0; i < R; i++) {
                int c = a.cm[(x0 + std::min(i, rows - 1)) * a.kw + tap % a.kw];
                ptrs[(size_t)tap * R + i] = r < 0 || c < 0 ? a.padvec : src + ((long)r * a.iw + c) * ic;
            }
        }
        run_tile(a.tier, ptrs.data(), taps, ic, wb, wstep, nblk, bb, part);
        long o = (long)x0 * a.oc + blk * Ob;
        epilogue(part, rows, lanes0, lanes1, orow + o, arow ? arow + o : nullptr, a.oc, a.act);
    }
}

// ---------------------------------------------------------------------------------------------
// Winograd F(4x4, 3x3) (Kernels/NhwcWinograd.cs). U = G g G^T in double then cast; V = B^T d B;
// M = sum_c V U per transformed element through the conv micro-kernel (zero bias);
// Y = A^T M A; epilogue = Y + bias (+ residual), activation.
// ---------------------------------------------------------------------------------------------
const double kG[6][3] = {
    {1.0 / 4, 0, 0},
    {-1.0 / 6, -1.0 / 6, -1.0 / 6},
    {-1.0 / 6, 1.0 / 6, -1.0 / 6},
    {1.0 / 24, 1.0 / 12, 1.0 / 6},
    {1.0 / 24, -1.0 / 12, 1.0 / 6},
    {0, 0, 1},
};

// PackWinograd (NhwcWinograd.cs:46-68): [36][nb(+1)][ic][16].
std::vector<float> pack_winograd(const float* w, int oc, int ic, int nb) {
    std::vector<float> u((size_t)36 * (nb + 1) * ic * Ob, 0.0f);
    double gg[18];
    for (int o = 0; o < oc; o++)
        for (int c = 0; c < ic; c++) {
            const float* k = w + ((size_t)o * ic + c) * 9;
            for (int i = 0; i < 6; i++)
                for (int j = 0; j < 3; j++)
                    gg[i * 3 + j] = kG[i][0] * k[j] + kG[i][1] * k[3 + j] + kG[i][2] * k[6 + j];
            for (int i = 0; i < 6; i++)
                for (int j = 0; j < 6; j++) {
                    double v = gg[i * 3] * kG[j][0] + gg[i * 3 + 1] * kG[j][1] + gg[i * 3 + 2] * kG[j][2];
                    u[(((size_t)(i * 6 + j) * (nb + 1) + o / Ob) * ic + c) * Ob + o % Ob] = (float)v;
                }
        }
    return u;
}

// InputTransform (NhwcWinograd.cs:254-291): v[xi*vstride + c].
void input_transform(const float* const* d, int ic, float* v, long vstride) {
    float t[36];
    for (int c = 0; c < ic; c++) {
        for (int j = 0; j < 6; j++) {
            float d0 = d[j][c], d1 = d[6 + j][c], d2 = d[12 + j][c], d3 = d[18 + j][c], d4 = d[24 + j][c],
                  d5 = d[30 + j][c];
            t[j] = 4.0f * d0 - 5.0f * d2 + d4;
            t[6 + j] = d3 + d4 - 4.0f * (d1 + d2);
            t[12 + j] = d4 - d3 + 4.0f * (d1 - d2);
            t[18 + j] = d4 - d2 + 2.0f * (d3 - d1);
            t[24 + j] = d4 - d2 - 2.0f * (d3 - d1);
            t[30 + j] = 4.0f * d1 - 5.0f * d3 + d5;
        }
        for (int i = 0; i < 6; i++) {
            float r0 = t[i * 6], r1 = t[i * 6 + 1], r2 = t[i * 6 + 2], r3 = t[i * 6 + 3], r4 = t[i * 6 + 4],
                  r5 = t[i * 6 + 5];
            float* o = v + c + (long)(i * 6) * vstride;
            o[0] = 4.0f * r0 - 5.0f * r2 + r4;
            o[vstride] = r3 + r4 - 4.0f * (r1 + r2);
            o[2 * vstride] = r4 - r3 + 4.0f * (r1 - r2);
            o[3 * vstride] = r4 - r2 + 2.0f * (r3 - r1);
            o[4 * vstride] = r4 - r2 - 2.0f * (r3 - r1);
            o[5 * vstride] = 4.0f * r1 - 5.0f * r3 + r5;
        }
    }
}

// OutputTransform (NhwcWinograd.cs:295-329): tmp[(py*4+px)*16 + l].
void output_transform(const float* m, long mstride, float* tmp) {
    float s[24];
    for (int l = 0; l < Ob; l++) {
        for (int j = 0; j < 6; j++) {
            float m0 = m[j * mstride + l], m1 = m[(6 + j) * mstride + l], m2 = m[(12 + j) * mstride + l],
                  m3 = m[(18 + j) * mstride + l], m4 = m[(24 + j) * mstride + l], m5 = m[(30 + j) * mstride + l];
            float a = m1 + m2, b = m1 - m2, c = m3 + m4, e = m3 - m4;
            s[j] = m0 + a + c;
            s[6 + j] = b + 2.0f * e;
            s[12 + j] = a + 4.0f * c;
            s[18 + j] = b + 8.0f * e + m5;
        }
        for (int i = 0; i < 4; i++) {
            float r0 = s[i * 6], r1 = s[i * 6 + 1], r2 = s[i * 6 + 2], r3 = s[i * 6 + 3], r4 = s[i * 6 + 4],
                  r5 = s[i * 6 + 5];
            float a = r1 + r2, b = r1 - r2, c = r3 + r4, e = r3 - r4;
            float* o = tmp + i * 4 * Ob + l;
            o[0] = r0 + a + c;
            o[Ob] = b + 2.0f * e;
            o[2 * Ob] = a + 4.0f * c;
            o[3 * Ob] = b + 8.0f * e + r5;
        }
    }
}

int winograd_conv(const float* src, int ih, int iw, int ic, const float* w, const float* bias, const float* add,
                  float* dst, int oh, int ow, int oc, const ora_conv_p* p, int tier) {
    int nb = (oc + Ob - 1) / Ob;
    std::vector<float> U = pack_winograd(w, oc, ic, nb);
    std::vector<float> pb((size_t)(nb + 1) * Ob, 0.0f);
    if (bias) memcpy(pb.data(), bias, sizeof(float) * oc);
    std::vector<float> padvec(ic, p->pad_value);
    int tw = (ow + 3) / 4, th = (oh + 3) / 4, nt = tw * th;
    int R = tier_rows(tier);
    const int T = R * 6;  // tiles per chunk (a multiple of the tile height)
    int chunks = (nt + T - 1) / T;
    bool refl = p->pad_mode == 1;
    int pad_t = p->pad_t, pad_l = p->pad_l;
#pragma omp parallel for schedule(dynamic) num_threads(threads())
    for (int chunk = 0; chunk < chunks; chunk++) {
        int t0 = chunk * T, tn = std::min(T, nt - t0);
        std::vector<float> V((size_t)36 * T * ic), M((size_t)36 * T * 32), zero(32, 0.0f);
        const float* d6[36];
        for (int t = 0; t < tn; t++) {
            int ty = (t0 + t) / tw, tx = (t0 + t) % tw;
            int iy0 = ty * 4 - pad_t, ix0 = tx * 4 - pad_l;
            for (int i = 0; i < 6; i++) {
                int yy = iy0 + i;
                int r = (unsigned)yy < (unsigned)ih ? yy : refl ? reflect_idx(yy, ih) : -1;
                for (int j = 0; j < 6; j++) {
                    int xx = ix0 + j;
                    int c = (unsigned)xx < (unsigned)iw ? xx : refl ? reflect_idx(xx, iw) : -1;
                    d6[i * 6 + j] = r < 0 || c < 0 ? padvec.data() : src + ((long)r * iw + c) * ic;
                }
            }
            input_transform(d6, ic, V.data() + (long)t * ic, (long)T * ic);
        }
        std::vector<const float*> ptrs(R);
        float part[10 * 32], tmp[16 * Ob];
        int step = tier_blocks(tier);
        for (int blk0 = 0; blk0 < nb; blk0 += step) {
            int nblk = std::min(step, nb - blk0);
            if (tier == ORA_TIER_AVX512) nblk = blk0 + 1 < nb ? 2 : 1;
            for (int xi = 0; xi < 36; xi++) {
                const float* wb = U.data() + ((size_t)xi * (nb + 1) + blk0) * ic * Ob;
                const float* vx = V.data() + (size_t)xi * T * ic;
                float* mx = M.data() + (size_t)xi * T * 32;
                for (int r0 = 0; r0 < tn; r0 += R) {
                    int rows = std::min(R, tn - r0);
                    for (int i = 0; i < R; i++) ptrs[i] = vx + (long)(r0 + std::min(i, rows - 1)) * ic;
                    run_tile(tier, ptrs.data(), 1, ic, wb, (long)ic * Ob, nblk, zero.data(), part);
                    for (int r = 0; r < rows; r++) memcpy(mx + (size_t)(r0 + r) * 32, part + r * 32, 32 * 4);
                }
            }
            for (int h = 0; h < nblk; h++) {
                int blk = blk0 + h, lanes = std::min(Ob, oc - blk * Ob);
                const float* bb = pb.data() + blk * Ob;
                for (int t = 0; t < tn; t++) {
                    int ty = (t0 + t) / tw, tx = (t0 + t) % tw;
                    output_transform(M.data() + (size_t)t * 32 + h * Ob, (long)T * 32, tmp);
                    for (int py = 0; py < 4; py++) {
                        int oy = ty * 4 + py;
                        if (oy >= oh) break;
                        for (int px = 0; px < 4; px++) {
                            int ox = tx * 4 + px;
                            if (ox >= ow) break;
                            long o = ((long)oy * ow + ox) * oc + blk * Ob;
                            const float* tp = tmp + (py * 4 + px) * Ob;
                            for (int l = 0; l < lanes; l++) {
                                float v = tp[l] + bb[l];
                                if (add) v = v + add[o + l];
                                dst[o + l] = act8(v, p->act);
                            }
                        }
                    }
                }
            }
        }
    }
    return 0;
}

// Depthwise (Nhwc.Depthwise / DwRow, Kernels/Nhwc.cs:496-631): acc = bias[c] + sum over taps
// (row-major) x*w, one FMA each; constant-0 padded rows are skipped (ClipRows).
int depthwise(const float* src, int ih, int iw, int c, const float* w, const float* bias, const float* add,
              float* dst, int oh, int ow, const ora_conv_p* p) {
    int kh = p->kh, kw = p->kw, taps = kh * kw;
    std::vector<int> rm = make_map(oh, kh, p->sh, p->pad_t, ih, p->pad_mode);
    std::vector<int> cm = make_map(ow, kw, p->sw, p->pad_l, iw, p->pad_mode);
    std::vector<float> pw((size_t)taps * c);
    for (int ch = 0; ch < c; ch++)
        for (int t = 0; t < taps; t++) pw[(size_t)t * c + ch] = w[(size_t)ch * taps + t];
    bool clip = p->pad_value == 0.0f;
#pragma omp parallel for schedule(static) num_threads(threads())
    for (int y = 0; y < oh; y++) {
        int kyB = 0, kyE = kh;
        if (clip) {
            while (kyB < kyE && rm[y * kh + kyB] < 0) kyB++;
            while (kyE > kyB && rm[y * kh + kyE - 1] < 0) kyE--;
        }
        for (int x = 0; x < ow; x++) {
            float* o = dst + ((long)y * ow + x) * c;
            const float* ad = add ? add + ((long)y * ow + x) * c : nullptr;
            for (int ch = 0; ch < c; ch++) {
                float acc = bias ? bias[ch] : 0.0f;
                for (int ky = kyB; ky < kyE; ky++) {
                    int r = rm[y * kh + ky];
                    for (int kx = 0; kx < kw; kx++) {
                        int cc = cm[x * kw + kx];
                        float xv = r < 0 || cc < 0 ? p->pad_value : src[((long)r * iw + cc) * c + ch];
                        acc = fmaf(xv, pw[(size_t)(ky * kw + kx) * c + ch], acc);
                    }
                }
                if (ad) acc = acc + ad[ch];
                o[ch] = act8(acc, p->act);
            }
        }
    }
    return 0;
}

}  // namespace

extern "C" {

int ora_tier_available(int tier) { return resolve_tier(tier) > 0 ? 1 : 0; }
void ora_set_threads(int t) { g_threads = t; }
int ora_get_threads(void) { return threads(); }

float ora_exp_core(float x) { return exp_core(x); }
float ora_erf_core(float x) { return erf_core(x); }
float ora_gelu_core(float x) { return gelu_core(x); }
float ora_sigmoid_core(float x) { return sigmoid_core(x); }
float ora_act(float x, int act) { return act8(x, act); }

int ora_winograd_eligible(const ora_conv_p* p, int ic) {
    // WinogradEligible (NhwcWinograd.cs:28-32) with Vector<float>.Count = 8 (AVX2 / AVX-512 hosts)
    return p->group == 1 && p->kh == 3 && p->kw == 3 && p->sh == 1 && p->sw == 1 && ic >= 16 && ic % 8 == 0 &&
           !p->pool;
}

int ora_conv(const float* src, int n, int ih, int iw, int ic, const float* w, const float* bias, const float* add,
             float* dst, int oh, int ow, int oc, const ora_conv_p* p, int algo, int tier) {
    tier = resolve_tier(tier);
    if (tier < 0) return -1;
    long in_img = (long)ih * iw * ic;
    if (p->group > 1) {
        if (p->group != ic || oc != ic || p->pool) return -2;  // NHWC grouped conv: depthwise only (Nhwc.cs:105-108)
        long out_img = (long)oh * ow * oc;
        for (int b = 0; b < n; b++)
            depthwise(src + b * in_img, ih, iw, ic, w, bias, add ? add + b * out_img : nullptr, dst + b * out_img, oh,
                      ow, p);
        return 0;
    }
    if (p->pool && add) return -3;  // ConvPool has no residual (Nhwc.cs:669-671)
    // conv geometry: with a fused pool, (oh, ow) is the pooled size and the conv output is twice that
    int coh = p->pool ? oh * 2 : oh, cow = p->pool ? ow * 2 : ow;
    long out_img = (long)oh * ow * oc, conv_img = (long)coh * cow * oc;
    if (!p->pool && algo == 0 && ora_winograd_eligible(p, ic)) {
        for (int b = 0; b < n; b++)
            winograd_conv(src + b * in_img, ih, iw, ic, w, bias, add ? add + b * out_img : nullptr, dst + b * out_img,
                          oh, ow, oc, p, tier);
        return 0;
    }
    int taps = p->kh * p->kw, nb;
    std::vector<float> pw, pb;
    pack_dense(w, oc, ic, taps, bias, pw, pb, nb);
    std::vector<int> rm = make_map(coh, p->kh, p->sh, p->pad_t, ih, p->pad_mode);
    std::vector<int> cm = make_map(cow, p->kw, p->sw, p->pad_l, iw, p->pad_mode);
    std::vector<float> padvec((size_t)ic + Ob, p->pad_value);
    DenseCtx a{src, ih, iw, ic, coh, cow, oc, p->kh, p->kw, nb, rm.data(), cm.data(), padvec.data(), pw.data(),
               pb.data(), p->act, tier};
    int step = tier_blocks(tier), npair = (nb + step - 1) / step;
    std::vector<float> full;
    if (p->pool) full.resize((size_t)conv_img * n);
    float* cdst = p->pool ? full.data() : dst;
    long tasks = (long)n * coh * npair;
#pragma omp parallel for schedule(static) num_threads(threads())
    for (long t = 0; t < tasks; t++) {
        int b = (int)(t / ((long)coh * npair));
        long rr = t % ((long)coh * npair);
        int y = (int)(rr / npair), blk = (int)(rr % npair) * step;
        int nblk = std::min(step, nb - blk);
        long o = b * conv_img + (long)y * cow * oc;
        dense_row(a, src + b * in_img, y, blk, nblk, cdst + o, add ? add + o : nullptr);
    }
    if (p->pool) {
        // PoolBand (Nhwc.cs:708-727): 2x2/2 max over conv row pairs, then the pool's relu
        for (int b = 0; b < n; b++)
            for (int y = 0; y < oh; y++)
                for (int x = 0; x < ow; x++)
                    for (int ch = 0; ch < oc; ch++) {
                        const float* base = full.data() + b * conv_img;
                        float s0 = base[((long)(2 * y) * cow + 2 * x) * oc + ch];
                        float s1 = base[((long)(2 * y) * cow + 2 * x + 1) * oc + ch];
                        float s2 = base[((long)(2 * y + 1) * cow + 2 * x) * oc + ch];
                        float s3 = base[((long)(2 * y + 1) * cow + 2 * x + 1) * oc + ch];
                        float v = fmaxf(fmaxf(fmaxf(s0, s1), s2), s3);
                        if (p->pool_relu) v = fmaxf(v, 0.0f);
                        dst[b * out_img + ((long)y * ow + x) * oc + ch] = v;
                    }
    }
    return 0;
}

int ora_gemm(const float* a, int m, int k, const float* b, int n, int trans_b, const float* bias, int act, float* dst,
             int tier) {
    tier = resolve_tier(tier);
    if (tier < 0) return -1;
    // PackGemm (Nhwc.cs:128-138): B -> [nb][k][16]
    int nb = (n + Ob - 1) / Ob;
    std::vector<float> pw((size_t)(nb + 1) * k * Ob, 0.0f), pb((size_t)(nb + 1) * Ob, 0.0f);
    for (int o = 0; o < n; o++)
        for (int c = 0; c < k; c++)
            pw[((size_t)(o / Ob) * k + c) * Ob + o % Ob] = trans_b ? b[(size_t)o * k + c] : b[(size_t)c * n + o];
    if (bias) memcpy(pb.data(), bias, sizeof(float) * n);
    int R = tier_rows(tier), step = tier_blocks(tier), npair = (nb + step - 1) / step;
    int tiles = (m + R - 1) / R;
    const int G = 8;  // row tiles per task sharing one weight panel walk (Nhwc.cs:146)
    int groups = (tiles + G - 1) / G;
    long wstep = (long)k * Ob;
#pragma omp parallel for schedule(static) num_threads(threads())
    for (long t = 0; t < (long)groups * npair; t++) {
        int g = (int)(t / npair), blk = (int)(t % npair) * step, nblk = std::min(step, nb - blk);
        const float* ptrs[10];
        float part[10 * 32];
        int lanes0 = std::min(Ob, n - blk * Ob), lanes1 = nblk == 2 ? std::min(Ob, n - (blk + 1) * Ob) : 0;
        for (int tile = g * G, te = std::min(tiles, tile + G); tile < te; tile++) {
            int m0 = tile * R, rows = std::min(R, m - m0);
            for (int i = 0; i < R; i++) ptrs[i] = a + (long)(m0 + std::min(i, rows - 1)) * k;
            run_tile(tier, ptrs, 1, k, pw.data() + blk * wstep, wstep, nblk, pb.data() + blk * Ob, part);
            epilogue(part, rows, lanes0, lanes1, dst + (long)m0 * n + blk * Ob, nullptr, n, act);
        }
    }
    return 0;
}

int ora_matmul(const float* a, const float* b, int batch, int m, int k, int n, float* c) {
    // Avx2Kernels.GemmKN per batch (Avx2Kernels.cs:503-556): acc = 0, k ascending, one FMA each
#pragma omp parallel for schedule(static) num_threads(threads())
    for (long t = 0; t < (long)batch * m; t++) {
        long bi = t / m, i = t % m;
        const float* ar = a + (bi * m + i) * k;
        const float* bb = b + bi * (long)k * n;
        float* cr = c + (bi * m + i) * n;
        for (int j = 0; j < n; j++) {
            float s = 0.0f;
            for (int kk = 0; kk < k; kk++) s = fmaf(ar[kk], bb[(long)kk * n + j], s);
            cr[j] = s;
        }
    }
    return 0;
}

int ora_conv_transpose(const float* src, int n, int ih, int iw, int ic, const float* w, int oc, int kh, int kw,
                       const float* bias, int act, float* dst) {
    int taps = kh * kw, ow = iw * kw, ohh = ih * kh;
    long in_img = (long)ih * iw * ic, out_img = (long)ohh * ow * oc;
    for (int b = 0; b < n; b++) {
        const float* sp = src + b * in_img;
        float* dp = dst + b * out_img;
        if (oc <= 4) {
            // ConvTDot (Nhwc.Det.cs:96-131): s = b + Sum(4-lane partial products) + tail, then act
#pragma omp parallel for schedule(static) num_threads(threads())
            for (int y = 0; y < ih; y++)
                for (int x = 0; x < iw; x++) {
                    const float* xp = sp + ((long)y * iw + x) * ic;
                    for (int t = 0; t < taps; t++) {
                        float* o = dp + ((long)(y * kh + t / kw) * ow + x * kw + t % kw) * oc;
                        for (int kk = 0; kk < oc; kk++) {
                            float lane[4] = {0, 0, 0, 0};
                            int c = 0;
                            for (; c + 4 <= ic; c += 4)
                                for (int l = 0; l < 4; l++)
                                    lane[l] = lane[l] + xp[c + l] * w[((long)(c + l) * oc + kk) * taps + t];
                            float s = bias ? bias[kk] : 0.0f;
                            s = s + ((lane[0] + lane[1]) + (lane[2] + lane[3]));
                            for (; c < ic; c++) s = s + xp[c] * w[((long)c * oc + kk) * taps + t];
                            o[kk] = act8(s, act);
                        }
                    }
                }
        } else {
            // per-tap Gemm panel through the conv micro-kernel: acc = bias, c ascending FMA, Store16
#pragma omp parallel for schedule(static) num_threads(threads())
            for (int y = 0; y < ih; y++)
                for (int x = 0; x < iw; x++) {
                    const float* xp = sp + ((long)y * iw + x) * ic;
                    for (int t = 0; t < taps; t++) {
                        float* o = dp + ((long)(y * kh + t / kw) * ow + x * kw + t % kw) * oc;
                        for (int kk = 0; kk < oc; kk++) {
                            float s = bias ? bias[kk] : 0.0f;
                            for (int c = 0; c < ic; c++) s = fmaf(xp[c], w[((long)c * oc + kk) * taps + t], s);
                            o[kk] = act8(s, act);
                        }
                    }
                }
        }
    }
    return 0;
}

int ora_global_avg_pool(const float* src, int hw, int c, float* dst) {
    // chunked partial sums reduced in chunk order (Nhwc.Det.cs:134-164)
    long chunks = std::max(1L, std::min((long)hw * c / 65536, (long)threads()));
    std::vector<float> part((size_t)chunks * c, 0.0f);
    for (long kk = 0; kk < chunks; kk++) {
        long p0 = kk * hw / chunks, p1 = (kk + 1) * hw / chunks;
        float* acc = part.data() + kk * c;
        for (long px = p0; px < p1; px++)
            for (int ch = 0; ch < c; ch++) acc[ch] = acc[ch] + src[px * c + ch];
    }
    float inv = 1.0f / hw;
    for (int ch = 0; ch < c; ch++) {
        float s = 0;
        for (long kk = 0; kk < chunks; kk++) s = s + part[kk * c + ch];
        dst[ch] = s * inv;
    }
    return 0;
}

int ora_channel_gate(const float* src, int hw, int c, const float* w1, const float* b1, const float* w2,
                     const float* b2, int r, int act1_relu, int hard, float alpha, float beta, float offset,
                     float* dst) {
    std::vector<float> mean(c), hid(r);
    ora_global_avg_pool(src, hw, c, mean.data());
    for (int j = 0; j < r; j++) {
        float s = b1 ? b1[j] : 0.0f;
        for (int kk = 0; kk < c; kk++) s = s + w1[(long)j * c + kk] * mean[kk];
        hid[j] = act1_relu ? fmaxf(s, 0.0f) : s;
    }
    for (int ch = 0; ch < c; ch++) {
        float z = b2 ? b2[ch] : 0.0f;
        for (int j = 0; j < r; j++) z = z + w2[(long)ch * r + j] * hid[j];
        float g = hard ? std::min(std::max(z * alpha + beta, 0.0f), 1.0f) : 1.0f / (1.0f + expf(-z));
        dst[ch] = g + offset;
    }
    return 0;
}

int ora_channel_broadcast(const float* full, const float* vec, float* dst, long rows, int c, int op, int rev,
                          int act) {
#pragma omp parallel for schedule(static) num_threads(threads())
    for (long r = 0; r < rows; r++)
        for (int ch = 0; ch < c; ch++) {
            float a = full[r * c + ch], b = vec[ch];
            if (rev) std::swap(a, b);
            float s = op == 0 ? a + b : op == 1 ? a - b : op == 2 ? a * b : a / b;
            dst[r * c + ch] = act == 1 ? fmaxf(s, 0.0f) : s;
        }
    return 0;
}

int ora_ew2(const float* a, const float* b, float* dst, long count, int op, int act) {
#pragma omp parallel for schedule(static) num_threads(threads())
    for (long i = 0; i < count; i++) {
        float s = op == 0 ? a[i] + b[i] : op == 1 ? a[i] - b[i] : op == 2 ? a[i] * b[i] : a[i] / b[i];
        dst[i] = act == 1 ? fmaxf(s, 0.0f) : s;
    }
    return 0;
}

int ora_resize_nearest(const float* src, int ih, int iw, int c, float* dst, int oh, int ow, float sy, float sx,
                       const float* add, int add_relu) {
    std::vector<int> xs(ow);
    for (int x = 0; x < ow; x++) xs[x] = std::min((int)floorf(x / sx), iw - 1);
#pragma omp parallel for schedule(static) num_threads(threads())
    for (int y = 0; y < oh; y++) {
        int ys = std::min((int)floorf(y / sy), ih - 1);
        for (int x = 0; x < ow; x++) {
            const float* s = src + ((long)ys * iw + xs[x]) * c;
            float* o = dst + ((long)y * ow + x) * c;
            const float* a = add ? add + ((long)y * ow + x) * c : nullptr;
            for (int ch = 0; ch < c; ch++) o[ch] = a ? s[ch] + (add_relu ? fmaxf(a[ch], 0.0f) : a[ch]) : s[ch];
        }
    }
    return 0;
}

int ora_concat_inner(const float* const* ins, const int* counts, int nin, long outer, float* dst) {
    long total = 0;
    for (int i = 0; i < nin; i++) total += counts[i];
    for (long o = 0; o < outer; o++) {
        float* d = dst + o * total;
        for (int i = 0; i < nin; i++) {
            memcpy(d, ins[i] + o * counts[i], sizeof(float) * counts[i]);
            d += counts[i];
        }
    }
    return 0;
}

int ora_hard_sigmoid(const float* src, long count, float alpha, float beta, float* dst) {
    for (long i = 0; i < count; i++) dst[i] = std::min(std::max(src[i] * alpha + beta, 0.0f), 1.0f);
    return 0;
}

int ora_activation(const float* src, long count, int act, float* dst) {
#pragma omp parallel for schedule(static) num_threads(threads())
    for (long i = 0; i < count; i++) dst[i] = act8(src[i], act);
    return 0;
}

int ora_layer_norm(const float* src, long rows, int len, const float* gamma, const float* beta, float eps,
                   float* dst) {
    // Avx2Kernels.LayerNorm (Avx2Kernels.cs:562-600): 8 lane partial sums, sum-of-squares by FMA
#pragma omp parallel for schedule(static) num_threads(threads())
    for (long r = 0; r < rows; r++) {
        const float* xr = src + r * len;
        float* dr = dst + r * len;
        float sum[8] = {0}, sq[8] = {0};
        int i = 0;
        for (; i + 8 <= len; i += 8)
            for (int l = 0; l < 8; l++) {
                float v = xr[i + l];
                sum[l] = sum[l] + v;
                sq[l] = fmaf(v, v, sq[l]);
            }
        float s = 0, ss = 0;
        for (int l = 0; l < 8; l++) { s = s + sum[l]; ss = ss + sq[l]; }
        for (; i < len; i++) { float v = xr[i]; s = s + v; ss = ss + v * v; }
        float mean = s / len;
        float inv = 1.0f / sqrtf(fmaxf(ss / len - mean * mean, 0.0f) + eps);
        for (i = 0; i + 8 <= len; i += 8)
            for (int l = 0; l < 8; l++) dr[i + l] = fmaf(xr[i + l] - mean, inv * gamma[i + l], beta[i + l]);
        for (; i < len; i++) dr[i] = (xr[i] - mean) * inv * gamma[i] + beta[i];
    }
    return 0;
}

static void softmax_row(const float* s, float* d, int c) {
    // SoftmaxRow (Ops.Seq.cs:39-72): 4-lane max and sum, ExpCore on the vector part, expf on the tail
    float mx = -INFINITY;
    int i = 0;
    if (c >= 4) {
        float vm[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
        for (; i + 4 <= c; i += 4)
            for (int l = 0; l < 4; l++) vm[l] = fmaxf(vm[l], s[i + l]);
        mx = fmaxf(fmaxf(vm[0], vm[1]), fmaxf(vm[2], vm[3]));
    }
    for (; i < c; i++) mx = fmaxf(mx, s[i]);
    float acc[4] = {0, 0, 0, 0};
    i = 0;
    for (; i + 4 <= c; i += 4)
        for (int l = 0; l < 4; l++) {
            float e = exp_core(s[i + l] - mx);
            d[i + l] = e;
            acc[l] = acc[l] + e;
        }
    float sum = (acc[0] + acc[1]) + (acc[2] + acc[3]);
    for (; i < c; i++) { float e = expf(s[i] - mx); d[i] = e; sum = sum + e; }
    float inv = 1.0f / sum;
    for (i = 0; i < c; i++) d[i] = d[i] * inv;
}

int ora_softmax(const float* src, long rows, int len, float* dst) {
#pragma omp parallel for schedule(static) num_threads(threads())
    for (long r = 0; r < rows; r++) softmax_row(src + r * len, dst + r * len, len);
    return 0;
}

int ora_attention(const float* q, const float* k, const float* v, int bh, int t, int s, int d, float scale,
                  float* out) {
#pragma omp parallel for schedule(static) num_threads(threads())
    for (long idx = 0; idx < (long)bh * t; idx++) {
        long b = idx / t, i = idx % t;
        const float* qr = q + (b * t + i) * d;
        std::vector<float> sc(s), p(s);
        for (int j = 0; j < s; j++) {
            const float* kr = k + (b * s + j) * d;
            float acc = 0.0f;
            for (int e = 0; e < d; e++) acc = fmaf(qr[e], kr[e], acc);
            sc[j] = acc * scale;
        }
        softmax_row(sc.data(), p.data(), s);
        float* o = out + (b * t + i) * d;
        for (int e = 0; e < d; e++) {
            float acc = 0.0f;
            for (int j = 0; j < s; j++) acc = fmaf(p[j], v[(b * s + j) * d + e], acc);
            o[e] = acc;
        }
    }
    return 0;
}

// IEEE binary32 -> binary16 (round to nearest, ties to even) -> binary32, in integer arithmetic.
static float round_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = x & 0x80000000u, ax = x & 0x7fffffffu;
    uint32_t out;
    if (ax >= 0x7f800000u) {
        out = ax > 0x7f800000u ? 0x7fc00000u : 0x7f800000u;  // NaN stays NaN, inf stays inf
    } else if (ax >= 0x477ff000u) {
        out = 0x7f800000u;  // at or above 65520: rounds to inf
    } else if (ax < 0x38800000u) {
        // subnormal half range: quantum 2^-24
        float q = 5.9604644775390625e-08f;  // 2^-24
        float a;
        memcpy(&a, &ax, 4);
        float r = nearbyintf(a / q) * q;  // a/q is exact (power of two scale); nearbyint ties to even
        memcpy(&out, &r, 4);
    } else {
        // normal: keep 10 mantissa bits
        uint32_t lsb = (ax >> 13) & 1u;
        uint32_t r = ax + 0xfffu + lsb;
        out = r & ~0x1fffu;
    }
    out |= sign;
    float res;
    memcpy(&res, &out, 4);
    return res;
}

void ora_round_f16(const float* src, float* dst, long count) {
    for (long i = 0; i < count; i++) dst[i] = round_f16(src[i]);
}


// ---------------------------------------------------------------------------------------------
// The rest of the GPU op surface (the ExecOp cases of Backends/Vulkan/VkGraph.cs:795-1068) as the
// CPU engine computes them (Engine/Session.cs:178-270, 345-410).
// ---------------------------------------------------------------------------------------------

// Nhwc.ResizeAxis (Kernels/Nhwc.cs:773-783): half-pixel source coordinate, both taps clamped.
static void resize_axis(int out_len, int in_len, float scale, int* i0, int* i1, float* wt) {
    for (int o = 0; o < out_len; o++) {
        float f = (o + 0.5f) / scale - 0.5f;
        float fl = floorf(f);
        i0[o] = std::min(std::max((int)fl, 0), in_len - 1);
        i1[o] = std::min(std::max((int)fl + 1, 0), in_len - 1);
        wt[o] = f - fl;
    }
}

int ora_resize_bilinear(const float* src, int ih, int iw, int c, float* dst, int oh, int ow, float sy, float sx,
                        int relu, const float* add, int add_relu) {
    std::vector<int> y0(oh), y1(oh), x0(ow), x1(ow);
    std::vector<float> wy(oh), wx(ow);
    resize_axis(oh, ih, sy, y0.data(), y1.data(), wy.data());
    resize_axis(ow, iw, sx, x0.data(), x1.data(), wx.data());
#pragma omp parallel for schedule(static) num_threads(threads())
    for (int y = 0; y < oh; y++) {
        const float* r0 = src + (long)y0[y] * iw * c;
        const float* r1 = src + (long)y1[y] * iw * c;
        for (int x = 0; x < ow; x++) {
            const float *a = r0 + (long)x0[x] * c, *b = r0 + (long)x1[x] * c;
            const float *e = r1 + (long)x0[x] * c, *f = r1 + (long)x1[x] * c;
            long ob = ((long)y * ow + x) * c;
            for (int ch = 0; ch < c; ch++) {  // Nhwc.ResizePixel (Kernels/Nhwc.cs:788-814)
                float top = a[ch] + (b[ch] - a[ch]) * wx[x];
                float bot = e[ch] + (f[ch] - e[ch]) * wx[x];
                float v = top + (bot - top) * wy[y];
                if (relu) v = fmaxf(v, 0.0f);
                if (add) v += add_relu ? fmaxf(add[ob + ch], 0.0f) : add[ob + ch];
                dst[ob + ch] = v;
            }
        }
    }
    return 0;
}

// Nhwc.Pad (Kernels/Nhwc.cs:877-900): spatial pad of one NHWC image; mode 0 constant, 1 reflect.
int ora_pad_nhwc(const float* src, int ih, int iw, int c, float* dst, int oh, int ow, int pad_t, int pad_l,
                 int mode, float value) {
    std::vector<int> rm = make_map(oh, 1, 1, pad_t, ih, mode), cm = make_map(ow, 1, 1, pad_l, iw, mode);
    for (int y = 0; y < oh; y++)
        for (int x = 0; x < ow; x++) {
            float* o = dst + ((long)y * ow + x) * c;
            if (rm[y] < 0 || cm[x] < 0)
                for (int ch = 0; ch < c; ch++) o[ch] = value;
            else
                memcpy(o, src + ((long)rm[y] * iw + cm[x]) * c, sizeof(float) * c);
        }
    return 0;
}

// Nhwc.MaxPool (Kernels/Nhwc.cs:729-769): out-of-image taps are skipped (constant pad map), the
// first in-image tap is copied and the rest folded in with max in (ky, kx) order; a window with no
// in-image tap is 0; the fused relu (PoolP.FuseRelu) is applied last.
int ora_max_pool_nhwc(const float* src, int ih, int iw, int c, float* dst, int oh, int ow, int kh, int kw, int sh,
                      int sw, int pad_t, int pad_l, int relu) {
    std::vector<int> rm = make_map(oh, kh, sh, pad_t, ih, 0), cm = make_map(ow, kw, sw, pad_l, iw, 0);
#pragma omp parallel for schedule(static) num_threads(threads())
    for (int y = 0; y < oh; y++)
        for (int x = 0; x < ow; x++) {
            float* o = dst + ((long)y * ow + x) * c;
            bool any = false;
            for (int ky = 0; ky < kh; ky++) {
                int r = rm[(long)y * kh + ky];
                if (r < 0) continue;
                for (int kx = 0; kx < kw; kx++) {
                    int cc = cm[(long)x * kw + kx];
                    if (cc < 0) continue;
                    const float* s = src + ((long)r * iw + cc) * c;
                    if (!any) {
                        memcpy(o, s, sizeof(float) * c);
                        any = true;
                        continue;
                    }
                    for (int ch = 0; ch < c; ch++) o[ch] = fmaxf(o[ch], s[ch]);
                }
            }
            if (!any)
                for (int ch = 0; ch < c; ch++) o[ch] = 0.0f;
            else if (relu)
                for (int ch = 0; ch < c; ch++) o[ch] = fmaxf(o[ch], 0.0f);
        }
    return 0;
}

// Nhwc.AvgPool (Kernels/Ops.Seq.cs:180-215): taps summed in (ky, kx) order, then one multiply by
// 1 / count (kh*kw with count_include_pad, else the in-bounds taps).
int ora_avg_pool_nhwc(const float* src, int ih, int iw, int c, float* dst, int oh, int ow, int kh, int kw, int sh,
                      int sw, int pad_t, int pad_l, int count_include_pad) {
    std::vector<int> rm = make_map(oh, kh, sh, pad_t, ih, 0), cm = make_map(ow, kw, sw, pad_l, iw, 0);
#pragma omp parallel for schedule(static) num_threads(threads())
    for (int y = 0; y < oh; y++)
        for (int x = 0; x < ow; x++) {
            float* o = dst + ((long)y * ow + x) * c;
            for (int ch = 0; ch < c; ch++) o[ch] = 0.0f;
            int cnt = 0;
            for (int ky = 0; ky < kh; ky++) {
                int r = rm[(long)y * kh + ky];
                if (r < 0) continue;
                for (int kx = 0; kx < kw; kx++) {
                    int cc = cm[(long)x * kw + kx];
                    if (cc < 0) continue;
                    const float* s = src + ((long)r * iw + cc) * c;
                    for (int ch = 0; ch < c; ch++) o[ch] += s[ch];
                    cnt++;
                }
            }
            float inv = 1.0f / (count_include_pad ? kh * kw : std::max(cnt, 1));
            for (int ch = 0; ch < c; ch++) o[ch] *= inv;
        }
    return 0;
}

// Nhwc.DepthToSpace / SpaceToDepth, NHWC (Kernels/Nhwc.Det.cs:210-282). dir 0: depth-to-space
// (src [ih][iw][ic] -> [ih*b][iw*b][ic/b^2]), 1: space-to-depth ([ih][iw][ic] -> [ih/b][iw/b][ic*b^2]).
int ora_depth_space(const float* src, int ih, int iw, int ic, float* dst, int b, int crd, int dir) {
    const int bb = b * b;
    if (dir == 0) {
        const int oc = ic / bb, oh = ih * b, ow = iw * b;
        for (int y = 0; y < oh; y++)
            for (int x = 0; x < ow; x++) {
                const float* s = src + ((long)(y / b) * iw + x / b) * ic;
                float* o = dst + ((long)y * ow + x) * oc;
                const int sub = (y % b) * b + x % b;
                for (int ch = 0; ch < oc; ch++) o[ch] = crd ? s[ch * bb + sub] : s[(long)sub * oc + ch];
            }
    } else {
        const int oc = ic * bb, oh = ih / b, ow = iw / b;
        for (int y = 0; y < oh; y++)
            for (int x = 0; x < ow; x++) {
                float* o = dst + ((long)y * ow + x) * oc;
                for (int sub = 0; sub < bb; sub++) {
                    const float* s = src + ((long)(y * b + sub / b) * iw + x * b + sub % b) * ic;
                    for (int ch = 0; ch < ic; ch++) {
                        if (crd) o[ch * bb + sub] = s[ch];
                        else o[(long)sub * ic + ch] = s[ch];
                    }
                }
            }
    }
    return 0;
}

// Act.ApplyLeakyRelu / ApplyTanh / ApplyClip / ApplyErf (Kernels/Act.cs:83-147), the vector forms:
// mode 0 leaky (max(x, a x) for a <= 1, else min), 1 tanh = 2o sigmoid(2i x) - o with the Cephes
// sigmoid core (a = i, b = o), 2 clip min(max(x, a), b), 3 erf (A&S 7.1.26 core).
int ora_unary2(const float* src, long count, int mode, float a, float b, float* dst) {
#pragma omp parallel for schedule(static) num_threads(threads())
    for (long i = 0; i < count; i++) {
        const float x = src[i];
        float y;
        switch (mode) {
            case 0: y = a <= 1.0f ? fmaxf(x, x * a) : fminf(x, x * a); break;
            case 1: y = sigmoid_core(x * (2.0f * a)) * (2.0f * b) - b; break;
            case 2: y = fminf(fmaxf(x, a), b); break;
            default: y = erf_core(x); break;
        }
        dst[i] = y;
    }
    return 0;
}

// CtcProjection.ArgMax, the scalar kernel (Decoding/Kernels/MatMul.ArgMax.cs:130-299, Row1): per row,
// logit = bias + sum_k x w (k ascending, one multiply and add each), UpdateArgMax (:267-278): a
// larger logit rescales the running sum by exp(max - logit) and adds 1, else adds exp(logit - max);
// ties keep the first column; probability = min(1, 1 / sum) (:287-292). Returns -1 on a non-finite
// logit or sum (the reference throws "Recognizer output is invalid.").
int ora_ctc_argmax(const float* x, const float* w, const float* bias, long rows, int inner, int columns, int* indices,
                   float* probs) {
    int bad = 0;
#pragma omp parallel for schedule(static) num_threads(threads()) reduction(| : bad)
    for (long r = 0; r < rows; r++) {
        const float* xr = x + r * inner;
        float mx = -INFINITY, sum = 0.0f;
        int best = 0;
        for (int col = 0; col < columns; col++) {
            float v = bias ? bias[col] : 0.0f;
            for (int k = 0; k < inner; k++) v += xr[k] * w[(long)k * columns + col];
            if (!std::isfinite(v)) {
                bad = 1;
                break;
            }
            if (v > mx) {
                sum = sum * expf(mx - v) + 1.0f;
                mx = v;
                best = col;
            } else {
                sum += expf(v - mx);
            }
        }
        if (!(sum > 0.0f) || std::isinf(sum)) bad = 1;
        indices[r] = best;
        probs[r] = std::min(1.0f, 1.0f / sum);
    }
    return bad ? -1 : 0;
}

// SafeDiv (Kernels/FusedKernels.cs:35-57): clamp(a / max(b, eps), lo, hi).
int ora_safediv(const float* a, const float* b, float* dst, long count, float eps, float lo, float hi) {
    for (long i = 0; i < count; i++) dst[i] = std::min(std::max(a[i] / std::max(b[i], eps), lo), hi);
    return 0;
}

// ChannelShift, NHWC, one image (Kernels/FusedKernels.cs:195-222).
int ora_channel_shift(const float* src, int h, int w, int c, float* dst, int axis, const int* ends, const int* offs,
                      int ngroups) {
    for (int y = 0; y < h; y++)
        for (int x = 0; x < w; x++) {
            float* o = dst + ((long)y * w + x) * c;
            int g0 = 0;
            for (int g = 0; g < ngroups; g++) {
                const int g1 = ends[g];
                const int sy = axis == 2 ? y + offs[g] : y, sx = axis == 2 ? x : x + offs[g];
                for (int ch = g0; ch < g1; ch++)
                    o[ch] = ((unsigned)sy < (unsigned)h && (unsigned)sx < (unsigned)w) ? src[((long)sy * w + sx) * c + ch] : 0.0f;
                g0 = g1;
            }
            for (int ch = g0; ch < c; ch++) o[ch] = src[((long)y * w + x) * c + ch];
        }
    return 0;
}

// UpHead, one image, the scalar path (Kernels/FusedKernels.cs:62-192): s = ResizePixel(x) with the
// skip as its addend, acc = bias then acc += s[c] w[o][c] in ascending c, then the activation.
int ora_uphead(const float* src, int ih, int iw, int c, const float* skip, float* dst, int oh, int ow, float sy,
               float sx, const float* w, const float* bias, int oc, int resize_relu, int skip_relu, int act) {
    if (oc > 8) return -1;
    std::vector<int> y0(oh), y1(oh), x0(ow), x1(ow);
    std::vector<float> wy(oh), wx(ow);
    resize_axis(oh, ih, sy, y0.data(), y1.data(), wy.data());
    resize_axis(ow, iw, sx, x0.data(), x1.data(), wx.data());
#pragma omp parallel for schedule(static) num_threads(threads())
    for (int y = 0; y < oh; y++) {
        std::vector<float> s(c);
        for (int x = 0; x < ow; x++) {
            const float* a = src + ((long)y0[y] * iw + x0[x]) * c;
            const float* b = src + ((long)y0[y] * iw + x1[x]) * c;
            const float* e = src + ((long)y1[y] * iw + x0[x]) * c;
            const float* f = src + ((long)y1[y] * iw + x1[x]) * c;
            const float* k = skip + ((long)y * ow + x) * c;
            for (int ch = 0; ch < c; ch++) {
                float top = a[ch] + (b[ch] - a[ch]) * wx[x];
                float bot = e[ch] + (f[ch] - e[ch]) * wx[x];
                float v = top + (bot - top) * wy[y];
                if (resize_relu) v = fmaxf(v, 0.0f);
                v += skip_relu ? fmaxf(k[ch], 0.0f) : k[ch];
                s[ch] = v;
            }
            float acc[8];
            for (int o = 0; o < oc; o++) acc[o] = bias ? bias[o] : 0.0f;
            for (int ch = 0; ch < c; ch++)
                for (int o = 0; o < oc; o++) acc[o] += s[ch] * w[(long)o * c + ch];
            float* out = dst + ((long)y * ow + x) * oc;
            for (int o = 0; o < oc; o++) out[o] = act8(acc[o], act);
        }
    }
    return 0;
}

}  // extern "C"
