/*
 * CPU oracle for the conv/GEMM hot path: a C++ restatement of SimdOnnx's NHWC CPU kernels.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product (simdonnx_amd/) links, loads or calls this
 * library. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, and there
 * only as the checker / the timed CPU baseline.
 *
 * Every entry point names the reference routine it restates (paths relative to the reference
 * repository root, src/Sdcb.SimdOnnx/...). Per-element arithmetic follows the reference order:
 * accumulators start at the bias, taps ascend, channels ascend, one fused multiply-add each
 * (Kernels/Nhwc.cs:343-373, Kernels/Nhwc.Avx512.cs:11-19). The scalar, AVX2 (6 px x 16 oc) and
 * AVX-512 (10 px x 32 oc) tiers keep that order, so they agree bit for bit.
 *
 * Layout: NHWC activations ([n][h][w][c]), ONNX weight layouts ([oc][ic/g][kh][kw] for Conv,
 * [ic][oc][kh][kw] for ConvTranspose, [K][N] or [N][K] for Gemm).
 * Return value: 0 on success, negative on an unsupported shape/argument.
 */
#ifndef SOX_ORACLE_H
#define SOX_ORACLE_H
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

/* ActivationKind (Engine/ExecPlan.cs:42). */
enum { ORA_ACT_NONE = 0, ORA_ACT_RELU = 1, ORA_ACT_SIGMOID = 2, ORA_ACT_GELU = 3, ORA_ACT_HARDSWISH = 4, ORA_ACT_SWISH = 5 };
/* Tier selection: 0 = best available, 1 = scalar, 2 = AVX2+FMA, 3 = AVX-512F. */
enum { ORA_TIER_AUTO = 0, ORA_TIER_SCALAR = 1, ORA_TIER_AVX2 = 2, ORA_TIER_AVX512 = 3 };

/* ConvP (Engine/ExecPlan.cs:50-65), spatial fields only. */
typedef struct ora_conv_p {
    int kh, kw;
    int sh, sw;
    int pad_t, pad_l, pad_b, pad_r;
    int group;
    int act;
    int pad_mode;    /* 0 constant, 1 reflect (PadMode, ExecPlan.cs:44) */
    float pad_value; /* constant-mode fill */
    int pool;        /* 1: fused 2x2/2 max pool epilogue (ConvP.Pool, Nhwc.ConvPool) */
    int pool_relu;   /* PoolP.FuseRelu */
} ora_conv_p;

int ora_tier_available(int tier);
void ora_set_threads(int threads); /* Par.Threads analogue (Kernels/Par.cs:11-58); <=0 = all CPUs */
int ora_get_threads(void);

/* Winograd eligibility (Kernels/NhwcWinograd.cs:28-32). */
int ora_winograd_eligible(const ora_conv_p* p, int ic);

/* Nhwc.Conv (Kernels/Nhwc.cs:172-217): dense / depthwise / Winograd, batch of n images.
 * algo: 0 = the reference's choice (Winograd when eligible), 1 = force direct.
 * add: same-shape residual (nullable), added before the activation. bias nullable. */
int ora_conv(const float* src, int n, int ih, int iw, int ic, const float* w, const float* bias,
             const float* add, float* dst, int oh, int ow, int oc, const ora_conv_p* p, int algo, int tier);

/* Nhwc.PackGemm + Nhwc.Gemm (Kernels/Nhwc.cs:128-168, Nhwc.Avx512.cs:241-266):
 * dst[m,n] = act(a[m,k] . B + bias); B is [k][n] or, with trans_b, [n][k]. */
int ora_gemm(const float* a, int m, int k, const float* b, int n, int trans_b, const float* bias, int act,
             float* dst, int tier);

/* Ops.MatMul (Kernels/Ops.Seq.cs:92-116), batched, no broadcast: c[b] = a[b] (m x k) . b[b] (k x n). */
int ora_matmul(const float* a, const float* b, int batch, int m, int k, int n, float* c);

/* Nhwc.ConvTranspose / ConvTDot (Kernels/Nhwc.Det.cs:26-131): stride == kernel, no pad, group 1.
 * w is [ic][oc][kh][kw]; dst is [ih*kh][iw*kw][oc] per image. */
int ora_conv_transpose(const float* src, int n, int ih, int iw, int ic, const float* w, int oc, int kh, int kw,
                       const float* bias, int act, float* dst);

/* Nhwc.GlobalAvgPool (Kernels/Nhwc.Det.cs:134-164), one image [hw][c] -> [c]. */
int ora_global_avg_pool(const float* src, int hw, int c, float* dst);

/* Nhwc.ChannelGate (Kernels/Nhwc.Det.cs:287-314), one image. w1 [r][c], w2 [c][r]. */
int ora_channel_gate(const float* src, int hw, int c, const float* w1, const float* b1, const float* w2,
                     const float* b2, int r, int act1_relu, int hard, float alpha, float beta, float offset, float* dst);

/* Nhwc.ChannelBroadcast (Kernels/Nhwc.Det.cs:317-351): dst[row,c] = full[row,c] op vec[c]
 * (vec op full when rev). op: 0 add, 1 sub, 2 mul, 3 div (EwOp). act: 0 or 1 (relu). */
int ora_channel_broadcast(const float* full, const float* vec, float* dst, long rows, int c, int op, int rev, int act);

/* Elementwise same-shape binary op (Kernels/Ew.cs), act 0/1. */
int ora_ew2(const float* a, const float* b, float* dst, long count, int op, int act);

/* Nhwc.ResizeNearest (Kernels/Nhwc.Det.cs:167-204): asymmetric / floor, optional addend. */
int ora_resize_nearest(const float* src, int ih, int iw, int c, float* dst, int oh, int ow, float sy, float sx,
                       const float* add, int add_relu);

/* Nhwc.ConcatInner (Kernels/Nhwc.Det.cs:354-370). */
int ora_concat_inner(const float* const* ins, const int* counts, int nin, long outer, float* dst);

/* Nhwc.HardSigmoid (Kernels/Nhwc.Det.cs:373-384). */
int ora_hard_sigmoid(const float* src, long count, float alpha, float beta, float* dst);

/* Unary activation over a buffer (Nhwc.Act8 / ActRow), act as ActivationKind. */
int ora_activation(const float* src, long count, int act, float* dst);

/* Ops.LayerNorm (Kernels/Ops.cs:544-574 -> Avx2Kernels.LayerNorm): rows x len, gamma/beta [len]. */
int ora_layer_norm(const float* src, long rows, int len, const float* gamma, const float* beta, float eps, float* dst);

/* Ops.Softmax over the last axis (Kernels/Ops.Seq.cs:28-72). */
int ora_softmax(const float* src, long rows, int len, float* dst);

/* Scaled dot-product attention as the CPU plan computes it (MatMul, scale, Softmax, MatMul;
 * Ops.Seq.cs:28-116). q,k,v,out are [batch*heads][t][d] contiguous. */
int ora_attention(const float* q, const float* k, const float* v, int bh, int t, int s, int d, float scale, float* out);

/* SimdMath scalar restatements of the vector cores (Kernels/SimdMath.cs:121-168). */
float ora_exp_core(float x);
float ora_erf_core(float x);
float ora_gelu_core(float x);
float ora_sigmoid_core(float x);
float ora_act(float x, int act);

/* IEEE binary16 round-to-nearest-even (the (Half) cast of Engine/Extensions.cs:315). */
void ora_round_f16(const float* src, float* dst, long count);

/* Nhwc.ResizeBilinear (Kernels/Nhwc.cs:773-870), one image: half-pixel coordinates clamped at the
 * borders; out = [relu](lerp) + [relu](add) (add nullable). */
int ora_resize_bilinear(const float* src, int ih, int iw, int c, float* dst, int oh, int ow, float sy, float sx,
                        int relu, const float* add, int add_relu);
/* Nhwc.Pad (Kernels/Nhwc.cs:877-900), spatial, one image; mode 0 constant, 1 reflect. */
int ora_pad_nhwc(const float* src, int ih, int iw, int c, float* dst, int oh, int ow, int pad_t, int pad_l,
                 int mode, float value);
/* Nhwc.AvgPool (Kernels/Ops.Seq.cs:180-215), one image. */
/* Nhwc.MaxPool (Kernels/Nhwc.cs:729-769), one image: taps outside the image skipped, an empty window
 * is 0, relu (PoolP.FuseRelu) last. */
int ora_max_pool_nhwc(const float* src, int ih, int iw, int c, float* dst, int oh, int ow, int kh, int kw, int sh,
                      int sw, int pad_t, int pad_l, int relu);
int ora_avg_pool_nhwc(const float* src, int ih, int iw, int c, float* dst, int oh, int ow, int kh, int kw, int sh,
                      int sw, int pad_t, int pad_l, int count_include_pad);
/* Nhwc.DepthToSpace (dir 0) / SpaceToDepth (dir 1), NHWC, one image (Kernels/Nhwc.Det.cs:210-282). */
int ora_depth_space(const float* src, int ih, int iw, int ic, float* dst, int b, int crd, int dir);
/* LeakyRelu (0) / Tanh (1) / Clip (2) / Erf (3) (Kernels/Act.cs:83-147). */
int ora_unary2(const float* src, long count, int mode, float a, float b, float* dst);

/* CtcProjection.ArgMax, scalar kernel (Decoding/Kernels/MatMul.ArgMax.cs:130-299): x [rows][inner],
 * w row-major [inner][columns], bias nullable. -1 on a non-finite logit. */
int ora_ctc_argmax(const float* x, const float* w, const float* bias, long rows, int inner, int columns, int* indices,
                   float* probs);

/* Built-in extension ops (Kernels/FusedKernels.cs): SafeDiv (:35-57), ChannelShift NHWC one image
 * (:195-222), UpHead one image with a stored skip (:62-192; w [oc][c], oc <= 8, bias nullable). */
int ora_safediv(const float* a, const float* b, float* dst, long count, float eps, float lo, float hi);
int ora_channel_shift(const float* src, int h, int w, int c, float* dst, int axis, const int* ends, const int* offs,
                      int ngroups);
int ora_uphead(const float* src, int ih, int iw, int c, const float* skip, float* dst, int oh, int ow, float sy,
               float sx, const float* w, const float* bias, int oc, int resize_relu, int skip_relu, int act);

#ifdef __cplusplus
}
#endif
#endif
