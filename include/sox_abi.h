/*
 * sox_abi.h - kernel argument blocks of the gfx950 code objects (one definition, shared by the
 * kernels, the host backend and any other host that launches them through sox_launch).
 *
 * Each kernel takes exactly one of these structs by value, so its kernarg segment IS the struct:
 * a host fills it and passes its bytes to sox_launch (hipModuleLaunchKernel with
 * HIP_LAUNCH_PARAM_BUFFER_POINTER), always sizeof the whole struct as declared here: the runtime
 * lays the block out as given, and a shorter one (a host built against an older copy of a struct
 * that has since grown) is not what the kernel reads. Field order is device pointers first, then the parameter
 * block, mirroring the reference's binding order + push-constant struct for the matching shader
 * (e.g. Backends/Vulkan/Shaders/conv_cm.comp:86-91 and its ND(...) call, Backends/Vulkan/VkGraph.cs:664-674).
 *
 * Storage types: "act" tensors are fp16 on fp16 graphs and fp32 on fp32 graphs; bias, norm and
 * SE parameters are always fp32 (ConstKind.F32, Engine/Extensions.cs:145).
 */
#ifndef SOX_ABI_H
#define SOX_ABI_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ActivationKind (Engine/ExecPlan.cs:42). */
enum sox_act { SOX_ACT_NONE = 0, SOX_ACT_RELU = 1, SOX_ACT_SIGMOID = 2, SOX_ACT_GELU = 3, SOX_ACT_HARDSWISH = 4, SOX_ACT_SWISH = 5 };

/* Epilogue flag bits, conv_cm's layout (VkGraph.cs:667-669): bias=1, residual=2, reflect=4, act<<4. */
#define SOX_F_BIAS 1
#define SOX_F_RESIDUAL 2
#define SOX_F_REFLECT 4
#define SOX_F_ACT_SHIFT 4
#define SOX_F_ACT_MASK 0xF0
#define SOX_F_DENSE_A 0x100 /* A is a plain row-major [M][lda] matrix (Gemm), not an NHWC image */
#define SOX_F_PAD_ROWS 0x400 /* LDS-DMA Gemm: output rows are padded to ldy >= N rounded up to 4, so the N tail
                                 is stored as whole 4-element groups (the pad columns take junk) */
#define SOX_F_POOL 0x800      /* direct conv kernels: 2x2/2 max pool of the (activated) conv output fused in
                                 (ConvP.Pool, Kernels/Nhwc.cs:661-727); m counts pooled pixels, oh / ow
                                 stay the conv output's size */
#define SOX_F_POOL_RELU 0x1000 /* with SOX_F_POOL: relu after the max (PoolP.FuseRelu) */
#define SOX_F_CONVT 0x200   /* LDS-DMA conv kernels: column n = tap * ct_oc + o of input pixel m is
                               ConvTranspose output (y * ct_kh + dy, x * ct_kw + dx, o), tap = dy * ct_kw + dx */

/*
 * Implicit-GEMM convolution / Gemm with fused epilogue (conv_cm.comp, gemm.comp).
 *   M = n*oh*ow output pixels (or Gemm rows), N = oc, K = kh*kw*ic (tap-major, channel fastest).
 *   w is [N][kpad] (k fastest: ConstKind.ConvWT / GemmNK, Engine/Extensions.cs:150-153).
 *   y[m*ldy + n] = act(sum_k A[m,k] w[n,k] (+ bias[n]) (+ add[m*ldy + n]))
 * The sox_gemm_ln_* kernels take A as the input of a LayerNorm over its rows (K) that the host folded
 * into the Gemm: w holds gamma-scaled weights, bias = b + beta . W, and
 *   y[m*ldy + n] = act(rstd_m (sum_k A[m,k] w[n,k] - mean_m ln_c[n]) + bias[n] (+ add)).
 * Grid: (ceil(M/BM), ceil(N/BN)); 256 threads.
 */
typedef struct sox_igemm_args {
    const void* x;
    const void* w;
    const float* bias;
    const void* add;
    void* y;
    const void* zeros; /* >= 16 zero bytes: the source of padding taps for LDS-DMA conv kernels */
    int32_t m, n, k, kpad;
    int32_t ih, iw, ic, oh, ow;
    int32_t kh, kw, sh, sw, pt, pl;
    int32_t flags;
    float pad_value;
    int32_t ldy;  /* output / residual row stride in elements (n, or a concat channel total) */
    int32_t lda;  /* SOX_F_DENSE_A: A row stride in elements */
    int32_t tiles_n; /* ceil(N/BN): tile-order remap of the 1-D grid */
    int32_t ct_kh, ct_kw, ct_oc; /* SOX_F_CONVT: the ConvTranspose kernel (stride == kernel) and its channels */
    float ln_eps;                /* sox_gemm_ln_*: the folded LayerNorm's epsilon */
    const float* ln_c;           /* sox_gemm_ln_*: [N] column sums of the gamma-scaled packed weights */
    /* sox_conv_halo_*_upcat: the input (x unused) is the channel concat of up_n sources of up_c channels
     * each, source s the nearest upsample by 2^up_shift[s] of up[s] = [n][ih >> shift][iw >> shift][up_c] */
    const void* up[4];
    int32_t up_n, up_c;
    int32_t up_shift[4];
    /* conv-ring kernels with a residual: res_shift > 0 reads it as the nearest upsample by 2^res_shift of
     * [n][oh >> res_shift][ow >> res_shift][ldy] (the FPN's top-down Add, fused) */
    int32_t res_shift, pad_;
} sox_igemm_args;

/*
 * Depthwise k x k conv, NHWC (depthwise.comp; Kernels/Nhwc.cs:496-631).
 *   w is [tap][c] (ConstKind.DwW). acc = bias[c] + sum_tap x * w; act.
 * Grid: 1-D over n*oh*ow*(c/cvec) work items.
 */
typedef struct sox_dw_args {
    const void* x;
    const void* w;
    const float* bias;
    const void* add;
    void* y;
    int32_t n, c, ih, iw, oh, ow;
    int32_t kh, kw, sh, sw, pt, pl;
    int32_t flags;
    float pad_value;
} sox_dw_args;

/*
 * Depthwise k x k over LDS tiles (k = 3 or 5, stride 1 or 2, c % 8 == 0, zero or reflect pad):
 * a workgroup computes an output tile of 8 x 8 pixels of 64 channels
 * from the tile's input halo staged once in LDS. Grid (tiles_x * tiles_y, ceil(c / 64), n).
 * gap = 1: the workgroup also writes the channel sums of its stored (rounded) outputs,
 * part[b][tile][c], the GAP partials of an SE gate that reads this conv's output.
 */
typedef struct sox_dwt_args {
    const void* x;
    const void* w;
    const float* bias;
    const void* add;
    void* y;
    float* part;
    int32_t n, c, ih, iw, oh, ow;
    int32_t kh, kw, sh, sw, pt, pl;
    int32_t flags;
    int32_t tiles_x, tiles_y;
    int32_t gap;
} sox_dwt_args;

/*
 * ConvTranspose with stride == kernel, no pad, group 1 (convt.comp; Kernels/Nhwc.Det.cs:51-131).
 *   w is [tap][ic][oc] (ConstKind.ConvTW). out[(y*kh+dy), (x*kw+dx), o] = act(b[o] + sum_c x[y,x,c] w[tap][c][o]).
 */
typedef struct sox_convt_args {
    const void* x;
    const void* w;
    const float* bias;
    void* y;
    int32_t n, ih, iw, ic, oc, kh, kw;
    int32_t flags;
} sox_convt_args;

/*
 * Two chained stride-2 2x2 ConvTransposes run as one kernel (the DB head's probability map: ConvT
 * ic -> oc1 + bias + act1, then ConvT oc1 -> 1 + bias + act2; the reference dispatches convt.comp
 * for each, Backends/Vulkan/VkGraph.cs:918-926). Per input pixel the first one's 4 x oc1 outputs
 * stay on chip (rounded to the storage type as the unfused path stores them) and the second one's
 * 16 outputs are written:
 * y[n][4 ih][4 iw][1]. w1 is the first ConvT as [tap * oc1 + o][kpad] (its Gemm packing), w2 the
 * second as [tap][oc1]. ic <= 32, ic % 8 == 0; oc1 % 8 == 0, oc1 <= 32.
 */
typedef struct sox_convt2_args {
    const void* x;
    const void* w1;
    const float* b1; /* [oc1] or null */
    const void* w2;
    const float* b2; /* [1] or null */
    void* y;
    int32_t n, ih, iw, ic, oc1, kpad;
    int32_t act1, act2;
} sox_convt2_args;

/* Per-channel mean partials over pixel chunks (gap_part.comp): part[n][chunk][c] (fp32). */
typedef struct sox_gap_args {
    const void* x;
    float* part;
    int32_t n, hw, c, chunks;
} sox_gap_args;

/*
 * Squeeze-excitation gate (se_gate.comp; Kernels/Nhwc.Det.cs:287-314) in two passes:
 *   sox_se_fc1: grid (groups, n), groups = ceil(c / 64). Workgroup g averages channels
 *               [64 g, 64 g + 64) over the GAP partials and writes its share of fc1,
 *               hid[b][g][j] = sum_{ch in group} W1[j][ch] mean[ch]                      256 threads
 *   sox_se_fc2: grid (ceil(c/4), n). h = act1(b1 + sum_g hid[b][g]); one wave per channel:
 *               z = b2 + W2 h; gate = sigmoid(z) or hard-sigmoid, + offset              256 threads
 *               and either s[b][ch] = gate, or (SOX_SE_FOLD, one image) column ch of the consumer
 *               1x1 conv's packed weights scaled by it: wdst[n][ch] = wsrc[n][ch] * gate.
 *   w1 [r][c] and w2 [c][r] keep their ONNX 1x1-conv layouts (fp32): one contiguous row per output.
 */
#define SOX_SE_FOLD 16
typedef struct sox_se_args {
    const float* part;
    const float* w1;
    const float* b1;
    const float* w2;
    const float* b2;
    void* s;           /* [n][c] in the graph's storage type */
    float* hid;        /* [n][groups][r] fp32 (scratch) */
    const void* wsrc;  /* SOX_SE_FOLD: the consumer's weights [wn][wk] (storage type) */
    void* wdst;        /* SOX_SE_FOLD: their gated copy (scratch) */
    int32_t c, r, chunks, hw, groups;
    int32_t wn, wk;
    int32_t flags; /* bit0 b1, bit1 b2, bit2 act1 relu, bit3 hard, SOX_SE_FOLD */
    float alpha, beta, offset;
} sox_se_args;

/*
 * Depthwise tiles (sox_dwt_args, dw.gap = 1) with the SE gate that reads their output run in the same
 * launch: depthwise.comp + gap_part.comp + se_gate.comp (VkGraph.cs:595-605, 949-965) as one dispatch.
 * Each workgroup stores its GAP partials and counts itself in sync[b][g] (a vector atomic increment
 * that wraps to 0 at its last arrival, with agent-scope release / acquire fences around it). The last
 * tile of channel group g runs sox_se_fc1's work for that group and counts in sync[b][groups]; the
 * last group's workgroup runs sox_se_fc2's for every channel of image b (the gates, then the folded
 * weights or s). No workgroup waits on another. The counters are 0 between launches; their memory
 * (SOX_SLOT_SYNC) belongs to the session, zeroed when it is made. Taken when SIMDONNX_HIP_SE_IN_DW is
 * set: the one-workgroup fc2 is slower than the separate passes on MI355X.
 *   kernels: sox_dwt_{f16,bf16,f32}_k{3,5}s{1,2}_se, grid as sox_dwt_*, 256 threads
 */
typedef struct sox_dwt_se_args {
    sox_dwt_args dw;
    sox_se_args se;
    uint32_t* sync; /* [n][groups + 1] */
} sox_dwt_se_args;

/* out[p, c] = act(x[p, c] op v[img(p), c]): NHWC per-channel broadcast (ew2 / ChannelBroadcast). */
typedef struct sox_chan_args {
    const void* x;
    const void* v; /* [n][c], storage type */
    void* y;
    int64_t rows;  /* n*h*w */
    int32_t c, hw;
    int32_t op;    /* EwOp: 0 add, 1 sub, 2 mul, 3 div */
    int32_t flags; /* bit0 reversed operands, bit1 v is one [c] vector for every image, act<<4 */
} sox_chan_args;

/* Same-shape elementwise binary op + act (ew2v.comp). */
typedef struct sox_ew_args {
    const void* a;
    const void* b;
    void* y;
    int64_t count;
    int32_t op;
    int32_t flags; /* act<<4 */
} sox_ew_args;

/* Unary activation / affine (unary.comp, unary2.comp, hsig.comp): y = act(alpha*x + beta) or hard-sigmoid. */
typedef struct sox_unary_args {
    const void* x;
    void* y;
    int64_t count;
    int32_t mode;  /* 0 act, 1 affine alpha*x+beta, 2 hard-sigmoid clamp(alpha*x+beta,0,1), 3 copy */
    int32_t act;
    float alpha, beta;
} sox_unary_args;

/* Nearest resize (asymmetric, floor) + optional [relu] addend (nearest.comp; Nhwc.Det.cs:167-204). */
typedef struct sox_nearest_args {
    const void* x;
    const void* add;
    void* y;
    int32_t n, ih, iw, c, oh, ow;
    float sy, sx;
    int32_t flags; /* bit0 addend, bit1 relu on addend */
    int32_t ldy, y_off; /* output pixel stride and channel offset (writes a concat slice) */
} sox_nearest_args;

/* Channel-slice copy: y[p*ldy + y_off + c] = x[p*c_in + c] (concat_ax.comp, NHWC channel concat). */
typedef struct sox_slice_copy_args {
    const void* x;
    void* y;
    int64_t rows;
    int32_t c, ldy, y_off;
} sox_slice_copy_args;

/* fp32 <-> fp16 staging conversion (f32to16.comp / f16to32.comp). */
typedef struct sox_cvt_args {
    const void* x;
    void* y;
    int64_t count;
} sox_cvt_args;

/* LayerNorm over the innermost dim, one wave per row (layernorm.comp; Kernels/Ops.cs:544-574). */
typedef struct sox_ln_args {
    const void* x;
    const float* gamma;
    const float* beta;
    void* y;
    int64_t rows;
    int32_t len;
    float eps;
} sox_ln_args;

/* Row softmax over the innermost dim (softmax.comp; Kernels/Ops.Seq.cs:28-72). */
typedef struct sox_softmax_args {
    const void* x;
    void* y;
    int64_t rows;
    int32_t len;
    int32_t staged; /* 1: the row is kept in dynamic LDS (len floats, granted at launch) */
    int32_t ldx;    /* input row stride in elements (>= len; the output rows are dense) */
    int32_t pad_;
} sox_softmax_args;

/*
 * Fused attention (attn.comp): out[b,h,t,:] = sum_s softmax_s(scale q.k) v over strided views.
 * Element (b, h, t, d) of operand i lives at base_i + b*sb_i + h*sh_i + t*st_i + d (d contiguous).
 */
typedef struct sox_attn_args {
    const void* q;
    const void* k;
    const void* v;
    void* o;
    int32_t batch, heads, t, s, d;
    float scale;
    int64_t q_sb, q_sh, q_st;
    int64_t k_sb, k_sh, k_st;
    int64_t v_sb, v_sh, v_st;
    int64_t o_sb, o_sh, o_st;
} sox_attn_args;

/* 2x2/2 max pool (+relu) of an NHWC tensor (the ConvP.Pool epilogue when it runs as its own pass). */
typedef struct sox_pool_args {
    const void* x;
    void* y;
    int32_t n, ih, iw, c, oh, ow;
    int32_t kh, kw, sh, sw, pt, pl;
    int32_t flags; /* bit0 relu */
} sox_pool_args;

/* ---- the rest of the ExecOp surface (Backends/Vulkan/VkGraph.cs:795-1068) ---- */

/* Bilinear resize, half-pixel source coordinates clamped at the borders (bilinear.comp;
 * Kernels/Nhwc.cs:773-870), out = [relu](lerp) + [relu](add). */
typedef struct sox_bilinear_args {
    const void* x;
    const void* add;
    void* y;
    int32_t n, ih, iw, c, oh, ow;
    float sy, sx;
    int32_t flags; /* bit0 relu on the resized value, bit1 addend, bit2 relu on the addend */
} sox_bilinear_args;

/* Rank-4 pad in physical (storage) order (pad.comp): source index o - pb per dim, out of range
 * -> value (constant) or the reflected index (reflect). */
typedef struct sox_pad_args {
    const void* x;
    void* y;
    int32_t id[4], od[4], pb[4];
    int32_t reflect;
    float value;
} sox_pad_args;

/* Strided gather, rank <= 6 (transpose.comp / slice.comp; Kernels/Ops.cs:798-883):
 * y[o] = x[base + sum_k o_k * str[k]], o_k the digits of the output index in od[]. */
typedef struct sox_gather_args {
    const void* x;
    void* y;
    int64_t count, base;
    int64_t str[6];
    int32_t od[6];
} sox_gather_args;

/* Batched 2D transpose (a permutation that swaps two contiguous groups of dims):
 * y[b][c][r] = x[b][r][c], grid (ceil(cols / 64), ceil(rows / 64), batch). */
typedef struct sox_transpose2d_args {
    const void* x;
    void* y;
    int32_t rows, cols;
} sox_transpose2d_args;

/* LeakyRelu (0) / Tanh (1, a = in scale, b = out scale) / Clip (2, a = min, b = max) / Erf (3)
 * (unary2.comp; Kernels/Act.cs:83-147). */
typedef struct sox_unary2_args {
    const void* x;
    void* y;
    int64_t count;
    int32_t mode;
    float a, b;
} sox_unary2_args;

/* DepthToSpace (s2d = 0) / SpaceToDepth (s2d = 1), NHWC, CRD or DCR (d2s.comp / s2d.comp;
 * Kernels/Nhwc.Det.cs:210-282). */
typedef struct sox_d2s_args {
    const void* x;
    void* y;
    int64_t count;
    int32_t n, ih, iw, ic, oh, ow, oc, block, crd, s2d;
} sox_d2s_args;

/* Average pool of an NHWC tensor (avgpool.comp; Kernels/Ops.Seq.cs:180-215). */
typedef struct sox_avgpool_args {
    const void* x;
    void* y;
    int32_t n, ih, iw, c, oh, ow;
    int32_t kh, kw, sh, sw, pt, pl;
    int32_t count_include_pad;
} sox_avgpool_args;

/* GlobalAvgPool finish (gap_sum.comp): y[b][c] = (sum over chunks of part[b][chunk][c]) * inv_hw,
 * chunks added in 4 interleaved phases, the phase sums in phase order. Grid (ceil(c / 64), n). */
typedef struct sox_gap_mean_args {
    const float* part;
    void* y;
    int32_t n, c, chunks;
    float inv_hw;
} sox_gap_mean_args;

/* Batched MatMul, activation x activation (the gemm.comp matmul route; Kernels/Ops.Seq.cs:92-116):
 * y[b] = a[b] (m x k) . b[b or 0] (k x n), element strides between batches (b_stride 0 = broadcast). */
typedef struct sox_matmul_args {
    const void* a;
    const void* b;
    void* y;
    int32_t batch, m, n, k;
    int64_t a_stride, b_stride, y_stride;
} sox_matmul_args;

/* CTC head, pass 1 (Decoding/Kernels/MatMul.ArgMax.cs:29-299): per (row block of 128, column range
 * of cols_per_split) the rows' (max, sum of exp(logit - max), argmax) over the range, logits =
 * x . W^T + bias. Grid (ceil(rows / 256), splits), 512 threads; cols_per_split * (inner * 2 + 4) <= 128 KiB. */
typedef struct sox_ctc_args {
    const void* x;      /* features fp16 [rows][inner] */
    const void* w;      /* weights fp16 [columns][ldw], the inner values of a column contiguous */
    const float* bias;  /* [columns] when has_bias */
    float* part;        /* [splits][rows][3]: max, sum (NaN: a non-finite logit), argmax (int bits) */
    int32_t* status;    /* cleared to 0 by workgroup (0, 0) (pass 2 sets it on a non-finite logit) */
    int32_t rows, inner, columns, ldw, cols_per_split, has_bias;
} sox_ctc_args;

/* CTC head, pass 2: the splits (<= 64) of a row merged by one wave; probability = min(1, 1 / sum);
 * *status = 1 when a logit or the sum was not finite. 256 threads, ceil(rows / 4) workgroups. */
typedef struct sox_ctc_merge_args {
    const float* part;
    int32_t* indices;
    float* probs;
    int32_t* status;
    int32_t rows, splits;
} sox_ctc_merge_args;

/* Built-in extension op SafeDiv (Engine/Fusions/SafeDivOp.cs; safediv.comp): y = clamp(a / max(b, eps),
 * lo, hi) in fp32 over same-shape operands. */
typedef struct sox_safediv_args {
    const void* a;
    const void* b;
    void* y;
    int64_t count;
    float eps, lo, hi;
} sox_safediv_args;

/* Built-in extension op ChannelShift (Engine/Fusions/ChannelShiftOp.cs; shift.comp), NHWC: channel group g
 * (channels [ends[g-1], ends[g])) reads the pixel offs[g] away along H (axis 2) or W (axis 3), zero
 * outside; channels past the last group end copy unshifted. */
typedef struct sox_shift_args {
    const void* x;
    void* y;
    int32_t n, h, w, c, axis, ngroups;
    int32_t ends[5], offs[5];
} sox_shift_args;

/* Built-in extension op UpHead (Engine/Fusions/UpHeadOp.cs; uphead.comp / uphead_sc.comp), NHWC, one
 * thread per output pixel: s[c] = [relu](bilinear(x)) + [relu](skip), out[o] = act(bias[o] +
 * sum_c w[o][c] s[c]) for o < oc <= 8. With a skip conv (flags bit 3) the skip is recomputed per pixel
 * from its input sk ([oh][ow][skc], stride 1) by the conv w_sc [c][skc][kh][kw] + b_sc (+ relu). */
typedef struct sox_uphead_args {
    const void* x;
    const void* skip;     /* the skip tensor [oh][ow][c], or the skip conv's input [oh][ow][skc] */
    const void* w;        /* [oc][c], storage type */
    const float* bias;    /* [oc] (flags bit 2) */
    void* y;
    const void* w_sc;     /* [c][skc][kh][kw], storage type */
    const float* b_sc;    /* [c] (sc_flags bit 0) */
    int32_t n, ih, iw, c, oh, ow, oc;
    float sy, sx;
    int32_t flags;        /* bit0 relu on the resize, bit1 relu on the skip, bit2 bias, bit3 skip conv, act << 4 */
    int32_t skc, kh, kw, pt, pl, sc_flags;  /* sc_flags: bit0 bias, bit1 reflect pad, bit2 relu */
    float sc_pad_value;
} sox_uphead_args;

/* Image session input (img2nhwc.comp): interleaved u8 pixels (bpp 3 or 4, rows `stride` bytes apart)
 * -> NHWC [oh][ow][3], tensor channel c = lut[c * 256 + byte], the image at (pt, pl) with its edge
 * repeated around it; swap = 1: tensor channel 0 is byte 2 of a pixel. Two flat tensor pixels per
 * thread, grid ceil(oh * ow / 512). */
typedef struct sox_img2nhwc_args {
    const uint8_t* src;
    void* y;
    const float* lut;  /* [3][256] */
    int32_t oh, ow, ih, iw, pt, pl, stride, bpp, swap;
} sox_img2nhwc_args;

/* Image session output (nhwc2img.comp): the ih x iw window at (pt, pl) of NHWC [h][w][3] -> tightly
 * packed u8, byte = clamp(int(v * scale + 0.5), 0, 255); one thread per 4-byte word (3 bpp: words
 * straddle pixels; 4 bpp: one pixel, alpha copied from the uploaded source `alpha`). */
typedef struct sox_nhwc2img_args {
    const void* x;
    uint32_t* dst;
    const uint32_t* alpha;
    int32_t h, w, ih, iw, pt, pl, nwords, bpp, swap;
    float scale;
} sox_nhwc2img_args;

/* Fused transformer MLP (mlp.hip): y = act2(GELU(rstd (x . W1 - mean c1) + b1) . W2 + b2 + res), the
 * LayerNorm folded into W1 / b1 / c1 at graph creation. sox_mlp_*: one 512-thread workgroup per 32 rows.
 * Split form for grids that would leave CUs idle: sox_mlpq_* runs one 512-thread workgroup per (32 rows,
 * part of the hidden width), each writing its part's fc2 sums to `part`; sox_mlp_sum_* (256 threads, 4
 * outputs each) then adds b2, the parts in order and the residual. */
typedef struct sox_mlp_args {
    const void* x;      /* fp16 [m][k1] */
    const void* w1;     /* fp16 gamma-scaled [k1][h] in 32x32x16 fragment order (32 columns x 16 k per KiB) */
    const float* b1;    /* [h]: b + beta W */
    const float* c1;    /* [h]: column sums of w1 as rounded */
    const void* w2;     /* fp16 [h][n2] in the same fragment order */
    const float* b2;    /* [n2] (flags bit0) */
    const void* res;    /* fp16 [m][n2] (flags bit1) */
    void* y;            /* fp16 [m][n2] */
    int32_t m, k1, h, n2, ldw1, ldw2;
    float eps;
    int32_t flags;      /* bit0 b2, bit1 residual, act2 << 4 */
    float* part;        /* sox_mlpq_* / sox_mlp_sum_*: fp32 [parts][m][n2], fc2 over each part of the hidden width */
    int32_t parts;
    /* sox_mlpqp_*: x is first computed as the preceding projection Gemm with its residual Add,
     * x = po . Wp^T + pb + px ([m][k1] each, Wp GemmNK-packed [k1][k1]); part 0 of every row block
     * stores it to xout (the MLP's residual, read by sox_mlp_sum_*). */
    int32_t pflags;     /* bit0 pb */
    const void* po;
    const void* pw;
    const float* pb;
    const void* px;
    void* xout;
} sox_mlp_args;

/* Matrix-core rate probe (sox_probe_mfma_f16 in the Gemm code object; a measurement kernel, no
 * counterpart in the reference): each of the grid's waves runs `iters` rounds of four independent
 * 32x32x16 fp16 MFMA chains on hashed register operands and writes one float per thread to out. */
typedef struct sox_mfma_probe_args {
    float* out;
    int32_t iters;
    uint32_t seed;
} sox_mfma_probe_args;

/*
 * LayerNorm -> qkv Gemm -> attention of a transformer block in one dispatch (qkv_attn.hip), one 576-thread
 * workgroup per (image, head): images of t <= 96 tokens of dim = heads * 32 channels, ViT-style packed qkv
 * (the SVTR mixer). For head h of image b:
 *   q, k, v = LN(x) . Wqkv[cols of h] + bqkv  with the LayerNorm folded: wqkv gamma-scaled, bqkv = b + beta W,
 *             cqkv = the column sums of wqkv as rounded (the sox_gemm_ln_* epilogue), rounded to the storage type;
 *   o[b][:, h] = softmax(q k^T * scale) v  (the sox_attn_*_mfma kernel), rounded.
 * wqkv is GemmNK-packed [3 dim][kpad]; the head's qkv columns never leave LDS.
 */
typedef struct sox_qkvattn_args {
    const void* x;      /* [n][t][dim] */
    const void* wqkv;
    const float* bqkv;  /* [3 dim] (flags bit1) */
    const float* cqkv;  /* [3 dim] */
    void* o;            /* [n][t][heads][32] */
    int32_t n, t, kpad;
    float eps, scale;
    int32_t flags;      /* bit1 bqkv */
} sox_qkvattn_args;

/* LDS and LDS-DMA throughput probes (sox_probe_lds_read / sox_probe_lds_dma in probe.hip; measurement
 * kernels, no counterpart in the reference). 1024 threads per workgroup (16 waves), one workgroup per
 * CU. read: every wave keeps 16 ds_read_b128 of 1 KiB in flight per round; dma: every wave issues 8
 * global_load_lds_dwordx4 of 1 KiB per round from a 64 KiB slice of src (L2-resident after the first
 * round) into LDS. `iters` rounds; out gets one float per thread. */
typedef struct sox_lds_probe_args {
    float* out;
    const void* src; /* >= 64 x 64 KiB (dma) */
    int32_t iters;
    int32_t pad_;
} sox_lds_probe_args;

#ifdef __cplusplus
}
#endif
#endif
