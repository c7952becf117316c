"""The benchmark workloads as fused NHWC ExecPlans (what GraphCompiler emits for them, PlanTarget.Hip).

Every workload returns ``(plan, inputs)``: the plan and its seeded fp32 inputs in physical layout.
Weights and inputs come from ``synth`` (a counter-based generator; the reference's System.Random
cannot be reproduced outside .NET). Workloads:

  conv3x3_bias_relu   1x64x64x64 NHWC fp32, Conv3x3 s1 p1 64->64 + bias + ReLU
  matmul_bias_gelu    A[16,512,768] x W[768,3072] + b[3072] -> GELU (Gemm after FuseBiasAdd / FuseGelu /
                      FuseLateAct, GraphCompiler.cs:1161-1213, 1058-1105, 800-874)
  mobilenetv3_small   MobileNetV3-small backbone at 3x640x640 (configs 3 / 4)
  dbnet               DBNet-style detector at 3x960x960 (config 4)
  svtr                SVTR/CRNN-style recognizer, batch 32 of 3x48x320 (config 5)
"""
from __future__ import annotations

import functools
import os

import numpy as np

from . import synth
from .plan import NHWC, PlanBuilder


class _Ids:
    """Sequential tensor ids for the generator."""

    def __init__(self):
        self.i = 0

    def __call__(self):
        self.i += 1
        return self.i


def conv3x3_bias_relu(seed: int = 1, n=1, h=64, w=64, cin=64, cout=64):
    """Single fused Conv2d 3x3 s1 p1 + bias + ReLU, NHWC; x, W ~ U(-1,1), b ~ U(-0.1,0.1)."""
    pb = PlanBuilder()
    x = pb.input((n, cin, h, w), NHWC, "x")
    W = synth.uniform(seed, 2, (cout, cin, 3, 3), -1.0, 1.0)
    b = synth.uniform(seed, 3, (cout,), -0.1, 0.1)
    y = pb.conv(x, W, b, stride=1, pad=1, act="relu", name="conv")
    plan = pb.build(y)
    xin = synth.uniform(seed, 1, (n, h, w, cin), -1.0, 1.0)
    return plan, [xin]


def conv3x3_flops(n=1, h=64, w=64, cin=64, cout=64):
    return 2 * n * h * w * cout * cin * 9


def matmul_bias_gelu(seed: int = 2, batch=16, seq=512, k=768, n=3072):
    """MatMul + bias + GELU: A ~ N(0,1), W ~ N(0, 0.02), b ~ U(-0.1, 0.1)."""
    pb = PlanBuilder()
    a = pb.input((batch, seq, k), None, "A")
    W = synth.normal(seed, 2, (k, n), 0.02)
    b = synth.uniform(seed, 3, (n,), -0.1, 0.1)
    y = pb.gemm(a, W, b, act="gelu", name="gemm_gelu")
    plan = pb.build(y)
    ain = synth.normal(seed, 1, (batch, seq, k), 1.0)
    return plan, [ain]


def matmul_flops(batch=16, seq=512, k=768, n=3072):
    return 2 * batch * seq * k * n


# ---------------------------------------------------------------------------------------------
# MobileNetV3-small backbone (configs 3 and 4). Layer table per Howard et al. 2019, Table 2, as
# the block stack the config names; BatchNorm is folded into the convs (OnnxRewrites.FoldConvBatchNorm,
# Onnx/OnnxRewrites.cs:71-111), so each conv carries a bias. Activations as the reference fuses them:
# ReLU / HardSwish epilogues (HardSigmoid(1/6, 0.5) * x -> HardSwish, GraphCompiler.cs:1225-1252),
# SE as ChannelGate + broadcast multiply, projection + skip Add as ConvP.AddValue (:956-1019).
# ---------------------------------------------------------------------------------------------
# (kernel, expanded, out, se, act, stride)
MBV3_SMALL = [
    (3, 16, 16, True, "relu", 2),
    (3, 72, 24, False, "relu", 2),
    (3, 88, 24, False, "relu", 1),
    (5, 96, 40, True, "hardswish", 2),
    (5, 240, 40, True, "hardswish", 1),
    (5, 240, 40, True, "hardswish", 1),
    (5, 120, 48, True, "hardswish", 1),
    (5, 144, 48, True, "hardswish", 1),
    (5, 288, 96, True, "hardswish", 2),
    (5, 576, 96, True, "hardswish", 1),
    (5, 576, 96, True, "hardswish", 1),
]
# blocks whose outputs are the detector's stride 4 / 8 / 16 / 32 taps
MBV3_TAPS = (0, 2, 7, 10)


# ---------------------------------------------------------------------------------------------
# BatchNorm folds of the random weights (configs 3 and 4). A trained MobileNetV3 / DBNet has a
# BatchNorm after every conv, which OnnxRewrites.FoldConvBatchNorm (Onnx/OnnxRewrites.cs:71-111)
# folds into the conv: per output channel, w' = w s and b' = b s + t. With He-normal weights and no
# BatchNorm the detector's activations grow through the residual and FPN sums to logits of |70|,
# where fp16 storage by itself moves the sigmoid output by 5e-2, so no fp16 engine could meet 2e-2.
# Here every conv carries the fold of a BatchNorm (gamma 1, beta 0) whose statistics were measured
# once with the CPU reference on the seeded N(0, 1) calibration image at the config's size: the
# pre-activation of each output channel (the conv part of a residual projection, the detector's
# logit) has mean 0 and standard deviation 1. The (s, t) pairs are
# committed in data/bn_calibration.npz, keyed "<model>/<layer>/s|t", by
# tests/golden/make_bn_calibration.py; the weights stay the seeded He-normal draws, rescaled.
# ---------------------------------------------------------------------------------------------
_CAL_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "data", "bn_calibration.npz")


@functools.lru_cache(maxsize=1)
def _bn_calibration() -> dict:
    with np.load(_CAL_PATH, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _bn_scale(scales, model: str, layer: str, w, b, transpose=False):
    """(w, b) with the layer's folded BatchNorm (w s, b s + t per output channel: axis 0 of a Conv
    weight, axis 1 of a ConvTranspose weight). scales None: the committed calibration; a dict: the
    calibration in progress (a missing layer is left as it is)."""
    key = f"{model}/{layer}"
    cal = _bn_calibration() if scales is None else scales
    if key + "/s" not in cal:
        if scales is None:
            raise KeyError(f"no BatchNorm calibration for {key}")
        return w, b
    sc = np.asarray(cal[key + "/s"], np.float64)
    sh = np.asarray(cal[key + "/t"], np.float64)
    shape = (1, -1, 1, 1) if transpose else (-1, 1, 1, 1)
    w2 = (w.astype(np.float64) * sc.reshape(shape)).astype(np.float32)
    b64 = np.zeros(len(sc)) if b is None else b.astype(np.float64)
    return w2, (b64 * sc + sh).astype(np.float32)


def _make_divisible(v, d=8):
    return max(d, int(v + d / 2) // d * d)


def _bias(seed, ids, c):
    return synth.uniform(seed, ids(), (c,), -0.1, 0.1)


def mobilenetv3_backbone(pb: PlanBuilder, x: int, seed: int, ids: _Ids, name="mbv3", model="mbv3", scales=None):
    """Emits the stem + 11 inverted-residual blocks; returns (last output, [tap outputs]). Every conv
    carries its folded BatchNorm (_bn_scale of `model`'s calibration)."""

    def conv(h, w, b, *, name, **kw):
        w, b = _bn_scale(scales, model, name, w, b)
        return pb.conv(h, w, b, name=name, **kw)

    c_in = 3
    y = conv(x, synth.he_normal(seed, ids(), (16, c_in, 3, 3)), _bias(seed, ids, 16), stride=2, pad=1,
             act="hardswish", name=f"{name}.stem")
    c_in = 16
    taps = []
    for bi, (k, exp, out, se, act, s) in enumerate(MBV3_SMALL):
        bname = f"{name}.b{bi}"
        h = y
        if exp != c_in:
            h = conv(h, synth.he_normal(seed, ids(), (exp, c_in, 1, 1)), _bias(seed, ids, exp), stride=1, pad=0,
                     act=act, name=f"{bname}.expand")
        h = conv(h, synth.he_normal(seed, ids(), (exp, 1, k, k)), _bias(seed, ids, exp), stride=s, pad=k // 2,
                 group=exp, act=act, name=f"{bname}.dw")
        if se:
            r = _make_divisible(exp // 4)
            w1 = synth.he_normal(seed, ids(), (r, exp, 1, 1))
            w2 = synth.he_normal(seed, ids(), (exp, r, 1, 1))
            gate = pb.channel_gate(h, w1, _bias(seed, ids, r), w2, _bias(seed, ids, exp), act1="relu", hard=True,
                                   alpha=1.0 / 6.0, beta=0.5, name=f"{bname}.se")
            h = pb.mul(h, gate, name=f"{bname}.se_scale")
        residual = y if (s == 1 and c_in == out) else None
        y = conv(h, synth.he_normal(seed, ids(), (out, exp, 1, 1)), _bias(seed, ids, out), stride=1, pad=0,
                 act="none", add=residual, name=f"{bname}.project")
        c_in = out
        if bi in MBV3_TAPS:
            taps.append(y)
    return y, taps


def mobilenetv3_small(seed: int = 3, n=1, size=640, scales=None, input_id=10_000):
    """Config 3: the MobileNetV3-small block stack at 3 x size x size, input ~ N(0,1), He-normal
    weights with folded BatchNorms (scales: see _bn_scale; {} = the plain He-normal weights). The input
    is tensor `input_id` of the seed: the default one is the calibration image, others are held out."""
    pb = PlanBuilder()
    ids = _Ids()
    x = pb.input((n, 3, size, size), NHWC, "image")
    y, _ = mobilenetv3_backbone(pb, x, seed, ids, model="mbv3", scales=scales)
    plan = pb.build(y)
    xin = synth.normal(seed, input_id, (n, size, size, 3), 1.0)
    return plan, [xin]


def dbnet(seed: int = 4, n=1, size=960, scales=None, logit=False, input_id=10_000):
    """Config 4: DBNet-style detector - MobileNetV3-small backbone, 4-level FPN (1x1 laterals to 96,
    nearest x2 + add top-down, 3x3 convs 96->24 per level, upsample + concat to 96 at 1/4 scale), head
    conv3x3 + BN + ReLU, ConvT 2x2 s2 + BN + ReLU, ConvT 2x2 s2 + bias + Sigmoid -> 1 x size x size.
    The BatchNormalization after the first ConvTranspose is not foldable (OnnxRewrites.cs:78-82) and
    lowers to per-channel Mul + Add(+ReLU) (GraphCompiler.cs:1898-1923). He-normal weights with the
    folded BatchNorms of every other conv (scales: see _bn_scale; {} = the plain He-normal weights);
    logit=True ends at the logit (no sigmoid), for calibration. The input is tensor `input_id` of the
    seed: the default one is the calibration image, others are held out."""
    pb = PlanBuilder()
    ids = _Ids()
    x = pb.input((n, 3, size, size), NHWC, "image")
    _, (c2, c3, c4, c5) = mobilenetv3_backbone(pb, x, seed, ids, model="dbnet", scales=scales)
    chans = [pb.values[v].phys[3] for v in (c2, c3, c4, c5)]
    oc = 96

    def conv(h, w, b, *, name, **kw):
        w, b = _bn_scale(scales, "dbnet", name, w, b)
        return pb.conv(h, w, b, name=name, **kw)

    def convt(h, w, b, *, name, **kw):
        w, b = _bn_scale(scales, "dbnet", name, w, b, transpose=True)
        return pb.conv_transpose(h, w, b, name=name, **kw)

    lat = [conv(v, synth.he_normal(seed, ids(), (oc, c, 1, 1)), None, stride=1, pad=0, name=f"fpn.lat{i}")
           for i, (v, c) in enumerate(zip((c2, c3, c4, c5), chans))]
    in2, in3, in4, in5 = lat
    out4 = pb.resize_nearest(in5, 2, add=in4, name="fpn.up5")
    out3 = pb.resize_nearest(out4, 2, add=in3, name="fpn.up4")
    out2 = pb.resize_nearest(out3, 2, add=in2, name="fpn.up3")
    q = oc // 4
    p5 = conv(in5, synth.he_normal(seed, ids(), (q, oc, 3, 3)), None, pad=1, name="fpn.p5")
    p4 = conv(out4, synth.he_normal(seed, ids(), (q, oc, 3, 3)), None, pad=1, name="fpn.p4")
    p3 = conv(out3, synth.he_normal(seed, ids(), (q, oc, 3, 3)), None, pad=1, name="fpn.p3")
    p2 = conv(out2, synth.he_normal(seed, ids(), (q, oc, 3, 3)), None, pad=1, name="fpn.p2")
    p5 = pb.resize_nearest(p5, 8, name="fpn.p5_up")
    p4 = pb.resize_nearest(p4, 4, name="fpn.p4_up")
    p3 = pb.resize_nearest(p3, 2, name="fpn.p3_up")
    fuse = pb.concat_channels([p5, p4, p3, p2], name="fpn.concat")
    h = conv(fuse, synth.he_normal(seed, ids(), (q, oc, 3, 3)), _bias(seed, ids, q), pad=1, act="relu",
             name="head.conv")
    h = convt(h, synth.he_normal(seed, ids(), (q, q, 2, 2)), _bias(seed, ids, q), name="head.convt1")
    bn_s = pb.const(synth.uniform(seed, ids(), (q, 1, 1), 0.5, 1.5), "head.bn_scale")
    bn_t = pb.const(synth.uniform(seed, ids(), (q, 1, 1), -0.1, 0.1), "head.bn_shift")
    h = pb.ew(h, bn_s, 2, name="head.bn_mul")
    h = pb.ew(h, bn_t, 0, act="relu", name="head.bn_add")
    y = convt(h, synth.he_normal(seed, ids(), (q, 1, 2, 2)), _bias(seed, ids, 1), act="none" if logit else "sigmoid",
              name="head.convt2")
    plan = pb.build(y)
    xin = synth.normal(seed, input_id, (n, size, size, 3), 1.0)
    return plan, [xin]


def svtr(seed: int = 5, n=32, h=48, w=320, dim=192, heads=6, depth=8, mlp=4, classes=6625, head="softmax"):
    """Config 5: SVTR/CRNN-style recognizer. Stem: two conv3x3 s2 + BN(folded) + GELU (3->32->64);
    the 64 x 12 x 80 map collapses its height with a 12x1 conv to dim (80 tokens x 192); 8 mixer
    blocks x = x + proj(attn(LN(x))), x = x + fc2(GELU(fc1(LN(x)))); final LN; linear head to
    `classes` + softmax. Weights ~ N(0, 0.02) for the mixer / head Gemms (He-normal for convs).
    head="features": the plan ends at the final LayerNorm (the [n*80, dim] features a CTC head reads)
    and the head's (weights [dim, classes], bias) come back as a third item."""
    pb = PlanBuilder()
    ids = _Ids()
    x = pb.input((n, 3, h, w), NHWC, "image")
    y = pb.conv(x, synth.he_normal(seed, ids(), (32, 3, 3, 3)), _bias(seed, ids, 32), stride=2, pad=1, act="gelu",
                name="stem.conv1")
    y = pb.conv(y, synth.he_normal(seed, ids(), (64, 32, 3, 3)), _bias(seed, ids, 64), stride=2, pad=1, act="gelu",
                name="stem.conv2")
    _, hh, ww, _ = pb.values[y].phys
    y = pb.conv(y, synth.he_normal(seed, ids(), (dim, 64, hh, 1)), _bias(seed, ids, dim), stride=1, pad=0,
                name="stem.collapse")  # [n, 1, ww, dim] NHWC == [n, ww, dim] tokens
    t = ww
    tok = pb.alias(y, (n, t, dim), None, "tokens")

    def lin(v, k, nout, act="none", name=""):
        return pb.gemm(v, synth.normal(seed, ids(), (k, nout), 0.02), _bias(seed, ids, nout), act=act, name=name)

    def ln(v, name):
        return pb.layer_norm(v, 1.0 + synth.uniform(seed, ids(), (dim,), -0.1, 0.1),
                             synth.uniform(seed, ids(), (dim,), -0.1, 0.1), 1e-6, name=name)

    d = dim // heads
    for b in range(depth):
        hn = ln(tok, f"blk{b}.ln1")
        qkv = lin(hn, dim, 3 * dim, name=f"blk{b}.qkv")
        att = pb.attention(qkv, heads, d, d ** -0.5, name=f"blk{b}.attn")
        proj = lin(att, dim, dim, name=f"blk{b}.proj")
        tok = pb.add(tok, proj, name=f"blk{b}.res1")
        hn = ln(tok, f"blk{b}.ln2")
        f1 = lin(hn, dim, dim * mlp, act="gelu", name=f"blk{b}.fc1")
        f2 = lin(f1, dim * mlp, dim, name=f"blk{b}.fc2")
        tok = pb.add(tok, f2, name=f"blk{b}.res2")
    tok = ln(tok, "norm")
    xin = synth.normal(seed, 10_000, (n, h, w, 3), 1.0)
    if head == "features":
        hw = synth.normal(seed, ids(), (dim, classes), 0.02)
        hb = _bias(seed, ids, classes)
        return pb.build(tok), [xin], (hw, hb)
    logits = lin(tok, dim, classes, name="head")
    y = pb.softmax(logits, name="softmax")
    plan = pb.build(y)
    return plan, [xin]


def plan_flops(plan) -> int:
    """Algorithmic FLOPs of a plan: 2*MACs of every conv / Gemm / ConvT / attention (epilogues ignored)."""
    total = 0
    for nd in plan.nodes:
        v = plan.values
        if nd.op == "Conv":
            w = v[nd.ins[1]].shape
            out = v[nd.outs[0]].phys
            if nd.p.pool is not None:
                out = (out[0], out[1] * 2, out[2] * 2, out[3])
            total += 2 * out[0] * out[1] * out[2] * out[3] * w[1] * w[2] * w[3]
        elif nd.op == "Gemm":
            k = v[nd.ins[0]].shape[-1]
            total += 2 * v[nd.outs[0]].count * k
        elif nd.op == "ConvTranspose":
            total += 2 * v[nd.outs[0]].count * v[nd.ins[1]].shape[0]
        elif nd.op == "Attention":
            nb, hh, t, dd = v[nd.outs[0]].shape
            total += 4 * nb * hh * t * t * dd
    return total


def node_cost(plan, node, es: int = 2):
    """Algorithmic (flops, bytes) of one node: 2*MACs, and every tensor it reads or writes counted
    once at its storage size (activations and weights `es` bytes; bias, LayerNorm and SE parameters
    fp32, ConstKind.F32)."""
    v = plan.values
    p = node.p
    f32_ids = set()
    if node.op in ("Conv", "Gemm", "ConvTranspose") and p.bias >= 0:
        f32_ids.add(p.bias)
    if node.op == "LayerNorm":
        f32_ids.update(node.ins[1:])
    if node.op == "ChannelGate":
        f32_ids.update(node.ins[1:])
        f32_ids.update(r for r in (p.b1, p.b2) if r >= 0)
    reads = list(dict.fromkeys(list(node.ins) + node.param_refs()))
    by = sum(v[i].count * (4 if i in f32_ids else es) for i in reads)
    by += sum(v[i].count * es for i in node.outs)
    fl = 0
    if node.op == "Conv":
        w = v[node.ins[1]].shape
        out = v[node.outs[0]].phys
        if p.pool is not None:
            out = (out[0], out[1] * 2, out[2] * 2, out[3])
        fl = 2 * out[0] * out[1] * out[2] * out[3] * w[1] * w[2] * w[3]
    elif node.op == "Gemm":
        fl = 2 * v[node.outs[0]].count * v[node.ins[0]].shape[-1]
    elif node.op == "ConvTranspose":
        fl = 2 * v[node.outs[0]].count * v[node.ins[1]].shape[0]
    elif node.op == "Attention":
        nb, hh, t, dd = v[node.outs[0]].shape
        fl = 4 * nb * hh * t * t * dd
        by = 4 * v[node.outs[0]].count * es  # q, k and v read once, output written once
    return fl, by
