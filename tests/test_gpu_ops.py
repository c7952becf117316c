"""HIP kernels for the rest of the ExecOp surface vs the CPU oracle (the GpuOpTests pattern,
tests/Sdcb.SimdOnnx.Tests/GpuOpTests.cs): bilinear resize (+relu, +addend), pad, transpose,
slice, LeakyRelu / Tanh / Clip / Erf, DepthToSpace / SpaceToDepth, average pool, global average
pool and batched MatMul, each as a one-node plan through HipBackend -> HipGraphModel ->
HipInferenceSession (include/sox_backend.h).

Bars: index / copy ops (pad, transpose, slice, depth-space) are bit-exact in both storage modes;
arithmetic ops meet max-rel 1e-4 with fp32 storage and 2e-3 with fp16 storage (operands rounded to
fp16 on both sides, fp32 math, one rounding of the output).
"""
import numpy as np
import pytest

import oracle as O
from simdonnx_amd import synth
from simdonnx_amd.backend import HipInferenceSession
from simdonnx_amd.plan import NHWC, PlanBuilder
from tests.conftest import max_rel

pytestmark = pytest.mark.gpu
TOL = {False: 1e-4, True: 2e-3}
HALF = pytest.mark.parametrize("half", [False, True], ids=["f32", "f16"])


def f16(a):
    return np.asarray(a, np.float32).astype(np.float16).astype(np.float32)


def run(hip, plan, inputs, half, kernel_prefix):
    print(f"[gpu] {plan.nodes[-1].op} f16={half} shapes={[np.shape(x) for x in inputs]}", flush=True)
    g = hip.graph(plan, half)
    names = [d[0] for d in g.dispatches]
    assert names and all(n.startswith(kernel_prefix) for n in names if n != "gap_part"), names
    with HipInferenceSession(g) as s:
        for i, x in enumerate(inputs):
            s.set_input(x, i)
        return s.run().copy()


def img(seed, shape, half):
    x = synth.normal(seed, 1, shape, 1.0)
    return f16(x) if half else x


@HALF
@pytest.mark.parametrize("n,h,w,c,scale,relu,addend,add_relu", [
    (1, 7, 9, 8, 2, False, False, False), (2, 5, 6, 3, 3, True, False, False), (1, 30, 40, 96, 2, True, True, True),
    (1, 120, 120, 24, 2, False, True, False), (1, 16, 12, 16, 0.5, False, False, False)])
def test_resize_bilinear(hip, n, h, w, c, scale, relu, addend, add_relu, half):
    x = img(1, (n, h, w, c), half)
    oh, ow = int(h * scale), int(w * scale)
    pb = PlanBuilder()
    xv = pb.input((n, c, h, w), NHWC, "x")
    ins, av, a = [x], None, None
    if addend:
        a = img(2, (n, oh, ow, c), half)
        av = pb.input((n, c, oh, ow), NHWC, "a")
        ins.append(a)
    y = pb.resize_bilinear(xv, scale, av, relu=relu, add_relu=add_relu, name="bil")
    got = run(hip, pb.build(y), ins, half, "bilinear")
    want = O.resize_bilinear(x, scale, scale, a, relu=relu, add_relu=add_relu)
    assert max_rel(got, want) < TOL[half]


@HALF
@pytest.mark.parametrize("shape,pads,mode,value", [
    ((1, 6, 7, 8), (1, 2, 0, 3), 0, 0.0), ((2, 5, 5, 3), (2, 1, 2, 1), 1, 0.0), ((1, 64, 48, 32), (3, 3, 3, 3), 1, 0.0),
    ((1, 9, 4, 16), (0, 3, 3, 0), 0, -1.5)])
def test_pad(hip, shape, pads, mode, value, half):
    n, h, w, c = shape
    x = img(3, shape, half)
    t, l, b, r = pads
    pb = PlanBuilder()
    xv = pb.input((n, c, h, w), NHWC, "x")
    y = pb.pad(xv, (0, 0, t, l, 0, 0, b, r), mode, value, name="pad")
    got = run(hip, pb.build(y), [x], half, "pad")
    assert np.array_equal(got, O.pad_nhwc(x, t, l, b, r, mode, value))


@HALF
@pytest.mark.parametrize("shape,perm", [((2, 13, 11, 40), (0, 3, 1, 2)), ((4, 80, 6, 32), (0, 2, 1, 3)),
                                        ((3, 5, 7), (2, 0, 1)), ((2, 3, 4, 5, 6, 7), (5, 3, 1, 0, 2, 4)),
                                        ((4, 80, 33), (0, 2, 1)), ((2, 24, 70, 65), (0, 2, 3, 1))])
def test_transpose(hip, shape, perm, half):
    """Swaps of two contiguous dim groups run the LDS-tiled 2D transpose, other perms the gather."""
    x = img(4, shape, half)
    pb = PlanBuilder()
    xv = pb.input(shape, None, "x")
    y = pb.transpose(xv, perm, name="tr")
    got = run(hip, pb.build(y), [x], half, "transpose")
    assert np.array_equal(got.reshape(-1), O.transpose(x, perm).reshape(-1))


@HALF
@pytest.mark.parametrize("shape,starts,ends,axes,steps", [
    ((2, 13, 11, 40), (1, 10, 3), (12, 2, 40), (1, 2, 3), (2, -3, 5)),
    ((4, 80, 576), (192,), (384,), (2,), (1,)), ((6, 9), (8,), (-1,), (1,), (-1,))])
def test_slice(hip, shape, starts, ends, axes, steps, half):
    x = img(5, shape, half)
    pb = PlanBuilder()
    xv = pb.input(shape, None, "x")
    y = pb.slice(xv, starts, ends, axes, steps, name="sl")
    got = run(hip, pb.build(y), [x], half, "slice")
    want = O.slice_(x, starts, ends, axes, steps)
    assert got.size == want.size and np.array_equal(got.reshape(-1), want.reshape(-1))


@HALF
@pytest.mark.parametrize("op,a,b", [("LeakyRelu", 0.1, 0.0), ("LeakyRelu", 2.0, 0.0), ("Tanh", 1.0, 1.0),
                                    ("Tanh", 2.0 / 3.0, 1.7159), ("Clip", -1.0, 0.75), ("Erf", 0.0, 0.0)])
def test_unary2(hip, op, a, b, half):
    x = synth.normal(6, 1, (3, 1001), 2.5)
    x = f16(x) if half else x
    pb = PlanBuilder()
    xv = pb.input(x.shape, None, "x")
    y = pb.scalar_act(op, xv, a, b, name="u")
    got = run(hip, pb.build(y), [x], half, "unary2")
    want = O.unary2(x, op, a, b)
    assert max_rel(got, want) < (TOL[half] if op in ("Tanh", "Erf") or half else 1e-6)


@HALF
@pytest.mark.parametrize("shape,block,crd,inverse", [
    ((1, 3, 4, 8), 2, True, False), ((2, 2, 3, 27), 3, False, False), ((1, 60, 60, 64), 2, False, False),
    ((1, 6, 8, 3), 2, True, True), ((2, 6, 9, 4), 3, False, True), ((1, 120, 120, 16), 2, True, True),
    ((1, 12, 12, 16), 2, False, True)])
def test_depth_space(hip, shape, block, crd, inverse, half):
    n, h, w, c = shape
    x = img(7, shape, half)
    pb = PlanBuilder()
    xv = pb.input((n, c, h, w), NHWC, "x")
    y = pb.depth_to_space(xv, block, crd, inverse, name="d2s")
    got = run(hip, pb.build(y), [x], half, "s2d" if inverse else "d2s")
    assert np.array_equal(got, O.depth_to_space(x, block, crd, inverse))


@HALF
@pytest.mark.parametrize("shape,k,s,pads,cip", [
    ((1, 9, 9, 8), 3, 2, (1, 1, 1, 1), False), ((2, 8, 10, 3), 2, 2, (0, 0, 0, 0), False),
    ((1, 11, 7, 16), 3, 1, (1, 1, 1, 1), True), ((1, 60, 60, 96), 5, 3, (2, 2, 2, 2), False)])
def test_avg_pool(hip, shape, k, s, pads, cip, half):
    n, h, w, c = shape
    x = img(8, shape, half)
    pb = PlanBuilder()
    xv = pb.input((n, c, h, w), NHWC, "x")
    y = pb.avg_pool(xv, (k, k), (s, s), pads, cip, name="avg")
    got = run(hip, pb.build(y), [x], half, "avgpool")
    assert max_rel(got, O.avg_pool(x, (k, k), (s, s), pads, cip)) < TOL[half]


@HALF
@pytest.mark.parametrize("shape", [(2, 13, 11, 40), (1, 240, 240, 16), (3, 7, 5, 3)])
def test_global_avg_pool(hip, shape, half):
    n, h, w, c = shape
    x = img(9, shape, half)
    pb = PlanBuilder()
    xv = pb.input((n, c, h, w), NHWC, "x")
    y = pb.global_avg_pool(xv, name="gap")
    got = run(hip, pb.build(y), [x], half, "gap_mean")
    assert max_rel(got.reshape(n, c), O.global_avg_pool(x)) < TOL[half]


@HALF
@pytest.mark.parametrize("batch,m,k,n,bcast", [(3, 17, 33, 21, False), (4, 80, 32, 80, True),
                                               (192, 80, 32, 80, False), (2, 300, 257, 130, True)])
def test_matmul(hip, batch, m, k, n, bcast, half):
    a = img(10, (batch, m, k), half)
    b = synth.normal(10, 2, (1 if bcast else batch, k, n), 0.2)
    b = f16(b) if half else b
    pb = PlanBuilder()
    av = pb.input(a.shape, None, "a")
    bv = pb.input(b.shape, None, "b")
    y = pb.matmul(av, bv, name="mm")
    got = run(hip, pb.build(y), [a, b], half, "matmul")
    assert max_rel(got, O.matmul_bcast(a, b)) < TOL[half]


@HALF
@pytest.mark.parametrize("shape,eps,lo,hi", [((2, 5, 7, 16), 1e-3, -4.0, 4.0), ((3, 1001), 1e-6, 0.0, 1.0)])
def test_safe_div(hip, shape, eps, lo, hi, half):
    a = img(11, shape, half)
    b = synth.uniform(11, 2, shape, -0.5, 2.0)
    b = f16(b) if half else b
    pb = PlanBuilder()
    av, bv = pb.input(shape, None, "a"), pb.input(shape, None, "b")
    y = pb.safe_div(av, bv, eps, lo, hi, name="sd")
    got = run(hip, pb.build(y), [a, b], half, "safediv")
    assert max_rel(got, O.safe_div(a, b, eps, lo, hi)) < TOL[half]


@HALF
@pytest.mark.parametrize("shape,axis,ends,offs", [((1, 6, 9, 20), 2, (4, 8, 12, 16, 20), (-2, -1, 0, 1, 2)),
                                                  ((2, 40, 40, 64), 3, (16, 32, 48, 56), (1, -1, 3, -3)),
                                                  ((1, 7, 5, 13), 3, (3, 9), (2, -1))])
def test_channel_shift(hip, shape, axis, ends, offs, half):
    n, h, w, c = shape
    x = img(12, shape, half)
    pb = PlanBuilder()
    xv = pb.input((n, c, h, w), NHWC, "x")
    y = pb.channel_shift(xv, axis, ends, offs, name="sh")
    got = run(hip, pb.build(y), [x], half, "shift")
    assert np.array_equal(got, O.channel_shift(x, axis, list(ends), list(offs)))


@HALF
@pytest.mark.parametrize("c,oc,act,skip_conv,hw", [(16, 1, "sigmoid", False, (12, 10)), (32, 2, "sigmoid", True, (12, 10)),
                                                   (96, 8, "relu", False, (30, 30)), (24, 1, "none", True, (60, 60))])
def test_up_head(hip, c, oc, act, skip_conv, hw, half):
    """UpHead with a stored skip and with the skip recomputed from its 3x3 conv's input (reflect pad in
    the last case)."""
    h, w = hw
    x = img(13, (1, h, w, c), half)
    wh = synth.normal(13, 3, (oc, c), 0.2)
    bh = synth.uniform(13, 4, (oc,), -0.1, 0.1)
    pb = PlanBuilder()
    xv = pb.input((1, c, h, w), NHWC, "x")
    if skip_conv:
        sk = img(14, (1, 2 * h, 2 * w, 3), half)
        w_sc = synth.normal(13, 5, (c, 3, 3, 3), 0.3)
        b_sc = synth.uniform(13, 6, (c,), -0.1, 0.1)
        mode = 1 if c == 24 else 0
        sv = pb.input((1, 3, 2 * h, 2 * w), NHWC, "skin")
        y = pb.up_head(xv, sv, wh, bh, 2, resize_relu=True, skip_relu=True, act=act,
                       skip_conv=(w_sc, b_sc, (1, 1, 1, 1), mode, 0.0, "relu"), name="uh")
        w_sc_r = f16(w_sc) if half else w_sc
        skip = O.conv(sk, w_sc_r, b_sc, None, stride=(1, 1), pads=(1, 1, 1, 1), act="relu", pad_mode=mode, algo=1)
    else:
        sk = img(14, (1, 2 * h, 2 * w, c), half)
        sv = pb.input((1, c, 2 * h, 2 * w), NHWC, "skip")
        y = pb.up_head(xv, sv, wh, bh, 2, resize_relu=True, skip_relu=True, act=act, name="uh")
        skip = sk
    got = run(hip, pb.build(y), [x, sk], half, "uphead")
    want = O.up_head(x, skip, f16(wh) if half else wh, bh, 2, resize_relu=True, skip_relu=True, act=act)
    assert max_rel(got, want) < TOL[half]


@HALF
@pytest.mark.parametrize("op", ["Relu", "Sigmoid", "Gelu", "HardSwish", "Swish", "HardSigmoid", "Copy"])
@pytest.mark.parametrize("shape", [(1, 17, 23, 24), (2, 5, 7, 3)], ids=["vec", "tail"])
def test_standalone_activation(hip, op, shape, half):
    """The activation ops that stay nodes of their own (not folded into a producer's epilogue),
    VkGraph.cs:495-553 (unary.comp / hsig.comp / copy): per element, fp32 math."""
    n, h, w, c = shape
    x = img(31, shape, half) * 4.0
    pb = PlanBuilder()
    xv = pb.input((n, c, h, w), NHWC, "x")
    if op == "HardSigmoid":
        y = pb.hard_sigmoid(xv, 0.25, 0.4, name="hsig")
    else:
        y = pb.unary(op, xv, name=op.lower())
    got = run(hip, pb.build(y), [x], half, "unary")
    if op == "Copy":
        assert np.array_equal(got, x)
        return
    want = O.hard_sigmoid(x, 0.25, 0.4) if op == "HardSigmoid" else O.activation(x, op.lower())
    assert max_rel(got, want) < TOL[half]


@HALF
@pytest.mark.parametrize("n,h,w,c,k,s,pads,relu", [
    (1, 32, 40, 16, 2, 2, (0, 0, 0, 0), False), (2, 15, 13, 24, 3, 2, (1, 1, 1, 1), True),
    (1, 9, 11, 3, 3, 1, (1, 1, 1, 1), False), (1, 12, 10, 8, 2, 2, (0, 0, 1, 1), True)])
def test_maxpool(hip, n, h, w, c, k, s, pads, relu, half):
    """MaxPool (+ the folded Relu, PoolP.FuseRelu) as its own node (maxpool.comp, VkGraph.cs:705-717):
    a max selects one of its inputs, so the result is bit-exact in both storage modes."""
    x = img(33, (n, h, w, c), half)
    pb = PlanBuilder()
    xv = pb.input((n, c, h, w), NHWC, "x")
    y = pb.max_pool(xv, (k, k), (s, s), pads, relu=relu, name="pool")
    got = run(hip, pb.build(y), [x], half, "maxpool")
    want = O.max_pool(x, (k, k), (s, s), pads, relu)
    assert got.shape == want.shape
    assert np.array_equal(got, f16(want) if half else want)


@HALF
@pytest.mark.parametrize("ic,oc,k,h,w,act,pool_relu", [
    (3, 16, 3, 64, 48, "relu", False), (3, 32, 3, 31, 40, "none", True), (4, 8, 3, 20, 18, "relu", True),
    (1, 16, 5, 24, 24, "none", False), (3, 64, 1, 16, 22, "relu", True)])
def test_conv_pool_fused(hip, ic, oc, k, h, w, act, pool_relu, half):
    """ConvP.Pool on a small-ic stem (the reference's GPU ConvPool, GraphCompiler.GpuSmallConv +
    VkGraph.cs:559-575; Nhwc.ConvPool, Kernels/Nhwc.cs:661-727): one dispatch that never stores the
    full-resolution conv, against the oracle's ConvPool. An odd conv height (31) floors the pool."""
    x = img(35, (1, h, w, ic), half)
    wt = synth.uniform(35, 2, (oc, ic, k, k), -0.5, 0.5)
    wt = f16(wt) if half else wt
    b = synth.uniform(35, 3, (oc,), -0.1, 0.1)
    pb = PlanBuilder()
    xv = pb.input((1, ic, h, w), NHWC, "x")
    y = pb.conv(xv, wt, b, stride=1, pad=k // 2, act=act, pool="relu" if pool_relu else True, name="stem")
    plan = pb.build(y)
    g = hip.graph(plan, half)
    names = [d[0] for d in g.dispatches]
    fused = ic % (8 if half else 4) != 0 and h % 2 == 0 and w % 2 == 0  # else conv to scratch + pool pass
    print(f"[gpu] convpool ic={ic} oc={oc} k={k} {h}x{w} f16={half} dispatches={names}", flush=True)
    if fused:
        assert names == ["convpool"], names
    with HipInferenceSession(g) as s:
        s.set_input(x)
        got = s.run().copy()
    want = O.conv(x, wt, b, stride=(1, 1), pads=(k // 2,) * 4, act=act, pool=True, pool_relu=pool_relu)
    assert got.shape == want.shape == (1, h // 2, w // 2, oc)
    assert max_rel(got, want) < TOL[half]
