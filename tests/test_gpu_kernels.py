"""HIP kernels vs the CPU oracle, one fused node at a time (the VkKernelTests / GpuOpTests pattern,
tests/Sdcb.SimdOnnx.Tests/VkKernelTests.cs:62-196, GpuOpTests.cs:17-325).

Every case builds a one-node ExecPlan, runs it through HipBackend -> HipGraphModel ->
HipInferenceSession (the C ABI of include/sox_backend.h) and compares with the oracle on the same
inputs. Tolerances, max-rel = max|gpu - cpu| / max|cpu|:
  fp32 storage: 1e-4;
  fp16 storage: operands pre-rounded to fp16 so both sides multiply identical values
  (VkKernelTests.cs:141-143), 2e-3 (fp32 accumulation, one fp16 rounding of the output).
"""
import os

import numpy as np
import pytest

import oracle as O
from simdonnx_amd import synth
from simdonnx_amd.backend import HipInferenceSession
from simdonnx_amd.plan import NHWC, PlanBuilder
from tests.conftest import max_rel

pytestmark = pytest.mark.gpu

G = np.load(os.path.join(os.path.dirname(__file__), "golden", "golden.npz"))
ACTS = ["none", "relu", "sigmoid", "gelu", "hardswish", "swish"]
TOL = {False: 1e-4, True: 2e-3}


def f16(a):
    return np.asarray(a, np.float32).astype(np.float16).astype(np.float32)


def run(hip, plan, inputs, f16_storage):
    print(f"[gpu] plan {len(plan.nodes)} nodes f16={f16_storage}", flush=True)
    with HipInferenceSession(hip.graph(plan, f16_storage)) as s:
        for i, x in enumerate(inputs):
            s.set_input(x, i)
        return s.run().copy()


def conv_plan(x, w, b, add, stride, pads, act, pad_mode, pad_value, group=1):
    pb = PlanBuilder()
    n, h, ww, c = x.shape
    xv = pb.input((n, c, h, ww), NHWC, "x")
    addv = None
    ins = [x]
    if add is not None:
        addv = pb.input((add.shape[0], add.shape[3], add.shape[1], add.shape[2]), NHWC, "add")
        ins.append(add)
    y = pb.conv(xv, w, b, stride=stride, pad=pads, group=group, act=act, add=addv, pad_mode=pad_mode,
                pad_value=pad_value, name="conv")
    return pb.build(y), ins


@pytest.mark.parametrize("half,path", [(False, "default"), (True, "default"), (True, "ring"), (True, "igemm")],
                         ids=["f32", "f16", "f16-ring", "f16-igemm"])
@pytest.mark.parametrize("i", range(int(G["conv_n"][0])))
def test_conv_matches_oracle(hip, i, half, path, monkeypatch):
    """Every golden conv case; fp16 through the default route (the direct kernel below 8 output
    channels, the LDS halo kernel for other 3x3 convs with few output channels, else the LDS-DMA implicit-GEMM ring when ic % 8 == 0), through the ring
    alone and through the register-staged implicit-GEMM kernel."""
    if path == "igemm":
        monkeypatch.setenv("SIMDONNX_HIP_IGEMM", "1")
    if path == "ring":
        monkeypatch.setenv("SIMDONNX_HIP_NOHALO", "1")
        monkeypatch.setenv("SIMDONNX_HIP_NONARROW", "1")
    ic, oc, k, s, h, w, mode, act, res = [int(v) for v in G[f"conv{i}_meta"]]
    pv = float(G[f"conv{i}_pv"][0])
    cv = f16 if half else (lambda a: a)
    x, wt, b = cv(G[f"conv{i}_x"]), cv(G[f"conv{i}_w"]), G[f"conv{i}_b"]
    add = cv(G[f"conv{i}_add"]) if res else None
    pads = (k // 2,) * 4
    plan, ins = conv_plan(x, wt, b, add, (s, s), pads, ACTS[act], mode, pv)
    got = run(hip, plan, ins, half)
    want = O.conv(x, wt, b, add, stride=(s, s), pads=pads, act=ACTS[act], pad_mode=mode, pad_value=pv)
    assert max_rel(got, want) < TOL[half]


@pytest.mark.parametrize("half", [False, True], ids=["f32", "f16"])
@pytest.mark.parametrize("case", [(3, 16, 2, 64, 40), (64, 128, 1, 33, 29), (32, 96, 2, 30, 22), (8, 64, 2, 21, 17),
                                  (128, 256, 1, 16, 16), (16, 160, 1, 24, 20), (64, 128, 1, 96, 96)])
def test_conv_shapes_batch(hip, case, half):
    """conv_cm route coverage (VkKernelTests.ConvCm_MatchesCpu shapes): stems, stride 2, wide oc, batch 2."""
    ic, oc, s, h, w = case
    cv = f16 if half else (lambda a: a)
    x = cv(synth.uniform(11, 1, (2, h, w, ic), -1, 1))
    wt = cv(synth.uniform(11, 2, (oc, ic, 3, 3), -0.25, 0.25))
    b = synth.uniform(11, 3, (oc,), -0.1, 0.1)
    plan, ins = conv_plan(x, wt, b, None, (s, s), (1, 1, 1, 1), "relu", 0, 0.0)
    got = run(hip, plan, ins, half)
    want = O.conv(x, wt, b, stride=(s, s), pads=(1, 1, 1, 1), act="relu")
    assert max_rel(got, want) < TOL[half]


@pytest.mark.parametrize("half", [False, True], ids=["f32", "f16"])
@pytest.mark.parametrize("i", range(int(G["gemm_n"][0])))
def test_gemm_matches_oracle(hip, i, half):
    m, k, n, tb, act = [int(v) for v in G[f"gemm{i}_meta"]]
    cv = f16 if half else (lambda a: a)
    a, bm, bias = cv(G[f"gemm{i}_a"]), cv(G[f"gemm{i}_b"]), G[f"gemm{i}_bias"]
    pb = PlanBuilder()
    av = pb.input((m, k), None, "a")
    y = pb.gemm(av, bm, bias, act=ACTS[act], trans_b=bool(tb), name="gemm")
    got = run(hip, pb.build(y), [a], half)
    want = O.gemm(a, bm, bias, trans_b=bool(tb), act=ACTS[act])
    assert max_rel(got, want) < TOL[half]


@pytest.mark.parametrize("half", [False, True], ids=["f32", "f16"])
@pytest.mark.parametrize("i", range(int(G["dw_n"][0])))
def test_depthwise_matches_oracle(hip, i, half):
    c, k, s, h, w, mode, act = [int(v) for v in G[f"dw{i}_meta"]]
    cv = f16 if half else (lambda a: a)
    x, wt, b = cv(G[f"dw{i}_x"]), cv(G[f"dw{i}_w"]), G[f"dw{i}_b"]
    plan, ins = conv_plan(x, wt, b, None, (s, s), (k // 2,) * 4, ACTS[act], mode, 0.0, group=c)
    got = run(hip, plan, ins, half)
    want = O.conv(x, wt, b, stride=(s, s), pads=(k // 2,) * 4, group=c, act=ACTS[act], pad_mode=mode)
    assert max_rel(got, want) < TOL[half]


DW_TILE_CASES = [  # (c, k, s, h, w, pad_mode, act, residual)
    (64, 3, 1, 16, 16, 0, "relu", False), (72, 3, 2, 240, 240, 0, "relu", False), (88, 3, 1, 37, 53, 1, "none", True),
    (96, 5, 2, 120, 120, 0, "hardswish", False), (240, 5, 1, 60, 60, 0, "hardswish", False),
    (16, 3, 2, 33, 17, 1, "relu", False), (576, 5, 1, 30, 30, 0, "hardswish", True), (120, 5, 2, 9, 23, 1, "swish", False)]


@pytest.mark.parametrize("rows", [8, 4], ids=["8x8", "4x8"])
@pytest.mark.parametrize("storage", ["f16", "bf16", "f32"])
@pytest.mark.parametrize("case", DW_TILE_CASES, ids=[f"c{c[0]}k{c[1]}s{c[2]}_{c[3]}x{c[4]}" for c in DW_TILE_CASES])
def test_depthwise_tiles_match_per_pixel_kernel(hip, case, storage, rows, monkeypatch):
    """The LDS-tile depthwise kernels (sox_dwt_*: 8 x 8 and 4 x 8 tiles, channel tails, reflect
    padding, residual, ragged tiles) give the per-pixel kernel's bits (same fma order per output) and
    meet the oracle."""
    monkeypatch.setenv("SIMDONNX_HIP_DWT_ROWS", str(rows))
    c, k, s, h, w, mode, act, res = case
    from oracle.interp import _bf16
    rnd = {"f16": f16, "bf16": _bf16, "f32": lambda a: a}[storage]
    x = rnd(synth.uniform(41, 1, (1, h, w, c), -1, 1))
    wt = rnd(synth.uniform(41, 2, (c, 1, k, k), -0.5, 0.5))
    b = synth.uniform(41, 3, (c,), -0.1, 0.1)
    oh, ow = (h + 2 * (k // 2) - k) // s + 1, (w + 2 * (k // 2) - k) // s + 1
    add = rnd(synth.uniform(41, 4, (1, oh, ow, c), -1, 1)) if res else None
    plan, ins = conv_plan(x, wt, b, add, (s, s), (k // 2,) * 4, act, mode, 0.0, group=c)
    g = hip.graph(plan, storage)
    assert g.kernels == [f"sox_dwt_{storage}_k{k}s{s}" + ("_h4" if rows == 4 else "")], g.kernels
    g.release()
    tiled = run(hip, plan, ins, storage)
    monkeypatch.setenv("SIMDONNX_HIP_DW_DIRECT", "1")
    g = hip.graph(plan, storage)
    assert g.kernels[0].startswith(f"sox_dw_{storage}_v"), g.kernels
    g.release()
    direct = run(hip, plan, ins, storage)
    assert np.array_equal(tiled, direct)
    want = O.conv(x, wt, b, add, stride=(s, s), pads=(k // 2,) * 4, group=c, act=act, pad_mode=mode)
    assert max_rel(tiled, want) < {"f16": 2e-3, "bf16": 4e-3, "f32": 1e-4}[storage]


STEM_CASES = [  # (oc, stride, h, w, pad_mode, act, residual)
    (16, 2, 97, 131, 0, "relu", False), (32, 2, 48, 320, 0, "gelu", False), (16, 1, 37, 23, 1, "hardswish", True),
    (8, 2, 33, 17, 1, "none", False), (24, 1, 40, 48, 0, "swish", False)]


@pytest.mark.parametrize("storage", ["f16", "bf16"])
@pytest.mark.parametrize("case", STEM_CASES, ids=[f"oc{c[0]}s{c[1]}_{c[2]}x{c[3]}" for c in STEM_CASES])
def test_rgb_stem_on_matrix_cores(hip, case, storage, monkeypatch):
    """3x3 convs over 3 channels in 16-bit graphs take the tiled matrix-core stem (sox_conv_stem_*:
    ragged 16 x 16 tiles, stride 1 / 2, zero and reflect padding, residual, oc below one 32-channel
    block) and meet the oracle, as the per-pixel fp32-FMA kernel (SIMDONNX_HIP_STEM_DIRECT) does; the two
    differ only by summation order."""
    oc, st, h, w, mode, act, res = case
    from oracle.interp import _bf16
    rnd = {"f16": f16, "bf16": _bf16}[storage]
    x = rnd(synth.uniform(44, 1, (1, h, w, 3), -1, 1))
    wt = rnd(synth.uniform(44, 2, (oc, 3, 3, 3), -0.5, 0.5))
    b = synth.uniform(44, 3, (oc,), -0.1, 0.1)
    oh, ow = (h + 2 - 3) // st + 1, (w + 2 - 3) // st + 1
    add = rnd(synth.uniform(44, 4, (1, oh, ow, oc), -1, 1)) if res else None
    plan, ins = conv_plan(x, wt, b, add, (st, st), (1, 1, 1, 1), act, mode, 0.0)
    g = hip.graph(plan, storage)
    assert g.kernels == [f"sox_conv_stem_s{st}_{storage}"], g.kernels
    g.release()
    tiled = run(hip, plan, ins, storage)
    monkeypatch.setenv("SIMDONNX_HIP_STEM_DIRECT", "1")
    g = hip.graph(plan, storage)
    assert g.kernels == [f"sox_conv_direct_333_{storage}"], g.kernels
    g.release()
    direct = run(hip, plan, ins, storage)
    want = O.conv(x, wt, b, add, stride=(st, st), pads=(1, 1, 1, 1), act=act, pad_mode=mode)
    tol = {"f16": 2e-3, "bf16": 8e-3}[storage]
    assert max_rel(tiled, want) < tol and max_rel(direct, want) < tol
    assert max_rel(tiled, direct) < tol


@pytest.mark.parametrize("storage", ["f16", "bf16", "f32"])
@pytest.mark.parametrize("case", [(240, 5, 1, 60, 60), (96, 5, 2, 120, 120), (576, 5, 1, 30, 30), (72, 3, 1, 44, 36),
                                  (16, 3, 2, 480, 480), (24, 3, 1, 100, 92), (16, 3, 1, 100, 92)])
def test_se_gap_partials_from_depthwise(hip, case, storage, monkeypatch):
    """Depthwise conv -> SE gate -> x * gate -> 1x1 projection (the MobileNetV3 block tail): the
    depthwise tiles write the gate's GAP partials (no gap_part dispatch), agreeing with the separate
    GAP pass (SIMDONNX_HIP_NO_DW_GAP) to fp32 summation order and with the oracle on the plan."""
    from oracle.interp import run_plan
    c, k, s, h, w = case
    r = max(8, (c // 4 + 4) // 8 * 8)
    pb = PlanBuilder()
    xv = pb.input((1, c, h, w), NHWC, "x")
    d = pb.conv(xv, synth.uniform(42, 1, (c, 1, k, k), -0.5, 0.5), synth.uniform(42, 2, (c,), -0.1, 0.1),
                stride=(s, s), pad=(k // 2,) * 4, group=c, act="hardswish", name="dw")
    gate = pb.channel_gate(d, synth.uniform(42, 3, (r, c, 1, 1), -0.3, 0.3), synth.uniform(42, 4, (r,), -0.1, 0.1),
                           synth.uniform(42, 5, (c, r, 1, 1), -0.3, 0.3), synth.uniform(42, 6, (c,), -0.1, 0.1),
                           act1="relu", hard=True, alpha=1.0 / 6.0, beta=0.5, name="se")
    m = pb.mul(d, gate, name="se_scale")
    y = pb.conv(m, synth.uniform(42, 7, (48, c, 1, 1), -0.2, 0.2), synth.uniform(42, 8, (48,), -0.1, 0.1),
                name="project")
    plan = pb.build(y)
    x = synth.uniform(42, 9, (1, h, w, c), -1, 1)
    g = hip.graph(plan, storage)
    names = [t[0] for t in g.dispatches]
    assert "gap_part" not in names and names[0] in ("depthwise", "depthwise_se"), names
    g.release()
    fused = run(hip, plan, [x], storage)
    monkeypatch.setenv("SIMDONNX_HIP_NO_DW_GAP", "1")
    g = hip.graph(plan, storage)
    assert "gap_part" in [t[0] for t in g.dispatches]
    g.release()
    sep = run(hip, plan, [x], storage)
    assert max_rel(fused, sep) < {"f16": 2e-3, "bf16": 1e-2, "f32": 1e-5}[storage]
    emu = {"f16": True, "bf16": "bf16", "f32": False}[storage]  # the storage contract
    want = run_plan(plan, [x], f16_storage=emu)
    assert max_rel(fused, want) < (1e-4 if storage == "f32" else 2e-2)


@pytest.mark.parametrize("half,path", [(False, "direct"), (True, "gemm"), (True, "direct")],
                         ids=["f32", "f16-gemm", "f16-direct"])
@pytest.mark.parametrize("i", range(int(G["ct_n"][0])))
def test_conv_transpose_matches_oracle(hip, i, half, path, monkeypatch):
    if path == "direct":
        monkeypatch.setenv("SIMDONNX_HIP_CONVT_DIRECT", "1")
    ic, oc, k, h, w, act = [int(v) for v in G[f"ct{i}_meta"]]
    cv = f16 if half else (lambda a: a)
    x, wt, b = cv(G[f"ct{i}_x"]), cv(G[f"ct{i}_w"]), G[f"ct{i}_b"]
    pb = PlanBuilder()
    xv = pb.input((1, ic, h, w), NHWC, "x")
    y = pb.conv_transpose(xv, wt, b, act=ACTS[act], name="convt")
    got = run(hip, pb.build(y), [x], half)
    want = O.conv_transpose(x, wt, b, act=ACTS[act])
    assert max_rel(got, want) < TOL[half]


# (batch, ic, oc, k, h, w, act): ConvTranspose (stride == kernel) shapes beyond the fixtures; oc = 1 with
# a 2x2 or 1x1 kernel takes the one-channel pixel kernel (the DB head's probability map)
CONVT_SHAPES = [(2, 32, 16, 3, 7, 5, "relu"), (1, 16, 5, 2, 33, 17, "sigmoid"), (1, 64, 96, 2, 13, 11, "none"),
                (1, 24, 1, 2, 45, 31, "sigmoid"), (2, 16, 1, 1, 9, 14, "relu"), (1, 8, 1, 3, 5, 6, "none")]


@pytest.mark.parametrize("half", [False, True], ids=["f32", "f16"])
@pytest.mark.parametrize("case", CONVT_SHAPES, ids=lambda c: "x".join(str(v) for v in c))
def test_conv_transpose_shapes(hip, case, half):
    n, ic, oc, k, h, w, act = case
    cv = f16 if half else (lambda a: a)
    x = cv(synth.uniform(12, 1, (n, h, w, ic), -1, 1))
    wt = cv(synth.normal(12, 2, (ic, oc, k, k), 0.2))
    b = synth.uniform(12, 3, (oc,), -0.2, 0.2)
    pb = PlanBuilder()
    xv = pb.input((n, ic, h, w), NHWC, "x")
    y = pb.conv_transpose(xv, wt, b, act=act, name="convt")
    got = run(hip, pb.build(y), [x], half)
    assert max_rel(got, O.conv_transpose(x, wt, b, act=act)) < TOL[half]


@pytest.mark.parametrize("half", [False, True], ids=["f32", "f16"])
def test_conv_transpose_then_channel_affine(hip, half):
    """ConvTranspose -> per-channel Mul -> per-channel Add + ReLU (an unfolded BatchNormalization)."""
    cv = f16 if half else (lambda a: a)
    ic, oc, h, w = 24, 24, 15, 13
    x = cv(synth.uniform(13, 1, (1, h, w, ic), -1, 1))
    wt = cv(synth.normal(13, 2, (ic, oc, 2, 2), 0.2))
    b = synth.uniform(13, 3, (oc,), -0.2, 0.2)
    s_, t_ = synth.uniform(13, 4, (oc, 1, 1), 0.5, 1.5), synth.uniform(13, 5, (oc, 1, 1), -0.3, 0.3)
    pb = PlanBuilder()
    xv = pb.input((1, ic, h, w), NHWC, "x")
    hv = pb.conv_transpose(xv, wt, b, name="convt")
    hv = pb.ew(hv, pb.const(s_, "bn_scale"), 2, name="bn_mul")
    y = pb.ew(hv, pb.const(t_, "bn_shift"), 0, act="relu", name="bn_add")
    got = run(hip, pb.build(y), [x], half)
    ref = O.conv_transpose(x, wt, b)
    if half:
        ref = f16(ref)
    want = np.maximum(ref * s_.reshape(-1) + t_.reshape(-1), 0.0)
    assert max_rel(got, want) < TOL[half]


@pytest.mark.parametrize("half", [False, True], ids=["f32", "f16"])
def test_se_block_matches_oracle(hip, half):
    """ChannelGate + broadcast multiply (the fused SE of GraphCompiler.cs:355, VkGraph.cs:547-551)."""
    cv = f16 if half else (lambda a: a)
    x = cv(G["se_x"])
    n, h, w, c = x.shape
    pb = PlanBuilder()
    xv = pb.input((n, c, h, w), NHWC, "x")
    gate = pb.channel_gate(xv, G["se_w1"], G["se_b1"], G["se_w2"], G["se_b2"], name="se")
    y = pb.mul(xv, gate, name="scale")
    got = run(hip, pb.build(y), [x], half)
    s = O.channel_gate(x, G["se_w1"], G["se_b1"], G["se_w2"], G["se_b2"])
    want = x * s[:, None, None, :]
    assert max_rel(got, want) < TOL[half]


# (n, h, w, c, shifts, oc): sources of c channels at (h >> s, w >> s), each upsampled (nearest) by 2^s,
# concatenated, then a 3x3 conv (+ bias, relu): the DB FPN's fuse conv at its full size and smaller
UPCAT_CASES = [(1, 240, 240, 24, (3, 2, 1, 0), 24), (1, 64, 64, 24, (3, 2, 1, 0), 24), (2, 48, 40, 16, (0, 1, 2), 40),
               (1, 36, 20, 32, (2, 2), 8)]


@pytest.mark.parametrize("storage", ["f16", "bf16"])
@pytest.mark.parametrize("case", UPCAT_CASES, ids=lambda c: "x".join(str(v) for v in c))
def test_conv_gathers_upsample_concat(hip, case, storage, monkeypatch):
    """A 3x3 conv over a channel concat of nearest upsamples runs as one halo-conv dispatch that reads each
    channel chunk from its source at (y >> s, x >> s) (sox_conv_halo_*_upcat): no upsample or concat is
    stored, and the output is the bits of the three-step path (SIMDONNX_HIP_NO_UPCAT) and the oracle's
    within the 16-bit contract."""
    from oracle.interp import run_plan
    n, h, w, c, shifts, oc = case
    pb = PlanBuilder()
    srcs, xs = [], []
    for i, sh in enumerate(shifts):
        v = pb.input((n, c, h >> sh, w >> sh), NHWC, f"p{i}")
        srcs.append(pb.resize_nearest(v, 1 << sh, name=f"up{i}") if sh else v)
        xs.append(synth.uniform(44, i, (n, h >> sh, w >> sh, c), -1, 1))
    fuse = pb.concat_channels(srcs, name="fuse")
    y = pb.conv(fuse, synth.uniform(44, 10, (oc, c * len(shifts), 3, 3), -0.1, 0.1),
                synth.uniform(44, 11, (oc,), -0.1, 0.1), pad=(1, 1, 1, 1), act="relu", name="conv")
    plan = pb.build(y)
    g = hip.graph(plan, storage)
    assert [d[0] for d in g.dispatches] == ["conv_halo"]
    assert g.kernels == [f"sox_conv_halo_{storage}_3x3s1_upcat"]
    g.release()
    got = run(hip, plan, xs, storage)
    monkeypatch.setenv("SIMDONNX_HIP_NO_UPCAT", "1")
    g = hip.graph(plan, storage)
    names = [d[0] for d in g.dispatches]
    assert "nearest" in names and names[-1] == "conv_halo", names
    g.release()
    ref = run(hip, plan, xs, storage)
    assert got.tobytes() == ref.tobytes()
    emu = {"f16": True, "bf16": "bf16"}[storage]
    assert max_rel(got, run_plan(plan, xs, f16_storage=emu)) < 2e-2


# (n, h, w, levels, ic, c): an FPN top-down chain over `levels` pyramid levels (the finest h x w): 1x1
# laterals of ic channels to c, then out_k = up2(out_{k+1}) + lat_k; the 4-level case is the detector's
UPADD_CASES = [(1, 240, 240, 4, 16, 96), (2, 40, 24, 3, 32, 64), (1, 36, 52, 2, 8, 16)]


@pytest.mark.parametrize("storage", ["f16", "bf16"])
@pytest.mark.parametrize("case", UPADD_CASES, ids=lambda c: "x".join(str(v) for v in c))
def test_fpn_topdown_add_in_lateral_conv(hip, case, storage, monkeypatch):
    """The FPN's nearest-upsample + Add runs inside the lateral 1x1 conv that produces the addend (the
    conv moves to the Add's place, the coarser level as its residual read at (y >> 1, x >> 1)): no upsample
    dispatch and no lateral output stored; within the 16-bit contract of the separate passes
    (SIMDONNX_HIP_NO_UPADD: the fused form rounds once) and of the oracle."""
    from oracle.interp import run_plan
    n, h, w, levels, ic, c = case
    pb = PlanBuilder()
    feats, xs = [], []
    for i in range(levels):
        ch = ic * (i + 1)
        feats.append(pb.input((n, ch, h >> i, w >> i), NHWC, f"c{i}"))
        xs.append(synth.uniform(45, i, (n, h >> i, w >> i, ch), -1, 1))
    lat = [pb.conv(f, synth.uniform(45, 10 + i, (c, ic * (i + 1), 1, 1), -0.3, 0.3), None, name=f"lat{i}")
           for i, f in enumerate(feats)]
    out = lat[-1]
    outs = []
    for i in range(levels - 2, -1, -1):
        out = pb.resize_nearest(out, 2, add=lat[i], name=f"up{i}")
        outs.append(out)
    plan = pb.build(outs[-1])  # each coarser level is read again as the next level's residual
    g = hip.graph(plan, storage)
    names = [d[0] for d in g.dispatches]
    g.release()
    assert "nearest" not in names and names == ["conv"] * levels, names
    got = run(hip, plan, xs, storage)
    monkeypatch.setenv("SIMDONNX_HIP_NO_UPADD", "1")
    g = hip.graph(plan, storage)
    assert [d[0] for d in g.dispatches].count("nearest") == levels - 1
    g.release()
    ref = run(hip, plan, xs, storage)
    assert max_rel(got, ref) < {"f16": 2e-3, "bf16": 1e-2}[storage]
    emu = {"f16": True, "bf16": "bf16"}[storage]
    assert max_rel(got, run_plan(plan, xs, f16_storage=emu)) < 2e-2


# (m, k, n): Gemm -> Softmax over rows whose N is not a multiple of 4 (the class head): the Gemm runs
# on the LDS-DMA ring into rows padded to a multiple of 8, the Softmax reads that stride
HEAD_CASES = [(300, 128, 1001), (2560, 192, 6625), (77, 64, 13)]


@pytest.mark.parametrize("case", HEAD_CASES, ids=lambda c: "x".join(str(v) for v in c))
def test_gemm_softmax_padded_rows(hip, case):
    m, k, n = case
    a = f16(synth.uniform(15, 1, (m, k), -1, 1))
    w = f16(synth.normal(15, 2, (k, n), 0.1))
    b = synth.uniform(15, 3, (n,), -0.5, 0.5)
    pb = PlanBuilder()
    av = pb.input((m, k), None, "a")
    y = pb.softmax(pb.gemm(av, w, b, name="head"), name="softmax")
    got = run(hip, pb.build(y), [a], True)
    want = O.softmax(f16(O.gemm(a, w, b)))
    assert max_rel(got, want) < TOL[True]


# (batch, ic, oc, k, stride, h, w, act, residual, reflect): fp32 convs with ic % 16 == 0, kh*kw*ic up to 576
# and zero padding take the short-K matrix-core kernel (whole tile in LDS, K split over the waves); pixel
# and channel tails, stride 2, residual; the reflect-padded case takes the general kernel
F32_SHORT_CASES = [(1, 64, 64, 3, 1, 64, 64, "relu", False, False), (2, 64, 96, 3, 2, 33, 29, "gelu", True, False),
                   (1, 64, 36, 1, 1, 10, 10, "none", False, False), (1, 16, 8, 4, 1, 12, 12, "hardswish", True, False),
                   (1, 64, 40, 3, 1, 15, 17, "sigmoid", False, True), (3, 128, 24, 1, 1, 7, 9, "relu", True, False)]


@pytest.mark.parametrize("case", F32_SHORT_CASES, ids=lambda c: "x".join(str(v) for v in c))
def test_conv_f32_short_route(hip, case):
    n, ic, oc, k, s, h, w, act, res, refl = case
    x = synth.uniform(17, 1, (n, h, w, ic), -1, 1)
    wt = synth.uniform(17, 2, (oc, ic, k, k), -0.25, 0.25)
    b = synth.uniform(17, 3, (oc,), -0.1, 0.1)
    pad = (k - 1) // 2 if k % 2 else k // 2
    pads = (pad, pad, k - 1 - pad, k - 1 - pad)
    oh, ow = (h + k - 1 - k) // s + 1, (w + k - 1 - k) // s + 1
    add = synth.uniform(17, 4, (n, oh, ow, oc), -1, 1) if res else None
    mode = 1 if refl else 0
    plan, ins = conv_plan(x, wt, b, add, (s, s), pads, act, mode, 0.0)
    g = hip.graph(plan, False)
    assert [d[0] for d in g.dispatches] == ["conv"]
    got = run(hip, plan, ins, False)
    want = O.conv(x, wt, b, add, stride=(s, s), pads=pads, act=act, pad_mode=mode)
    assert got.shape == want.shape
    assert max_rel(got, want) < TOL[False]


# (rows, k, n, act, trans_b, tail, mean): a LayerNorm whose output only a Gemm reads folds into the Gemm
# (sox_gemm_ln_*, one dispatch). tail: "softmax" (the class head: N % 4 != 0, padded rows), "residual"
# (the block's Add of the LayerNorm's own input in the Gemm epilogue); mean: an offset added to every
# input row (the single-pass variance against a mean 8x the spread). The last two cases stay unfolded:
# K % 64 != 0 and fewer than 64 rows.
LN_GEMM_CASES = [(2560, 192, 576, "none", 0, None, 0.0), (2560, 192, 768, "gelu", 0, None, 0.0),
                 (300, 192, 6625, "none", 0, "softmax", 0.0), (1000, 128, 256, "relu", 1, None, 8.0),
                 (2560, 192, 192, "none", 0, "residual", 0.5), (200, 40, 64, "none", 0, None, 0.0),
                 (40, 64, 64, "none", 0, None, 0.0)]


@pytest.mark.parametrize("case", LN_GEMM_CASES, ids=lambda c: "x".join(str(v) for v in c))
def test_layernorm_folded_into_gemm(hip, case):
    m, k, n, act, tb, tail, mean = case
    x = f16(synth.uniform(16, 1, (m, k), -1, 1) + mean)
    gam = 1.0 + synth.uniform(16, 2, (k,), -0.2, 0.2)
    bet = synth.uniform(16, 3, (k,), -0.2, 0.2)
    w = f16(synth.normal(16, 4, (n, k) if tb else (k, n), 0.1))
    b = synth.uniform(16, 5, (n,), -0.2, 0.2)
    pb = PlanBuilder()
    xv = pb.input((m, k), None, "x")
    h = pb.layer_norm(xv, gam, bet, 1e-5, name="ln")
    y = pb.gemm(h, w, b, act=act if tail != "residual" else "none", trans_b=bool(tb), name="gemm")
    if tail == "softmax":
        y = pb.softmax(y, name="softmax")
    elif tail == "residual":
        y = pb.add(xv, y, name="res")
    plan = pb.build(y)
    g = hip.graph(plan, True)
    folded = k % 64 == 0 and m >= 64
    names = [d[0] for d in g.dispatches]
    assert names == (["gemm_ln"] if folded else ["layernorm", "gemm"]) + (["softmax"] if tail == "softmax" else [])
    got = run(hip, plan, [x], True)
    wk = w.T if tb else w
    want = O.gemm(O.layer_norm(x, gam, bet, 1e-5), np.ascontiguousarray(wk), b, act=act if tail != "residual" else "none")
    if tail == "softmax":
        want = O.softmax(f16(want))
    elif tail == "residual":
        want = x + f16(want)
    assert max_rel(got, want) < TOL[True]


# (batch, ic, oc, stride, h, w, act, residual): 3x3 zero-padded convs on the halo route (stride 1),
# with tile, output-channel and input-channel-block tails; the stride-2 case takes the ring
HALO_CASES = [(1, 96, 24, 1, 30, 30, "none", False), (2, 40, 40, 1, 17, 35, "relu", True),
              (1, 32, 64, 2, 33, 47, "hardswish", False), (1, 8, 16, 1, 9, 8, "gelu", True),
              (1, 64, 72, 1, 12, 20, "none", False)]


@pytest.mark.parametrize("case", HALO_CASES, ids=lambda c: "x".join(str(v) for v in c))
def test_conv_halo_route(hip, case):
    n, ic, oc, s, h, w, act, res = case
    x = f16(synth.uniform(14, 1, (n, h, w, ic), -1, 1))
    wt = f16(synth.normal(14, 2, (oc, ic, 3, 3), 0.1))
    b = synth.uniform(14, 3, (oc,), -0.2, 0.2)
    oh, ow = (h + 2 - 3) // s + 1, (w + 2 - 3) // s + 1
    add = f16(synth.uniform(14, 4, (n, oh, ow, oc), -1, 1)) if res else None
    plan, ins = conv_plan(x, wt, b, add, (s, s), (1, 1, 1, 1), act, 0, 0.0)
    got = run(hip, plan, ins, True)
    want = O.conv(x, wt, b, add, stride=(s, s), pads=(1, 1, 1, 1), act=act)
    assert max_rel(got, want) < TOL[True]


# (batch, c, r, h, w, out, residual): one image with c % 8 == 0 folds the gate into the projection's
# weights; two images, or c % 8 != 0, keep the broadcast multiply
SE_PROJ = [(1, 96, 24, 9, 11, 40, False), (1, 576, 144, 5, 7, 96, True), (1, 16, 8, 33, 31, 16, True),
           (2, 96, 24, 9, 11, 40, False), (1, 36, 12, 6, 5, 24, False)]


@pytest.mark.parametrize("half", [False, True], ids=["f32", "f16"])
@pytest.mark.parametrize("case", SE_PROJ, ids=lambda c: "x".join(str(int(v)) for v in c))
def test_se_then_projection(hip, case, half):
    """ChannelGate -> x * gate -> 1x1 conv (+ residual), the MobileNetV3 block tail."""
    n, c, r, h, w, out, res = case
    cv = f16 if half else (lambda a: a)
    x = cv(synth.uniform(11, c, (n, h, w, c), -1, 1))
    w1 = synth.normal(11, 2, (r, c, 1, 1), 0.2)
    w2 = synth.normal(11, 3, (c, r, 1, 1), 0.2)
    b1, b2 = synth.uniform(11, 4, (r,), -0.1, 0.1), synth.uniform(11, 5, (c,), -0.1, 0.1)
    wp = cv(synth.normal(11, 6, (out, c, 1, 1), 0.1))
    bp = synth.uniform(11, 7, (out,), -0.1, 0.1)
    add = cv(synth.uniform(11, 8, (n, h, w, out), -1, 1)) if res else None
    pb = PlanBuilder()
    xv = pb.input((n, c, h, w), NHWC, "x")
    av = pb.input((n, out, h, w), NHWC, "add") if res else None
    gate = pb.channel_gate(xv, w1, b1, w2, b2, act1="relu", hard=True, alpha=1.0 / 6.0, beta=0.5, name="se")
    hv = pb.mul(xv, gate, name="se_scale")
    y = pb.conv(hv, wp, bp, stride=1, pad=0, add=av, name="project")
    got = run(hip, pb.build(y), [x, add] if res else [x], half)
    s = O.channel_gate(x, w1.reshape(r, c), b1, w2.reshape(c, r), b2)
    scaled = cv(x * s[:, None, None, :])
    want = O.conv(scaled, wp, bp, add)
    assert max_rel(got, want) < TOL[half]


@pytest.mark.parametrize("half", [False, True], ids=["f32", "f16"])
def test_se_fold_with_projection_planned_over_its_input(hip, half):
    """The gate's input x is an intermediate value, dead after x * s, so the arena packer places the
    projection's output over x. The folded projection reads x while it writes its output, so that
    output moves to a buffer of its own and the fold still happens: no broadcast multiply dispatch,
    and the result matches the unfused oracle."""
    c, r, h, w, out = 96, 24, 9, 11, 40
    cv = f16 if half else (lambda a: a)
    x0 = cv(synth.uniform(12, 1, (1, h, w, c), -1, 1))
    w1 = synth.normal(12, 2, (r, c, 1, 1), 0.2)
    w2 = synth.normal(12, 3, (c, r, 1, 1), 0.2)
    b1, b2 = synth.uniform(12, 4, (r,), -0.1, 0.1), synth.uniform(12, 5, (c,), -0.1, 0.1)
    wp = cv(synth.normal(12, 6, (out, c, 1, 1), 0.1))
    bp = synth.uniform(12, 7, (out,), -0.1, 0.1)
    pb = PlanBuilder()
    x0v = pb.input((1, c, h, w), NHWC, "x0")
    xv = pb.unary("Relu", x0v, name="x")
    gate = pb.channel_gate(xv, w1, b1, w2, b2, act1="relu", hard=True, alpha=1.0 / 6.0, beta=0.5, name="se")
    hv = pb.mul(xv, gate, name="se_scale")
    y = pb.conv(hv, wp, bp, stride=1, pad=0, name="project")
    plan = pb.build(y)
    vals = {v.name: v for v in plan.values}
    off = plan.buf_offset
    assert off[vals["x"].buf] == off[vals["project"].buf], "the packer no longer overlaps them: case untested"
    g = hip.graph(plan, half)
    names = [d[0] for d in g.dispatches]
    assert "ew2" not in names, names
    with HipInferenceSession(g) as s:
        s.set_input(x0)
        got = s.run().copy()
    x = np.maximum(x0, 0)
    s_ = O.channel_gate(x, w1.reshape(r, c), b1, w2.reshape(c, r), b2)
    want = O.conv(cv(x * s_[:, None, None, :]), wp, bp, None)
    assert max_rel(got, want) < TOL[half]


@pytest.mark.parametrize("half", [False, True], ids=["f32", "f16"])
def test_nearest_add_and_concat(hip, half):
    cv = f16 if half else (lambda a: a)
    x, add = cv(G["near_x"]), cv(G["near_add"])
    pb = PlanBuilder()
    xv = pb.input((1, 16, 7, 9), NHWC, "x")
    av = pb.input((1, 16, 14, 18), NHWC, "add")
    up = pb.resize_nearest(xv, 2, add=av, add_relu=True, name="up")
    y = pb.concat_channels([up, av], name="cat")
    got = run(hip, pb.build(y), [x, add], half)
    want = np.concatenate([O.resize_nearest(x, 2, 2, add, True), add], axis=-1)
    assert max_rel(got, want) < TOL[half]


@pytest.mark.parametrize("half", [False, True], ids=["f32", "f16"])
def test_layernorm_softmax(hip, half):
    cv = f16 if half else (lambda a: a)
    x = cv(G["ln_x"])
    pb = PlanBuilder()
    xv = pb.input((37, 192), None, "x")
    y = pb.layer_norm(xv, G["ln_g"], G["ln_b"], 1e-5, name="ln")
    got = run(hip, pb.build(y), [x], half)
    assert max_rel(got, O.layer_norm(x, G["ln_g"], G["ln_b"], 1e-5)) < TOL[half]
    x = cv(G["sm_x"])
    pb = PlanBuilder()
    xv = pb.input(x.shape, None, "x")
    y = pb.softmax(xv, name="softmax")
    got = run(hip, pb.build(y), [x], half)
    assert max_rel(got, O.softmax(x)) < TOL[half]


@pytest.mark.parametrize("half", [False, True], ids=["f32", "f16"])
@pytest.mark.parametrize("rows,len_", [(37, 1), (37, 13), (3, 8), (19, 2048), (19, 2049), (9, 4000), (23, 6625),
                                       (5, 8192), (5, 8193), (3, 20000)])
def test_softmax_lengths(hip, rows, len_, half):
    """Row softmax on the LDS-staged kernel (rows <= 16384, including the class head's 6625), the
    register-held rows (16-bit, stride a multiple of 8, <= 8192: 8, 2048, 4000, 8192) and the streaming
    one past 16384, with a per-row offset spread so the max subtraction matters."""
    cv = f16 if half else (lambda a: a)
    x = cv(synth.uniform(18, 1, (rows, len_), -4, 4) + synth.uniform(18, 2, (rows, 1), -20, 20))
    pb = PlanBuilder()
    xv = pb.input((rows, len_), None, "x")
    y = pb.softmax(xv, name="softmax")
    got = run(hip, pb.build(y), [x], half)
    assert max_rel(got, O.softmax(x)) < TOL[half]


@pytest.mark.parametrize("half", [False, True], ids=["f32", "f16"])
@pytest.mark.parametrize("shape", [(4, 80, 6, 32), (2, 37, 3, 64), (3, 128, 2, 32), (1, 20, 4, 64), (2, 64, 2, 64),
                                   (5, 50, 1, 32), (2, 130, 2, 32)], ids=lambda c: "x".join(str(v) for v in c))
def test_attention_packed_qkv(hip, half, shape):
    """Fused attention over a packed [N, T, 3*H*D] qkv (GpuOpTests attention packed-qkv case): the
    fp16 matrix-core kernel for every key-count bucket (32 / 64 / 80 / 128, with key tails) and head
    size 32 / 64, and the general kernel past 128 keys."""
    nb, t, heads, d = shape
    cv = f16 if half else (lambda a: a)
    qkv = cv(synth.uniform(5, 1, (nb, t, 3 * heads * d), -1, 1))
    pb = PlanBuilder()
    xv = pb.input(qkv.shape, None, "qkv")
    y = pb.attention(xv, heads, d, d ** -0.5, name="attn")
    got = run(hip, pb.build(y), [qkv], half)
    q5 = qkv.reshape(nb, t, 3, heads, d)
    q, k, v = (np.ascontiguousarray(q5[:, :, j].transpose(0, 2, 1, 3)).reshape(nb * heads, t, d) for j in range(3))
    want = O.attention(q, k, v, d ** -0.5).reshape(nb, heads, t, d).transpose(0, 2, 1, 3).reshape(nb, t, heads * d)
    assert max_rel(got.reshape(want.shape), want) < TOL[half]


def test_replay_matches_direct(hip):
    """A HIP-graph replay of the dispatch list gives the direct launches' bits on every replay."""
    x = f16(G["conv12_x"])
    plan, ins = conv_plan(x, f16(G["conv12_w"]), G["conv12_b"], None, (1, 1), (1, 1, 1, 1), "relu", 0, 0.0)
    with HipInferenceSession(hip.graph(plan, True)) as s:
        s.set_input(x)
        direct = s.run().copy()
        s.set_replay(True)
        for _ in range(3):
            s.set_input(x)
            assert np.array_equal(s.run(), direct)


GEMM_KERNELS = ["sox_gemm_f16_256x192_k32s5", "sox_gemm_f16_256x128_w8k64s2", "sox_gemm_f16_128x128_k64s2",
                "sox_gemm_f16_128x64_k64s2", "sox_gemm_f16_64x64_k64s2", "sox_gemm_f16_256x192_k32s4",
                "sox_gemm_f16_256x192_w8k64s2", "sox_gemm_f16_256x256_w8k32s4", "sox_gemm_f16_256x256_w8k64s2",
                "sox_gemm_f16_256x128_k32s3", "sox_gemm_f16_256x128_k32s5", "sox_gemm_f16_128x128_k32s4",
                "sox_gemm_f16_64x64_k64s4", "sox_gemm_f16_128x64_k64s4", "sox_gemm_f16_128x192_k32s3"]


@pytest.mark.parametrize("kernel", GEMM_KERNELS)
@pytest.mark.parametrize("act,shape", [("gelu", (4100, 192, 776)), ("relu", (4100, 192, 776)),
                                       ("none", (16400, 64, 200)), ("hardswish", (16400, 128, 520)),
                                       ("none", (2560, 192, 6625)), ("relu", (300, 64, 13))])
def test_pipelined_gemm_variants(hip, kernel, act, shape, monkeypatch):
    """Every LDS-DMA Gemm tiling against the oracle, with M and N tails. The M=16400 cases give every
    tiling more tiles than resident workgroups, so one workgroup's K-slice ring crosses tile borders
    (with K=64 a border every slice); hardswish takes the runtime-activation epilogue; N=6625 (the
    recognizer head) and N=13 take the unaligned-row store path and the zero-padded bias groups."""
    monkeypatch.setenv("SIMDONNX_HIP_GEMM", kernel)
    m, k, n = shape
    a = f16(synth.uniform(21, 1, (m, k), -1, 1))
    w = f16(synth.normal(21, 2, (k, n), 0.1))
    b = synth.uniform(21, 3, (n,), -0.1, 0.1)
    pb = PlanBuilder()
    av = pb.input((m, k), None, "a")
    y = pb.gemm(av, w, b, act=act, name="gemm")
    plan = pb.build(y)
    g = hip.graph(plan, True)
    assert g.dispatches[0][0] == "gemm"
    with HipInferenceSession(g) as s:
        s.set_input(a)
        got = s.run().copy()
    want = O.gemm(a, w, b, act=act)
    assert max_rel(got, want) < TOL[True]


@pytest.mark.parametrize("half", [False, True], ids=["f32", "f16"])
@pytest.mark.parametrize("m,k,n,act", [(2560, 192, 576, "none"), (2560, 768, 192, "relu"), (300, 40, 24, "none")])
def test_gemm_residual_add_fused(hip, m, k, n, act, half):
    """Gemm followed by Add(gemm, residual) [+ReLU] runs as one dispatch (the Add in the epilogue) through
    the LDS-DMA kernel (fp16, K % 64 == 0) or the implicit-GEMM kernel, against the unfused oracle."""
    cv = f16 if half else (lambda v: v)
    a = cv(synth.uniform(31, 1, (m, k), -1, 1))
    r = cv(synth.uniform(31, 2, (m, n), -1, 1))
    w = cv(synth.normal(31, 3, (k, n), 0.1))
    b = synth.uniform(31, 4, (n,), -0.1, 0.1)
    pb = PlanBuilder()
    av = pb.input((m, k), None, "a")
    rv = pb.input((m, n), None, "r")
    y = pb.gemm(av, w, b, name="gemm")
    z = pb.add(y, rv, act=act, name="res")
    plan = pb.build(z)
    g = hip.graph(plan, half)
    assert [d[0] for d in g.dispatches] == ["gemm"]
    got = run(hip, plan, [a, r], half)
    g1 = O.gemm(a, w, b)
    want = O.ew2(O.round_f16(g1) if half else g1, r, op=0, act=1 if act == "relu" else 0)
    assert max_rel(got, want) < (2e-2 if half else 1e-4)


# (batch, ic, oc, k, stride, h, w, act, residual, pad_mode, pad_value): fp16 convs with fewer than 8
# output channels take the one-pixel-per-item direct kernel; K = 9 * 128 is its largest reduction
NARROW_CASES = [(1, 8, 3, 3, 1, 37, 61, "none", False, 0, 0.0), (2, 16, 1, 3, 1, 20, 18, "sigmoid", True, 0, 0.0),
                (1, 24, 5, 3, 2, 33, 29, "relu", False, 0, 0.0), (1, 8, 7, 5, 1, 15, 22, "hardswish", True, 1, 0.0),
                (1, 128, 2, 3, 1, 9, 10, "gelu", False, 0, 0.0), (1, 8, 4, 3, 1, 11, 13, "none", False, 0, -0.5),
                (1, 16, 3, 3, 1, 21, 17, "none", False, 0, 0.1)]


@pytest.mark.parametrize("case", NARROW_CASES, ids=lambda c: "x".join(str(v) for v in c))
def test_conv_narrow_route(hip, case):
    n, ic, oc, k, s, h, w, act, res, mode, pv = case
    x = f16(synth.uniform(19, 1, (n, h, w, ic), -1, 1))
    wt = f16(synth.normal(19, 2, (oc, ic, k, k), 0.15))
    b = synth.uniform(19, 3, (oc,), -0.2, 0.2)
    p = k // 2
    pads = (p, p, p, p)
    oh, ow = (h + 2 * p - k) // s + 1, (w + 2 * p - k) // s + 1
    add = f16(synth.uniform(19, 4, (n, oh, ow, oc), -1, 1)) if res else None
    plan, ins = conv_plan(x, wt, b, add, (s, s), pads, act, mode, pv)
    g = hip.graph(plan, True)
    assert [d[0] for d in g.dispatches] == ["conv_narrow"]
    got = run(hip, plan, ins, True)
    want = O.conv(x, wt, b, add, stride=(s, s), pads=pads, act=act, pad_mode=mode, pad_value=pv)
    assert got.shape == want.shape
    assert max_rel(got, want) < TOL[True]


def test_conv_narrow_pad_value_is_fp32(hip):
    """The constant pad value enters the narrow kernel's FMAs in fp32, as in the other routes and the
    oracle: two pad values inside one fp16 rounding interval (0.09996 and 0.1 both round to
    0.0999756) must still give different border outputs, each within the fp16 bar of the oracle."""
    x = f16(synth.uniform(20, 1, (1, 24, 20, 16), -1, 1))
    wt = f16(synth.normal(20, 2, (3, 16, 3, 3), 0.15))
    b = synth.uniform(20, 3, (3,), -0.2, 0.2)
    assert np.float16(0.09996) == np.float16(0.1)
    outs = []
    for pv in (0.09996, 0.1):
        plan, ins = conv_plan(x, wt, b, None, (1, 1), (1, 1, 1, 1), "none", 0, pv)
        assert [d[0] for d in hip.graph(plan, True).dispatches] == ["conv_narrow"]
        got = run(hip, plan, ins, True)
        want = O.conv(x, wt, b, stride=(1, 1), pads=(1, 1, 1, 1), pad_value=pv)
        assert max_rel(got, want) < TOL[True]
        outs.append(got)
    assert not np.array_equal(outs[0], outs[1])
    assert np.array_equal(outs[0][:, 1:-1, 1:-1], outs[1][:, 1:-1, 1:-1])  # interior pixels see no padding


@pytest.mark.parametrize("storage", ["f16", "bf16"])
@pytest.mark.parametrize("route", ["ring", "pp"])
def test_gemm_gelu_epilogue_within_one_ulp(hip, storage, route, monkeypatch):
    """The 16-bit Gemm epilogue's GELU (one exp2 per element) over every fp16 value in [-8, 8] (every
    bf16 value for bf16): A = x e_0, W row 0 = 1, so each output is GELU(x) of one exact fp32
    accumulator. Against the float64 erf-GELU (scipy's erfc) it is within one ulp of the 16-bit
    output at the exact value, or 1e-6 absolute where that is larger (outputs of |x| > 5.5 and
    fp16's subnormal range: the A&S 7.1.26 form of the reference is itself ~3e-7 off there)."""
    from scipy.special import erfc
    from oracle.interp import _bf16
    pos = np.arange(0, np.float16(8.0).view(np.uint16), dtype=np.uint16).view(np.float16)
    x = np.unique(np.concatenate([pos, -pos]).astype(np.float32))
    if storage == "bf16":
        x = np.unique(_bf16(np.linspace(-8, 8, 200001, dtype=np.float32)))
    # the ring (K = 64), or the epilogue-under-MFMA kernel (K = 768, 256 x 128 tiles, >= 256 of them)
    k, n = (64, 64) if route == "ring" else (768, 512)
    if route == "pp":
        monkeypatch.setenv("SIMDONNX_HIP_GEMMPP", "1")
    m = max((len(x) + 255) // 256 * 256, 64 if route == "ring" else 16384)  # pp: >= 256 tiles (zero rows)
    a = np.zeros((m, k), np.float32)
    a[: len(x), 0] = x
    w = np.zeros((k, n), np.float32)
    w[0, :] = 1.0
    pb = PlanBuilder()
    av = pb.input((m, k), None, "a")
    y = pb.gemm(av, w, None, act="gelu", name="gemm")
    g = hip.graph(pb.build(y), storage)
    assert [d[0] for d in g.dispatches] == ["gemm"]
    assert g.kernels[0].startswith("sox_gemmpp_" if route == "pp" else "sox_gemm_"), g.kernels
    with HipInferenceSession(g) as s:
        s.set_input(a)
        got = s.run().copy()[: len(x)]
    assert np.all(got == got[:, :1])
    got = got[:, 0].astype(np.float64)
    xd = x.astype(np.float64)
    ref = xd * 0.5 * erfc(-xd / np.sqrt(2.0))
    mag = np.abs(ref)
    exp = np.floor(np.log2(np.maximum(mag, 1e-300)))
    ulp = np.ldexp(1.0, (exp - (10 if storage == "f16" else 7)).astype(np.int32))
    bad = np.abs(got - ref) > np.maximum(ulp, 1e-6)
    assert not bad.any(), (x[bad][:8], got[bad][:8], ref[bad][:8])


@pytest.mark.parametrize("storage", ["f16", "bf16"])
@pytest.mark.parametrize("m,n,act,bias", [(4096, 2048, "gelu", True), (8192, 3072, "gelu", True),
                                          (6144, 1536, "relu", True), (6144, 1536, "none", False)],
                         ids=["1-tile-per-cu", "config2", "uneven-relu", "uneven-none-nobias"])
def test_gemm_pp_matches_ring_bitwise(hip, m, n, act, bias, storage, monkeypatch):
    """Under SIMDONNX_HIP_GEMMPP, whole 256 x 128 tiles with K = 768 take the kernel that runs each
    tile's epilogue under the next tile's MFMAs (gemm_pp.h). It accumulates the same 32x32x16 steps from
    the bias in the same k order and applies the same activation as the LDS-DMA ring (the default), so
    the two agree bit for bit; both within the fp16 (2e-3) / bf16 (8e-3) contract of the oracle on the rounded operands.
    Shapes: one tile per workgroup (first tile and the trailing epilogue only), config 2 (three per
    workgroup), and 288 tiles over 256 workgroups (one or two each)."""
    from oracle.interp import _bf16
    k = 768
    rnd = f16 if storage == "f16" else _bf16
    a = rnd(synth.normal(71, 1, (m, k), 1.0))
    w = rnd(synth.normal(71, 2, (k, n), 0.05))
    b = synth.uniform(71, 3, (n,), -0.1, 0.1) if bias else None
    pb = PlanBuilder()
    av = pb.input((m, k), None, "a")
    y = pb.gemm(av, w, b, act=act, name="gemm")
    plan = pb.build(y)
    print(f"[gpu] gemm_pp {m}x{n}x{k} {act} bias={bias} {storage}", flush=True)
    monkeypatch.setenv("SIMDONNX_HIP_GEMMPP", "1")
    g = hip.graph(plan, storage)
    assert g.kernels == [f"sox_gemmpp_{storage}_256x128_k768_{act}"], g.kernels
    with HipInferenceSession(g) as s:
        s.set_input(a)
        got = s.run().copy()
    g.release()
    monkeypatch.delenv("SIMDONNX_HIP_GEMMPP")
    g2 = hip.graph(plan, storage)
    assert g2.kernels[0].startswith(f"sox_gemm_{storage}_"), g2.kernels
    with HipInferenceSession(g2) as s:
        s.set_input(a)
        ring = s.run().copy()
    g2.release()
    assert got.tobytes() == ring.tobytes(), f"max diff {np.abs(got - ring).max()}"
    want = O.gemm(a, w, b, act=act)
    assert max_rel(got, want) < (2e-3 if storage == "f16" else 8e-3)


@pytest.mark.parametrize("kernel", ["", "sox_conv_f16_256x128_w8k64s2", "sox_conv_f16_256x256_w8k64s2"],
                         ids=["default", "w8-256x128", "w8-256x256"])
@pytest.mark.parametrize("storage", ["f16", "bf16"])
def test_conv_large_channels(hip, storage, kernel, monkeypatch):
    """The large conv of the bench (3x3 s1 p1 + bias + ReLU, 256 -> 256 channels), at batch 1 and 48x40
    so the oracle stays quick, on the default route and forced onto the ring's 8-wave tilings (the
    bench's 8x128x128 size takes the halo tile, tested by test_conv_halo_tile_matches_ring)."""
    if kernel:
        monkeypatch.setenv("SIMDONNX_HIP_CONV", kernel)
    from oracle.interp import _bf16
    cv = f16 if storage == "f16" else _bf16
    x = cv(synth.normal(64, 3, (1, 48, 40, 256), 1.0))
    wt = cv(synth.he_normal(64, 1, (256, 256, 3, 3)))
    b = synth.uniform(64, 2, (256,), -0.1, 0.1)
    plan, ins = conv_plan(x, wt, b, None, (1, 1), (1, 1, 1, 1), "relu", 0, 0.0)
    g = hip.graph(plan, storage)
    assert [d[0] for d in g.dispatches] == ["conv"]
    got = run(hip, plan, ins, storage)
    want = O.conv(x, wt, b, stride=(1, 1), pads=(1, 1, 1, 1), act="relu")
    assert max_rel(got, want) < (TOL[True] if storage == "f16" else 4e-3)


@pytest.mark.parametrize("storage", ["f16", "bf16"])
@pytest.mark.parametrize("shape,mode,act,res", [((1, 48, 40), 0, "relu", False), ((2, 33, 31), 0, "relu", False),
                                                ((2, 33, 31), 1, "relu", False), ((1, 48, 40), 0, "gelu", False),
                                                ((2, 33, 31), 0, "relu", True)],
                         ids=["48x40", "2x33x31-ragged", "2x33x31-reflect", "48x40-gelu", "2x33x31-residual"])
def test_conv_256x256_tile_matches_256x128(hip, storage, shape, mode, act, res, monkeypatch):
    """The 256 x 256 conv tile (8 waves of 128 x 64, 32-bit input offsets, 16-byte stores from
    registers; 8-byte stores with a residual) and the 256 x 128 one (image-base pointers, LDS-staged
    stores; register stores with a residual) run the same k-steps in the same order from the same bias
    and round the activation to fp32 before the 16-bit conversion: the outputs are equal bit for bit,
    on whole and ragged row tiles, with zero and reflect padding (the second image's reflected rows find
    their image's base from the 32-bit offset), GELU, and a fused residual Add; the reflect case also
    against the oracle."""
    from oracle.interp import _bf16
    n, h, w = shape
    cv = f16 if storage == "f16" else _bf16
    x = cv(synth.normal(65, 3, (n, h, w, 256), 1.0))
    wt = cv(synth.he_normal(65, 1, (256, 256, 3, 3)))
    b = synth.uniform(65, 2, (256,), -0.1, 0.1)
    add = cv(synth.uniform(65, 4, (n, h, w, 256), -1, 1)) if res else None
    plan, ins = conv_plan(x, wt, b, add, (1, 1), (1, 1, 1, 1), act, mode, 0.0)
    outs = []
    for k in ("sox_conv_f16_256x256_w8k64s2", "sox_conv_f16_256x128_w8k64s2"):
        monkeypatch.setenv("SIMDONNX_HIP_CONV", k)
        g = hip.graph(plan, storage)
        assert g.kernels == [k.replace("_f16_", f"_{storage}_")], g.kernels
        g.release()
        outs.append(run(hip, plan, ins, storage))
    assert outs[0].tobytes() == outs[1].tobytes(), f"max diff {np.abs(outs[0] - outs[1]).max()}"
    if mode:
        want = O.conv(x, wt, b, stride=(1, 1), pads=(1, 1, 1, 1), act="relu", pad_mode=mode)
        assert max_rel(outs[0], want) < (TOL[True] if storage == "f16" else 4e-3)


# (batch, h, w, ic, oc, act, residual): 3x3 convs on the halo tile (sox_conv_*_h256): ragged row tiles
# (h % 8 != 0), partial column tiles (w % 32 != 0), one and four 64-channel blocks, two 256-channel
# blocks of output (grid.y = 2), GELU and a fused residual (8-byte stores), several tiles per workgroup
H256_CASES = [(2, 33, 64, 256, 256, "relu", False), (1, 16, 32, 64, 256, "gelu", False),
              (1, 19, 96, 128, 512, "relu", False), (2, 24, 32, 192, 256, "none", True),
              (2, 17, 40, 128, 256, "relu", False), (1, 9, 71, 64, 256, "gelu", True)]


@pytest.mark.parametrize("storage", ["f16", "bf16"])
@pytest.mark.parametrize("case", H256_CASES, ids=lambda c: "x".join(str(v) for v in c[:5]) + f"-{c[5]}" + ("-res" if c[6] else ""))
def test_conv_halo_tile_matches_ring(hip, storage, case, monkeypatch):
    """The halo-tile large conv (8 x 32 pixels x 256 channels per workgroup, input halos in LDS) adds
    each output's channel blocks, taps and k-steps in the implicit-GEMM ring's order from the same
    bias, so it equals the 256 x 128 ring tile bit for bit, and meets the oracle."""
    from oracle.interp import _bf16
    n, h, w, ic, oc, act, res = case
    cv = f16 if storage == "f16" else _bf16
    x = cv(synth.normal(66, 3, (n, h, w, ic), 1.0))
    wt = cv(synth.he_normal(66, 1, (oc, ic, 3, 3)))
    b = synth.uniform(66, 2, (oc,), -0.1, 0.1)
    add = cv(synth.uniform(66, 4, (n, h, w, oc), -1, 1)) if res else None
    plan, ins = conv_plan(x, wt, b, add, (1, 1), (1, 1, 1, 1), act, 0, 0.0)
    outs = []
    for k in ("sox_conv_f16_h256", "sox_conv_f16_256x128_w8k64s2"):
        monkeypatch.setenv("SIMDONNX_HIP_CONV", k)
        g = hip.graph(plan, storage)
        assert g.kernels == [k.replace("_f16_", f"_{storage}_")], g.kernels
        g.release()
        outs.append(run(hip, plan, ins, storage))
    assert outs[0].tobytes() == outs[1].tobytes(), f"max diff {np.abs(outs[0] - outs[1]).max()}"
    want = O.conv(x, wt, b, add, stride=(1, 1), pads=(1, 1, 1, 1), act=act)
    assert max_rel(outs[0], want) < (TOL[True] if storage == "f16" else 4e-3)


# (batch, ic, oc1, h, w, bn): two chained 2x2 ConvTransposes, the second to one channel (the DB head's
# probability map); bn: an unfolded BatchNorm + ReLU between them (folded into the first), else ReLU on
# the first. Ragged pixel counts leave partial 128-pixel blocks.
CONVT_CHAIN = [(1, 24, 24, 60, 60, True), (2, 16, 8, 9, 13, False), (1, 32, 32, 17, 11, True), (1, 8, 16, 5, 7, False)]


@pytest.mark.parametrize("storage", ["f16", "bf16"])
@pytest.mark.parametrize("case", CONVT_CHAIN, ids=lambda c: "x".join(str(v) for v in c[:5]) + ("-bn" if c[5] else ""))
def test_convt_chain_matches_unfused(hip, storage, case, monkeypatch):
    """The fused pair (sox_convt2_*) against the two separate ConvTranspose dispatches bit for bit (the
    first as the same matrix product from zero with its bias after, rounded to the storage type; the
    second in sox_convt_one_*'s order), and against the fp32 oracle of the chain."""
    from oracle.interp import _bf16
    n, ic, oc1, h, w, bn = case
    cv = f16 if storage == "f16" else _bf16
    x = cv(synth.uniform(66, 1, (n, h, w, ic), -1, 1))
    w1 = cv(synth.normal(66, 2, (ic, oc1, 2, 2), 0.3))
    b1 = synth.uniform(66, 3, (oc1,), -0.2, 0.2)
    w2 = cv(synth.normal(66, 4, (oc1, 1, 2, 2), 0.3))
    b2 = synth.uniform(66, 5, (1,), -0.2, 0.2)
    s_, t_ = synth.uniform(66, 6, (oc1, 1, 1), 0.5, 1.5), synth.uniform(66, 7, (oc1, 1, 1), -0.3, 0.3)
    pb = PlanBuilder()
    xv = pb.input((n, ic, h, w), NHWC, "x")
    hv = pb.conv_transpose(xv, w1, b1, act="none" if bn else "relu", name="convt1")
    if bn:
        hv = pb.ew(hv, pb.const(s_, "bn_scale"), 2, name="bn_mul")
        hv = pb.ew(hv, pb.const(t_, "bn_shift"), 0, act="relu", name="bn_add")
    y = pb.conv_transpose(hv, w2, b2, act="sigmoid", name="convt2")
    plan = pb.build(y)
    g = hip.graph(plan, storage)
    assert g.kernels == [f"sox_convt2_{storage}_n{oc1 // 8}"], g.kernels
    g.release()
    got = run(hip, plan, [x], storage)
    monkeypatch.setenv("SIMDONNX_HIP_NO_CONVT_CHAIN", "1")
    g = hip.graph(plan, storage)
    assert len(g.kernels) == 2 and g.kernels[1] == f"sox_convt_one_{storage}", g.kernels
    g.release()
    unfused = run(hip, plan, [x], storage)
    assert got.shape == (n, 4 * h, 4 * w, 1)
    assert got.tobytes() == unfused.tobytes(), f"max diff {np.abs(got - unfused).max()}"
    ref = O.conv_transpose(x, w1, b1)
    ref = np.maximum(ref * s_.reshape(-1) + t_.reshape(-1), 0.0) if bn else np.maximum(ref, 0.0)
    want = O.conv_transpose(ref, w2, b2, act="sigmoid")
    assert max_rel(got, want) < (5e-3 if storage == "f16" else 2e-2)
