"""Pins the CPU oracle (oracle/) before it is trusted as the parity reference.

  * against the committed torch-float64 golden vectors (tests/golden/make_golden.py): the closed
    forms of every restated routine;
  * tier invariants of the reference: AVX-512 == AVX2 (== scalar) bit for bit
    (Avx512KernelTests.cs:7-33), Winograd within 1e-4 * max|out| of direct (EngineTests.cs:184-212);
  * the shared transcendental cores against math.erf / math.exp within their published bounds;
  * planted mistakes in a copy of the restatement fail these checks (the mutation guard,
    tests/test_oracle_mutation.py: seven mutants, each caught; the unmutated copy passes).
"""
import math
import os

import numpy as np
import pytest

import oracle as O
from tests.conftest import max_rel

G = np.load(os.path.join(os.path.dirname(__file__), "golden", "golden.npz"))
ACTS = ["none", "relu", "sigmoid", "gelu", "hardswish", "swish"]


def _conv_case(i):
    ic, oc, k, s, h, w, mode, act, res = [int(v) for v in G[f"conv{i}_meta"]]
    pv = float(G[f"conv{i}_pv"][0])
    add = G[f"conv{i}_add"] if res else None
    return dict(x=G[f"conv{i}_x"], w=G[f"conv{i}_w"], b=G[f"conv{i}_b"], add=add, stride=(s, s),
                pads=(k // 2,) * 4, act=ACTS[act], pad_mode=mode, pad_value=pv), G[f"conv{i}_y"]


@pytest.mark.parametrize("i", range(int(G["conv_n"][0])))
@pytest.mark.parametrize("algo", [0, 1])
def test_conv_matches_golden(i, algo):
    c, want = _conv_case(i)
    got = O.conv(c["x"], c["w"], c["b"], c["add"], stride=c["stride"], pads=c["pads"], act=c["act"],
                 pad_mode=c["pad_mode"], pad_value=c["pad_value"], algo=algo)
    tol = 2e-6 if algo == 1 else 2e-5
    assert max_rel(got, want) < tol


@pytest.mark.parametrize("i", range(int(G["conv_n"][0])))
def test_conv_tiers_bitwise(i):
    c, _ = _conv_case(i)
    outs = []
    for tier in (O.TIER_SCALAR, O.TIER_AVX2, O.TIER_AVX512):
        if not O.tier_available(tier):
            pytest.skip("tier not available on this CPU")
        for algo in (0, 1):
            outs.append((tier, algo, O.conv(c["x"], c["w"], c["b"], c["add"], stride=c["stride"], pads=c["pads"],
                                            act=c["act"], pad_mode=c["pad_mode"], pad_value=c["pad_value"],
                                            algo=algo, tier=tier)))
    for algo in (0, 1):
        same = [o for t, a, o in outs if a == algo]
        for o in same[1:]:
            assert np.array_equal(o.view(np.uint32), same[0].view(np.uint32))


@pytest.mark.parametrize("i", range(int(G["conv_n"][0])))
def test_winograd_vs_direct(i):
    c, _ = _conv_case(i)
    kh = c["w"].shape[2]
    if not O.winograd_eligible(kh, kh, c["stride"][0], c["stride"][1], 1, c["x"].shape[-1]):
        pytest.skip("not Winograd-eligible")
    kw = dict(stride=c["stride"], pads=c["pads"], act=c["act"], pad_mode=c["pad_mode"], pad_value=c["pad_value"])
    direct = O.conv(c["x"], c["w"], c["b"], c["add"], algo=1, **kw)
    wino = O.conv(c["x"], c["w"], c["b"], c["add"], algo=0, **kw)
    assert np.abs(wino - direct).max() < 1e-4 * np.abs(direct).max()


@pytest.mark.parametrize("i", range(int(G["dw_n"][0])))
def test_depthwise_matches_golden(i):
    c, k, s, h, w, mode, act = [int(v) for v in G[f"dw{i}_meta"]]
    got = O.conv(G[f"dw{i}_x"], G[f"dw{i}_w"], G[f"dw{i}_b"], stride=(s, s), pads=(k // 2,) * 4, group=c,
                 act=ACTS[act], pad_mode=mode)
    assert max_rel(got, G[f"dw{i}_y"]) < 2e-6


@pytest.mark.parametrize("i", range(int(G["gemm_n"][0])))
def test_gemm_matches_golden_and_tiers(i):
    m, k, n, tb, act = [int(v) for v in G[f"gemm{i}_meta"]]
    outs = [O.gemm(G[f"gemm{i}_a"], G[f"gemm{i}_b"], G[f"gemm{i}_bias"], trans_b=bool(tb), act=ACTS[act], tier=t)
            for t in (O.TIER_SCALAR, O.TIER_AVX2, O.TIER_AVX512) if O.tier_available(t)]
    assert max_rel(outs[-1], G[f"gemm{i}_y"]) < 2e-6
    for o in outs[1:]:
        assert np.array_equal(o.view(np.uint32), outs[0].view(np.uint32))


@pytest.mark.parametrize("i", range(int(G["ct_n"][0])))
def test_conv_transpose_matches_golden(i):
    ic, oc, k, h, w, act = [int(v) for v in G[f"ct{i}_meta"]]
    got = O.conv_transpose(G[f"ct{i}_x"], G[f"ct{i}_w"], G[f"ct{i}_b"], act=ACTS[act])
    assert max_rel(got, G[f"ct{i}_y"]) < 2e-6


def test_layer_norm_softmax_matmul_attention():
    assert max_rel(O.layer_norm(G["ln_x"], G["ln_g"], G["ln_b"], 1e-5), G["ln_y"]) < 2e-5
    assert max_rel(O.softmax(G["sm_x"]), G["sm_y"]) < 2e-6
    assert max_rel(O.matmul(G["mm_a"], G["mm_b"]), G["mm_y"]) < 2e-6
    got = O.attention(G["attn_q"], G["attn_k"], G["attn_v"], 32 ** -0.5)
    assert max_rel(got, G["attn_y"]) < 2e-6


def test_gap_se_nearest():
    assert max_rel(O.global_avg_pool(G["gap_x"]), G["gap_y"]) < 2e-6
    got = O.channel_gate(G["se_x"], G["se_w1"], G["se_b1"], G["se_w2"], G["se_b2"], act1_relu=True, hard=True)
    assert max_rel(got, G["se_y"]) < 2e-6
    got = O.resize_nearest(G["near_x"], 2.0, 2.0, G["near_add"], add_relu=True)
    assert max_rel(got, G["near_y"]) < 1e-7


def test_conv_pool_equals_conv_then_pool():
    """ConvPool keeps the per-element math of Conv -> MaxPool (Nhwc.cs:661-727)."""
    c, _ = _conv_case(1)
    kw = dict(stride=c["stride"], pads=c["pads"], act="relu", pad_mode=c["pad_mode"])
    full = O.conv(c["x"], c["w"], c["b"], **kw)
    n, h, w, oc = full.shape
    pooled = full[:, :h // 2 * 2, :w // 2 * 2].reshape(n, h // 2, 2, w // 2, 2, oc).max(axis=(2, 4))
    got = O.conv(c["x"], c["w"], c["b"], pool=True, **kw)
    assert np.array_equal(got, pooled)


def test_one_by_one_conv_equals_gemm():
    """A 1x1 stride-1 conv is the Gemm of pixels x channels (Nhwc.cs:177-183 batch folding)."""
    x = G["conv6_x"]
    w = G["conv6_w"]
    y = O.conv(x, w, G["conv6_b"], algo=1)
    g = O.gemm(x.reshape(-1, x.shape[-1]), w[:, :, 0, 0], G["conv6_b"], trans_b=True)
    assert np.array_equal(y.reshape(g.shape), g)


def test_math_cores():
    xs = np.linspace(-9, 9, 20001)
    err_erf = max(abs(O.erf_core(x) - math.erf(x)) for x in xs)
    assert err_erf < 5e-7  # A&S 7.1.26: |eps| <= 1.5e-7 (plus float32 rounding)
    xs = np.linspace(-80, 80, 4001).astype(np.float32).astype(np.float64)  # exact float32 arguments
    rel = max(abs(O.exp_core(x) - math.exp(x)) / math.exp(x) for x in xs)
    assert rel < 5e-7  # Cephes degree-5 polynomial: ~2 ulp
    assert O.exp_core(-100.0) == pytest.approx(math.exp(-87.3), rel=1e-6)  # clamp
    xs = np.linspace(-6, 6, 1201)
    g = max(abs(O.gelu_core(x) - 0.5 * x * (1 + math.erf(x / math.sqrt(2)))) for x in xs)
    assert g < 2e-6


def test_round_f16_matches_ieee():
    x = np.concatenate([np.linspace(-70000, 70000, 10001), np.linspace(-1e-4, 1e-4, 10001)]).astype(np.float32)
    with np.errstate(over="ignore"):
        assert np.array_equal(O.round_f16(x), x.astype(np.float16).astype(np.float32))


def test_elementwise_broadcast_concat_against_numpy():
    """Elementwise Add/Sub/Mul/Div (+ReLU), per-channel broadcast both operand orders, channel concat and
    HardSigmoid against numpy's own float32 arithmetic (one rounding per op, so bit-exact)."""
    rng = np.random.default_rng(7)
    a = rng.uniform(-2, 2, (3, 5, 7, 12)).astype(np.float32)
    b = rng.uniform(0.5, 2, (3, 5, 7, 12)).astype(np.float32)
    ops = [np.add, np.subtract, np.multiply, np.divide]
    for op, fn in enumerate(ops):
        assert np.array_equal(O.ew2(a, b, op=op), fn(a, b))
        assert np.array_equal(O.ew2(a, b, op=op, act=1), np.maximum(fn(a, b), np.float32(0)))
        v = b[0, 0, 0]
        assert np.array_equal(O.channel_broadcast(a, v, op=op), fn(a, v))
        assert np.array_equal(O.channel_broadcast(a, v, op=op, rev=True), fn(v, a))
    parts = [a[..., :3], b[..., :5], a[..., 5:9]]
    assert np.array_equal(O.concat_channels(parts), np.concatenate(parts, axis=-1))
    hs = O.hard_sigmoid(a, 1 / 6, 0.5)
    assert np.array_equal(hs, np.clip(a * np.float32(1 / 6) + np.float32(0.5), 0, 1))


def test_activation_kinds_closed_forms():
    """ActivationKind epilogues (Kernels/Nhwc.cs:83-99) against their float64 closed forms."""
    x = np.linspace(-12, 12, 4801).astype(np.float32)
    x64 = x.astype(np.float64)
    sig = 1 / (1 + np.exp(-x64))
    want = {"relu": np.maximum(x64, 0), "sigmoid": sig, "hardswish": x64 * np.clip(x64 / 6 + 0.5, 0, 1),
            "swish": x64 * sig, "gelu": 0.5 * x64 * (1 + np.vectorize(math.erf)(x64 / math.sqrt(2)))}
    for act, w in want.items():
        got = O.activation(x, act).astype(np.float64)
        assert np.max(np.abs(got - w)) <= 4e-6 * max(1.0, np.max(np.abs(w))), act


def test_bn_calibration_normalises_preactivations():
    """The committed BatchNorm folds of configs 3 / 4 (simdonnx_amd/data/bn_calibration.npz, from
    tests/golden/make_bn_calibration.py) do what they claim: at the calibration size every conv's
    pre-activation channels have mean ~0 and std ~1 (bar the epsilon-floored near-constant ones), and
    the fp16 storage contract emulated on the CPU stays within the 2e-2 bar of the fp32 detector."""
    import sys
    sys.path.insert(0, os.path.join(os.path.dirname(__file__), "golden"))
    import make_bn_calibration as M
    from oracle.interp import run_plan
    from simdonnx_amd import graphs
    for build in (lambda: graphs.mobilenetv3_small(size=640), lambda: graphs.dbnet(size=960, logit=True)):
        plan, ins = build()
        _, env = run_plan(plan, ins, keep=True)
        stds = []
        for nd in plan.nodes:
            if nd.op in ("Conv", "ConvTranspose"):
                y = M.preactivation(plan, env, nd).astype(np.float64)
                y = y.reshape(-1, y.shape[-1])
                assert np.abs(y.mean(axis=0)).max() < 2e-3, nd.name
                stds.append(y.std(axis=0))
        stds = np.concatenate(stds)
        assert np.abs(stds - 1.0).max() < 2e-3 or (np.abs(stds - 1.0) > 2e-3).mean() < 0.02
    plan, ins = graphs.dbnet()
    want = run_plan(plan, ins)
    emu = run_plan(plan, ins, f16_storage=True)
    assert max_rel(emu, want) < 2e-2


def test_bf16_storage_rounding_matches_torch():
    """The oracle's bf16 storage emulation (round to nearest even, the v_cvt_pk_bf16_f32 rounding)
    equals torch's float32 -> bfloat16 cast, ties and subnormals included."""
    import torch
    from oracle.interp import _bf16
    x = np.random.default_rng(0).standard_normal(200000).astype(np.float32) * 100
    x[:6] = [1.00390625, 1.01171875, -1.00390625, -2.5e-39, 3.0e38, 0.0]  # exact ties, subnormal, large
    assert np.array_equal(_bf16(x), torch.from_numpy(x).to(torch.bfloat16).float().numpy())
