"""The SE gate inside the launch of the depthwise conv that produces its input (sox_dwt_*_se, taken
under SIMDONNX_HIP_SE_IN_DW; slower than the separate passes on MI355X, so not the default): the
reference's depthwise.comp, gap_part.comp and se_gate.comp (Backends/Vulkan/VkGraph.cs:595-605,
949-965) as one dispatch. Every tile workgroup stores its GAP partials and counts itself with a vector
atomic; the last tile of a 64-channel group runs fc1 for the group, the last group's workgroup runs
fc2 for the image. Checked:
  - one depthwise_se dispatch per block, no gap_part / se_gate dispatch;
  - the output equals the separate passes' (the default) bit for bit: the same sums in
    the same order, so any partial read before its tile stored it, or a count that missed, shows;
  - five runs in a row, runs of a captured replay, and a unit-runner wave beside other units give the
    same bits (the counters return to 0 after every launch);
  - the oracle on the plan within the storage contract (1e-4 fp32, 2e-2 16-bit).
Cases: 1, 2 and 9 channel groups (c = 16, 96, 576: the largest MobileNetV3-small gate), r up to 256,
k3 / k5, stride 1 / 2, folded into the projection (one image) and not folded (two images, the gate
feeding a channel broadcast).
"""
import numpy as np
import pytest

from oracle.interp import run_plan
from simdonnx_amd import synth
from simdonnx_amd.backend import HipInferenceSession, HipUnitRunner
from simdonnx_amd.plan import NHWC, PlanBuilder
from tests.conftest import max_rel

pytestmark = pytest.mark.gpu

CASES = {  # c, r, k, stride, h, w, images
    "c16-k3s2": (16, 8, 3, 2, 160, 160, 1),
    "c96-k5s2": (96, 24, 5, 2, 80, 80, 1),
    "c240-k5s1": (240, 64, 5, 1, 40, 40, 1),
    "c576-k5s1": (576, 144, 5, 1, 20, 20, 1),
    "c576-r256-k3s1": (576, 256, 3, 1, 20, 20, 1),
    "c72-k3s1-2img": (72, 24, 3, 1, 44, 36, 2),
    "c576-k5s1-2img": (576, 144, 5, 1, 20, 20, 2),
}


def se_block(c, r, k, s, h, w, n, seed=91):
    """Depthwise k x k + hardswish -> SE gate (ReLU, hard sigmoid) -> x * gate -> 1x1 projection."""
    pb = PlanBuilder()
    xv = pb.input((n, c, h, w), NHWC, "x")
    d = pb.conv(xv, synth.uniform(seed, 1, (c, 1, k, k), -0.5, 0.5), synth.uniform(seed, 2, (c,), -0.1, 0.1),
                stride=(s, s), pad=(k // 2,) * 4, group=c, act="hardswish", name="dw")
    gate = pb.channel_gate(d, synth.uniform(seed, 3, (r, c, 1, 1), -0.3, 0.3),
                           synth.uniform(seed, 4, (r,), -0.1, 0.1), synth.uniform(seed, 5, (c, r, 1, 1), -0.3, 0.3),
                           synth.uniform(seed, 6, (c,), -0.1, 0.1), act1="relu", hard=True, alpha=1.0 / 6.0,
                           beta=0.5, name="se")
    m = pb.mul(d, gate, name="se_scale")
    y = pb.conv(m, synth.uniform(seed, 7, (48, c, 1, 1), -0.2, 0.2), synth.uniform(seed, 8, (48,), -0.1, 0.1),
                name="project")
    x = synth.uniform(seed, 9, (n, h, w, c), -1, 1)
    return pb.build(y), x


@pytest.fixture(autouse=True)
def _se_in_depthwise(monkeypatch):
    monkeypatch.setenv("SIMDONNX_HIP_SE_IN_DW", "1")


def _runs(g, x, times, replay=False):
    with HipInferenceSession(g) as s:
        if replay:
            s.set_replay(True)
        s.set_input(x)
        return [s.run().copy() for _ in range(times)]


@pytest.mark.parametrize("storage", ["f16", "bf16", "f32"])
@pytest.mark.parametrize("case", list(CASES))
def test_se_in_depthwise_launch_matches_separate_passes(hip, case, storage, monkeypatch):
    c, r, k, s, h, w, n = CASES[case]
    plan, x = se_block(c, r, k, s, h, w, n)
    print(f"[gpu] se in depthwise {case} {storage}", flush=True)
    g = hip.graph(plan, storage)
    labels = [d[0] for d in g.dispatches]
    assert labels.count("depthwise_se") == 1 and "se_gate" not in labels and "gap_part" not in labels, labels
    assert g.sync_bytes >= n * ((c + 63) // 64 + 1) * 4
    runs = _runs(g, x, 5)
    replays = _runs(g, x, 3, replay=True)
    g.release()
    monkeypatch.delenv("SIMDONNX_HIP_SE_IN_DW")
    monkeypatch.setenv("SIMDONNX_HIP_DWT_ROWS", "8")  # the fused gate's tiling: the same GAP partial sums
    g2 = hip.graph(plan, storage)
    labels2 = [d[0] for d in g2.dispatches]
    assert "depthwise_se" not in labels2 and "se_gate" in labels2, labels2
    sep = _runs(g2, x, 1)[0]
    g2.release()
    for i, got in enumerate(runs + replays):
        assert got.tobytes() == sep.tobytes(), f"run {i}: max diff {np.abs(got - sep).max()}"
    emu = {"f16": True, "bf16": "bf16", "f32": False}[storage]  # the storage contract
    want = run_plan(plan, [x], f16_storage=emu)
    err = max_rel(runs[0], want)
    print(f"[gpu] {case} {storage}: vs oracle {err:.2e}", flush=True)
    assert err < (1e-4 if storage == "f32" else 2e-2)


def test_se_in_depthwise_launch_in_unit_runner(hip):
    """Units of SE blocks of three sizes, two of each, in one wave on four streams (each unit with its
    own counters): every output equals a session's of the same graph."""
    cases = ["c96-k5s2", "c576-k5s1", "c72-k3s1-2img"]
    built = [se_block(*CASES[cs]) for cs in cases]
    graphs = [hip.graph(p, "f16") for p, _ in built]
    want = [_runs(g, x, 1)[0] for g, (_, x) in zip(graphs, built)]
    r = HipUnitRunner(hip, streams=4)
    order = [0, 1, 2, 1, 0, 2]
    for rep in range(2):
        print(f"[gpu] se units run {rep}", flush=True)
        r.clear()
        for i in order:
            r.add(graphs[i])
        for k, i in enumerate(order):
            r.input(k)[:] = built[i][1].reshape(-1)
        r.submit()
        r.wait()
        for k, i in enumerate(order):
            assert r.output(k).tobytes() == want[i].tobytes(), (rep, k, i)
    r.close()
    for g in graphs:
        g.release()
