"""The HIP unit runner (sox_unit_runner_*, HipUnitRunner; VkUnitRunner's contract,
Backends/Vulkan/VkUnitRunner.cs:5-337): units of different shapes in two waves on several streams
give, each, the bits a session of the same graph gives (the same kernels on the same inputs), and
match the oracle; a second run after Clear with other units reuses the grown buffers."""
import numpy as np
import pytest

from oracle.interp import run_plan
from simdonnx_amd import synth
from simdonnx_amd.backend import HipInferenceSession, HipUnitRunner
from simdonnx_amd.plan import NHWC, PlanBuilder
from tests.conftest import max_rel

pytestmark = pytest.mark.gpu


def line_plan(w, seed=71):
    """A small recognizer-like unit: a text line [1, 3, 32, w] -> conv 3x3 s2 + GELU -> 1x1 conv ->
    [1, 16, 16, w/2]."""
    pb = PlanBuilder()
    x = pb.input((1, 3, 32, w), NHWC, "line")
    y = pb.conv(x, synth.he_normal(seed, 1, (32, 3, 3, 3)), synth.uniform(seed, 2, (32,), -0.1, 0.1), stride=2, pad=1,
                act="gelu", name="c1")
    y = pb.conv(y, synth.he_normal(seed, 3, (16, 32, 1, 1)), None, name="c2")
    return pb.build(y)


@pytest.mark.parametrize("half", [False, True], ids=["f32", "f16"])
def test_unit_runner_waves_match_sessions(hip, half):
    widths = [64, 160, 320, 96, 480, 256]
    plans = [line_plan(w) for w in widths]
    graphs = [hip.graph(p, half) for p in plans]
    xs = [synth.normal(72, i, (1, 32, w, 3), 1.0) for i, w in enumerate(widths)]
    r = HipUnitRunner(hip, streams=4)
    for run in range(2):
        order = list(range(len(widths))) if run == 0 else [5, 2, 0]
        r.clear()
        for k, i in enumerate(order):
            r.add(graphs[i])
            if k == 2:
                r.cut()  # two waves: the first three units, then the rest
        for k, i in enumerate(order):
            r.input(k)[:] = xs[i].reshape(-1)
        print(f"[gpu] unit runner run {run} f16={half} units={order} waves={r.waves}", flush=True)
        r.submit()
        r.wait(0)
        r.wait()
        for k, i in enumerate(order):
            with HipInferenceSession(graphs[i]) as s:
                s.set_input(xs[i])
                want = s.run().copy()
            got = r.output(k)
            assert np.array_equal(got, want), (run, i)
            ref = run_plan(plans[i], [xs[i]], f16_storage=half)
            assert max_rel(got, ref) < (2e-2 if half else 1e-4)
    r.close()
