"""The consumer extension hook and lost-device recovery through the C ABI (include/sox_backend.h).

Extension (tests/Sdcb.SimdOnnx.Tests/Api/ExtensionTests.cs:15-60, 86-120; Engine/Extensions.cs:41-50):
a consumer op "MyHardSigmoid" replaces the built-in HardSigmoid of conv -> mul -> hardsigmoid -> conv.
Its kernel lives in a code object of its own (csrc/ext_example/my_hard_sigmoid.hip, built apart from
the embedded ones and loaded with sox_backend_load_module); its emitter, registered with
sox_backend_register_ext, binds the node's values and dispatches with sox_graph_dispatch. The graph
must run it (the emitter was called, its kernel is in the dispatch list) and give the built-in's bits,
through a session and through the unit runner, and match the oracle.

Device loss (tests/Sdcb.SimdOnnx.Tests/VkDeviceLossTests.cs:13-42): the host marks the device lost;
Run then fails with DeviceLostError; Default hands out a new backend, whose session gives the bits
the first one gave before the loss.
"""
import struct

import numpy as np
import pytest

from oracle.interp import run_plan
from simdonnx_amd import build as B
from simdonnx_amd import native as N
from simdonnx_amd import synth
from simdonnx_amd.backend import HipBackend, HipInferenceSession, HipUnitRunner
from simdonnx_amd.plan import NHWC, PlanBuilder
from tests.conftest import max_rel

pytestmark = pytest.mark.gpu


def model(ext: bool):
    """ExtensionTests.Model: Conv 3x3 8->16 (+bias) -> Mul by a [1,16,1,1] const -> HardSigmoid(0.25, 0.4)
    -> Conv 1x1 16->8, input [1, 8, 12, 16]."""
    pb = PlanBuilder()
    x = pb.input((1, 8, 12, 16), NHWC, "x")
    c1 = pb.conv(x, synth.uniform(7, 1, (16, 8, 3, 3), -1, 1), synth.uniform(7, 2, (16,), -1, 1), pad=1, name="c1")
    m = pb.mul(c1, pb.const(synth.uniform(7, 3, (16, 1, 1), -1, 1), "K"), name="m")
    if ext:
        r = pb.ext("MyHardSigmoid", [m], (1, 16, 12, 16), bytes(N.HardSigmoidP(0.25, 0.4)), NHWC, "r")
    else:
        r = pb.hard_sigmoid(m, 0.25, 0.4, name="r")
    y = pb.conv(r, synth.uniform(7, 4, (8, 16, 1, 1), -1, 1), None, pad=0, name="y")
    return pb.build(y)


class MyHardSigmoid:
    """The consumer's op: EmitHip = one dispatch of its own kernel over the node's values."""

    def __init__(self, hip: HipBackend):
        with open(B.ext_example_path("my_hard_sigmoid"), "rb") as f:
            self.module = hip.load_module(f.read())
        self.emits = 0
        hip.register_ext("MyHardSigmoid", self.emit)

    def emit(self, g, node):
        self.emits += 1
        _, params = g.node(node)
        hs = N.HardSigmoidP.from_buffer_copy(params)
        ins, outs = g.node_values(node)
        count = int(np.prod(g.shape(outs[0])))
        # kernarg = the two binds, then {count, alpha, beta} and the struct's tail padding
        kp = struct.pack("<Iff4x", count, hs.alpha, hs.beta)
        return g.dispatch(node, "my_hsig_" + g.storage, [g.bind(ins[0]), g.bind(outs[0])], kp,
                          grid=((count + 255) // 256, 1, 1), module=self.module)


def run_session(graph, x, replay=False):
    with HipInferenceSession(graph) as s:
        s.set_replay(replay)
        s.set_input(x)
        s.run()
        s.set_input(x)
        return s.run().copy()


@pytest.mark.parametrize("half", [False, True, "bf16"], ids=["f32", "f16", "bf16"])
def test_extension_matches_builtin(hip, half):
    op = MyHardSigmoid(hip)
    x = np.sin(np.arange(8 * 12 * 16, dtype=np.float32) * 0.37).reshape(1, 8, 12, 16).transpose(0, 2, 3, 1).copy()
    plain_plan, ext_plan = model(False), model(True)
    plain_g = hip.graph(plain_plan, half)
    ext_g = hip.graph(ext_plan, half)
    names = [d[0] for d in ext_g.dispatches]
    print(f"[gpu] extension f16={half} dispatches={names}", flush=True)
    assert op.emits == 1 and ("my_hsig_" + {False: "f32", True: "f16", "bf16": "bf16"}[half]) in names
    assert "unary" not in names and "unary" in [d[0] for d in plain_g.dispatches]
    want = run_session(plain_g, x)
    got = run_session(ext_g, x)
    assert np.array_equal(got, want)  # same fp32 formula on the same stored operands
    assert np.array_equal(run_session(ext_g, x, replay=True), want)
    ref = run_plan(plain_plan, [x], f16_storage=half)
    assert max_rel(got, ref) < {False: 1e-4, True: 2e-3, "bf16": 1.6e-2}[half]
    # the unit runner relocates the extension dispatch's binds into its own arena window
    r = HipUnitRunner(hip, streams=2)
    r.add(plain_g)
    r.add(ext_g)
    r.input(0)[:] = x.reshape(-1)
    r.input(1)[:] = x.reshape(-1)
    r.submit()
    r.wait()
    assert np.array_equal(r.output(0), want) and np.array_equal(r.output(1), want)
    r.close()
    plain_g.release()
    ext_g.release()


def test_default_backend_recreated_after_loss(hip):
    plan = model(False)
    x = synth.normal(8, 1, (1, 12, 16, 8), 1.0)
    before = HipBackend.default()
    with HipInferenceSession(before.graph(plan, True)) as s:
        s.set_input(x)
        want = s.run().copy()
        print("[gpu] device loss: marking the device lost", flush=True)
        HipBackend.mark_lost()
        assert before.is_lost
        s.set_input(x)
        with pytest.raises(N.DeviceLostError):
            s.run()
    after = HipBackend.default()
    assert after.h.value != before.h.value
    assert not after.is_lost
    with HipInferenceSession(after.graph(plan, True)) as s2:
        s2.set_input(x)
        assert np.array_equal(s2.run(), want)
