"""Shared session buffers (sox_buffer_pool: VkBufferPool / VkSessionBuffers, Backends/Vulkan/VkBatch.cs:6-25,
VkSession.cs:10-55), as tests/Sdcb.SimdOnnx.Tests/Api/VkBatchTests.cs:55-83 checks them:
  - a small session on a pool runs and matches a session with its own slab, bit for bit;
  - a larger session on the same pool regrows the buffers: the small one is then stale and running it
    fails (SOX_E_INVALID, the reference's InvalidOperationException);
  - the large session, and a small session made after the growth, match their own-slab runs bit for
    bit, and nothing goes stale then;
  - the pool holds one slab the size of the largest session's.
"""
import numpy as np
import pytest

from simdonnx_amd import native as N
from simdonnx_amd import synth
from simdonnx_amd.backend import HipInferenceSession
from simdonnx_amd.plan import NHWC, PlanBuilder

pytestmark = pytest.mark.gpu


def _model(h, w, seed=111):
    """A two-conv model of the test's shape (8 -> 16 -> 4 channels, 3x3 then 1x1)."""
    pb = PlanBuilder()
    x = pb.input((1, 8, h, w), NHWC, "x")
    y = pb.conv(x, synth.normal(seed, 1, (16, 8, 3, 3), 0.2), synth.uniform(seed, 2, (16,), -0.1, 0.1), pad=1,
                act="relu", name="c1")
    z = pb.conv(y, synth.normal(seed, 3, (4, 16, 1, 1), 0.2), synth.uniform(seed, 4, (4,), -0.1, 0.1), name="c2")
    return pb.build(z)


def _own(hip, plan, x, storage):
    with HipInferenceSession(hip.graph(plan, storage)) as s:
        s.set_input(x)
        return s.run().copy()


@pytest.mark.parametrize("storage", ["f32", "f16"])
def test_pool_growth_makes_earlier_sessions_stale(hip, storage):
    small, large = _model(6, 5), _model(24, 20)
    xs = synth.normal(112, 1, (1, 6, 5, 8), 1.0)
    xl = synth.normal(112, 2, (1, 24, 20, 8), 1.0)
    print(f"[gpu] buffer pool {storage}", flush=True)
    with hip.create_buffer_pool() as pool:
        gs, gl = hip.graph(small, storage), hip.graph(large, storage)
        s1 = HipInferenceSession(gs, pool)
        s1.set_input(xs)
        s1.submit()
        s1.wait()
        assert s1.output.tobytes() == _own(hip, small, xs, storage).tobytes()
        assert not s1.is_stale
        gen = pool.generation

        s2 = HipInferenceSession(gl, pool)
        assert s1.is_stale, "a larger session should regrow the pool"
        assert pool.generation > gen
        with pytest.raises(N.SoxError, match="stale"):
            s1.run()
        with pytest.raises(N.SoxError):
            s1.set_input(xs)
        s2.set_input(xl)
        got = s2.run().copy()
        assert got.tobytes() == _own(hip, large, xl, storage).tobytes()

        # a session made after the growth fits in the grown buffers: nothing goes stale
        s3 = HipInferenceSession(gs, pool)
        assert not s2.is_stale and not s3.is_stale
        s3.set_input(xs)
        assert s3.run().tobytes() == _own(hip, small, xs, storage).tobytes()
        s2.set_input(xl)
        assert s2.run().tobytes() == got.tobytes()
        # one slab: the largest session's (grown by at least half), not one per session
        assert gl.arena_bytes <= pool.arena_bytes < gl.arena_bytes + gs.arena_bytes + gl.arena_bytes // 2 + 256
        for s in (s1, s2, s3):
            s.close()
        gs.release()
        gl.release()


def test_pool_outlives_its_last_session(hip):
    """Destroying the pool while a session still borrows it keeps the buffers until that session goes."""
    plan = _model(6, 5)
    x = synth.normal(113, 1, (1, 6, 5, 8), 1.0)
    pool = hip.create_buffer_pool()
    g = hip.graph(plan, True)
    s = HipInferenceSession(g, pool)
    pool.close()
    s.set_input(x)
    assert s.run().tobytes() == _own(hip, plan, x, True).tobytes()
    s.close()
    g.release()
