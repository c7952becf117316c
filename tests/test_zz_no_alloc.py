"""The allocation-free CTC head (sox_ctc_argmax_noalloc, include/sox_backend.h) against the allocating
one (sox_ctc_argmax) through the C ABI: two calls in a row, the second on a smaller input, give the
same indices and probabilities bit for bit (same kernels, same column ranges; the partials live in the
GPU's static scratch instead of a per-object workspace), the status word is cleared by every call,
and a call whose partials exceed the scratch is refused with an error. The calls make no device or
pinned allocation (sox_alloc_count unchanged), and a call captured into a HIP graph replays to the
same bits, three times, with eager work between the replays."""
import ctypes

import numpy as np
import pytest

from simdonnx_amd import native as N
from simdonnx_amd import synth
from simdonnx_amd.backend import HipCtcProjection, HipInferenceSession
from simdonnx_amd.plan import PlanBuilder

pytestmark = pytest.mark.gpu


def f16(a):
    return np.asarray(a, np.float32).astype(np.float16).astype(np.float32)


def features_session(hip, x):
    pb = PlanBuilder()
    xv = pb.input(x.shape, None, "features")
    y = pb.unary("Copy", xv, name="copy")
    s = HipInferenceSession(hip.graph(pb.build(y), True))
    s.set_input(x)
    s.run()
    return s, xv


class DeviceOut:
    """Caller-owned device outputs (the entry point allocates nothing itself)."""

    def __init__(self, rows):
        self.rows = rows
        self.ptrs = []
        for nbytes in (rows * 4, rows * 4, 4):
            p = N.c_void_p()
            N.check(N.thin().sox_malloc(ctypes.byref(p), nbytes), "sox_malloc")
            self.ptrs.append(p)

    def read(self, stream):
        idx = np.empty(self.rows, np.int32)
        prob = np.empty(self.rows, np.float32)
        st = np.empty(1, np.int32)
        for host, dev, nb in ((idx, self.ptrs[0], self.rows * 4), (prob, self.ptrs[1], self.rows * 4), (st, self.ptrs[2], 4)):
            N.check(N.thin().sox_memcpy_d2h(host.ctypes.data, dev, nb, stream), "d2h")
        N.check(N.thin().sox_stream_sync(stream), "sync")
        return idx, prob, int(st[0])

    def free(self):
        for p in self.ptrs:
            N.thin().sox_free(p)


def noalloc(ctc, s, xv, batch, rows, out):
    before = N.thin().sox_alloc_count()
    rc = N.backend().sox_ctc_argmax_noalloc(ctc.h, s.h, xv, batch, rows, out.ptrs[0], out.ptrs[1], out.ptrs[2])
    assert N.thin().sox_alloc_count() == before, "the allocation-free entry point allocated"
    return rc


def test_ctc_noalloc_matches_allocating_entry(hip):
    inner, columns = 192, 6625
    w = f16(synth.normal(51, 2, (inner, columns), 0.1))
    b = synth.uniform(51, 3, (columns,), -0.5, 0.5)
    ctc = HipCtcProjection(hip, w, b, inner, columns)
    for call, (batch, rows) in enumerate(((32, 80), (1, 70))):  # the second call is smaller
        x = f16(synth.normal(51, 10 + call, (batch * rows, inner), 1.0))
        s, xv = features_session(hip, x)
        out = DeviceOut(batch * rows)
        with s:
            print(f"[gpu] no-alloc ctc call {call}: {batch} x {rows} rows", flush=True)
            want_i, want_p = ctc.argmax(s, xv, batch, rows)
            N.check(noalloc(ctc, s, xv, batch, rows, out), "sox_ctc_argmax_noalloc")
            idx, prob, status = out.read(N.backend().sox_session_stream(s.h))
        out.free()
        assert status == 0
        assert np.array_equal(idx, want_i)
        assert np.array_equal(prob, want_p)
    ctc.close()


def test_ctc_noalloc_status_and_limit(hip):
    inner, columns = 64, 1100
    w = f16(synth.normal(52, 2, (inner, columns), 0.1))
    ctc = HipCtcProjection(hip, w, None, inner, columns)
    x = f16(synth.normal(52, 1, (64, inner), 1.0))
    bad = x.copy()
    bad[10, 3] = np.inf
    out = DeviceOut(64)
    for data, want_status in ((bad, 1), (x, 0)):  # the second call clears what the first set
        s, xv = features_session(hip, data)
        with s:
            print(f"[gpu] no-alloc ctc status case {want_status}", flush=True)
            N.check(noalloc(ctc, s, xv, 1, 64, out), "sox_ctc_argmax_noalloc")
            idx, prob, status = out.read(N.backend().sox_session_stream(s.h))
            assert status == want_status
            if want_status == 0:
                want_i, want_p = ctc.argmax(s, xv, 1, 64)
                assert np.array_equal(idx, want_i) and np.array_equal(prob, want_p)
    out.free()
    ctc.close()
    # partials beyond the static scratch (>= 21 column ranges of the 6625-class head x 40000 rows x 12
    # bytes > 8 MiB): refused before anything is launched
    wide = HipCtcProjection(hip, f16(synth.normal(52, 3, (192, 6625), 0.1)), None, 192, 6625)
    big_rows = 40000
    s, xv = features_session(hip, np.zeros((big_rows, 192), np.float32))
    outb = DeviceOut(big_rows)
    with s:
        rc = noalloc(wide, s, xv, 1, big_rows, outb)
        assert rc == N.SOX_E_INVALID
        assert b"scratch" in N.backend().sox_last_error()
    outb.free()
    wide.close()


def test_ctc_noalloc_under_graph_capture(hip):
    """The entry point called while the session's stream captures a HIP graph: the graph replays the
    two passes into the caller's arrays. Three replays, each after the outputs were overwritten and an
    eager (allocating) call ran, give the eager result bit for bit."""
    inner, columns, batch, rows = 192, 6625, 8, 80
    w = f16(synth.normal(53, 2, (inner, columns), 0.1))
    b = synth.uniform(53, 3, (columns,), -0.5, 0.5)
    ctc = HipCtcProjection(hip, w, b, inner, columns)
    x = f16(synth.normal(53, 1, (batch * rows, inner), 1.0))
    s, xv = features_session(hip, x)
    out = DeviceOut(batch * rows)
    T = N.thin()
    with s:
        stream = N.backend().sox_session_stream(s.h)
        want_i, want_p = ctc.argmax(s, xv, batch, rows)
        print("[gpu] no-alloc ctc under capture", flush=True)
        N.check(T.sox_graph_begin(stream), "capture")
        rc = noalloc(ctc, s, xv, batch, rows, out)
        ex = N.c_void_p()
        N.check(T.sox_graph_end(stream, ctypes.byref(ex)), "capture end")
        N.check(rc, "sox_ctc_argmax_noalloc under capture")
        junk = np.full(batch * rows, -7, np.int32)
        try:
            for rep in range(3):
                for p in out.ptrs[:2]:
                    N.check(T.sox_memcpy_h2d(p, junk.ctypes.data, junk.nbytes, stream), "overwrite")
                N.check(T.sox_memcpy_h2d(out.ptrs[2], junk.ctypes.data, 4, stream), "overwrite")
                ei, ep = ctc.argmax(s, xv, batch, rows)  # eager work between the replays
                assert np.array_equal(ei, want_i) and np.array_equal(ep, want_p)
                N.check(T.sox_graph_launch(ex, stream), "replay")
                idx, prob, status = out.read(stream)
                assert status == 0, rep
                assert np.array_equal(idx, want_i) and np.array_equal(prob, want_p), rep
        finally:
            T.sox_graph_destroy(ex)
    out.free()
    ctc.close()
