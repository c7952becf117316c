"""The CTC head on the device (sox_ctc_*, HipCtcProjection) vs the oracle's CtcProjection.ArgMax
(Decoding/Kernels/MatMul.ArgMax.cs; the reference's CTC tests compare fused and unfused heads the
same way). Both sides see the same fp16-rounded features and weights and compute in fp32, so the
logits differ only in summation order: indices must match except on rows whose two best float64
logits are closer than 1e-3 (such rows are counted and must be rare), probabilities within 1e-3."""
import numpy as np
import pytest

import oracle as O
from simdonnx_amd import graphs, synth
from simdonnx_amd.backend import HipCtcProjection, HipInferenceSession
from simdonnx_amd.native import SoxError
from simdonnx_amd.plan import PlanBuilder
from tests.conftest import max_rel

pytestmark = pytest.mark.gpu


def f16(a):
    return np.asarray(a, np.float32).astype(np.float16).astype(np.float32)


def features_session(hip, x):
    """A session whose arena holds x (fp16) as its input value 0."""
    pb = PlanBuilder()
    xv = pb.input(x.shape, None, "features")
    y = pb.unary("Copy", xv, name="copy")
    s = HipInferenceSession(hip.graph(pb.build(y), True))
    s.set_input(x)
    s.run()
    return s, xv


def check(x, w, b, idx, prob):
    want_i, want_p = O.ctc_argmax(x, w, b)
    lg = x.astype(np.float64) @ w.astype(np.float64) + (0 if b is None else b.astype(np.float64))
    top2 = np.sort(lg, axis=1)[:, -2:]
    near = (top2[:, 1] - top2[:, 0]) < 1e-3
    mism = idx != want_i
    assert not (mism & ~near).any(), np.nonzero(mism & ~near)[0][:10]
    assert mism.sum() <= max(2, len(idx) // 500)
    assert max_rel(prob[~mism], want_p[~mism]) < 1e-3


@pytest.mark.parametrize("rows,inner,columns,bias", [(70, 64, 1100, True), (2560, 192, 6625, True),
                                                     (333, 256, 2048, False), (128, 80, 1030, True)])
def test_ctc_matches_oracle(hip, rows, inner, columns, bias):
    x = f16(synth.normal(41, 1, (rows, inner), 1.0))
    w = f16(synth.normal(41, 2, (inner, columns), 0.1))
    b = synth.uniform(41, 3, (columns,), -0.5, 0.5) if bias else None
    print(f"[gpu] ctc rows={rows} inner={inner} columns={columns}", flush=True)
    ctc = HipCtcProjection(hip, w, b, inner, columns)
    assert ctc.is_fused
    s, xv = features_session(hip, x)
    with s:
        idx, prob = ctc.argmax(s, xv, 1, rows)
    check(x, w, b, idx, prob)


def test_ctc_ties_invalid_and_unfused(hip):
    x = f16(synth.normal(42, 1, (64, 64), 1.0))
    w = f16(synth.normal(42, 2, (64, 1100), 0.1))
    w[:, 900] = w[:, 5]
    b = np.zeros(1100, np.float32)
    b[5] = b[900] = 100.0
    ctc = HipCtcProjection(hip, w, b, 64, 1100)
    s, xv = features_session(hip, x)
    with s:
        idx, prob = ctc.argmax(s, xv, 2, 32)
        assert (idx == 5).all() and np.allclose(prob, 0.5, rtol=1e-3)
    x[10, 3] = np.inf
    s, xv = features_session(hip, x)
    with s:
        with pytest.raises(SoxError, match="invalid"):
            ctc.argmax(s, xv, 1, 64)
    narrow = HipCtcProjection(hip, w[:, :1000], b[:1000], 64, 1000)  # columns < 1024: not fused
    assert not narrow.is_fused
    s, xv = features_session(hip, f16(synth.normal(42, 3, (64, 64), 1.0)))
    with s:
        assert narrow.argmax(s, xv, 1, 64) is None


def test_recognizer_features_to_ctc(hip):
    """The recognizer (batch 32) up to its final LayerNorm, then the fused head on those device
    features, against the oracle head on the same features read back."""
    plan, ins, (hw, hb) = graphs.svtr(head="features")
    ctc = HipCtcProjection(hip, f16(hw), hb, hw.shape[0], hw.shape[1])
    with HipInferenceSession(hip.graph(plan, True)) as s:
        s.set_input(ins[0])
        s.run()
        feats = s.read_value(plan.output).reshape(-1, hw.shape[0])
        idx, prob = ctc.argmax(s, plan.output, 32, feats.shape[0] // 32)
    check(feats, f16(hw), hb, idx, prob)


def test_ctc_few_rows_many_columns(hip):
    """One short line against the full 6625-class head: the column ranges are capped at 64 (one merge
    wave per row) instead of one per CU."""
    x = f16(synth.normal(43, 1, (40, 192), 1.0))
    w = f16(synth.normal(43, 2, (192, 6625), 0.1))
    b = synth.uniform(43, 3, (6625,), -0.5, 0.5)
    ctc = HipCtcProjection(hip, w, b, 192, 6625)
    s, xv = features_session(hip, x)
    with s:
        res = ctc.argmax(s, xv, 1, 40)
    assert res is not None
    check(x, w, b, *res)


def test_ctc_rejects_overwritten_and_fp32_features(hip):
    """A mid-graph value whose arena range a later node reuses, and an fp32 session, are errors
    (SOX_E_INVALID), not the unfused head's None."""
    x = f16(synth.normal(44, 1, (64, 64), 1.0))
    w = f16(synth.normal(44, 2, (64, 1100), 0.1))
    ctc = HipCtcProjection(hip, w, None, 64, 1100)
    pb = PlanBuilder()
    xv = pb.input(x.shape, None, "x")
    a = pb.unary("Relu", xv, name="a")
    bb = pb.unary("Sigmoid", a, name="b")
    c = pb.unary("Copy", bb, name="c")  # reuses a's buffer once a is dead
    plan = pb.build(c)
    assert plan.buf_offset[plan.values[a].buf] == plan.buf_offset[plan.values[c].buf]
    with HipInferenceSession(hip.graph(plan, True)) as s:
        s.set_input(x)
        s.run()
        with pytest.raises(SoxError, match="overwrites"):
            ctc.argmax(s, a, 1, 64)
        assert ctc.argmax(s, c, 1, 64) is not None
    with HipInferenceSession(hip.graph(plan, False)) as s:
        s.set_input(x)
        s.run()
        with pytest.raises(SoxError, match="fp16"):
            ctc.argmax(s, c, 1, 64)
