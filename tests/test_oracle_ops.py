"""Pins the oracle's restatement of the rest of the GPU op surface (bilinear resize, pad, average
pool, DepthToSpace / SpaceToDepth, LeakyRelu / Tanh / Clip / Erf, global average pool, batched
MatMul with a broadcast operand, transpose, slice) before it checks the HIP kernels.

Expected values are the committed torch-float64 golden vectors of tests/golden/make_golden_ops.py
(library routines and the ONNX definitions), plus invariants: SpaceToDepth inverts DepthToSpace in
both channel orders, a transpose twice with inverse perms is the identity, a slice equals numpy's.
"""
import os

import numpy as np
import pytest

import oracle as O
from tests.conftest import max_rel

G = np.load(os.path.join(os.path.dirname(__file__), "golden", "golden_ops.npz"))


def _n(prefix):
    return len({k.split("_")[0] for k in G.files if k.startswith(prefix) and k[len(prefix)].isdigit()})


@pytest.mark.parametrize("i", range(_n("bil")))
def test_resize_bilinear_golden(i):
    s, relu, has_add, add_relu = G[f"bil{i}_meta"]
    add = G[f"bil{i}_add"] if has_add else None
    got = O.resize_bilinear(G[f"bil{i}_x"], float(s), float(s), add, relu=bool(relu), add_relu=bool(add_relu))
    assert got.shape == G[f"bil{i}_y"].shape
    assert max_rel(got, G[f"bil{i}_y"]) < 2e-6


@pytest.mark.parametrize("i", range(_n("pad")))
def test_pad_golden(i):
    t, l, b, r, mode, value = G[f"pad{i}_meta"]
    got = O.pad_nhwc(G[f"pad{i}_x"], int(t), int(l), int(b), int(r), int(mode), float(value))
    assert np.array_equal(got, G[f"pad{i}_y"])  # copies and fills only


@pytest.mark.parametrize("i", range(_n("avg")))
def test_avg_pool_golden(i):
    k, s, t, l, b, r, cip = (int(v) for v in G[f"avg{i}_meta"])
    got = O.avg_pool(G[f"avg{i}_x"], (k, k), (s, s), (t, l, b, r), bool(cip))
    assert got.shape == G[f"avg{i}_y"].shape
    assert max_rel(got, G[f"avg{i}_y"]) < 2e-6


@pytest.mark.parametrize("i", range(_n("d2s")))
def test_depth_to_space_golden_and_inverse(i):
    x, b = G[f"d2s{i}_x"], int(G[f"d2s{i}_meta"][0])
    for crd, key in ((True, "crd"), (False, "dcr")):
        y = O.depth_to_space(x, b, crd)
        assert np.array_equal(y, G[f"d2s{i}_{key}"])
        assert np.array_equal(O.depth_to_space(y, b, crd, inverse=True), x)


@pytest.mark.parametrize("i", range(_n("s2d")))
def test_space_to_depth_golden(i):
    x, b = G[f"s2d{i}_x"], int(G[f"s2d{i}_meta"][0])
    for crd, key in ((True, "crd"), (False, "dcr")):
        assert np.array_equal(O.depth_to_space(x, b, crd, inverse=True), G[f"s2d{i}_{key}"])


def test_unary2_golden():
    x = G["un_x"]
    assert max_rel(O.unary2(x, "LeakyRelu", 0.1), G["un_leaky01"]) < 1e-6
    assert max_rel(O.unary2(x, "LeakyRelu", 2.0), G["un_leaky2"]) < 1e-6  # the a > 1 (min) branch
    assert max_rel(O.unary2(x, "Tanh", 1.0, 1.0), G["un_tanh"]) < 1e-6
    assert max_rel(O.unary2(x, "Tanh", 2.0 / 3.0, 1.7159), G["un_tanh_scaled"]) < 1e-6
    assert np.array_equal(O.unary2(x, "Clip", -1.0, 0.75), G["un_clip"])
    assert max_rel(O.unary2(x, "Erf"), G["un_erf"]) < 5e-7  # A&S 7.1.26: |err| <= 1.5e-7


def test_gap_and_matmul_broadcast_golden():
    assert max_rel(O.global_avg_pool(G["gap_x"]), G["gap_y"]) < 1e-6
    for i in range(_n("mm")):
        assert max_rel(O.matmul_bcast(G[f"mm{i}_a"], G[f"mm{i}_b"]), G[f"mm{i}_y"]) < 1e-5


def test_transpose_slice_index_ops():
    x = G["gap_x"]  # [2, 13, 11, 40]
    perm = (0, 3, 1, 2)
    y = O.transpose(x, perm)
    assert y.shape == (2, 40, 13, 11) and y[1, 7, 4, 9] == x[1, 4, 9, 7]
    assert np.array_equal(O.transpose(y, np.argsort(perm)), x)
    s = O.slice_(x, (1, 10, 3), (12, 2, 40), (1, 2, 3), (2, -3, 5))
    assert np.array_equal(s, x[:, 1:12:2, 10:2:-3, 3:40:5])


def test_ctc_argmax_golden():
    """Fused projection + argmax + softmax probability (CtcProjection.ArgMax) vs torch float64."""
    idx, prob = O.ctc_argmax(G["ctc_x"], G["ctc_w"], G["ctc_b"])
    assert np.array_equal(idx, G["ctc_idx"])
    assert max_rel(prob, G["ctc_prob"]) < 1e-5


def test_ctc_argmax_ties_and_invalid():
    """Equal logits keep the first column; a non-finite logit raises (MatMul.ArgMax.cs:267-278)."""
    x, w, b = G["ctc_x"][:8].copy(), G["ctc_w"].copy(), G["ctc_b"].copy()
    w[:, 900] = w[:, 5]
    b[5] = b[900] = 100.0  # both dominate every row, exactly equal
    idx, prob = O.ctc_argmax(x, w, b)
    assert (idx == 5).all() and np.allclose(prob, 0.5, rtol=1e-5)
    x[3, 7] = np.inf
    with pytest.raises(ValueError):
        O.ctc_argmax(x, w, b)


def test_builtin_ext_ops_golden():
    """SafeDiv, ChannelShift and UpHead (Engine/Fusions/*.cs, Kernels/FusedKernels.cs) vs torch / numpy."""
    assert max_rel(O.safe_div(G["sd_a"], G["sd_b"], 1e-3, -4.0, 4.0), G["sd_y"]) < 1e-6
    ends, offs = [4, 8, 12, 16, 20], [-2, -1, 0, 1, 2]
    for axis in (2, 3):
        assert np.array_equal(O.channel_shift(G["sh_x"], axis, ends, offs), G[f"sh_y{axis}"])
    # a stored skip; and the skip recomputed by its conv (the oracle's direct conv, then the stored form)
    got0 = O.up_head(G["uh0_x"], G["uh0_skip"], G["uh0_w"], G["uh0_b"], 2.0, resize_relu=True, skip_relu=True,
                     act="sigmoid")
    assert max_rel(got0, G["uh0_y"]) < 2e-6
    skip = O.conv(G["uh1_skin"], G["uh1_wsc"], G["uh1_bsc"], None, stride=(1, 1), pads=(1, 1, 1, 1), act="relu",
                  algo=1)
    got1 = O.up_head(G["uh1_x"], skip, G["uh1_w"], G["uh1_b"], 2.0, resize_relu=True, skip_relu=True, act="sigmoid")
    assert max_rel(got1, G["uh1_y"]) < 2e-6


def test_pixels_tensor_round_trip_and_channel_order():
    """ImageTensor.FromPixels / ToPixels (Imaging/ImageTensor.cs:322-430): with the unit table
    (byte / 255) a padded tensor cropped back gives the original bytes (both channel orders, 3 and 4
    bytes per pixel, alpha from the source); tensor channel 0 is byte 0 of a pixel for BGR bytes with
    a BGR table and byte 2 when they differ; the padding repeats the edge pixel."""
    rng = np.random.default_rng(5)
    unit = np.tile(np.arange(256, dtype=np.float32) / np.float32(255), 3)
    for bpp in (3, 4):
        for swap in (0, 1):
            src = rng.integers(0, 256, (7, 9 * bpp), dtype=np.uint8)
            t = O.from_pixels(src, 9, 7, bpp, unit, swap, 16, 12, pad_left=3, pad_top=2)
            assert t[0, 0, 0] == unit[src[0, 2 * swap]] and t[11, 15, 1] == unit[src[6, (8 * bpp) + 1]]
            back = O.to_pixels(t, 9, 7, bpp, swap, 3, 2, 255.0, alpha=src if bpp == 4 else None)
            assert np.array_equal(back, src)
    # ToByte rounds half up and clamps: 0.5/255 -> 1 (0.5 + 0.5), -0.1 -> 0, 1.2 -> 255
    t = np.array([[[0.5 / 255, -0.1, 1.2]]], np.float32)
    assert O.to_pixels(t, 1, 1, 3, 0).tolist() == [[1, 0, 255]]


@pytest.mark.parametrize("k,s,pads,relu", [((2, 2), (2, 2), (0, 0, 0, 0), False), ((3, 3), (2, 2), (1, 1, 1, 1), True),
                                           ((3, 3), (1, 1), (1, 1, 1, 1), False), ((2, 3), (2, 1), (0, 1, 1, 1), True)])
def test_max_pool_matches_torch(k, s, pads, relu):
    """Nhwc.MaxPool against torch's max_pool2d in float64 over an explicit -inf padding (taps outside
    the image never win), then the fused relu."""
    import torch
    x = np.random.default_rng(5).standard_normal((2, 13, 11, 24)).astype(np.float32)
    got = O.max_pool(x, k, s, pads, relu)
    t = torch.from_numpy(x.astype(np.float64)).permute(0, 3, 1, 2)
    t = torch.nn.functional.pad(t, (pads[1], pads[3], pads[0], pads[2]), value=float("-inf"))
    want = torch.nn.functional.max_pool2d(t, k, s).permute(0, 2, 3, 1).numpy()
    if relu:
        want = np.maximum(want, 0.0)
    assert got.shape == want.shape
    assert np.array_equal(got, want.astype(np.float32))  # a max selects one of its inputs


def test_max_pool_empty_window_is_zero():
    """A window lying wholly in the padding outputs 0 (Nhwc.cs:765), not -inf: a 1x1 pool with pad 1
    gives a zero border around the (relu'd) image, checked element by element."""
    x = np.random.default_rng(6).standard_normal((1, 4, 5, 3)).astype(np.float32)
    got = O.max_pool(x, (1, 1), (1, 1), (1, 1, 1, 1), relu=True)
    want = np.zeros((1, 6, 7, 3), np.float32)
    want[:, 1:5, 1:6] = np.maximum(x, 0.0)
    assert np.array_equal(got, want)
