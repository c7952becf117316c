"""Writes the golden vectors that pin the CPU oracle: closed forms computed by torch in float64.

The reference ships no numeric vectors for this path (its tests draw inputs from System.Random and
compare kernels with each other or with hand loops; EngineTests.cs:131-212, Avx512KernelTests.cs),
so the vectors are the mathematics itself: cross-correlation with zero / constant / reflect padding,
ConvTranspose, Gemm, batched MatMul, LayerNorm, softmax, scaled-dot-product attention, global
average pooling, the SE gate and nearest resize, each with the ONNX-defined activation. Inputs come
from simdonnx_amd.synth (seeded); the file stores the inputs and the float64 results rounded to float32.

Run:  python tests/golden/make_golden.py      (writes tests/golden/golden.npz, ~3 MB)
"""
from __future__ import annotations

import os
import sys

import numpy as np
import torch
import torch.nn.functional as F

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from simdonnx_amd import synth  # noqa: E402

ACTS = ["none", "relu", "sigmoid", "gelu", "hardswish", "swish"]


def act64(y, act):
    if act == "relu":
        return torch.relu(y)
    if act == "sigmoid":
        return torch.sigmoid(y)
    if act == "gelu":
        return 0.5 * y * (1.0 + torch.erf(y / np.sqrt(2.0)))
    if act == "hardswish":
        return y * torch.clamp(y / 6.0 + 0.5, 0.0, 1.0)
    if act == "swish":
        return y * torch.sigmoid(y)
    return y


def t64(a):
    return torch.from_numpy(np.asarray(a, dtype=np.float64))


def conv_ref(x, w, b, stride, pads, group, act, pad_mode, pad_value, add=None):
    """x NHWC, w [oc, ic/g, kh, kw]; pads (top, left, bottom, right)."""
    xt = t64(x).permute(0, 3, 1, 2)
    pt, pl, pb, pr = pads
    if pad_mode == 1:
        xt = F.pad(xt, (pl, pr, pt, pb), mode="reflect")
    else:
        xt = F.pad(xt, (pl, pr, pt, pb), mode="constant", value=float(pad_value))
    y = F.conv2d(xt, t64(w), None if b is None else t64(b), stride=stride, groups=group)
    y = y.permute(0, 2, 3, 1)
    if add is not None:
        y = y + t64(add)
    return act64(y, act).numpy()


def main():
    out = {}
    seed = 7
    tid = [100]

    def U(shape, a=-1.0, b=1.0):
        tid[0] += 1
        return synth.uniform(seed, tid[0], shape, a, b)

    # dense conv cases: (ic, oc, k, stride, h, w, pad_mode, pad_value, residual, act) - the shape/flag
    # coverage of Avx512KernelTests.Conv_Direct_MatchesAvx2 and the Winograd cases of EngineTests
    conv_cases = [
        (3, 16, 3, 1, 37, 23, 1, 0.0, False, "none"),
        (6, 32, 3, 1, 29, 41, 1, 0.0, False, "relu"),
        (16, 48, 3, 1, 11, 13, 0, 0.25, True, "relu"),
        (20, 20, 3, 2, 17, 19, 0, 0.0, True, "sigmoid"),
        (32, 64, 3, 2, 12, 31, 1, 0.0, False, "gelu"),
        (24, 3, 3, 1, 9, 10, 0, 0.0, False, "none"),
        (40, 36, 1, 1, 7, 33, 0, 0.0, True, "relu"),
        (8, 32, 5, 1, 14, 9, 1, 0.0, False, "relu"),
        (16, 16, 3, 1, 9, 11, 0, 0.0, False, "none"),
        (24, 20, 3, 1, 13, 6, 1, 0.0, True, "relu"),
        (32, 48, 3, 1, 22, 18, 0, 0.5, False, "gelu"),
        (64, 16, 3, 1, 17, 23, 1, 0.0, True, "none"),
        (64, 64, 3, 1, 16, 16, 0, 0.0, False, "relu"),
        (16, 24, 3, 1, 10, 12, 0, 0.0, False, "hardswish"),
        (16, 24, 1, 1, 10, 12, 0, 0.0, False, "swish"),
    ]
    for i, (ic, oc, k, s, h, w, mode, pv, res, act) in enumerate(conv_cases):
        pad = k // 2
        oh, ow = (h + 2 * pad - k) // s + 1, (w + 2 * pad - k) // s + 1
        x, wt, b = U((1, h, w, ic)), U((oc, ic, k, k)), U((oc,))
        add = U((1, oh, ow, oc)) if res else None
        y = conv_ref(x, wt, b, s, (pad,) * 4, 1, act, mode, pv, add)
        out[f"conv{i}_meta"] = np.array([ic, oc, k, s, h, w, mode, ACTS.index(act), int(res)], np.int64)
        out[f"conv{i}_pv"] = np.array([pv], np.float64)
        out[f"conv{i}_x"], out[f"conv{i}_w"], out[f"conv{i}_b"], out[f"conv{i}_y"] = x, wt, b, y
        if res:
            out[f"conv{i}_add"] = add
    out["conv_n"] = np.array([len(conv_cases)])

    # depthwise: (c, k, stride, h, w, pad_mode, act)
    dw_cases = [(16, 3, 1, 20, 20, 0, "relu"), (24, 3, 2, 17, 15, 0, "none"), (40, 5, 1, 12, 13, 0, "hardswish"),
                (48, 5, 2, 11, 10, 1, "relu"), (7, 3, 1, 9, 8, 0, "none")]
    for i, (c, k, s, h, w, mode, act) in enumerate(dw_cases):
        pad = k // 2
        x, wt, b = U((1, h, w, c)), U((c, 1, k, k)), U((c,))
        y = conv_ref(x, wt, b, s, (pad,) * 4, c, act, mode, 0.0)
        out[f"dw{i}_meta"] = np.array([c, k, s, h, w, mode, ACTS.index(act)], np.int64)
        out[f"dw{i}_x"], out[f"dw{i}_w"], out[f"dw{i}_b"], out[f"dw{i}_y"] = x, wt, b, y
    out["dw_n"] = np.array([len(dw_cases)])

    # Gemm (m, k, n, transB, act) - Avx512KernelTests.Gemm_MatchesAvx2 shapes
    gemm_cases = [(57, 128, 128, False, "none"), (23, 160, 48, True, "gelu"), (5, 64, 20, False, "relu"),
                  (64, 96, 40, False, "gelu")]
    for i, (m, k, n, tb, act) in enumerate(gemm_cases):
        a, bm, bias = U((m, k)), U((n, k) if tb else (k, n)), U((n,))
        B = t64(bm).T if tb else t64(bm)
        y = act64(t64(a) @ B + t64(bias), act).numpy()
        out[f"gemm{i}_meta"] = np.array([m, k, n, int(tb), ACTS.index(act)], np.int64)
        out[f"gemm{i}_a"], out[f"gemm{i}_b"], out[f"gemm{i}_bias"], out[f"gemm{i}_y"] = a, bm, bias, y
    out["gemm_n"] = np.array([len(gemm_cases)])

    # ConvTranspose stride == kernel: (ic, oc, k, h, w, act)
    ct_cases = [(24, 24, 2, 9, 7, "relu"), (24, 1, 2, 8, 6, "sigmoid"), (8, 3, 2, 5, 5, "none")]
    for i, (ic, oc, k, h, w, act) in enumerate(ct_cases):
        x, wt, b = U((1, h, w, ic)), U((ic, oc, k, k)), U((oc,))
        y = F.conv_transpose2d(t64(x).permute(0, 3, 1, 2), t64(wt), t64(b), stride=k).permute(0, 2, 3, 1)
        out[f"ct{i}_meta"] = np.array([ic, oc, k, h, w, ACTS.index(act)], np.int64)
        out[f"ct{i}_x"], out[f"ct{i}_w"], out[f"ct{i}_b"], out[f"ct{i}_y"] = x, wt, b, act64(y, act).numpy()
    out["ct_n"] = np.array([len(ct_cases)])

    # LayerNorm, softmax, matmul, attention, GAP, SE gate, nearest + add
    x = U((37, 192))
    g, be = U((192,)), U((192,))
    xt = t64(x)
    out["ln_x"], out["ln_g"], out["ln_b"] = x, g, be
    out["ln_y"] = F.layer_norm(xt, (192,), t64(g), t64(be), eps=1e-5).numpy()
    x = U((9, 6625), -8, 8)
    out["sm_x"], out["sm_y"] = x, torch.softmax(t64(x), -1).numpy()
    a, b = U((3, 17, 24)), U((3, 24, 13))
    out["mm_a"], out["mm_b"], out["mm_y"] = a, b, (t64(a) @ t64(b)).numpy()
    q, k, v = U((12, 80, 32)), U((12, 80, 32)), U((12, 80, 32))
    sc = torch.softmax((t64(q) @ t64(k).transpose(1, 2)) * (32 ** -0.5), -1)
    out["attn_q"], out["attn_k"], out["attn_v"], out["attn_y"] = q, k, v, (sc @ t64(v)).numpy()
    x = U((2, 13, 11, 40))
    out["gap_x"], out["gap_y"] = x, t64(x).mean(dim=(1, 2)).numpy()
    c, r = 40, 10
    w1, b1, w2, b2 = U((r, c)), U((r,)), U((c, r)), U((c,))
    m = t64(x).mean(dim=(1, 2))
    hid = torch.relu(m @ t64(w1).T + t64(b1))
    z = hid @ t64(w2).T + t64(b2)
    out["se_x"], out["se_w1"], out["se_b1"], out["se_w2"], out["se_b2"] = x, w1, b1, w2, b2
    out["se_y"] = torch.clamp(z / 6.0 + 0.5, 0, 1).numpy()
    x, add = U((1, 7, 9, 16)), U((1, 14, 18, 16))
    up = t64(x).repeat_interleave(2, 1).repeat_interleave(2, 2)
    out["near_x"], out["near_add"], out["near_y"] = x, add, (up + torch.relu(t64(add))).numpy()

    # expected values are stored as float32: their rounding (6e-8 relative) is far below every tolerance
    out = {k: (v.astype(np.float32) if v.dtype == np.float64 and not k.endswith("_pv") else v) for k, v in out.items()}
    path = os.path.join(HERE, "golden.npz")
    np.savez_compressed(path, **out)
    print("wrote", path, os.path.getsize(path), "bytes,", len(out), "arrays")


if __name__ == "__main__":
    main()
