"""Writes the golden vectors that pin the oracle's restatement of the rest of the GPU op surface:
bilinear resize (+ relu, + addend), constant / reflect pad, average pool (with and without the
padded taps counted), DepthToSpace / SpaceToDepth (CRD and DCR), LeakyRelu / Tanh / Clip / Erf,
global average pool, batched MatMul with a broadcast right operand, the CTC head's fused
projection + argmax + softmax probability, and the built-in extension ops SafeDiv, ChannelShift and
UpHead (with a stored skip and with the skip recomputed by its 3x3 conv).

Each expected output is a library routine or the ONNX definition evaluated by torch in float64:
F.interpolate(bilinear, align_corners=False), F.pad(constant / reflect), F.avg_pool2d,
F.pixel_shuffle / pixel_unshuffle (CRD) and the ONNX DCR reshape-transpose, F.leaky_relu,
torch.tanh / clamp / erf, mean over H W, torch.matmul, and for the CTC head torch.argmax / softmax of
the float64 logits. Inputs come from simdonnx_amd.synth (seeded);
the file stores the inputs and the float64 results rounded to float32.

Run:  python tests/golden/make_golden_ops.py      (writes tests/golden/golden_ops.npz)
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


def t64(a):
    return torch.from_numpy(np.asarray(a, dtype=np.float64))


def nchw(x):
    return t64(x).permute(0, 3, 1, 2)


def nhwc(y):
    return y.permute(0, 2, 3, 1).contiguous().numpy().astype(np.float32)


# (n, h, w, c, scale, relu, addend, add_relu)
BILINEAR = [(1, 7, 9, 8, 2.0, False, False, False), (2, 5, 6, 3, 3.0, True, False, False),
            (1, 8, 12, 16, 0.5, False, True, True), (1, 12, 10, 32, 2.0, True, True, False)]
# (n, h, w, c, (t, l, b, r), mode, value)
PAD = [(1, 6, 7, 8, (1, 2, 0, 3), 0, 0.0), (2, 5, 5, 3, (2, 1, 2, 1), 1, 0.0), (1, 9, 4, 16, (0, 3, 3, 0), 0, -1.5)]
# (n, h, w, c, k, s, (t, l, b, r), count_include_pad)
AVGPOOL = [(1, 9, 9, 8, 3, 2, (1, 1, 1, 1), False), (2, 8, 10, 3, 2, 2, (0, 0, 0, 0), False),
           (1, 11, 7, 16, 3, 1, (1, 1, 1, 1), True), (1, 12, 12, 24, 5, 3, (2, 2, 2, 2), False)]
# (n, h, w, c_in, block)
D2S = [(1, 3, 4, 8, 2), (2, 2, 3, 27, 3), (1, 5, 5, 64, 2)]
S2D = [(1, 6, 8, 3, 2), (2, 6, 9, 4, 3), (1, 10, 10, 16, 2)]
# (batch, m, k, n, broadcast_b)
MATMUL = [(3, 17, 33, 21, False), (4, 80, 32, 80, True), (2, 64, 128, 96, False)]


def main():
    out = {}
    for i, (n, h, w, c, s, relu, has_add, add_relu) in enumerate(BILINEAR):
        x = synth.normal(900 + i, 1, (n, h, w, c), 1.0)
        oh, ow = int(h * s), int(w * s)
        y = F.interpolate(nchw(x), scale_factor=(s, s), mode="bilinear", align_corners=False,
                          recompute_scale_factor=False)
        if relu:
            y = torch.relu(y)
        out[f"bil{i}_x"] = x
        if has_add:
            a = synth.normal(900 + i, 2, (n, oh, ow, c), 1.0)
            out[f"bil{i}_add"] = a
            at = nchw(a)
            y = y + (torch.relu(at) if add_relu else at)
        out[f"bil{i}_meta"] = np.array([s, relu, has_add, add_relu], np.float32)
        out[f"bil{i}_y"] = nhwc(y)
    for i, (n, h, w, c, pads, mode, value) in enumerate(PAD):
        x = synth.normal(910 + i, 1, (n, h, w, c), 1.0)
        t, l, b, r = pads
        xt = nchw(x)
        y = F.pad(xt, (l, r, t, b), mode="reflect") if mode == 1 else F.pad(xt, (l, r, t, b), value=value)
        out[f"pad{i}_x"], out[f"pad{i}_y"] = x, nhwc(y)
        out[f"pad{i}_meta"] = np.array([t, l, b, r, mode, value], np.float32)
    for i, (n, h, w, c, k, s, pads, cip) in enumerate(AVGPOOL):
        x = synth.normal(920 + i, 1, (n, h, w, c), 1.0)
        t, l, b, r = pads
        assert t == b and l == r
        y = F.avg_pool2d(nchw(x), k, s, (t, l), count_include_pad=cip)
        out[f"avg{i}_x"], out[f"avg{i}_y"] = x, nhwc(y)
        out[f"avg{i}_meta"] = np.array([k, s, t, l, b, r, cip], np.float32)
    for i, (n, h, w, c, b) in enumerate(D2S):
        x = synth.normal(930 + i, 1, (n, h, w, c), 1.0)
        xt = nchw(x)
        crd = F.pixel_shuffle(xt, b)
        # ONNX DepthToSpace DCR: reshape [n, b, b, c/b^2, h, w] -> transpose [0, 3, 4, 1, 5, 2] -> [n, c/b^2, h b, w b]
        dcr = xt.reshape(n, b, b, c // (b * b), h, w).permute(0, 3, 4, 1, 5, 2).reshape(n, c // (b * b), h * b, w * b)
        out[f"d2s{i}_x"], out[f"d2s{i}_crd"], out[f"d2s{i}_dcr"] = x, nhwc(crd), nhwc(dcr)
        out[f"d2s{i}_meta"] = np.array([b], np.float32)
    for i, (n, h, w, c, b) in enumerate(S2D):
        x = synth.normal(940 + i, 1, (n, h, w, c), 1.0)
        xt = nchw(x)
        crd = F.pixel_unshuffle(xt, b)
        # ONNX SpaceToDepth (DCR order): reshape [n, c, h/b, b, w/b, b] -> transpose [0, 3, 5, 1, 2, 4]
        dcr = xt.reshape(n, c, h // b, b, w // b, b).permute(0, 3, 5, 1, 2, 4).reshape(n, c * b * b, h // b, w // b)
        out[f"s2d{i}_x"], out[f"s2d{i}_crd"], out[f"s2d{i}_dcr"] = x, nhwc(crd), nhwc(dcr)
        out[f"s2d{i}_meta"] = np.array([b], np.float32)
    u = synth.normal(950, 1, (4096,), 2.5)
    ut = t64(u)
    out["un_x"] = u
    out["un_leaky01"] = F.leaky_relu(ut, 0.1).numpy().astype(np.float32)
    out["un_leaky2"] = F.leaky_relu(ut, 2.0).numpy().astype(np.float32)
    out["un_tanh"] = torch.tanh(ut).numpy().astype(np.float32)
    out["un_tanh_scaled"] = (1.7159 * torch.tanh(ut * (2.0 / 3.0))).numpy().astype(np.float32)
    out["un_clip"] = torch.clamp(ut, -1.0, 0.75).numpy().astype(np.float32)
    out["un_erf"] = torch.erf(ut).numpy().astype(np.float32)
    g = synth.normal(960, 1, (2, 13, 11, 40), 1.0)
    out["gap_x"] = g
    out["gap_y"] = t64(g).mean(dim=(1, 2)).numpy().astype(np.float32)
    for i, (bt, m, k, nn, bc) in enumerate(MATMUL):
        a = synth.normal(970 + i, 1, (bt, m, k), 1.0)
        b = synth.normal(970 + i, 2, (1 if bc else bt, k, nn), 0.2)
        out[f"mm{i}_a"], out[f"mm{i}_b"] = a, b
        out[f"mm{i}_y"] = torch.matmul(t64(a), t64(b)).numpy().astype(np.float32)
    # CTC head: logits = x W + b, the first index of the row maximum and softmax(logits)[argmax]
    x = synth.normal(980, 1, (70, 64), 1.0)
    w = synth.normal(980, 2, (64, 1100), 0.1)
    b = synth.uniform(980, 3, (1100,), -0.1, 0.1)
    lg = t64(x) @ t64(w) + t64(b)
    out["ctc_x"], out["ctc_w"], out["ctc_b"] = x, w, b
    out["ctc_idx"] = torch.argmax(lg, dim=1).numpy().astype(np.int32)
    out["ctc_prob"] = torch.softmax(lg, dim=1).max(dim=1).values.numpy().astype(np.float32)
    # built-in extension ops: SafeDiv, ChannelShift (zero-filled shifts per channel group), UpHead
    a = synth.normal(990, 1, (2, 5, 7, 16), 1.0)
    b = synth.uniform(990, 2, (2, 5, 7, 16), -0.5, 2.0)
    out["sd_a"], out["sd_b"] = a, b
    out["sd_y"] = torch.clamp(t64(a) / torch.clamp(t64(b), min=1e-3), -4.0, 4.0).numpy().astype(np.float32)
    x = synth.normal(991, 1, (1, 6, 9, 20), 1.0)
    out["sh_x"] = x
    ends, offs = [4, 8, 12, 16, 20], [-2, -1, 0, 1, 2]
    for axis in (2, 3):
        y = np.zeros_like(x, dtype=np.float64)
        g0 = 0
        for g1, o in zip(ends, offs):
            src = np.roll(x[..., g0:g1].astype(np.float64), -o, axis=axis - 1)
            if o > 0:
                sl = [slice(None)] * 4
                sl[axis - 1] = slice(x.shape[axis - 1] - o, None)
                src[tuple(sl)] = 0
            elif o < 0:
                sl = [slice(None)] * 4
                sl[axis - 1] = slice(0, -o)
                src[tuple(sl)] = 0
            y[..., g0:g1] = src
            g0 = g1
        out[f"sh_y{axis}"] = y.astype(np.float32)
    for i, (c, oc, sc) in enumerate([(16, 1, False), (32, 2, True)]):
        x = synth.normal(992 + i, 1, (1, 12, 10, c), 1.0)
        w = synth.normal(992 + i, 3, (oc, c), 0.2)
        bb = synth.uniform(992 + i, 4, (oc,), -0.1, 0.1)
        r = F.interpolate(nchw(x), scale_factor=(2.0, 2.0), mode="bilinear", align_corners=False,
                          recompute_scale_factor=False)
        r = torch.relu(r)
        if sc:
            sk_in = synth.normal(992 + i, 2, (1, 24, 20, 3), 1.0)
            w_sc = synth.normal(992 + i, 5, (c, 3, 3, 3), 0.3)
            b_sc = synth.uniform(992 + i, 6, (c,), -0.1, 0.1)
            skip = torch.relu(F.conv2d(nchw(sk_in), t64(w_sc), t64(b_sc), padding=1))
            out[f"uh{i}_skin"], out[f"uh{i}_wsc"], out[f"uh{i}_bsc"] = sk_in, w_sc, b_sc
        else:
            sk = synth.normal(992 + i, 2, (1, 24, 20, c), 1.0)
            skip = nchw(sk)
            out[f"uh{i}_skip"] = sk
        s_ = r + torch.relu(skip)
        y = torch.sigmoid(F.conv2d(s_, t64(w).reshape(oc, c, 1, 1), t64(bb)))
        out[f"uh{i}_x"], out[f"uh{i}_w"], out[f"uh{i}_b"], out[f"uh{i}_y"] = x, w, bb, nhwc(y)
    path = os.path.join(HERE, "golden_ops.npz")
    np.savez_compressed(path, **out)
    print("wrote", path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
