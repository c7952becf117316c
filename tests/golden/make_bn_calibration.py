"""Measures the folded BatchNorms of the configs 3 and 4 models (simdonnx_amd/graphs.py) and writes
simdonnx_amd/data/bn_calibration.npz. Test infrastructure: it runs the CPU oracle.

A trained network's BatchNorm normalises each conv output channel over the data; folded into the conv
(OnnxRewrites.FoldConvBatchNorm, Onnx/OnnxRewrites.cs:71-111) it is w' = w s, b' = b s + t per output
channel. Here the statistics come from the seeded N(0, 1) calibration image at the config's size: for
every Conv / ConvTranspose, in plan order, the pre-activation of each output channel (the conv alone,
without its activation or skip add) is recomputed with the oracle from the layer's input and brought
to mean 0 and standard deviation 1 (the detector's logit included), one layer at a time, each after
the layers before it are normalised.

    python tests/golden/make_bn_calibration.py
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

import oracle as O  # noqa: E402
from oracle.interp import run_plan  # noqa: E402
from simdonnx_amd import graphs  # noqa: E402

OUT = os.path.join(ROOT, "simdonnx_amd", "data", "bn_calibration.npz")


def preactivation(plan, env, nd):
    v = plan.values
    x = env[nd.ins[0]]
    w = v[nd.ins[1]].data
    b = v[nd.p.bias].data if nd.p.bias >= 0 else None
    if nd.op == "ConvTranspose":
        return O.conv_transpose(x, w, b, act="none")
    p = nd.p
    return O.conv(x, w, b, None, stride=p.strides, pads=p.pads, group=p.group, act="none", pad_mode=p.pad_mode,
                  pad_value=p.pad_value)


def calibrate(model, build):
    """One layer at a time, in plan order: each is normalised against the already normalised layers
    before it (a rerun of the plan per layer), so one pass is the fixed point."""
    cal = {}
    plan, _ = build(cal)
    names = [nd.name for nd in plan.nodes if nd.op in ("Conv", "ConvTranspose") and nd.name]
    for name in names:
        plan, ins = build(cal)
        _, env = run_plan(plan, ins, keep=True)
        nd = next(n for n in plan.nodes if n.name == name)
        y = preactivation(plan, env, nd).astype(np.float64)
        y = y.reshape(-1, y.shape[-1])
        mu, sd = y.mean(axis=0), y.std(axis=0)
        # a channel that barely varies (a depthwise channel over a mostly-zero ReLU input) is not
        # amplified more than 10x: BatchNorm's epsilon plays this part in a trained network
        f = 1.0 / np.maximum(sd, 0.1)
        key = f"{model}/{name}"
        s0 = cal.get(key + "/s", np.ones_like(f))
        t0 = cal.get(key + "/t", np.zeros_like(f))
        # y = s0 raw + t0  ->  (y - mu) f = (s0 f) raw + (t0 - mu) f
        cal[key + "/s"], cal[key + "/t"] = s0 * f, (t0 - mu) * f
    print(f"{model}: {len(names)} layers", flush=True)
    return cal


def main():
    cal = {}
    cal.update(calibrate("mbv3", lambda c: graphs.mobilenetv3_small(size=640, scales=c)))
    cal.update(calibrate("dbnet", lambda c: graphs.dbnet(size=960, scales=c, logit=True)))
    os.makedirs(os.path.dirname(OUT), exist_ok=True)
    np.savez_compressed(OUT, **{k: v.astype(np.float32) for k, v in cal.items()})
    print("wrote", OUT, len(cal) // 2, "layers")


if __name__ == "__main__":
    main()
