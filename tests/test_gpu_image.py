"""The HIP image session (sox_image_session_*, HipImageSession) vs the oracle's FromPixels -> plan ->
ToPixels (VkImageSession's contract, Backends/Vulkan/VkImageSession.cs:7-297; the reference's image
session tests compare the GPU session with the CPU pipeline the same way).

A copy model must give back the input bytes exactly (every format, both paddings, row strides wider
than the row, alpha kept); a 3x3 conv model must match the oracle within 1 (fp32) / 2 (fp16) per byte."""
import numpy as np
import pytest

import oracle as O
from oracle.interp import run_plan
from simdonnx_amd import synth
from simdonnx_amd.backend import HipImageSession
from simdonnx_amd.plan import NHWC, PlanBuilder

pytestmark = pytest.mark.gpu
UNIT = np.tile(np.arange(256, dtype=np.float32) / np.float32(255), 3)


def copy_plan(h, w):
    pb = PlanBuilder()
    x = pb.input((1, 3, h, w), NHWC, "image")
    return pb.build(pb.unary("Copy", x, name="copy"))


def conv_plan(h, w):
    pb = PlanBuilder()
    x = pb.input((1, 3, h, w), NHWC, "image")
    y = pb.conv(x, synth.normal(51, 1, (8, 3, 3, 3), 0.3), synth.uniform(51, 2, (8,), -0.1, 0.1), act="relu",
                name="c1")
    y = pb.conv(y, synth.normal(51, 3, (3, 8, 3, 3), 0.2), synth.uniform(51, 4, (3,), 0.2, 0.4), act="sigmoid",
                name="c2")
    return pb.build(y)


@pytest.mark.parametrize("half", [False, True], ids=["f32", "f16"])
@pytest.mark.parametrize("fmt,bpp", [("Bgr24", 3), ("Rgb24", 3), ("Bgra32", 4), ("Rgba32", 4)])
@pytest.mark.parametrize("top_left", [False, True])
def test_image_session_copy_is_identity(hip, fmt, bpp, top_left, half):
    width, height, stride = 37, 23, 37 * bpp + 5
    src = np.random.default_rng(7).integers(0, 256, (height, stride), dtype=np.uint8)
    s = HipImageSession(hip, UNIT, rgb_order=False, pad_multiple=16, pad_top_left=top_left)
    th, tw = s.tensor_size(width, height)
    assert (th, tw) == (32, 48)
    print(f"[gpu] image session copy {fmt} f16={half}", flush=True)
    g = hip.graph(copy_plan(th, tw), half)
    out = s.run(g, src, width, height, fmt)
    assert np.array_equal(out[:, :width * bpp], src[:, :width * bpp])
    out2 = s.run(g, src, width, height, fmt)  # the bound graph and buffers are reused
    assert np.array_equal(out2[:, :width * bpp], out[:, :width * bpp])
    s.close()


@pytest.mark.parametrize("half", [False, True], ids=["f32", "f16"])
@pytest.mark.parametrize("fmt,bpp,size", [("Bgr24", 3, (61, 45)), ("Rgba32", 4, (200, 120)), ("Rgb24", 3, (33, 7))])
def test_image_session_conv_model(hip, fmt, bpp, size, half):
    width, height = size
    src = np.random.default_rng(8).integers(0, 256, (height, width * bpp), dtype=np.uint8)
    s = HipImageSession(hip, UNIT, rgb_order=True, pad_multiple=1 if width % 2 else 8)  # odd tensor widths too
    th, tw = s.tensor_size(width, height)
    plan = conv_plan(th, tw)
    print(f"[gpu] image session conv {fmt} {size} f16={half}", flush=True)
    out = s.run(hip.graph(plan, half), src, width, height, fmt)
    swap = 1 if fmt in ("Bgr24", "Bgra32") else 0  # the table is in RGB order
    t = O.from_pixels(src, width, height, bpp, UNIT, swap, tw, th)
    y = run_plan(plan, [t[None]], f16_storage=half).reshape(th, tw, 3)
    want = O.to_pixels(y, width, height, bpp, swap, alpha=src if bpp == 4 else None)
    diff = np.abs(out.astype(int) - want.astype(int))
    assert diff.max() <= (2 if half else 1), diff.max()
    if bpp == 4:
        assert np.array_equal(out.reshape(height, width, 4)[..., 3], src.reshape(height, width, 4)[..., 3])
    s.close()
