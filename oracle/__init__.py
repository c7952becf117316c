"""CPU oracle for the conv/GEMM hot path (test infrastructure only).

A C++ restatement of SimdOnnx's NHWC CPU kernels (``oracle/src/oracle.cpp``; each entry point names
the reference routine it follows, e.g. ``Kernels/Nhwc.cs:172-217`` for ``Nhwc.Conv``). Only
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` import this
package, and only to check the HIP path or to time the CPU baseline beside it. The product package
``simdonnx_amd`` never imports it.

Pinning (see tests/test_oracle.py):
  * dense / depthwise / Winograd conv, Gemm, ConvTranspose, MatMul, LayerNorm, softmax, attention,
    GAP, SE gate, nearest resize: against committed torch-float64 golden vectors
    (tests/golden/make_golden.py) and closed forms;
  * the scalar, AVX2 and AVX-512 tiers agree bit for bit (reference Avx512KernelTests.cs:7-33);
  * Winograd vs direct conv <= 1e-4 * max|out| (reference EngineTests.cs:184-212);
  * the A&S erf / Cephes exp cores against math.erf / math.exp within their published error.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# SIMDONNX_ORACLE_LIB: another build of the restatement (the mutation guard loads planted-mistake
# copies through it)
_LIB_PATH = os.environ.get("SIMDONNX_ORACLE_LIB") or os.path.join(_HERE, "build", "liboracle.so")
_lib = None

ACT = {"none": 0, "relu": 1, "sigmoid": 2, "gelu": 3, "hardswish": 4, "swish": 5}
TIER_AUTO, TIER_SCALAR, TIER_AVX2, TIER_AVX512 = 0, 1, 2, 3


class ConvP(ctypes.Structure):
    """``ora_conv_p``: ConvP's spatial fields (Engine/ExecPlan.cs:50-65)."""

    _fields_ = [
        ("kh", ctypes.c_int), ("kw", ctypes.c_int), ("sh", ctypes.c_int), ("sw", ctypes.c_int),
        ("pad_t", ctypes.c_int), ("pad_l", ctypes.c_int), ("pad_b", ctypes.c_int), ("pad_r", ctypes.c_int),
        ("group", ctypes.c_int), ("act", ctypes.c_int), ("pad_mode", ctypes.c_int),
        ("pad_value", ctypes.c_float), ("pool", ctypes.c_int), ("pool_relu", ctypes.c_int),
    ]


def build() -> str:
    """Compiles liboracle.so with the committed Makefile (g++ only)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        for name in ("ora_exp_core", "ora_erf_core", "ora_gelu_core", "ora_sigmoid_core"):
            getattr(_lib, name).restype = ctypes.c_float
            getattr(_lib, name).argtypes = [ctypes.c_float]
        _lib.ora_act.restype = ctypes.c_float
        _lib.ora_act.argtypes = [ctypes.c_float, ctypes.c_int]
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _f32(a):
    return None if a is None else np.ascontiguousarray(a, dtype=np.float32)


def _check(rc, what):
    if rc != 0:
        raise ValueError(f"oracle {what} rejected its arguments (status {rc})")


def set_threads(n: int) -> None:
    lib().ora_set_threads(int(n))


def get_threads() -> int:
    return lib().ora_get_threads()


def tier_available(tier: int) -> bool:
    return bool(lib().ora_tier_available(int(tier)))


def conv_out_size(i, k, s, p0, p1):
    return (i + p0 + p1 - k) // s + 1


def conv(x, w, bias=None, add=None, *, stride=(1, 1), pads=(0, 0, 0, 0), group=1, act="none",
         pad_mode=0, pad_value=0.0, pool=False, pool_relu=False, algo=0, tier=TIER_AUTO):
    """Nhwc.Conv (Kernels/Nhwc.cs:172-217). x: [n,h,w,c] fp32; w: ONNX [oc, ic/g, kh, kw]."""
    x, w, bias, add = _f32(x), _f32(w), _f32(bias), _f32(add)
    n, ih, iw, ic = x.shape
    oc, _, kh, kw = w.shape
    pt, pl, pb, pr = pads
    oh, ow = conv_out_size(ih, kh, stride[0], pt, pb), conv_out_size(iw, kw, stride[1], pl, pr)
    if pool:
        oh, ow = oh // 2, ow // 2
    p = ConvP(kh, kw, stride[0], stride[1], pt, pl, pb, pr, group, ACT[act] if isinstance(act, str) else act,
              pad_mode, pad_value, int(pool), int(pool_relu))
    out = np.empty((n, oh, ow, oc), np.float32)
    rc = lib().ora_conv(_p(x), n, ih, iw, ic, _p(w), _p(bias), _p(add), _p(out), oh, ow, oc, ctypes.byref(p),
                        algo, tier)
    _check(rc, "conv")
    return out


def winograd_eligible(kh, kw, sh, sw, group, ic, pool=False) -> bool:
    p = ConvP(kh, kw, sh, sw, 0, 0, 0, 0, group, 0, 0, 0.0, int(pool), 0)
    return bool(lib().ora_winograd_eligible(ctypes.byref(p), ic))


def gemm(a, b, bias=None, *, trans_b=False, act="none", tier=TIER_AUTO):
    """Nhwc.Gemm (Kernels/Nhwc.cs:141-168): act(a[m,k] . B + bias)."""
    a, b, bias = _f32(a), _f32(b), _f32(bias)
    k = a.shape[-1]
    m = a.size // k
    n = b.shape[0] if trans_b else b.shape[1]
    out = np.empty(a.shape[:-1] + (n,), np.float32)
    rc = lib().ora_gemm(_p(a), m, k, _p(b), n, int(trans_b), _p(bias), ACT[act] if isinstance(act, str) else act,
                        _p(out), tier)
    _check(rc, "gemm")
    return out


def matmul(a, b):
    """Ops.MatMul (Kernels/Ops.Seq.cs:92-116) over equal batch dims."""
    a, b = _f32(a), _f32(b)
    m, k = a.shape[-2:]
    n = b.shape[-1]
    batch = int(np.prod(a.shape[:-2])) if a.ndim > 2 else 1
    out = np.empty(a.shape[:-2] + (m, n), np.float32)
    _check(lib().ora_matmul(_p(a), _p(b), batch, m, k, n, _p(out)), "matmul")
    return out


def conv_transpose(x, w, bias=None, *, act="none"):
    """Nhwc.ConvTranspose (Kernels/Nhwc.Det.cs:51-131); w [ic, oc, kh, kw], stride == kernel."""
    x, w, bias = _f32(x), _f32(w), _f32(bias)
    n, ih, iw, ic = x.shape
    _, oc, kh, kw = w.shape
    out = np.empty((n, ih * kh, iw * kw, oc), np.float32)
    rc = lib().ora_conv_transpose(_p(x), n, ih, iw, ic, _p(w), oc, kh, kw, _p(bias),
                                  ACT[act] if isinstance(act, str) else act, _p(out))
    _check(rc, "conv_transpose")
    return out


def global_avg_pool(x):
    x = _f32(x)
    n, h, w, c = x.shape
    out = np.empty((n, c), np.float32)
    for i in range(n):
        lib().ora_global_avg_pool(_p(x[i]), h * w, c, _p(out[i]))
    return out


def channel_gate(x, w1, b1, w2, b2, *, act1_relu=True, hard=True, alpha=1.0 / 6, beta=0.5, offset=0.0):
    """Nhwc.ChannelGate (Kernels/Nhwc.Det.cs:287-314); w1 [r, c], w2 [c, r]. Returns [n, c]."""
    x, w1, b1, w2, b2 = _f32(x), _f32(w1), _f32(b1), _f32(w2), _f32(b2)
    n, h, w, c = x.shape
    r = w1.shape[0]
    out = np.empty((n, c), np.float32)
    for i in range(n):
        xi = np.ascontiguousarray(x[i])
        oi = np.empty(c, np.float32)
        lib().ora_channel_gate(_p(xi), h * w, c, _p(w1), _p(b1), _p(w2), _p(b2), r, int(act1_relu), int(hard),
                               ctypes.c_float(alpha), ctypes.c_float(beta), ctypes.c_float(offset), _p(oi))
        out[i] = oi
    return out


def channel_broadcast(full, vec, *, op=2, rev=False, act=0):
    full, vec = _f32(full), _f32(vec)
    c = full.shape[-1]
    out = np.empty_like(full)
    lib().ora_channel_broadcast(_p(full), _p(vec), _p(out), ctypes.c_long(full.size // c), c, op, int(rev), act)
    return out


def ew2(a, b, *, op=0, act=0):
    a, b = _f32(a), _f32(b)
    out = np.empty_like(a)
    lib().ora_ew2(_p(a), _p(b), _p(out), ctypes.c_long(a.size), op, act)
    return out


def resize_nearest(x, scale_y, scale_x, add=None, add_relu=False):
    x, add = _f32(x), _f32(add)
    n, ih, iw, c = x.shape
    oh, ow = int(ih * scale_y), int(iw * scale_x)
    out = np.empty((n, oh, ow, c), np.float32)
    for i in range(n):
        oi = np.empty((oh, ow, c), np.float32)
        ai = None if add is None else np.ascontiguousarray(add[i])
        lib().ora_resize_nearest(_p(np.ascontiguousarray(x[i])), ih, iw, c, _p(oi), oh, ow, ctypes.c_float(scale_y),
                                 ctypes.c_float(scale_x), _p(ai), int(add_relu))
        out[i] = oi
    return out


def concat_channels(xs):
    xs = [_f32(x) for x in xs]
    outer = xs[0].size // xs[0].shape[-1]
    counts = (ctypes.c_int * len(xs))(*[x.shape[-1] for x in xs])
    ptrs = (ctypes.c_void_p * len(xs))(*[x.ctypes.data for x in xs])
    out = np.empty(xs[0].shape[:-1] + (sum(x.shape[-1] for x in xs),), np.float32)
    lib().ora_concat_inner(ptrs, counts, len(xs), ctypes.c_long(outer), _p(out))
    return out


def activation(x, act):
    x = _f32(x)
    out = np.empty_like(x)
    lib().ora_activation(_p(x), ctypes.c_long(x.size), ACT[act] if isinstance(act, str) else act, _p(out))
    return out


def hard_sigmoid(x, alpha, beta):
    x = _f32(x)
    out = np.empty_like(x)
    lib().ora_hard_sigmoid(_p(x), ctypes.c_long(x.size), ctypes.c_float(alpha), ctypes.c_float(beta), _p(out))
    return out


def layer_norm(x, gamma, beta, eps=1e-5):
    x, gamma, beta = _f32(x), _f32(gamma), _f32(beta)
    n = x.shape[-1]
    out = np.empty_like(x)
    lib().ora_layer_norm(_p(x), ctypes.c_long(x.size // n), n, _p(gamma), _p(beta), ctypes.c_float(eps), _p(out))
    return out


def softmax(x):
    x = _f32(x)
    n = x.shape[-1]
    out = np.empty_like(x)
    lib().ora_softmax(_p(x), ctypes.c_long(x.size // n), n, _p(out))
    return out


def attention(q, k, v, scale):
    """softmax(scale * q k^T) v; q [bh, t, d], k/v [bh, s, d]."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    bh, t, d = q.shape
    s = k.shape[1]
    out = np.empty_like(q)
    lib().ora_attention(_p(q), _p(k), _p(v), bh, t, s, d, ctypes.c_float(scale), _p(out))
    return out


def round_f16(x):
    x = _f32(x)
    out = np.empty_like(x)
    lib().ora_round_f16(_p(x), _p(out), ctypes.c_long(x.size))
    return out


def exp_core(x):
    return lib().ora_exp_core(float(x))


def erf_core(x):
    return lib().ora_erf_core(float(x))


def gelu_core(x):
    return lib().ora_gelu_core(float(x))


# ---- the rest of the GPU op surface (Engine/Session.cs:178-270, 345-410) ----

def resize_bilinear(x, scale_y, scale_x, add=None, *, relu=False, add_relu=False):
    """Nhwc.ResizeBilinear (Kernels/Nhwc.cs:773-870), NHWC batch."""
    x, add = _f32(x), _f32(add)
    n, ih, iw, c = x.shape
    oh, ow = int(ih * scale_y), int(iw * scale_x)
    out = np.empty((n, oh, ow, c), np.float32)
    for i in range(n):
        oi = np.empty((oh, ow, c), np.float32)
        ai = None if add is None else np.ascontiguousarray(add[i])
        _check(lib().ora_resize_bilinear(_p(np.ascontiguousarray(x[i])), ih, iw, c, _p(oi), oh, ow,
                                         ctypes.c_float(scale_y), ctypes.c_float(scale_x), int(relu), _p(ai),
                                         int(add_relu)), "resize_bilinear")
        out[i] = oi
    return out


def pad_nhwc(x, pad_t, pad_l, pad_b, pad_r, mode=0, value=0.0):
    """Nhwc.Pad (Kernels/Nhwc.cs:877-900): spatial pad of an NHWC batch, constant (0) or reflect (1)."""
    x = _f32(x)
    n, ih, iw, c = x.shape
    oh, ow = ih + pad_t + pad_b, iw + pad_l + pad_r
    out = np.empty((n, oh, ow, c), np.float32)
    for i in range(n):
        oi = np.empty((oh, ow, c), np.float32)
        _check(lib().ora_pad_nhwc(_p(np.ascontiguousarray(x[i])), ih, iw, c, _p(oi), oh, ow, pad_t, pad_l, mode,
                                  ctypes.c_float(value)), "pad")
        out[i] = oi
    return out


def max_pool(x, kernel, stride, pads, relu=False):
    """Nhwc.MaxPool (Kernels/Nhwc.cs:729-769), NHWC batch, pads (t, l, b, r), PoolP.FuseRelu."""
    x = _f32(x)
    n, ih, iw, c = x.shape
    oh = conv_out_size(ih, kernel[0], stride[0], pads[0], pads[2])
    ow = conv_out_size(iw, kernel[1], stride[1], pads[1], pads[3])
    out = np.empty((n, oh, ow, c), np.float32)
    for i in range(n):
        oi = np.empty((oh, ow, c), np.float32)
        _check(lib().ora_max_pool_nhwc(_p(np.ascontiguousarray(x[i])), ih, iw, c, _p(oi), oh, ow, kernel[0],
                                       kernel[1], stride[0], stride[1], pads[0], pads[1], int(relu)), "max_pool")
        out[i] = oi
    return out


def avg_pool(x, kernel, stride, pads, count_include_pad=False):
    """Nhwc.AvgPool (Kernels/Ops.Seq.cs:180-215), NHWC batch, pads (t, l, b, r)."""
    x = _f32(x)
    n, ih, iw, c = x.shape
    oh = conv_out_size(ih, kernel[0], stride[0], pads[0], pads[2])
    ow = conv_out_size(iw, kernel[1], stride[1], pads[1], pads[3])
    out = np.empty((n, oh, ow, c), np.float32)
    for i in range(n):
        oi = np.empty((oh, ow, c), np.float32)
        _check(lib().ora_avg_pool_nhwc(_p(np.ascontiguousarray(x[i])), ih, iw, c, _p(oi), oh, ow, kernel[0],
                                       kernel[1], stride[0], stride[1], pads[0], pads[1], int(count_include_pad)),
               "avg_pool")
        out[i] = oi
    return out


def depth_to_space(x, block, crd=False, inverse=False):
    """Nhwc.DepthToSpace / SpaceToDepth (Kernels/Nhwc.Det.cs:210-282), NHWC batch."""
    x = _f32(x)
    n, ih, iw, ic = x.shape
    bb = block * block
    shape = (n, ih // block, iw // block, ic * bb) if inverse else (n, ih * block, iw * block, ic // bb)
    out = np.empty(shape, np.float32)
    for i in range(n):
        oi = np.empty(shape[1:], np.float32)
        _check(lib().ora_depth_space(_p(np.ascontiguousarray(x[i])), ih, iw, ic, _p(oi), block, int(crd),
                                     int(inverse)), "depth_space")
        out[i] = oi
    return out


UNARY2 = {"LeakyRelu": 0, "Tanh": 1, "Clip": 2, "Erf": 3}


def unary2(x, op, a=0.0, b=0.0):
    """Act.ApplyLeakyRelu / ApplyTanh / ApplyClip / ApplyErf (Kernels/Act.cs:83-147)."""
    x = _f32(x)
    out = np.empty_like(x)
    _check(lib().ora_unary2(_p(x), ctypes.c_long(x.size), UNARY2[op], ctypes.c_float(a), ctypes.c_float(b),
                            _p(out)), "unary2")
    return out


def transpose(x, perm):
    """Ops.Transpose (Kernels/Ops.cs:798-868): an index permutation, no arithmetic."""
    return np.ascontiguousarray(np.transpose(_f32(x), perm))


def slice_(x, starts, ends, axes, steps):
    """Ops.Slice (Kernels/Ops.cs:870-883): a strided gather from resolved starts; no arithmetic."""
    x = _f32(x)
    sl = [slice(None)] * x.ndim
    for s0, e0, a, st in zip(starts, ends, axes, steps):
        sl[a] = slice(s0, e0 if e0 >= 0 else None, st)
    return np.ascontiguousarray(x[tuple(sl)])


def matmul_bcast(a, b):
    """Ops.MatMul with B broadcast over A's batch (one B) or matched batches (Kernels/Ops.Seq.cs:92-116)."""
    a, b = _f32(a), _f32(b)
    m, k = a.shape[-2:]
    n = b.shape[-1]
    batch = a.size // (m * k)
    bb = b.size // (k * n)
    a3 = a.reshape(batch, m, k)
    b3 = np.broadcast_to(b.reshape(bb, k, n), (batch, k, n)) if bb == 1 else b.reshape(batch, k, n)
    return matmul(a3, np.ascontiguousarray(b3)).reshape(a.shape[:-2] + (m, n))


def ctc_argmax(x, w, bias=None):
    """CtcProjection.ArgMax (Decoding/Kernels/MatMul.ArgMax.cs:130-299): (indices, probabilities) per
    row of x [rows, inner] against w [inner, columns]; raises ValueError on a non-finite logit."""
    x, w, bias = _f32(x), _f32(w), _f32(bias)
    rows, inner = x.shape[0], x.shape[1]
    columns = w.shape[1]
    idx = np.empty(rows, np.int32)
    prob = np.empty(rows, np.float32)
    rc = lib().ora_ctc_argmax(_p(x), _p(w), _p(bias), ctypes.c_long(rows), inner, columns,
                              idx.ctypes.data_as(ctypes.c_void_p), _p(prob))
    if rc != 0:
        raise ValueError("Recognizer output is invalid.")
    return idx, prob


def safe_div(a, b, eps, lo, hi):
    """SafeDiv (Kernels/FusedKernels.cs:35-57)."""
    a, b = _f32(a), _f32(b)
    out = np.empty_like(a)
    lib().ora_safediv(_p(a), _p(b), _p(out), ctypes.c_long(a.size), ctypes.c_float(eps), ctypes.c_float(lo),
                      ctypes.c_float(hi))
    return out


def channel_shift(x, axis, ends, offs):
    """ChannelShift (Kernels/FusedKernels.cs:195-222), NHWC batch."""
    x = _f32(x)
    n, h, w, c = x.shape
    e = (ctypes.c_int * 5)(*ends)
    o = (ctypes.c_int * 5)(*offs)
    out = np.empty_like(x)
    for i in range(n):
        oi = np.empty((h, w, c), np.float32)
        lib().ora_channel_shift(_p(np.ascontiguousarray(x[i])), h, w, c, _p(oi), axis, e, o, len(ends))
        out[i] = oi
    return out


def up_head(x, skip, w, bias, scale, *, resize_relu=False, skip_relu=False, act="none"):
    """UpHead with a stored skip (Kernels/FusedKernels.cs:62-192), NHWC batch; w [oc, c]."""
    x, skip, w, bias = _f32(x), _f32(skip), _f32(w), _f32(bias)
    n, ih, iw, c = x.shape
    oc = w.shape[0]
    oh, ow = int(ih * scale), int(iw * scale)
    out = np.empty((n, oh, ow, oc), np.float32)
    for i in range(n):
        oi = np.empty((oh, ow, oc), np.float32)
        _check(lib().ora_uphead(_p(np.ascontiguousarray(x[i])), ih, iw, c, _p(np.ascontiguousarray(skip[i])), _p(oi),
                                oh, ow, ctypes.c_float(scale), ctypes.c_float(scale), _p(w.reshape(oc, c)), _p(bias),
                                oc, int(resize_relu), int(skip_relu), ACT[act] if isinstance(act, str) else act),
               "up_head")
        out[i] = oi
    return out


def from_pixels(src, width, height, bpp, lut, swap, tensor_w, tensor_h, pad_left=0, pad_top=0):
    """ImageTensor.FromPixels, NHWC (Imaging/ImageTensor.cs:322-365): byte rows -> [th, tw, 3] float32,
    the image at (pad_left, pad_top) with its edge repeated; channel c = lut[c][byte], channel 0 from
    byte 2 of a pixel when swap. Index and table work only."""
    src = np.asarray(src, np.uint8)
    lut = np.asarray(lut, np.float32).reshape(3, 256)
    ys = np.clip(np.arange(tensor_h) - pad_top, 0, height - 1)
    xs = np.clip(np.arange(tensor_w) - pad_left, 0, width - 1)
    px = src[ys[:, None, None], xs[None, :, None] * bpp + np.arange(3)[None, None, :]]  # [th, tw, 3] bytes
    o0 = 2 if swap else 0
    out = np.empty((tensor_h, tensor_w, 3), np.float32)
    out[..., 0] = lut[0][px[..., o0]]
    out[..., 1] = lut[1][px[..., 1]]
    out[..., 2] = lut[2][px[..., 2 - o0]]
    return out


def to_pixels(x, width, height, bpp, swap, crop_left=0, crop_top=0, scale=255.0, alpha=None):
    """ImageTensor.ToPixels, NHWC (Imaging/ImageTensor.cs:376-430): the width x height window at
    (crop_left, crop_top) of [th, tw, 3] -> uint8 [height, width * bpp], byte = clamp((int)(v * scale +
    0.5f), 0, 255) in float32 (multiply, then add, then truncate toward zero); 4-byte pixels take alpha
    from `alpha` ([height, width * 4]) or 255."""
    x = np.asarray(x, np.float32)[crop_top:crop_top + height, crop_left:crop_left + width]
    t = (x * np.float32(scale)).astype(np.float32) + np.float32(0.5)
    b = np.clip(np.trunc(t), 0, 255).astype(np.uint8)
    out = np.empty((height, width, bpp), np.uint8)
    o0 = 2 if swap else 0
    out[..., o0], out[..., 1], out[..., 2 - o0] = b[..., 0], b[..., 1], b[..., 2]
    if bpp == 4:
        out[..., 3] = 255 if alpha is None else np.asarray(alpha, np.uint8).reshape(height, width, 4)[..., 3]
    return out.reshape(height, width * bpp)

