"""ExecPlan: the executable IR the backend consumes, restated from Engine/ExecPlan.cs.

A plan is what SimdOnnx's GraphCompiler hands a GPU backend (PlanTarget != Cpu, NHWC layout
planned, fusions applied): values (``CValue``, ExecPlan.cs:202-220), nodes (``ExecNode``,
:235-276) with their parameter records (``ConvP`` :50-65, ``GemmP`` :87-93, ...), and the arena
plan (``BufOffset`` / ``ArenaFloats``, :283-285).

``PlanBuilder`` emits the fused nodes that GraphCompiler produces for the patterns it fuses
(Conv+bias+act+residual, Gemm+bias+GELU, HardSigmoid*x -> HardSwish epilogue, SE -> ChannelGate,
Resize(nearest)+Add, ConvTranspose+bias+act; GraphCompiler.cs:272-1332) and lays the activations
out in one arena with the lifetime packing of ``PlanArena`` (GraphCompiler.cs:1336-1474:
32-element aligned first fit over [first def, last use] intervals).
"""
from __future__ import annotations

import dataclasses
from dataclasses import dataclass, field
from typing import Optional

import numpy as np

from . import native as N

NHWC = (0, 2, 3, 1)  # Layout.Nhwc (Engine/Layout.cs:15): physical [n,h,w,c] of logical [n,c,h,w]
ACT = N.ACT


@dataclass
class Value:
    """CValue: logical shape, physical layout, arena buffer id or const data."""

    shape: tuple
    layout: Optional[tuple] = None
    buf: int = -1
    data: Optional[np.ndarray] = None
    name: str = ""
    alias_of: int = -1

    @property
    def is_const(self) -> bool:
        return self.data is not None

    @property
    def count(self) -> int:
        return int(np.prod(self.shape)) if self.shape else 1

    @property
    def phys(self) -> tuple:
        if self.layout is None:
            return tuple(self.shape)
        return tuple(self.shape[i] for i in self.layout)


@dataclass
class ConvP:
    pads: tuple  # top, left, bottom, right
    strides: tuple
    kernel: tuple
    dilations: tuple = (1, 1)
    group: int = 1
    act: str = "none"
    pad_mode: int = 0
    pad_value: float = 0.0
    bias: int = -1
    add: int = -1
    pool: Optional[tuple] = None  # (kernel, strides, pads, relu) of a fused max pool

    def native(self):
        p = N.ConvP()
        p.pads[:] = list(self.pads)
        p.strides[:] = list(self.strides)
        p.dilations[:] = list(self.dilations)
        p.kernel[:] = list(self.kernel)
        p.group, p.act, p.pad_mode, p.pad_value = self.group, ACT[self.act], self.pad_mode, self.pad_value
        p.bias_value, p.add_value = self.bias, self.add
        if self.pool is not None:
            k, s, pd, relu = self.pool
            p.has_pool = 1
            p.pool_kernel[:] = list(k)
            p.pool_strides[:] = list(s)
            p.pool_pads[:] = list(pd)
            p.pool_relu = int(relu)
        return p


@dataclass
class GemmP:
    trans_b: bool = False
    bias: int = -1
    act: str = "none"

    def native(self):
        return N.GemmP(int(self.trans_b), self.bias, ACT[self.act])


@dataclass
class ConvTP:
    kernel: tuple
    bias: int = -1
    act: str = "none"

    def native(self):
        p = N.ConvTP()
        p.kernel[:] = list(self.kernel)
        p.bias_value, p.act = self.bias, ACT[self.act]
        return p


@dataclass
class EwP:
    op: int  # EwOp: 0 add, 1 sub, 2 mul, 3 div
    act: str = "none"

    def native(self):
        return N.EwP(self.op, ACT[self.act])


@dataclass
class LnP:
    eps: float = 1e-5

    def native(self):
        return N.LnP(self.eps)


@dataclass
class ResizeNearestP:
    scales: tuple
    add_relu: bool = False

    def native(self):
        p = N.ResizeNearestP()
        sc = list(self.scales) + [1.0] * (4 - len(self.scales))
        p.scales[:] = sc[:4]
        p.add_relu = int(self.add_relu)
        return p


@dataclass
class ChannelGateP:
    b1: int = -1
    b2: int = -1
    act1: str = "relu"
    hard: bool = True
    alpha: float = 1.0 / 6.0
    beta: float = 0.5
    offset: float = 0.0

    def native(self):
        return N.ChannelGateP(self.b1, self.b2, ACT[self.act1], int(self.hard), self.alpha, self.beta, self.offset)


@dataclass
class ConcatP:
    axis: int

    def native(self):
        return N.ConcatP(self.axis)


@dataclass
class HardSigmoidP:
    alpha: float
    beta: float

    def native(self):
        return N.HardSigmoidP(self.alpha, self.beta)


@dataclass
class AttentionP:
    scale: float
    dims: tuple  # 3 x (n, h, t|s, d) logical axes
    fix_axis: tuple = (-1, -1, -1)
    fix_index: tuple = (0, 0, 0)
    out_layout: Optional[tuple] = None

    def native(self):
        p = N.AttentionP()
        p.scale = self.scale
        for i in range(3):
            p.dims[i][:] = list(self.dims[i])
        p.fix_axis[:] = list(self.fix_axis)
        p.fix_index[:] = list(self.fix_index)
        p.out_layout[:] = list(self.out_layout) if self.out_layout is not None else [-1, -1, -1, -1]
        return p


@dataclass
class PoolP:
    kernel: tuple
    strides: tuple
    pads: tuple
    relu: bool = False
    count_include_pad: bool = False

    def native(self):
        p = N.PoolP()
        p.kernel[:] = list(self.kernel)
        p.strides[:] = list(self.strides)
        p.pads[:] = list(self.pads)
        p.fuse_relu = int(self.relu)
        p.count_include_pad = int(self.count_include_pad)
        return p


@dataclass
class ResizeP:
    """ResizeP (ExecPlan.cs:95-101): bilinear; out = [relu](resize(x)) + [relu](In[1])."""
    scales: tuple
    fuse_relu: bool = False
    add_relu: bool = False

    def native(self):
        p = N.ResizeP()
        p.scales[:] = list(self.scales)
        p.fuse_relu, p.add_relu = int(self.fuse_relu), int(self.add_relu)
        return p


@dataclass
class PadP:
    """PadP (ExecPlan.cs:176-181): logical [2*rank] begin.., end.. pads, constant or reflect."""
    pads: tuple
    mode: int = 0
    value: float = 0.0

    def native(self):
        p = N.PadP()
        p.rank = len(self.pads) // 2
        p.pads[:len(self.pads)] = list(self.pads)
        p.mode, p.value = self.mode, self.value
        return p


@dataclass
class TransposeP:
    """TransposeP (ExecPlan.cs:183-186), a physical permutation."""
    perm: tuple

    def native(self):
        p = N.TransposeP()
        p.rank = len(self.perm)
        p.perm[:len(self.perm)] = list(self.perm)
        return p


@dataclass
class SliceP:
    """SliceP (ExecPlan.cs:188-194), physical axes, starts already clamped."""
    starts: tuple
    ends: tuple
    axes: tuple
    steps: tuple

    def native(self):
        p = N.SliceP()
        k = len(self.axes)
        p.naxes = k
        p.starts[:k], p.ends[:k], p.axes[:k], p.steps[:k] = (list(self.starts), list(self.ends), list(self.axes),
                                                               list(self.steps))
        return p


@dataclass
class ScalarP:
    """LeakyReluP (alpha), TanhP (in_scale, out_scale), ClipP (min, max) (ExecPlan.cs:123-138)."""
    kind: str
    a: float = 0.0
    b: float = 0.0

    def native(self):
        if self.kind == "LeakyRelu":
            return N.LeakyReluP(self.a)
        if self.kind == "Tanh":
            return N.TanhP(self.a, self.b)
        return N.ClipP(self.a, self.b)


@dataclass
class DepthToSpaceP:
    """DepthToSpaceP (ExecPlan.cs:139-145)."""
    block: int
    crd: bool = False

    def native(self):
        return N.DepthToSpaceP(self.block, int(self.crd))


@dataclass
class Node:
    """ExecNode: op + value ids (+ params)."""

    op: str
    ins: list
    outs: list
    p: object = None
    name: str = ""
    ext: str = ""

    def param_refs(self):
        """Value ids read through the params (ExecNode.ParamRefs, ExecPlan.cs:246-263)."""
        p = self.p
        refs = []
        if isinstance(p, ConvP):
            refs = [p.bias, p.add]
        elif isinstance(p, (GemmP, ConvTP)):
            refs = [p.bias]
        elif isinstance(p, ChannelGateP):
            refs = [p.b1, p.b2]
        return [r for r in refs if r >= 0]


@dataclass
class ExecPlan:
    values: list
    nodes: list
    buf_offset: list
    arena_floats: int
    inputs: list
    output: int
    nhwc: bool = True

    def buffer_of(self, vid: int) -> int:
        return self.values[vid].buf

    def to_native(self):
        """Marshals the plan into a native ``sox_plan`` (the C# side would do the same from its ExecPlan)."""
        lib = N.backend()
        h = N.c_void_p()
        N.check(lib.sox_plan_create(ctypes_byref(h)), "sox_plan_create")
        try:
            for v in self.values:
                shape = (N.c_int32 * max(len(v.shape), 1))(*v.shape)
                layout = (N.c_int32 * len(v.layout))(*v.layout) if v.layout is not None else None
                data = None
                nf = 0
                if v.is_const:
                    arr = np.ascontiguousarray(v.data, dtype=np.float32)
                    data = arr.ctypes.data_as(N.c_void_p)
                    nf = arr.size
                vid = N.c_int32()
                N.check(lib.sox_plan_add_value(h, shape, len(v.shape), layout, v.buf, data, nf, v.name.encode(),
                                               ctypes_byref(vid)), f"value {v.name}")
            for n in self.nodes:
                ins = (N.c_int32 * max(len(n.ins), 1))(*n.ins)
                outs = (N.c_int32 * len(n.outs))(*n.outs)
                if n.p is None:
                    pb, pn = None, 0
                elif isinstance(n.p, (bytes, bytearray)):
                    buf = ctypes_buffer(n.p)
                    pb, pn = ctypes_addr(buf), len(n.p)
                else:
                    rec = n.p.native()
                    pb, pn = ctypes_addr(rec), ctypes_sizeof(rec)
                    n._rec = rec  # keep alive through the call
                nid = N.c_int32()
                N.check(lib.sox_plan_add_node(h, N.OP[n.op], ins, len(n.ins), outs, len(n.outs), pb, pn,
                                              n.ext.encode() if n.ext else None, ctypes_byref(nid)),
                        f"node {n.name or n.op}")
            offs = (N.c_int64 * max(len(self.buf_offset), 1))(*self.buf_offset)
            N.check(lib.sox_plan_set_arena(h, offs, len(self.buf_offset), self.arena_floats), "arena")
            ins = (N.c_int32 * len(self.inputs))(*self.inputs)
            N.check(lib.sox_plan_set_io(h, ins, len(self.inputs), self.output), "io")
        except Exception:
            lib.sox_plan_destroy(h)
            raise
        return h


def ctypes_byref(x):
    import ctypes
    return ctypes.byref(x)


def ctypes_buffer(b):
    import ctypes
    return ctypes.create_string_buffer(bytes(b), len(b))


def ctypes_addr(x):
    import ctypes
    return ctypes.cast(ctypes.pointer(x), N.c_void_p) if not isinstance(x, ctypes.Array) else ctypes.cast(x, N.c_void_p)


def ctypes_sizeof(x):
    import ctypes
    return ctypes.sizeof(x)


def _out_size(i, k, s, p0, p1):
    return (i + p0 + p1 - k) // s + 1


class PlanBuilder:
    """Builds fused NHWC ExecPlans node by node (what GraphCompiler emits for PlanTarget.Hip)."""

    def __init__(self):
        self.values: list = []
        self.nodes: list = []
        self._nbuf = 0
        self.inputs: list = []

    # ---- values ----
    def _new_buf(self) -> int:
        b = self._nbuf
        self._nbuf += 1
        return b

    def activation(self, shape, layout=None, name="") -> int:
        self.values.append(Value(tuple(int(s) for s in shape), layout, self._new_buf(), None, name))
        return len(self.values) - 1

    def image(self, n, c, h, w, name="") -> int:
        """A rank-4 NHWC activation (logical [n,c,h,w], physical [n,h,w,c])."""
        return self.activation((n, c, h, w), NHWC, name)

    def input(self, shape, layout=None, name="input") -> int:
        v = self.activation(shape, layout, name)
        self.inputs.append(v)
        return v

    def const(self, data, name="") -> int:
        arr = np.ascontiguousarray(data, dtype=np.float32)
        self.values.append(Value(tuple(arr.shape), None, -1, arr, name))
        return len(self.values) - 1

    def alias(self, v, shape, layout=None, name="") -> int:
        """Zero-copy reshape view (CValue.AliasOf): same buffer, new logical shape."""
        src = self.values[v]
        assert int(np.prod(shape)) == src.count, "alias must keep the element count"
        self.values.append(Value(tuple(shape), layout, src.buf, None, name or src.name + "_view", alias_of=v))
        return len(self.values) - 1

    def nhwc_shape(self, v):
        val = self.values[v]
        return val.phys if len(val.shape) == 4 else None

    def _node(self, op, ins, outs, p=None, name="", ext=""):
        self.nodes.append(Node(op, list(ins), list(outs), p, name, ext))
        return outs[0]

    # ---- ops (fused forms) ----
    def conv(self, x, w, b=None, *, stride=1, pad=None, group=1, act="none", add=None, pad_mode=0, pad_value=0.0,
             pool=None, name=""):
        """Conv (+bias)(+residual before act)(+act) [+ fused 2x2/2 max pool] (ConvP)."""
        n, ih, iw, ic = self.values[x].phys
        wv = w if isinstance(w, int) else self.const(w, name + ".w")
        oc, _, kh, kw = self.values[wv].shape
        s = (stride, stride) if isinstance(stride, int) else tuple(stride)
        if pad is None:
            pad = (kh // 2, kw // 2, kh // 2, kw // 2)
        elif isinstance(pad, int):
            pad = (pad, pad, pad, pad)
        oh, ow = _out_size(ih, kh, s[0], pad[0], pad[2]), _out_size(iw, kw, s[1], pad[1], pad[3])
        bv = -1 if b is None else (b if isinstance(b, int) else self.const(b, name + ".b"))
        pp = None
        if pool is not None:
            pp = ((2, 2), (2, 2), (0, 0, 0, 0), bool(pool == "relu"))
            oh, ow = oh // 2, ow // 2
        y = self.image(n, oc, oh, ow, name)
        p = ConvP(tuple(pad), s, (kh, kw), group=group, act=act, pad_mode=pad_mode, pad_value=pad_value, bias=bv,
                  add=-1 if add is None else add, pool=pp)
        return self._node("Conv", [x, wv], [y], p, name)

    def gemm(self, a, w, b=None, *, act="none", trans_b=False, name=""):
        """Gemm: act(A[..., K] . B + bias) with B a [K, N] (or [N, K]) const (GemmP)."""
        av = self.values[a]
        wv = w if isinstance(w, int) else self.const(w, name + ".w")
        wshape = self.values[wv].shape
        nn = wshape[0] if trans_b else wshape[1]
        bv = -1 if b is None else (b if isinstance(b, int) else self.const(b, name + ".b"))
        y = self.activation(tuple(av.shape[:-1]) + (nn,), None, name)
        return self._node("Gemm", [a, wv], [y], GemmP(trans_b, bv, act), name)

    def conv_transpose(self, x, w, b=None, *, act="none", name=""):
        """ConvTranspose, stride == kernel, no pad (ConvTP)."""
        n, ih, iw, ic = self.values[x].phys
        wv = w if isinstance(w, int) else self.const(w, name + ".w")
        _, oc, kh, kw = self.values[wv].shape
        bv = -1 if b is None else (b if isinstance(b, int) else self.const(b, name + ".b"))
        y = self.image(n, oc, ih * kh, iw * kw, name)
        return self._node("ConvTranspose", [x, wv], [y], ConvTP((kh, kw), bv, act), name)

    def channel_gate(self, x, w1, b1, w2, b2, *, act1="relu", hard=True, alpha=1.0 / 6.0, beta=0.5, offset=0.0,
                     name=""):
        """SE gate: GAP -> 1x1 (+act1) -> 1x1 -> (hard) sigmoid (+offset) -> [N,C,1,1] (ChannelGateP)."""
        n, h, w, c = self.values[x].phys
        w1v, w2v = self.const(w1, name + ".w1"), self.const(w2, name + ".w2")
        b1v = -1 if b1 is None else self.const(b1, name + ".b1")
        b2v = -1 if b2 is None else self.const(b2, name + ".b2")
        y = self.image(n, c, 1, 1, name)
        return self._node("ChannelGate", [x, w1v, w2v], [y], ChannelGateP(b1v, b2v, act1, hard, alpha, beta, offset),
                          name)

    def ew(self, a, b, op, *, act="none", name=""):
        """Elementwise Add/Sub/Mul/Div with broadcast (EwP). Output takes the larger operand's shape."""
        va, vb = self.values[a], self.values[b]
        big = va if va.count >= vb.count else vb
        y = self.activation(big.shape, big.layout, name)
        return self._node("Elementwise", [a, b], [y], EwP(op, act), name)

    def add(self, a, b, **kw):
        return self.ew(a, b, 0, **kw)

    def mul(self, a, b, **kw):
        return self.ew(a, b, 2, **kw)

    def resize_nearest(self, x, scale, add=None, add_relu=False, name=""):
        """Nearest x`scale` upsample (+ [relu] same-shape addend) (ResizeNearestP)."""
        n, h, w, c = self.values[x].phys
        y = self.image(n, c, h * scale, w * scale, name)
        ins = [x] if add is None else [x, add]
        return self._node("ResizeNearest", ins, [y], ResizeNearestP((1.0, 1.0, float(scale), float(scale)), add_relu),
                          name)

    def concat_channels(self, xs, name=""):
        n, h, w, _ = self.values[xs[0]].phys
        c = sum(self.values[x].phys[3] for x in xs)
        y = self.image(n, c, h, w, name)
        return self._node("Concat", xs, [y], ConcatP(1), name)

    def layer_norm(self, x, gamma, beta, eps=1e-5, name=""):
        gv, bv = self.const(gamma, name + ".g"), self.const(beta, name + ".b")
        val = self.values[x]
        y = self.activation(val.shape, val.layout, name)
        return self._node("LayerNorm", [x, gv, bv], [y], LnP(eps), name)

    def softmax(self, x, name=""):
        val = self.values[x]
        y = self.activation(val.shape, val.layout, name)
        return self._node("Softmax", [x], [y], None, name)

    def unary(self, op, x, name=""):
        val = self.values[x]
        y = self.activation(val.shape, val.layout, name)
        return self._node(op, [x], [y], None, name)

    def hard_sigmoid(self, x, alpha=0.2, beta=0.5, name=""):
        """HardSigmoid: clamp(alpha x + beta, 0, 1) (HardSigmoidP, ExecPlan.cs:103-106)."""
        val = self.values[x]
        y = self.activation(val.shape, val.layout, name)
        return self._node("HardSigmoid", [x], [y], HardSigmoidP(alpha, beta), name)

    def attention(self, qkv, heads, head_dim, scale, name=""):
        """Fused attention over a packed [N, T, 3*H*D] QKV tensor viewed as [N, T, 3, H, D]
        (AttentionP with FixAxis 2 = 0/1/2); output [N, H, T, D] stored as [N, T, H, D]."""
        nb, t, c3 = self.values[qkv].shape
        view = self.alias(qkv, (nb, t, 3, heads, head_dim), None, name + ".qkv5")
        y = self.activation((nb, heads, t, head_dim), (0, 2, 1, 3), name)
        dims = ((0, 3, 1, 4),) * 3
        p = AttentionP(scale, dims, (2, 2, 2), (0, 1, 2), (0, 2, 1, 3))
        self._node("Attention", [view, view, view], [y], p, name)
        # [N, T, H*D] token view of the output (its transpose dissolved into the layout)
        return self.alias(y, (nb, t, heads * head_dim), None, name + ".tokens")

    def resize_bilinear(self, x, scale, add=None, *, relu=False, add_relu=False, name=""):
        """Bilinear x`scale` resize (+ [relu]) (+ [relu] same-shape addend) (ResizeP)."""
        n, h, w, c = self.values[x].phys
        oh, ow = int(h * scale), int(w * scale)
        y = self.image(n, c, oh, ow, name)
        ins = [x] if add is None else [x, add]
        return self._node("ResizeBilinear", ins, [y], ResizeP((1.0, 1.0, float(scale), float(scale)), relu, add_relu),
                          name)

    def pad(self, x, pads, mode=0, value=0.0, name=""):
        """Pad with logical [2*rank] pads (begin.., end..) (PadP)."""
        v = self.values[x]
        r = len(v.shape)
        shape = tuple(v.shape[d] + pads[d] + pads[r + d] for d in range(r))
        y = self.activation(shape, v.layout, name)
        return self._node("Pad", [x], [y], PadP(tuple(pads), mode, value), name)

    def transpose(self, x, perm, name=""):
        """Transpose of an identity-layout value (TransposeP; the perm is then also physical)."""
        v = self.values[x]
        assert v.layout is None
        y = self.activation(tuple(v.shape[p] for p in perm), None, name)
        return self._node("Transpose", [x], [y], TransposeP(tuple(perm)), name)

    def slice(self, x, starts, ends, axes, steps, name=""):
        """Slice of an identity-layout value with resolved (clamped) starts / ends (SliceP)."""
        v = self.values[x]
        assert v.layout is None
        shape = list(v.shape)
        for s0, e0, a, st in zip(starts, ends, axes, steps):
            shape[a] = max(0, (e0 - s0 + (st - (1 if st > 0 else -1))) // st)
        y = self.activation(tuple(shape), None, name)
        return self._node("Slice", [x], [y], SliceP(tuple(starts), tuple(ends), tuple(axes), tuple(steps)), name)

    def scalar_act(self, op, x, a=0.0, b=0.0, name=""):
        """LeakyRelu (a = alpha) / Tanh (a = in scale, b = out scale) / Clip (a = min, b = max) / Erf."""
        val = self.values[x]
        y = self.activation(val.shape, val.layout, name)
        return self._node(op, [x], [y], None if op == "Erf" else ScalarP(op, a, b), name)

    def depth_to_space(self, x, block, crd=False, inverse=False, name=""):
        """DepthToSpace (or SpaceToDepth with inverse=True) of an NHWC image (DepthToSpaceP)."""
        n, h, w, c = self.values[x].phys
        if inverse:
            y = self.image(n, c * block * block, h // block, w // block, name)
        else:
            y = self.image(n, c // (block * block), h * block, w * block, name)
        return self._node("SpaceToDepth" if inverse else "DepthToSpace", [x], [y], DepthToSpaceP(block, crd), name)

    def max_pool(self, x, kernel, stride, pads, relu=False, name=""):
        """MaxPool of an NHWC image, pads (t, l, b, r), PoolP.FuseRelu (GraphCompiler.EmitPool,
        GraphCompiler.cs:1805-1825; the Relu fold of :312-315)."""
        n, h, w, c = self.values[x].phys
        oh = _out_size(h, kernel[0], stride[0], pads[0], pads[2])
        ow = _out_size(w, kernel[1], stride[1], pads[1], pads[3])
        y = self.image(n, c, oh, ow, name)
        return self._node("MaxPool", [x], [y], PoolP(tuple(kernel), tuple(stride), tuple(pads), relu), name)

    def avg_pool(self, x, kernel, stride, pads, count_include_pad=False, name=""):
        """AveragePool of an NHWC image, pads (t, l, b, r) (PoolP)."""
        n, h, w, c = self.values[x].phys
        oh = _out_size(h, kernel[0], stride[0], pads[0], pads[2])
        ow = _out_size(w, kernel[1], stride[1], pads[1], pads[3])
        y = self.image(n, c, oh, ow, name)
        return self._node("AvgPool", [x], [y], PoolP(tuple(kernel), tuple(stride), tuple(pads), False,
                                                    count_include_pad), name)

    def global_avg_pool(self, x, name=""):
        n, h, w, c = self.values[x].phys
        y = self.image(n, c, 1, 1, name)
        return self._node("GlobalAvgPool", [x], [y], None, name)

    def matmul(self, a, b, name=""):
        """Batched MatMul [.., M, K] x [.., K, N] (B may have one batch), identity layouts."""
        va, vb = self.values[a], self.values[b]
        y = self.activation(tuple(va.shape[:-1]) + (vb.shape[-1],), None, name)
        return self._node("MatMul", [a, b], [y], None, name)

    # ---- the built-in extension ops (ExecOp.Ext, Engine/Fusions/*.cs) ----
    def safe_div(self, a, b, eps, lo, hi, name=""):
        """SafeDiv: clamp(a / max(b, eps), lo, hi) over same-shape operands (SafeDivP)."""
        v = self.values[a]
        return self.ext("SafeDiv", [a, b], v.shape, bytes(N.SafeDivP(eps, lo, hi)), v.layout, name or "safediv")

    def channel_shift(self, x, axis, group_ends, offsets, name=""):
        """ChannelShift of an NHWC image: channel group g shifted by offsets[g] along H (axis 2) or W (3)."""
        v = self.values[x]
        p = N.ShiftP()
        p.axis, p.ngroups = axis, len(group_ends)
        p.group_ends[:len(group_ends)] = list(group_ends)
        p.offsets[:len(offsets)] = list(offsets)
        return self.ext("ChannelShift", [x], v.shape, bytes(p), v.layout, name or "shift")

    def up_head(self, x, skip, w, b, scale, *, resize_relu=False, skip_relu=False, act="none", skip_conv=None,
                name=""):
        """UpHead: act(bias + W . ([relu](bilinear x`scale`(x)) + [relu](skip))), W [oc, c] (UpHeadP). With
        skip_conv = (w_sc [c, skc, kh, kw], b_sc, pads (t, l, b, r), pad_mode, pad_value, act) the `skip`
        argument is that stride-1 conv's input and the skip is recomputed from it."""
        n, h, ww, c = self.values[x].phys
        oc = np.asarray(w).shape[0]
        wv = self.const(np.asarray(w, np.float32).reshape(oc, c, 1, 1), name + ".w")
        ins = [x, skip, wv] + ([] if b is None else [self.const(b, name + ".b")])
        p = N.UpHeadP()
        p.scales[:] = [1.0, 1.0, float(scale), float(scale)]
        p.resize_relu, p.skip_relu, p.act = int(resize_relu), int(skip_relu), ACT[act]
        p.skip_w = p.skip_b = -1
        if skip_conv is not None:
            w_sc, b_sc, pads, pad_mode, pad_value, sc_act = skip_conv
            kh, kw = np.asarray(w_sc).shape[2:]
            p.has_skip_conv = 1
            p.skip_conv = ConvP(tuple(pads), (1, 1), (kh, kw), act=sc_act, pad_mode=pad_mode, pad_value=pad_value).native()
            p.skip_w = self.const(w_sc, name + ".w_sc")
            p.skip_b = -1 if b_sc is None else self.const(b_sc, name + ".b_sc")
        y = self.activation((n, oc, int(h * scale), int(ww * scale)), NHWC, name or "uphead")
        self._node("Ext", ins, [y], bytes(p), name or "uphead", ext="UpHead")
        return y

    def ext(self, name, ins, out_shape, params: bytes = b"", layout=None, node_name=""):
        """ExecOp.Ext node of a consumer-registered operator."""
        y = self.activation(out_shape, layout, node_name or name)
        return self._node("Ext", ins, [y], bytes(params), node_name or name, ext=name)

    # ---- finish: arena planning ----
    def build(self, output: int) -> ExecPlan:
        return plan_arena(self.values, self.nodes, self.inputs, output, self._nbuf)


def plan_arena(values, nodes, inputs, output, nbuf, align=32) -> ExecPlan:
    """Lifetime-packed arena (the PlanArena analogue, GraphCompiler.cs:1336-1474): each buffer is
    live from its producing node to its last reader (inputs from the start, the output to the end);
    first-fit placement at `align`-element granularity; no buffer overlaps a live one."""
    size = [0] * nbuf
    for v in values:
        if v.buf >= 0:
            size[v.buf] = max(size[v.buf], v.count)
    first = [None] * nbuf
    last = [-1] * nbuf
    for b in {values[i].buf for i in inputs}:
        first[b] = -1
    for i, n in enumerate(nodes):
        for vid in list(n.ins) + n.param_refs():
            b = values[vid].buf
            if b >= 0:
                last[b] = max(last[b], i)
        for vid in n.outs:
            b = values[vid].buf
            if first[b] is None:
                first[b] = i
    end = len(nodes)
    last[values[output].buf] = end
    for b in {values[i].buf for i in inputs}:
        last[b] = end  # inputs stay intact for the whole run (CompileOptions.ReleaseInputs = false)
    offset = [0] * nbuf
    live: list = []  # (start, stop, buf)
    order = sorted((b for b in range(nbuf) if first[b] is not None), key=lambda b: (first[b], -size[b]))
    top = 0
    for b in order:
        live = [iv for iv in live if last[iv[2]] >= first[b]]
        sz = (size[b] + align - 1) // align * align
        cand = 0
        for s, e, _ in sorted(live):
            if cand + sz <= s:
                break
            cand = max(cand, e)
        offset[b] = cand
        live.append((cand, cand + sz, b))
        top = max(top, cand + sz)
    return ExecPlan(values, nodes, offset, top, list(inputs), output)
