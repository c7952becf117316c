"""Runs an ExecPlan on the CPU oracle: the restatement of InferenceSession.ExecNhwc
(Engine/Session.cs:322-427) over the oracle kernels. Test infrastructure only.

Values are kept as fp32 numpy arrays in their physical layout; zero-copy views (CValue.AliasOf)
are reshapes of the same data. Fused GPU-plan ops are computed with the CPU formulas they fuse:
HardSwish as a conv epilogue (Nhwc.Act8), Attention as MatMul -> scale -> Softmax -> MatMul
(Ops.Seq.cs:28-116), ChannelGate as Nhwc.ChannelGate.
"""
from __future__ import annotations

import numpy as np

import oracle as O


def _phys(plan, vid, arr):
    return np.ascontiguousarray(arr, dtype=np.float32).reshape(plan.values[vid].phys)


def f32_params(plan):
    """Value ids a GPU plan keeps in fp32 on fp16 graphs: bias, LayerNorm and SE parameters
    (ConstKind.F32, Engine/Extensions.cs:145)."""
    ids = set()
    for n in plan.nodes:
        if n.op in ("Conv", "Gemm", "ConvTranspose") and n.p.bias >= 0:
            ids.add(n.p.bias)
        if n.op == "LayerNorm":
            ids.update(n.ins[1:])
        if n.op == "ChannelGate":
            ids.update(n.ins[1:])
            ids.update(r for r in (n.p.b1, n.p.b2) if r >= 0)
        if n.op == "Ext" and n.ext == "UpHead":
            from simdonnx_amd import native as N
            q = N.UpHeadP.from_buffer_copy(n.p)
            ids.update(n.ins[3:])
            if q.skip_b >= 0:
                ids.add(q.skip_b)
    return ids


def _f16(a):
    return np.asarray(a, np.float32).astype(np.float16).astype(np.float32)


def _bf16(a):
    """IEEE fp32 -> bfloat16 round to nearest even -> fp32 (the bf16 storage contract)."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = np.where(nan, u | 0x400000, r)
    return (r & 0xFFFFFFFF).astype(np.uint32).view(np.float32).reshape(np.shape(a))


def run_plan(plan, inputs, keep=False, f16_storage=False):
    """Returns the output (physical layout); with keep=True also the dict of every value.

    f16_storage=True applies the reference GPU numeric contract on the CPU: graph inputs, weights
    and every stored activation are rounded to IEEE fp16 (round to nearest even) at the points the
    GPU stores them (Backends/Vulkan/VkGraph.cs:33-43, Engine/Extensions.cs:311-316), while bias /
    norm / SE parameters stay fp32 and all math stays fp32. f16_storage="bf16" rounds to bfloat16
    at the same points instead (the bf16 graph mode)."""
    env = {}
    vals = plan.values
    keep32 = f32_params(plan) if f16_storage else set()
    rnd = _bf16 if f16_storage == "bf16" else _f16 if f16_storage else (lambda a: a)
    consts = {}

    def get(vid):
        v = vals[vid]
        if v.is_const:
            if f16_storage and vid not in keep32:
                if vid not in consts:
                    consts[vid] = rnd(v.data)
                return consts[vid]
            return v.data
        if vid in env:
            return env[vid]
        if v.alias_of >= 0:
            return get(v.alias_of).reshape(v.phys)
        raise KeyError(f"value {vid} ({v.name}) read before written")

    for vid, x in zip(plan.inputs, inputs):
        env[vid] = rnd(_phys(plan, vid, x))
    for node in plan.nodes:
        p = node.p
        out = node.outs[0]
        oshape = vals[out].phys
        if node.op == "Conv":
            x = get(node.ins[0])
            w = get(node.ins[1])
            bias = get(p.bias) if p.bias >= 0 else None
            add = get(p.add) if p.add >= 0 else None
            pool_relu = p.pool[3] if p.pool is not None else False
            y = O.conv(x, w, bias, add, stride=p.strides, pads=p.pads, group=p.group, act=p.act,
                       pad_mode=p.pad_mode, pad_value=p.pad_value, pool=p.pool is not None, pool_relu=pool_relu)
        elif node.op == "Gemm":
            a = get(node.ins[0])
            bias = get(p.bias) if p.bias >= 0 else None
            y = O.gemm(a.reshape(-1, a.shape[-1]), get(node.ins[1]), bias, trans_b=p.trans_b, act=p.act)
        elif node.op == "ConvTranspose":
            y = O.conv_transpose(get(node.ins[0]), get(node.ins[1]), get(p.bias) if p.bias >= 0 else None, act=p.act)
        elif node.op == "ChannelGate":
            x = get(node.ins[0])
            w1, w2 = get(node.ins[1]), get(node.ins[2])
            r, c = w1.shape[0], w2.shape[0]
            y = O.channel_gate(x, w1.reshape(r, c), get(p.b1) if p.b1 >= 0 else None, w2.reshape(c, r),
                               get(p.b2) if p.b2 >= 0 else None, act1_relu=p.act1 == "relu", hard=p.hard,
                               alpha=p.alpha, beta=p.beta, offset=p.offset)
        elif node.op == "Elementwise":
            a, b = get(node.ins[0]), get(node.ins[1])
            act = 1 if p.act == "relu" else 0
            if a.size == b.size:
                y = O.ew2(a.reshape(-1), b.reshape(-1), op=p.op, act=act)
            elif b.size == 1 or a.size == 1:
                f = np.float32
                s = (b if b.size == 1 else a).reshape(-1)[0]
                x = a if b.size == 1 else b
                rev = a.size == 1
                y = {0: lambda: x + f(s), 1: lambda: (f(s) - x) if rev else (x - f(s)), 2: lambda: x * f(s),
                     3: lambda: (f(s) / x) if rev else (x / f(s))}[p.op]()
            else:
                # NHWC per-channel broadcast [N,H,W,C] op [N,C]
                full, vec, rev = (a, b, False) if a.size > b.size else (b, a, True)
                nb = full.shape[0]
                c = full.shape[-1]
                vec = np.broadcast_to(vec.reshape(-1, c), (nb, c))  # [N,C,1,1] gate or a [C,1,1] const
                y = np.concatenate([O.channel_broadcast(full[i].reshape(-1, c), vec[i], op=p.op, rev=rev, act=act)
                                    .reshape(1, -1) for i in range(nb)])
        elif node.op in ("Relu", "Sigmoid", "Gelu", "HardSwish", "Swish"):
            y = O.activation(get(node.ins[0]), node.op.lower())
        elif node.op == "HardSigmoid":
            y = O.hard_sigmoid(get(node.ins[0]), p.alpha, p.beta)
        elif node.op == "Copy":
            y = get(node.ins[0]).copy()
        elif node.op == "ResizeNearest":
            x = get(node.ins[0])
            add = get(node.ins[1]) if len(node.ins) > 1 else None
            y = O.resize_nearest(x, p.scales[-2], p.scales[-1], add, p.add_relu)
        elif node.op == "Concat":
            y = O.concat_channels([get(v) for v in node.ins])
        elif node.op == "LayerNorm":
            y = O.layer_norm(get(node.ins[0]), get(node.ins[1]), get(node.ins[2]), p.eps)
        elif node.op == "Softmax":
            y = O.softmax(get(node.ins[0]))
        elif node.op == "Attention":
            qkv = get(node.ins[0])  # [N, T, 3, H, D] (identity layout)
            nb, t, _, h, d = qkv.shape
            q = np.ascontiguousarray(qkv[:, :, 0].transpose(0, 2, 1, 3)).reshape(nb * h, t, d)
            k = np.ascontiguousarray(qkv[:, :, 1].transpose(0, 2, 1, 3)).reshape(nb * h, t, d)
            v = np.ascontiguousarray(qkv[:, :, 2].transpose(0, 2, 1, 3)).reshape(nb * h, t, d)
            o = O.attention(q, k, v, p.scale).reshape(nb, h, t, d)
            y = np.ascontiguousarray(o.transpose(0, 2, 1, 3))  # stored [N, T, H, D]
        elif node.op == "ResizeBilinear":
            x = get(node.ins[0])
            add = get(node.ins[1]) if len(node.ins) > 1 else None
            y = O.resize_bilinear(x, p.scales[-2], p.scales[-1], add, relu=p.fuse_relu, add_relu=p.add_relu)
        elif node.op == "Pad":
            x = get(node.ins[0])  # NHWC, spatial pads only (Kernels/Nhwc.cs:877-900)
            r = len(p.pads) // 2
            assert r == 4 and p.pads[0] == p.pads[1] == p.pads[4] == p.pads[5] == 0
            y = O.pad_nhwc(x, p.pads[2], p.pads[3], p.pads[6], p.pads[7], p.mode, p.value)
        elif node.op == "Transpose":
            y = O.transpose(get(node.ins[0]), p.perm)
        elif node.op == "Slice":
            y = O.slice_(get(node.ins[0]), p.starts, p.ends, p.axes, p.steps)
        elif node.op in ("LeakyRelu", "Tanh", "Clip", "Erf"):
            y = O.unary2(get(node.ins[0]), node.op, *((p.a, p.b) if p is not None else (0.0, 0.0)))
        elif node.op in ("DepthToSpace", "SpaceToDepth"):
            y = O.depth_to_space(get(node.ins[0]), p.block, p.crd, node.op == "SpaceToDepth")
        elif node.op == "MaxPool":
            y = O.max_pool(get(node.ins[0]), p.kernel, p.strides, p.pads, p.relu)
        elif node.op == "AvgPool":
            y = O.avg_pool(get(node.ins[0]), p.kernel, p.strides, p.pads, p.count_include_pad)
        elif node.op == "GlobalAvgPool":
            y = O.global_avg_pool(get(node.ins[0]))
        elif node.op == "MatMul":
            y = O.matmul_bcast(get(node.ins[0]), get(node.ins[1]))
        elif node.op == "Ext" and node.ext in ("SafeDiv", "ChannelShift", "UpHead"):
            from simdonnx_amd import native as N  # the records' layout only
            if node.ext == "SafeDiv":
                q = N.SafeDivP.from_buffer_copy(node.p)
                y = O.safe_div(get(node.ins[0]), get(node.ins[1]), q.eps, q.lo, q.hi)
            elif node.ext == "ChannelShift":
                q = N.ShiftP.from_buffer_copy(node.p)
                y = O.channel_shift(get(node.ins[0]), q.axis, list(q.group_ends)[:q.ngroups], list(q.offsets)[:q.ngroups])
            else:
                q = N.UpHeadP.from_buffer_copy(node.p)
                skip = get(node.ins[1])
                if q.has_skip_conv:  # recomputed by the stem conv's direct kernel (FusedKernels.cs:81-83)
                    sc = q.skip_conv
                    acts = {v: k for k, v in O.ACT.items()}
                    skip = O.conv(skip, get(q.skip_w), get(q.skip_b) if q.skip_b >= 0 else None, None, stride=(1, 1),
                                  pads=tuple(sc.pads), act=acts[sc.act], pad_mode=sc.pad_mode, pad_value=sc.pad_value,
                                  algo=1)
                w = get(node.ins[2])
                y = O.up_head(get(node.ins[0]), skip, w.reshape(w.shape[0], -1),
                              get(node.ins[3]) if len(node.ins) > 3 else None, q.scales[3],
                              resize_relu=bool(q.resize_relu), skip_relu=bool(q.skip_relu), act=q.act)
        else:
            raise NotImplementedError(f"oracle interpreter: {node.op}")
        env[out] = rnd(np.ascontiguousarray(y, dtype=np.float32).reshape(oshape))
    res = get(plan.output)
    return (res, env) if keep else res
