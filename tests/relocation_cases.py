"""Plans in which a graph-creation rewrite moves its output to a buffer of its own while a zero-copy
view of that output (CValue.AliasOf: Reshape / Squeeze / Unsqueeze / Identity, Engine/ExecPlan.cs:207,
211) is read by a later node. Views share their source's buffer id and are bound through that buffer's
offset (Backends/Vulkan/VkGraph.cs:365-367), so the move must take the views along.

Each case is built twice over the same values: ``forced``, whose arena plan puts the rewritten output
over the rewrite's input (legal for the unfused plan, where that input is dead by then, so the rewrite
has to move the output), and ``natural``, the lifetime packer's own plan. Both run the same kernels on
the same data, so their outputs must be equal bit for bit; a view left at the old place reads
something else. Used by tests/test_host_lowering.py (the places and binds, on the CPU) and
tests/test_gpu_relocation.py (the numbers, on the GPU). Not collected by pytest itself.
"""
from __future__ import annotations

import copy
from dataclasses import dataclass

import numpy as np

from simdonnx_amd import synth
from simdonnx_amd.plan import NHWC, PlanBuilder


@dataclass
class Case:
    name: str
    plan: object          # ExecPlan
    inputs: list
    moved: int            # the value the rewrite relocates (forced plan)
    over: int             # the value it was planned over
    view: int             # a view of `moved` read by a later node
    switch: str           # env var that turns the rewrite off
    fused_label: str      # a dispatch label that shows the rewrite was taken
    storages: tuple       # storage modes the rewrite applies to


def lifetimes(plan):
    """[first writer, last reader] node index per buffer, as the lifetime packer counts them
    (graph inputs from -1 and, with the output, to the end; an unread value at its writer)."""
    nb = len(plan.buf_offset)
    first, last = [None] * nb, [-1] * nb
    for i in plan.inputs:
        first[plan.values[i].buf] = -1
    for k, n in enumerate(plan.nodes):
        for v in list(n.ins) + n.param_refs():
            b = plan.values[v].buf
            if b >= 0:
                last[b] = max(last[b], k)
        for v in n.outs:
            b = plan.values[v].buf
            if first[b] is None:
                first[b] = k
    end = len(plan.nodes)
    last[plan.values[plan.output].buf] = end
    for i in plan.inputs:
        last[plan.values[i].buf] = end
    for bi in range(nb):  # a value nothing reads is still live where it is written
        if first[bi] is not None:
            last[bi] = max(last[bi], first[bi])
    return first, last


def buffer_sizes(plan):
    size = [0] * len(plan.buf_offset)
    for v in plan.values:
        if v.buf >= 0:
            size[v.buf] = max(size[v.buf], v.count)
    return size


def conflicts(plan):
    """Pairs of buffers live at the same node whose arena ranges overlap (an invalid arena plan)."""
    first, last = lifetimes(plan)
    size = buffer_sizes(plan)
    live = [b for b in range(len(size)) if first[b] is not None]
    out = []
    for i, a in enumerate(live):
        for b in live[i + 1:]:
            if first[a] <= last[b] and first[b] <= last[a]:
                oa, ob = plan.buf_offset[a], plan.buf_offset[b]
                if oa < ob + size[b] and ob < oa + size[a]:
                    out.append((a, b))
    return out


def place_over(plan, v, over, shift=0):
    """Puts value v's buffer at value `over`'s offset (+ shift elements); any other buffer that then
    collides with a buffer live beside it moves past the end of the arena. Returns the new plan."""
    p = copy.deepcopy(plan)
    bv, bo = p.values[v].buf, p.values[over].buf
    p.buf_offset[bv] = p.buf_offset[bo] + shift
    size = buffer_sizes(p)
    top = max(p.arena_floats, max(p.buf_offset[b] + size[b] for b in range(len(size))))
    for _ in range(len(size)):
        bad = conflicts(p)
        if not bad:
            break
        a, b = bad[0]
        m = b if a == bv else a  # v's buffer stays where it was put
        p.buf_offset[m] = (top + 63) // 64 * 64
        top = p.buf_offset[m] + size[m]
    assert not conflicts(p), "could not make the forced arena plan valid"
    p.arena_floats = max(top, max(p.buf_offset[b] + size[b] for b in range(len(size))))
    first, last = lifetimes(p)
    assert last[bo] < first[bv], "the forced placement must be legal for the unfused plan"
    return p


def overlaps(plan, a, b):
    va, vb = plan.values[a], plan.values[b]
    oa, ob = plan.buf_offset[va.buf], plan.buf_offset[vb.buf]
    return oa < ob + vb.count and ob < oa + va.count


def residual_gemm(seed=101, rows=512, c=256):
    """Gemm (no activation) + Add of a residual: the Add runs in the Gemm epilogue and writes its
    output while other workgroups still read the Gemm's input A, so an output planned over A moves
    (plan_residual_adds). A Reshape of the Add's output feeds the next Gemm."""
    pb = PlanBuilder()
    x = pb.input((rows, c), None, "x")
    r = pb.input((rows, c), None, "r")
    a = pb.unary("Relu", x, name="a")
    y = pb.gemm(a, synth.normal(seed, 1, (c, c), 0.05), synth.uniform(seed, 2, (c,), -0.1, 0.1), name="fc")
    o = pb.add(y, r, name="res")
    v = pb.alias(o, (rows // 2, 2 * c), name="res.view")
    z = pb.gemm(v, synth.normal(seed, 3, (2 * c, 64), 0.05), synth.uniform(seed, 4, (64,), -0.1, 0.1), name="next")
    plan = pb.build(z)
    ins = [synth.normal(seed, 5, (rows, c), 1.0), synth.normal(seed, 6, (rows, c), 1.0)]
    return Case("residual_gemm", plan, ins, o, a, v, "SIMDONNX_HIP_NO_RES_FUSE", "gemm", ("f32", "f16", "bf16"))


def convt_affine(seed=102, c=24, hw=40):
    """ConvTranspose 2x2/2 + per-channel Mul + Add + ReLU (an unfolded BatchNorm): the pair folds into
    the ConvTranspose, which writes the Add's output; an output planned over the ConvTranspose's input
    moves (fold_affine_after_convt). A flattening view of it feeds a Gemm over its pixels."""
    pb = PlanBuilder()
    x = pb.input((1, c, hw, hw), NHWC, "x")
    a = pb.unary("Relu", x, name="a")
    y = pb.conv_transpose(a, synth.normal(seed, 1, (c, c, 2, 2), 0.2), synth.uniform(seed, 2, (c,), -0.1, 0.1),
                          name="convt")
    s = pb.const(synth.uniform(seed, 3, (c, 1, 1), 0.5, 1.5), "bn.s")
    t = pb.const(synth.uniform(seed, 4, (c, 1, 1), -0.1, 0.1), "bn.t")
    m = pb.ew(y, s, 2, name="bn.mul")
    o = pb.ew(m, t, 0, act="relu", name="bn.add")
    v = pb.alias(o, (4 * hw * hw, c), name="bn.pixels")
    z = pb.gemm(v, synth.normal(seed, 5, (c, 32), 0.2), synth.uniform(seed, 6, (32,), -0.1, 0.1), name="head")
    plan = pb.build(z)
    ins = [synth.normal(seed, 7, (1, hw, hw, c), 1.0)]
    return Case("convt_affine", plan, ins, o, a, v, "SIMDONNX_HIP_NO_CONVT_FOLD", "convt", ("f32", "f16", "bf16"))


def layernorm_gemm(seed=103, rows=256, k=192):
    """LayerNorm -> Gemm: the LayerNorm folds into the Gemm, which reads the LayerNorm's input; a Gemm
    output planned over that input moves (fold_layernorm_into_gemm, 16-bit graphs). A Reshape of the
    output feeds the next Gemm."""
    pb = PlanBuilder()
    x = pb.input((rows, k), None, "x")
    a = pb.unary("Relu", x, name="a")
    h = pb.layer_norm(a, 1.0 + synth.uniform(seed, 1, (k,), -0.1, 0.1), synth.uniform(seed, 2, (k,), -0.1, 0.1), 1e-6,
                      name="ln")
    y = pb.gemm(h, synth.normal(seed, 3, (k, k), 0.05), synth.uniform(seed, 4, (k,), -0.1, 0.1), name="qkv")
    v = pb.alias(y, (rows * k // 64, 64), name="qkv.view")
    z = pb.gemm(v, synth.normal(seed, 5, (64, 64), 0.1), synth.uniform(seed, 6, (64,), -0.1, 0.1), name="next")
    plan = pb.build(z)
    ins = [synth.normal(seed, 7, (rows, k), 1.0)]
    return Case("layernorm_gemm", plan, ins, y, a, v, "SIMDONNX_HIP_NO_LN_FOLD", "gemm_ln", ("f16", "bf16"))


def mlp(seed=104, rows=512, k=192, hidden=768):
    """LayerNorm -> fc1 + GELU -> fc2 as one kernel (plan_fused_mlp, 16-bit graphs): each workgroup reads
    its rows of x while others write the output, so an output planned over x at another offset moves.
    A Reshape of the output feeds the next Gemm."""
    pb = PlanBuilder()
    x = pb.input((rows, k), None, "x")
    a = pb.unary("Relu", x, name="a")
    h = pb.layer_norm(a, 1.0 + synth.uniform(seed, 1, (k,), -0.1, 0.1), synth.uniform(seed, 2, (k,), -0.1, 0.1), 1e-6,
                      name="ln")
    f1 = pb.gemm(h, synth.normal(seed, 3, (k, hidden), 0.05), synth.uniform(seed, 4, (hidden,), -0.1, 0.1),
                 act="gelu", name="fc1")
    f2 = pb.gemm(f1, synth.normal(seed, 5, (hidden, k), 0.05), synth.uniform(seed, 6, (k,), -0.1, 0.1), name="fc2")
    v = pb.alias(f2, (rows * k // 64, 64), name="fc2.view")
    z = pb.gemm(v, synth.normal(seed, 7, (64, 64), 0.1), synth.uniform(seed, 8, (64,), -0.1, 0.1), name="next")
    plan = pb.build(z)
    ins = [synth.normal(seed, 9, (rows, k), 1.0)]
    return Case("mlp", plan, ins, f2, a, v, "SIMDONNX_HIP_NO_MLP_FUSE", "mlp", ("f16", "bf16"))


CASES = {f.__name__: f for f in (residual_gemm, convt_affine, layernorm_gemm, mlp)}
# the MLP output is planned over x shifted by a few rows (the same rows at the same offset are allowed)
SHIFT = {"mlp": 64 * 192}


def forced(case: Case):
    """The case's plan with the rewritten output planned over the rewrite's input."""
    return place_over(case.plan, case.moved, case.over, SHIFT.get(case.name, 0))


def upsample_add_after_fused_write(seed=105, c=64, hw=16, rows=512, k=192, hidden=768):
    """The FPN Add o = up(u) + conv1x1(xi) runs the conv in the Add's place (plan_upsample_add), so xi
    must survive until then. Between the conv and the Add a transformer MLP (LayerNorm -> fc1 + GELU ->
    fc2) runs as one kernel at fc1's place (plan_fused_mlp): fc2 is folded and its output f2 is written
    by fc1's dispatch. Returns (plan, inputs, xi, f2, the Resize+Add node): the forced plan puts f2 over
    xi, which the unfused order allows (xi is dead after the conv there) and the fused one must undo by
    moving f2."""
    pb = PlanBuilder()
    x = pb.input((1, c, hw, hw), NHWC, "x")
    u = pb.input((1, c, hw // 2, hw // 2), NHWC, "u")
    t = pb.input((rows, k), None, "t")
    xi = pb.unary("Relu", x, name="xi")
    a = pb.conv(xi, synth.normal(seed, 1, (c, c, 1, 1), 0.1), synth.uniform(seed, 2, (c,), -0.1, 0.1), name="lat")
    h = pb.layer_norm(t, 1.0 + synth.uniform(seed, 3, (k,), -0.1, 0.1), synth.uniform(seed, 4, (k,), -0.1, 0.1), 1e-6,
                      name="ln")
    f1 = pb.gemm(h, synth.normal(seed, 5, (k, hidden), 0.05), synth.uniform(seed, 6, (hidden,), -0.1, 0.1),
                 act="gelu", name="fc1")
    f2 = pb.gemm(f1, synth.normal(seed, 7, (hidden, k), 0.05), synth.uniform(seed, 8, (k,), -0.1, 0.1), name="fc2")
    o = pb.resize_nearest(u, 2, add=a, name="up")
    plan = pb.build(o)
    ins = [synth.normal(seed, 9, (1, hw, hw, c), 1.0), synth.normal(seed, 10, (1, hw // 2, hw // 2, c), 1.0),
           synth.normal(seed, 11, (rows, k), 1.0)]
    up = next(i for i, n in enumerate(plan.nodes) if o in n.outs)
    return plan, ins, xi, f2, up
