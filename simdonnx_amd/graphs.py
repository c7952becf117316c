"""The benchmark workloads as fused NHWC ExecPlans (what GraphCompiler emits for them, PlanTarget.Hip).

Every workload returns ``(plan, inputs)``: the plan and its seeded fp32 inputs in physical layout.
Weights and inputs come from ``synth`` (a counter-based generator; the reference's System.Random
cannot be reproduced outside .NET). Workloads:

  conv3x3_bias_relu   1x64x64x64 NHWC fp32, Conv3x3 s1 p1 64->64 + bias + ReLU
  matmul_bias_gelu    A[16,512,768] x W[768,3072] + b[3072] -> GELU (Gemm after FuseBiasAdd / FuseGelu /
                      FuseLateAct, GraphCompiler.cs:1161-1213, 1058-1105, 800-874)
  mobilenetv3_small   MobileNetV3-small backbone at 3x640x640 (configs 3 / 4)
  dbnet               DBNet-style detector at 3x960x960 (config 4)
  svtr                SVTR/CRNN-style recognizer, batch 32 of 3x48x320 (config 5)
"""
from __future__ import annotations

import numpy as np

from . import synth
from .plan import NHWC, PlanBuilder


class _Ids:
    """Sequential tensor ids for the generator."""

    def __init__(self):
        self.i = 0

    def __call__(self):
        self.i += 1
        return self.i


def conv3x3_bias_relu(seed: int = 1, n=1, h=64, w=64, cin=64, cout=64):
    """Single fused Conv2d 3x3 s1 p1 + bias + ReLU, NHWC; x, W ~ U(-1,1), b ~ U(-0.1,0.1)."""
    pb = PlanBuilder()
    x = pb.input((n, cin, h, w), NHWC, "x")
    W = synth.uniform(seed, 2, (cout, cin, 3, 3), -1.0, 1.0)
    b = synth.uniform(seed, 3, (cout,), -0.1, 0.1)
    y = pb.conv(x, W, b, stride=1, pad=1, act="relu", name="conv")
    plan = pb.build(y)
    xin = synth.uniform(seed, 1, (n, h, w, cin), -1.0, 1.0)
    return plan, [xin]


def conv3x3_flops(n=1, h=64, w=64, cin=64, cout=64):
    return 2 * n * h * w * cout * cin * 9


def matmul_bias_gelu(seed: int = 2, batch=16, seq=512, k=768, n=3072):
    """MatMul + bias + GELU: A ~ N(0,1), W ~ N(0, 0.02), b ~ U(-0.1, 0.1)."""
    pb = PlanBuilder()
    a = pb.input((batch, seq, k), None, "A")
    W = synth.normal(seed, 2, (k, n), 0.02)
    b = synth.uniform(seed, 3, (n,), -0.1, 0.1)
    y = pb.gemm(a, W, b, act="gelu", name="gemm_gelu")
    plan = pb.build(y)
    ain = synth.normal(seed, 1, (batch, seq, k), 1.0)
    return plan, [ain]


def matmul_flops(batch=16, seq=512, k=768, n=3072):
    return 2 * batch * seq * k * n
