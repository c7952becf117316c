"""Workload-level parity on the GPU: each benchmark configuration through the backend vs the oracle
on the same seeded inputs and weights (max-rel: 1e-4 fp32 paths, 2e-2 fp16/bf16 MFMA paths)."""
import numpy as np
import pytest

from oracle.interp import run_plan
from simdonnx_amd import graphs
from simdonnx_amd.backend import HipInferenceSession
from tests.conftest import max_rel

pytestmark = pytest.mark.gpu


def run_gpu(hip, plan, inputs, f16):
    print(f"[gpu] workload {len(plan.nodes)} nodes f16={f16}", flush=True)
    with HipInferenceSession(hip.graph(plan, f16)) as s:
        for i, x in enumerate(inputs):
            s.set_input(x, i)
        return s.run().copy()


def test_conv3x3_bias_relu_fp32(hip):
    plan, ins = graphs.conv3x3_bias_relu()
    got = run_gpu(hip, plan, ins, False)
    want = run_plan(plan, ins)
    assert max_rel(got, want) <= 1e-4


def test_matmul_bias_gelu_fp16(hip):
    plan, ins = graphs.matmul_bias_gelu()
    got = run_gpu(hip, plan, ins, True)
    want = run_plan(plan, ins)
    assert max_rel(got, want) <= 2e-2


def test_matmul_bias_gelu_fp32(hip):
    plan, ins = graphs.matmul_bias_gelu(batch=2)
    got = run_gpu(hip, plan, ins, False)
    want = run_plan(plan, ins)
    assert max_rel(got, want) <= 1e-4
