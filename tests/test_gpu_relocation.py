"""A rewritten output moved to a buffer of its own, read through a view by a later node, on the GPU.

Four graph-creation rewrites write an output where the unfused plan's arena may have put it over the
rewrite's input (the residual Add in the Gemm epilogue, the BatchNorm folded into a ConvTranspose, a
LayerNorm folded into its Gemm, the fused transformer MLP). The output then moves, and a view of it
(a Reshape feeding the next Gemm, CValue.AliasOf, Engine/ExecPlan.cs:207, 211) must move with it. For
each case (tests/relocation_cases.py):
  - the forced plan (output planned over the input) equals the packer's own plan bit for bit: the same
    kernels on the same data, so a view left at the old place would show;
  - it matches the unfused graph (the rewrite's SIMDONNX_HIP_NO_* switch): bit for bit for the
    residual Add on fp32 graphs (the epilogue adds in the unfused order), else within the rounding the
    rewrite changes (1e-5 fp32, 4e-3 fp16, 2e-2 bf16: a few storage ulps of the largest output);
  - it matches the oracle on the unfused plan: 1e-4 (fp32) / 2e-2 (16-bit storage contract).
"""
import numpy as np
import pytest

from oracle.interp import run_plan
from simdonnx_amd.backend import HipInferenceSession
from tests import relocation_cases as RC
from tests.conftest import max_rel

pytestmark = pytest.mark.gpu

UNFUSED_TOL = {"f32": 1e-5, "f16": 4e-3, "bf16": 2e-2}
ORACLE_TOL = {"f32": 1e-4, "f16": 2e-2, "bf16": 2e-2}


def _run(hip, plan, inputs, storage):
    g = hip.graph(plan, storage)
    try:
        with HipInferenceSession(g) as s:
            for i, x in enumerate(inputs):
                s.set_input(x, i)
            return s.run().copy()
    finally:
        g.release()


@pytest.mark.parametrize("storage", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("case", list(RC.CASES))
def test_relocated_output_read_through_view(hip, case, storage, monkeypatch):
    c = RC.CASES[case]()
    if storage not in c.storages:
        pytest.skip(f"the rewrite is not taken on {storage} graphs")
    print(f"[gpu] relocation case {case} {storage}", flush=True)
    forced = RC.forced(c)
    assert RC.overlaps(forced, c.moved, c.over)
    g = hip.graph(forced, storage)
    try:
        place = g.value_place(c.moved)
        assert g.value_place(c.view)[0] == place[0], "the view stayed behind"
        assert place[0] >= forced.arena_floats * (4 if storage == "f32" else 2), "the rewrite did not move its output"
        with HipInferenceSession(g) as s:
            for i, x in enumerate(c.inputs):
                s.set_input(x, i)
            got = s.run().copy()
    finally:
        g.release()
    natural = _run(hip, c.plan, c.inputs, storage)
    assert got.tobytes() == natural.tobytes(), f"max diff {np.abs(got - natural).max()}"
    monkeypatch.setenv(c.switch, "1")
    unfused = _run(hip, forced, c.inputs, storage)
    err_unfused = max_rel(got, unfused)
    want = run_plan(c.plan, c.inputs, f16_storage={"f32": False, "f16": True, "bf16": "bf16"}[storage])
    err_oracle = max_rel(got, want)
    print(f"[gpu] {case} {storage}: vs unfused {err_unfused:.2e}, vs oracle {err_oracle:.2e}", flush=True)
    if case == "residual_gemm" and storage == "f32":
        assert got.tobytes() == unfused.tobytes()
    assert err_unfused <= UNFUSED_TOL[storage]
    assert err_oracle < ORACLE_TOL[storage]


@pytest.mark.parametrize("storage", ["f16", "bf16"])
def test_upsample_add_input_survives_fused_mlp(hip, storage, monkeypatch):
    """The lateral conv of an FPN Add runs at the Add's place; a fused transformer MLP in between writes
    fc2's output from fc1's dispatch. With that output planned over the conv's input (forced), the
    result equals the packer's own plan bit for bit, the unfused Add (SIMDONNX_HIP_NO_UPADD) within the
    rounding the fusion changes, and the oracle within the 16-bit contract."""
    plan, ins, xi, f2, up = RC.upsample_add_after_fused_write()
    forced = RC.place_over(plan, f2, xi)
    print(f"[gpu] upsample add after fused MLP {storage}", flush=True)
    got = _run(hip, forced, ins, storage)
    natural = _run(hip, plan, ins, storage)
    assert got.tobytes() == natural.tobytes(), f"max diff {np.abs(got - natural).max()}"
    monkeypatch.setenv("SIMDONNX_HIP_NO_UPADD", "1")
    unfused = _run(hip, forced, ins, storage)
    want = run_plan(plan, ins, f16_storage={"f16": True, "bf16": "bf16"}[storage])
    print(f"[gpu] vs unfused {max_rel(got, unfused):.2e}, vs oracle {max_rel(got, want):.2e}", flush=True)
    assert max_rel(got, unfused) <= UNFUSED_TOL[storage]
    assert max_rel(got, want) < ORACLE_TOL[storage]
