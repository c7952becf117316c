"""The host lowering on the CPU, with no device: every workload plan goes through graph creation on a
backend built by sox_backend_create_offline (the graph-creation rewrites, the arena moves, const
packing, the kernel choice against the embedded code objects' symbol tables), and the result is
checked for what can be checked without running it:
  - every dispatch's kernel exists in the embedded code objects, and every arena / const binding lies
    inside the slab / the const store;
  - a rewritten output moved to a buffer of its own takes its zero-copy views along (Engine/ExecPlan.cs:
    207, 211; Backends/Vulkan/VkGraph.cs:365-367), and the node reading the view binds the new place.
The same file then runs again in a child process against the host-sanitizer build of the library
(AddressSanitizer + UndefinedBehaviorSanitizer, simdonnx_amd.build.build_sanitized_backend), the HIP
counterpart of the reference's validation-layer mode (Backends/Vulkan/VkDevice.cs:176).
"""
import functools
import os
import subprocess
import sys

import pytest

from simdonnx_amd import graphs
from simdonnx_amd import native as N
from simdonnx_amd.backend import HipBackend
from tests import relocation_cases as RC

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
STORAGES = ["f32", "f16", "bf16"]


@functools.lru_cache(maxsize=None)
def _workload(name):
    return {
        "conv3x3": graphs.conv3x3_bias_relu,
        "matmul_gelu": graphs.matmul_bias_gelu,
        "mobilenetv3": graphs.mobilenetv3_small,
        "dbnet": graphs.dbnet,
        "svtr": graphs.svtr,
        "svtr_features": lambda: graphs.svtr(head="features")[:2],
    }[name]()[0]


@pytest.fixture(scope="module")
def offline():
    b = HipBackend.offline()
    yield b
    b.close()


def _check_binds(g):
    arena, consts, sync = g.arena_bytes, g.const_bytes, g.sync_bytes
    for i in range(len(g.dispatches)):
        for slot, off, size in g.binds(i):
            if slot == N.SLOT_ARENA:
                assert off + size <= arena, (i, g.kernels[i], off, size, arena)
            elif slot == N.SLOT_CONSTS:
                assert off + size <= consts, (i, g.kernels[i], off, size, consts)
            elif slot == N.SLOT_SYNC:
                assert off + size <= sync, (i, g.kernels[i], off, size, sync)
            else:
                assert slot == N.SLOT_DUMMY, (i, g.kernels[i], slot)


def test_sanitizer_build_is_the_one_loaded_when_asked():
    """Under SIMDONNX_HIP_BACKEND_LIB (the child run below) the sanitizer build and its runtime are
    the ones mapped into the process."""
    want = os.environ.get("SIMDONNX_HIP_BACKEND_LIB")
    if not want:
        pytest.skip("runs in the sanitizer child process")
    N.backend()
    maps = open("/proc/self/maps").read()
    assert os.path.realpath(want) in maps
    assert "libclang_rt.asan" in maps


@pytest.mark.parametrize("storage", STORAGES)
@pytest.mark.parametrize("name", ["conv3x3", "matmul_gelu", "mobilenetv3", "dbnet", "svtr", "svtr_features"])
def test_workload_lowers_without_device(offline, name, storage):
    g = offline.graph(_workload(name), storage)
    try:
        kernels = g.kernels
        assert kernels and all(k.startswith("sox_") for k in kernels)
        _check_binds(g)
    finally:
        g.release()


@pytest.mark.parametrize("storage", STORAGES)
@pytest.mark.parametrize("name", ["mobilenetv3", "dbnet"])
def test_se_in_depthwise_lowers_without_device(offline, name, storage, monkeypatch):
    """Under SIMDONNX_HIP_SE_IN_DW every SE gate of the convnets runs in its depthwise conv's launch:
    nine depthwise_se dispatches, no gap_part / se_gate, each with its own counters in the session's
    counter block (33 dispatches for MobileNetV3-small, 44 for the fp16 / bf16 detector)."""
    monkeypatch.setenv("SIMDONNX_HIP_SE_IN_DW", "1")
    g = offline.graph(_workload(name), storage)
    try:
        labels = [d[0] for d in g.dispatches]
        assert labels.count("depthwise_se") == 9 and "se_gate" not in labels and "gap_part" not in labels, labels
        if storage != "f32":
            assert len(labels) == {"mobilenetv3": 33, "dbnet": 43}[name], labels
        _check_binds(g)
        syncs = [(off, size) for i in range(len(labels)) for slot, off, size in g.binds(i) if slot == N.SLOT_SYNC]
        assert len(syncs) == 9 and len({off for off, _ in syncs}) == 9
        assert sum(size for _, size in syncs) <= g.sync_bytes
    finally:
        g.release()


def test_offline_backend_refuses_device_work(offline):
    from simdonnx_amd.backend import HipInferenceSession
    g = offline.graph(_workload("conv3x3"), "f16")
    try:
        with pytest.raises(N.NotSupportedError):
            HipInferenceSession(g)
        with pytest.raises(N.NotSupportedError):
            offline.create_buffer_pool()
    finally:
        g.release()


@pytest.mark.parametrize("storage", STORAGES)
@pytest.mark.parametrize("case", list(RC.CASES))
def test_relocated_output_keeps_its_views(offline, case, storage, monkeypatch):
    c = RC.CASES[case]()
    if storage not in c.storages:
        pytest.skip(f"the rewrite is not taken on {storage} graphs")
    p = RC.forced(c)
    assert RC.overlaps(p, c.moved, c.over) and not RC.conflicts(p)
    es = 4 if storage == "f32" else 2
    g = offline.graph(p, storage)
    monkeypatch.setenv(c.switch, "1")
    g_off = offline.graph(p, storage)
    try:
        labels, labels_off = [d[0] for d in g.dispatches], [d[0] for d in g_off.dispatches]
        assert len(labels) < len(labels_off) or (c.fused_label in labels and c.fused_label not in labels_off), \
            f"the rewrite was not taken: {labels} / {labels_off}"
        _check_binds(g)
        place = g.value_place(c.moved)
        assert g.value_place(c.view)[0] == place[0], "the view stayed behind"
        assert place[0] != p.buf_offset[p.values[c.moved].buf] * es, "the output was not moved"
        assert place[0] >= p.arena_floats * es, "the new place is past the planned activations"
        # the unfused graph keeps the planned place
        assert g_off.value_place(c.moved)[0] == p.buf_offset[p.values[c.moved].buf] * es
        reader = next(k for k, n in enumerate(p.nodes) if c.view in n.ins)
        binds = [b for i, d in enumerate(g.dispatches) if d[2] == reader for b in g.binds(i)]
        assert (N.SLOT_ARENA, place[0]) in [(s, o) for s, o, _ in binds], binds
    finally:
        g.release()
        g_off.release()


def test_host_lowering_under_sanitizers():
    """This file's other tests again, in a child process that loads the ASan + UBSan build of the
    backend library; any sanitizer report fails the child."""
    if os.environ.get("SIMDONNX_HIP_BACKEND_LIB"):
        pytest.skip("already the sanitizer child")
    from simdonnx_amd import build as B
    rt = B.sanitizer_runtime()
    if not rt:
        pytest.skip("the host compiler has no shared AddressSanitizer runtime")
    src = os.path.join(B.HDIR, "backend.cpp")
    if not os.path.exists(B.SAN_BACKEND) or os.path.getmtime(B.SAN_BACKEND) < os.path.getmtime(src):
        B.build_sanitized_backend()
    env = dict(os.environ)
    env["LD_PRELOAD"] = rt + (":" + env["LD_PRELOAD"] if env.get("LD_PRELOAD") else "")
    env["ASAN_OPTIONS"] = "detect_leaks=0:halt_on_error=1"
    env["UBSAN_OPTIONS"] = "halt_on_error=1:print_stacktrace=1"
    env["SIMDONNX_HIP_BACKEND_LIB"] = B.SAN_BACKEND
    r = subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider", os.path.abspath(__file__),
                        "-k", "not under_sanitizers"], cwd=ROOT, env=env, capture_output=True, text=True, timeout=1200)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-6000:]
    for marker in ("AddressSanitizer", "runtime error:", "LeakSanitizer"):
        assert marker not in out, out[-6000:]


@pytest.mark.parametrize("storage", ["f16", "bf16"])
def test_upsample_add_input_survives_fused_writes(offline, storage):
    """plan_upsample_add runs the lateral conv at the Add's place, so its input must survive what the
    dispatches in between write, including outputs written by a fused dispatch for a folded node (the
    transformer MLP writes fc2's output from fc1's place): an fc2 output planned over the conv's input
    moves to a buffer of its own (tests/relocation_cases.py: upsample_add_after_fused_write)."""
    plan, ins, xi, f2, up = RC.upsample_add_after_fused_write()
    p = RC.place_over(plan, f2, xi)
    assert RC.overlaps(p, f2, xi) and not RC.conflicts(p)
    g = offline.graph(p, storage)
    try:
        labels = [d[0] for d in g.dispatches]
        assert "mlp" in labels and "nearest" not in labels and labels[-1] == "conv", labels
        _check_binds(g)
        (xo, xb), (fo, fb) = g.value_place(xi), g.value_place(f2)
        assert fo + fb <= xo or xo + xb <= fo, "the fused MLP writes over the lateral conv's input"
        conv = len(labels) - 1
        assert (N.SLOT_ARENA, xo) in [(s, o) for s, o, _ in g.binds(conv)]
    finally:
        g.release()


def _conv3x3_256(n, h, w, stride=1):
    import numpy as np
    from simdonnx_amd.plan import NHWC, PlanBuilder
    pb = PlanBuilder()
    x = pb.input((n, 256, h, w), NHWC, "x")
    y = pb.conv(x, np.zeros((256, 256, 3, 3), np.float32), np.zeros(256, np.float32), stride=stride, pad=1, act="relu",
                name="c")
    return pb.build(y)


def test_large_conv_takes_the_halo_tile(offline, monkeypatch):
    """A large 3x3 stride-1 conv over 256 channels takes the halo tile (sox_conv_*_h256), also with a
    partial last tile per row (264 = 8.25 tiles of 32 pixels), and the ring under SIMDONNX_HIP_NO_H256;
    forcing the halo tile onto a conv it does not take (stride 2) is refused at graph creation."""
    for storage in ("f16", "bf16"):
        for w in (256, 264):
            g = offline.graph(_conv3x3_256(2, 256, w), storage)
            assert g.kernels == [f"sox_conv_{storage}_h256"], g.kernels
            g.release()
    monkeypatch.setenv("SIMDONNX_HIP_NO_H256", "1")
    g = offline.graph(_conv3x3_256(2, 256, 256), "f16")
    assert g.kernels == ["sox_conv_f16_256x256_w8k64s2"], g.kernels
    g.release()
    monkeypatch.delenv("SIMDONNX_HIP_NO_H256")
    monkeypatch.setenv("SIMDONNX_HIP_CONV", "sox_conv_f16_h256")
    with pytest.raises(N.NotSupportedError):
        offline.graph(_conv3x3_256(2, 256, 256, stride=2), "f16")


def test_large_conv_tile_takes_inputs_under_2_pow_31_elements(offline, monkeypatch):
    """The 256x256 conv tile keeps one 32-bit offset into the whole input per DMA row: a large conv takes
    it below 2^31 input elements and the 256x128 tile (64-bit image bases) from there; forcing the
    256x256 tile onto a larger input is refused at graph creation, not run."""
    monkeypatch.setenv("SIMDONNX_HIP_NO_H256", "1")  # the ring's choice
    g = offline.graph(_conv3x3_256(2, 256, 256), "f16")
    assert g.kernels == ["sox_conv_f16_256x256_w8k64s2"], g.kernels
    g.release()
    big = _conv3x3_256(1, 1024, 8448)  # 2^31 + 2^26 input elements
    g = offline.graph(big, "f16")
    assert g.kernels == ["sox_conv_f16_256x128_w8k64s2"], g.kernels
    g.release()
    monkeypatch.setenv("SIMDONNX_HIP_CONV", "sox_conv_f16_256x256_w8k64s2")
    with pytest.raises(N.NotSupportedError):
        offline.graph(big, "f16")
