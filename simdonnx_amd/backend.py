"""Python face of the HIP backend: HipBackend / HipGraphModel / HipInferenceSession.

Thin wrappers over include/sox_backend.h with the reference's member names and semantics
(Backends/Vulkan/VkBackend.cs:11-267, VkGraph.cs:44-1233, VkSession.cs:63-571). All GPU work is
done by the native library; nothing here computes anything itself, and there is no fallback: a
missing library or device raises.
"""
from __future__ import annotations

import ctypes
from typing import Optional

import numpy as np

from . import native as N
from .plan import ExecPlan


STORAGE = {"f32": 0, "f16": 1, "bf16": 2}  # SOX_STORAGE_* of include/sox_backend.h


def storage_mode(f16) -> int:
    """The storage mode of a graph: True / "f16" = fp16, "bf16" = bfloat16, False / "f32" = fp32."""
    if isinstance(f16, str):
        return STORAGE[f16]
    return STORAGE["f16"] if f16 else STORAGE["f32"]


class GpuDeviceInfo:
    """GpuDeviceInfo (Backends/GpuDeviceInfo.cs:12-20)."""

    def __init__(self, info: N.DeviceInfo):
        self.name = info.name.decode()
        self.arch = info.arch.decode()
        self.compute_units = info.compute_units
        self.lds_per_cu = info.lds_per_cu
        self.clock_khz = info.clock_khz
        self.wave_size = info.warp_size
        self.vendor_id = info.vendor_id
        self.hbm_bytes = info.hbm_bytes
        self.xcds = info.xcds

    def __repr__(self):
        return (f"GpuDeviceInfo({self.name!r}, {self.arch}, {self.compute_units} CUs, "
                f"{self.hbm_bytes / 2**30:.0f} GiB, wave{self.wave_size})")


class HipBackend:
    """VkBackend analogue: one per device; ``default()`` re-creates it after a device loss."""

    _default: Optional["HipBackend"] = None

    def __init__(self, handle):
        self.h = handle
        info = N.DeviceInfo()
        N.check(N.backend().sox_backend_info(self.h, ctypes.byref(info)), "sox_backend_info")
        self.device = GpuDeviceInfo(info)
        self._ext_keep = []

    @classmethod
    def default(cls) -> "HipBackend":
        h = N.c_void_p()
        N.check(N.backend().sox_backend_default(ctypes.byref(h)), "HipBackend.Default")
        if cls._default is None or cls._default.h.value != h.value:
            cls._default = HipBackend(h)
        return cls._default

    @classmethod
    def offline(cls, info: Optional[N.DeviceInfo] = None) -> "HipBackend":
        """A backend that touches no device (sox_backend_create_offline): graphs lower completely and
        can be inspected, but cannot run. ``info`` None describes an MI355X."""
        h = N.c_void_p()
        N.check(N.backend().sox_backend_create_offline(ctypes.byref(info) if info is not None else None,
                                                       ctypes.byref(h)), "HipBackend.offline")
        b = cls(h)
        b._offline = True
        return b

    def close(self):
        """Frees an offline backend (the device backend lives for the process)."""
        if getattr(self, "_offline", False) and self.h:
            N.backend().sox_backend_destroy(self.h)
            self.h = None

    def create_buffer_pool(self) -> "HipBufferPool":
        """CreateBufferPool (VkBackend.cs:220): buffers shared by sessions that run one at a time."""
        return HipBufferPool(self)

    @classmethod
    def try_default(cls) -> Optional["HipBackend"]:
        """TryGetDefault (VkBackend.cs:75-86): None when no device can be opened."""
        try:
            return cls.default()
        except (N.SoxError, OSError, RuntimeError):
            return None

    @property
    def is_lost(self) -> bool:
        return bool(N.backend().sox_backend_is_lost(self.h))

    @staticmethod
    def mark_lost():
        """Sets the process-wide lost flag from the host (VkDevice.Lost = true, the hook
        VkDeviceLossTests.cs:33 uses): every later submit returns DeviceLostError and ``default()``
        builds a new backend."""
        N.thin().sox_device_mark_lost()

    def graph(self, plan: ExecPlan, f16=True) -> "HipGraphModel":
        """f16: True / "f16" (fp16 storage), "bf16" (bfloat16 storage) or False / "f32"."""
        return HipGraphModel(self, plan, f16)

    def new_session(self, plan: ExecPlan, f16=True, pool: Optional["HipBufferPool"] = None) -> "HipInferenceSession":
        """NewSession(model, shape, opt[, pool]) (VkBackend.cs:205-243) for an already compiled plan."""
        g = self.graph(plan, f16)
        s = HipInferenceSession(g, pool)
        g.release()  # the session holds its own reference
        return s

    def load_module(self, image: bytes):
        """Loads an extension's code object (sox_backend_load_module)."""
        buf = ctypes.create_string_buffer(image, len(image))
        m = N.c_void_p()
        N.check(N.backend().sox_backend_load_module(self.h, buf, len(image), ctypes.byref(m)), "load_module")
        self._ext_keep.append(buf)
        return m

    def register_ext(self, name: str, emit, consts=None):
        """Registers an extension op's HIP emitter (the ExtOp.EmitHip hook)."""
        def _emit(user, g, node):
            try:
                rc = emit(HipGraphView(g), node)
                return N.SOX_OK if rc is None else int(rc)
            except Exception as e:  # an exception must not cross the C ABI: the build fails with it
                print(f"extension {name} emit failed: {e!r}", flush=True)
                return N.SOX_E_INVALID
        emit_fn = N.EXT_EMIT_FN(_emit)
        if consts is None:
            consts_fn = N.EXT_CONSTS_FN(lambda *a: 0)
        else:
            def _c(user, plan, node, vals, kinds, cap):
                items = consts(node)
                for i, (v, k) in enumerate(items[:cap]):
                    vals[i], kinds[i] = v, N.CK[k] if isinstance(k, str) else k
                return min(len(items), cap)
            consts_fn = N.EXT_CONSTS_FN(_c)
        self._ext_keep += [emit_fn, consts_fn]
        N.check(N.backend().sox_backend_register_ext(self.h, name.encode(), emit_fn, consts_fn, None),
                "register_ext")


class HipBufferPool:
    """VkBufferPool analogue (Backends/Vulkan/VkBatch.cs:6-25): the arena slab and staging shared by
    the sessions of one owner that run one at a time; grows to the largest, making earlier sessions
    stale. Not thread-safe."""

    def __init__(self, backend: HipBackend):
        self.backend = backend
        h = N.c_void_p()
        N.check(N.backend().sox_buffer_pool_create(backend.h, ctypes.byref(h)), "CreateBufferPool")
        self.h = h

    @property
    def arena_bytes(self) -> int:
        n = N.c_uint64()
        N.check(N.backend().sox_buffer_pool_info(self.h, ctypes.byref(n), None), "pool info")
        return int(n.value)

    @property
    def generation(self) -> int:
        g = N.c_int32()
        N.check(N.backend().sox_buffer_pool_info(self.h, None, ctypes.byref(g)), "pool info")
        return int(g.value)

    def close(self):
        if self.h:
            N.backend().sox_buffer_pool_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()


class HipGraphView:
    """The graph handed to an extension emitter: Bind / Scratch / Dispatch (VkGraph.cs:355-400, 1117-1123)."""

    def __init__(self, g):
        self.h = g

    @property
    def f16(self) -> bool:
        """16-bit storage (fp16 or bf16)."""
        return bool(N.backend().sox_graph_is_f16(self.h))

    @property
    def storage(self) -> str:
        """"f32", "f16" or "bf16" (sox_graph_is_f16's storage mode)."""
        return {v: k for k, v in STORAGE.items()}[N.backend().sox_graph_is_f16(self.h)]

    def bind(self, value: int, kind="raw") -> N.Bind:
        b = N.Bind()
        N.check(N.backend().sox_graph_bind(self.h, value, N.CK[kind] if isinstance(kind, str) else kind,
                                           ctypes.byref(b)), "Bind")
        return b

    def node_values(self, node: int):
        """(input value ids, output value ids) of a plan node (sox_graph_node_values)."""
        ins, outs = (N.c_int32 * 16)(), (N.c_int32 * 16)()
        ni, no = N.c_int32(), N.c_int32()
        N.check(N.backend().sox_graph_node_values(self.h, node, ins, 16, ctypes.byref(ni), outs, 16, ctypes.byref(no)),
                "node_values")
        return list(ins[: ni.value]), list(outs[: no.value])

    def node(self, node: int):
        """(ExecOp, params bytes) of a plan node (sox_graph_node_info)."""
        op = N.c_int32()
        pp = N.c_void_p()
        nb = N.c_size_t()
        N.check(N.backend().sox_graph_node_info(self.h, node, ctypes.byref(op), ctypes.byref(pp), ctypes.byref(nb)),
                "node_info")
        return op.value, ctypes.string_at(pp.value, nb.value) if nb.value else b""

    def shape(self, value: int):
        s = (N.c_int32 * 8)()
        r = N.c_int32()
        N.check(N.backend().sox_graph_value_shape(self.h, value, s, 8, ctypes.byref(r)), "shape")
        return tuple(s[: r.value])

    def dispatch(self, node: int, kernel: str, binds, params: bytes, grid, block=(256, 1, 1), lds=0, module=None):
        arr = (N.Bind * max(len(binds), 1))(*binds)
        g3 = (N.c_uint32 * 3)(*grid)
        b3 = (N.c_uint32 * 3)(*block)
        pbuf = ctypes.create_string_buffer(params, max(len(params), 1))
        return N.backend().sox_graph_dispatch(self.h, node, module, kernel.encode(), arr, len(binds), pbuf,
                                              len(params), g3, b3, lds)


class HipGraphModel:
    """VkGraphModel analogue: packed consts + the dispatch list of one plan."""

    def __init__(self, backend: HipBackend, plan: ExecPlan, f16=True):
        self.backend = backend
        self.plan = plan
        self.f16 = f16
        ph = plan.to_native()
        try:
            h = N.c_void_p()
            N.check(N.backend().sox_graph_create(backend.h, ph, storage_mode(f16), ctypes.byref(h)), "HipGraphModel")
            self.h = h
        finally:
            N.backend().sox_plan_destroy(ph)

    def release(self):
        if self.h:
            N.backend().sox_graph_release(self.h)
            self.h = None

    def __del__(self):
        try:
            self.release()
        except Exception:
            pass

    @property
    def dispatches(self):
        out = []
        lib = N.backend()
        for i in range(lib.sox_graph_dispatch_count(self.h)):
            name = ctypes.create_string_buffer(128)
            grid = (N.c_uint32 * 3)()
            node = N.c_int32()
            lib.sox_graph_dispatch_info(self.h, i, name, 128, grid, ctypes.byref(node))
            out.append((name.value.decode(), tuple(grid), node.value))
        return out

    @property
    def kernels(self):
        """The code object function of each dispatch (its tiling), in dispatch order."""
        out = []
        lib = N.backend()
        for i in range(lib.sox_graph_dispatch_count(self.h)):
            name = ctypes.create_string_buffer(128)
            N.check(lib.sox_graph_dispatch_kernel(self.h, i, name, 128), "dispatch_kernel")
            out.append(name.value.decode())
        return out

    @property
    def arena_bytes(self) -> int:
        return int(N.backend().sox_graph_arena_bytes(self.h))

    def value_place(self, value: int):
        """(byte offset, bytes) of an activation in a session's slab after the graph-creation rewrites."""
        off, n = N.c_uint64(), N.c_uint64()
        N.check(N.backend().sox_graph_value_place(self.h, value, ctypes.byref(off), ctypes.byref(n)), "value_place")
        return int(off.value), int(n.value)

    def binds(self, index: int):
        """The (slot, offset, size) bindings dispatch `index` is patched with, in kernarg order."""
        n = N.c_int32()
        N.check(N.backend().sox_graph_dispatch_binds(self.h, index, None, 0, ctypes.byref(n)), "dispatch_binds")
        arr = (N.Bind * max(n.value, 1))()
        N.check(N.backend().sox_graph_dispatch_binds(self.h, index, arr, n.value, ctypes.byref(n)), "dispatch_binds")
        return [(b.slot, int(b.offset), int(b.size)) for b in arr[: n.value]]

    @property
    def const_bytes(self) -> int:
        return int(N.backend().sox_graph_const_bytes(self.h))

    @property
    def sync_bytes(self) -> int:
        """Bytes of cross-workgroup counters each session holds (the depthwise launches that run their SE
        gate)."""
        return int(N.backend().sox_graph_sync_bytes(self.h))


class HipInferenceSession:
    """VkInferenceSession analogue: one arena slab, mapped fp32 staging; not thread-safe."""

    def __init__(self, graph: HipGraphModel, pool: Optional[HipBufferPool] = None):
        self.graph = graph
        self.pool = pool
        h = N.c_void_p()
        if pool is None:
            N.check(N.backend().sox_session_create(graph.h, ctypes.byref(h)), "HipInferenceSession")
        else:
            N.check(N.backend().sox_session_create_pooled(graph.h, pool.h, ctypes.byref(h)), "HipInferenceSession")
        self.h = h
        self._inputs = []
        lib = N.backend()
        for i in range(len(graph.plan.inputs)):
            p = ctypes.POINTER(N.c_float)()
            n = N.c_int64()
            N.check(lib.sox_session_input(self.h, i, ctypes.byref(p), ctypes.byref(n)), "input")
            self._inputs.append(np.ctypeslib.as_array(p, shape=(n.value,)))
        p = ctypes.POINTER(N.c_float)()
        n = N.c_int64()
        N.check(lib.sox_session_output(self.h, ctypes.byref(p), ctypes.byref(n)), "output")
        self._output = np.ctypeslib.as_array(p, shape=(n.value,))

    def close(self):
        if self.h:
            N.backend().sox_session_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    @property
    def is_stale(self) -> bool:
        """IsStale (VkSession.cs:178-180): a later session on the same buffer pool grew its buffers."""
        return bool(N.backend().sox_session_is_stale(self.h))

    def _current(self):
        # the staging windows of a stale pooled session were freed by the growth: refuse, as Run does
        if self.pool is not None and self.is_stale:
            p = ctypes.POINTER(N.c_float)()
            N.check(N.backend().sox_session_input(self.h, 0, ctypes.byref(p), None), "stale session")

    @property
    def input(self) -> np.ndarray:
        """Mapped fp32 staging of input 0, in the plan's physical layout (flat)."""
        self._current()
        return self._inputs[0]

    def get_input(self, i: int) -> np.ndarray:
        self._current()
        return self._inputs[i]

    @property
    def output(self) -> np.ndarray:
        self._current()
        return self._output

    def set_input(self, x: np.ndarray, i: int = 0):
        self._current()
        self._inputs[i][:] = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)

    def run(self) -> np.ndarray:
        N.check(N.backend().sox_session_run(self.h), "Run")
        shape = self.graph.plan.values[self.graph.plan.output].phys
        return self._output.reshape(shape)

    def submit(self):
        N.check(N.backend().sox_session_submit(self.h), "Submit")

    def wait(self):
        N.check(N.backend().sox_session_wait(self.h), "Wait")

    def set_replay(self, on: bool):
        N.check(N.backend().sox_session_set_replay(self.h, int(on)), "replay")

    @property
    def replaying(self) -> bool:
        """Whether runs replay a captured HIP graph (off while a rocprofiler-sdk tool is loaded)."""
        return bool(N.backend().sox_session_is_replaying(self.h))

    def time(self, iters: int, staging: bool = False) -> float:
        """Device ms for `iters` back-to-back enqueues, measured with HIP events on the session stream."""
        ms = N.c_float()
        flags = N.RUN_DISPATCHES | (N.RUN_STAGING if staging else 0)
        N.check(N.backend().sox_session_time(self.h, iters, flags, ctypes.byref(ms)), "time")
        return ms.value

    def profile(self, reps: int = 5):
        """DebugProfile: [(dispatch name, node, min ms)]."""
        d = self.graph.dispatches
        ms = (N.c_float * max(len(d), 1))()
        N.check(N.backend().sox_session_profile(self.h, reps, ms, len(d)), "profile")
        return [(name, node, ms[i]) for i, (name, grid, node) in enumerate(d)]

    def read_value(self, vid: int) -> np.ndarray:
        v = self.graph.plan.values[vid]
        out = np.empty(v.count, np.float32)
        N.check(N.backend().sox_session_read_value(self.h, vid, out.ctypes.data_as(ctypes.POINTER(N.c_float)),
                                                   v.count), "read_value")
        return out.reshape(v.phys)


class HipCtcProjection:
    """CtcProjection (Decoding/CtcProjection.cs:12-75) on the device: the CTC head's class projection
    fused with the per-row argmax and the winner's softmax probability, over a session's features
    (sox_ctc_* of include/sox_backend.h). One object serves any number of sessions."""

    def __init__(self, backend: HipBackend, weights: np.ndarray, bias: Optional[np.ndarray], inner: int, columns: int):
        w = np.ascontiguousarray(weights, dtype=np.float32)
        if w.size != inner * columns:
            raise ValueError("weights must hold inner x columns floats")
        b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
        if b is not None and b.size != columns:
            raise ValueError("bias must hold columns floats")
        h = N.c_void_p()
        N.check(N.backend().sox_ctc_create(backend.h, w.ctypes.data, None if b is None else b.ctypes.data, inner,
                                           columns, ctypes.byref(h)), "CtcProjection")
        self.h, self.inner, self.columns = h, inner, columns

    @property
    def is_fused(self) -> bool:
        return bool(N.backend().sox_ctc_is_fused(self.h))

    def argmax(self, session: "HipInferenceSession", feature_value: int, batch: int, rows: int):
        """(indices int32 [batch*rows], probabilities float32 [batch*rows]) of the session's features,
        or None when the head is not fused (the reference's false). A non-finite logit raises."""
        idx = np.empty(batch * rows, np.int32)
        prob = np.empty(batch * rows, np.float32)
        rc = N.backend().sox_ctc_argmax(self.h, session.h, feature_value, batch, rows, idx.ctypes.data, prob.ctypes.data)
        if rc == N.SOX_E_UNSUPPORTED:
            return None
        N.check(rc, "CtcProjection.ArgMax")
        return idx, prob

    def close(self):
        if self.h:
            N.backend().sox_ctc_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class HipImageSession:
    """VkImageSession (Backends/Vulkan/VkImageSession.cs:7-297) on HIP: 8-bit pixels in, the same
    format out, the pixel conversions on the device in the model's stream (sox_image_session_*).
    `lut` is PixelNormalization.Table ([3][256]); the caller builds the graph of the tensor size
    `tensor_size(width, height)` gives, as VkBackend.AcquireGraph does."""

    def __init__(self, backend: HipBackend, lut: np.ndarray, rgb_order: bool = False, output_scale: float = 255.0,
                 pad_multiple: int = 1, pad_top_left: bool = False):
        t = np.ascontiguousarray(lut, dtype=np.float32).reshape(-1)
        if t.size != 768:
            raise ValueError("lut must hold 3 x 256 floats")
        h = N.c_void_p()
        N.check(N.backend().sox_image_session_create(backend.h, t.ctypes.data, int(rgb_order), output_scale,
                                                     pad_multiple, int(pad_top_left), ctypes.byref(h)), "ImageSession")
        self.h = h

    def tensor_size(self, width: int, height: int):
        th, tw = N.c_int32(), N.c_int32()
        N.check(N.backend().sox_image_session_tensor_size(self.h, width, height, ctypes.byref(th), ctypes.byref(tw)),
                "ImageSession.Pads")
        return th.value, tw.value

    def run(self, graph: "HipGraphModel", src: np.ndarray, width: int, height: int, fmt: str = "Bgr24",
            dst: Optional[np.ndarray] = None) -> np.ndarray:
        """src: uint8 [height, stride] rows; returns (or fills) dst of the same shape and stride."""
        src = np.ascontiguousarray(src, dtype=np.uint8)
        out = np.empty_like(src) if dst is None else dst
        N.check(N.backend().sox_image_session_run(self.h, graph.h, src.ctypes.data, width, height, src.shape[1],
                                                  out.ctypes.data, out.shape[1], N.PIX[fmt]), "ImageSession.Run")
        return out

    def close(self):
        if self.h:
            N.backend().sox_image_session_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class HipUnitRunner:
    """VkUnitRunner (Backends/Vulkan/VkUnitRunner.cs:5-337) on HIP: several graph units per call in
    waves, over one grow-only arena and pinned staging, the units of a wave spread over `streams` HIP
    streams so small units run side by side (sox_unit_runner_*). Not thread-safe."""

    def __init__(self, backend: HipBackend, streams: int = 4):
        h = N.c_void_p()
        N.check(N.backend().sox_unit_runner_create(backend.h, streams, ctypes.byref(h)), "UnitRunner")
        self.h = h
        self._graphs = []

    def clear(self):
        N.check(N.backend().sox_unit_runner_clear(self.h), "UnitRunner.Clear")
        self._graphs = []

    def add(self, graph: "HipGraphModel") -> int:
        u = N.c_int32()
        N.check(N.backend().sox_unit_runner_add(self.h, graph.h, ctypes.byref(u)), "UnitRunner.Add")
        self._graphs.append(graph)
        return u.value

    def cut(self):
        N.check(N.backend().sox_unit_runner_cut(self.h), "UnitRunner.Cut")

    @property
    def waves(self) -> int:
        return N.backend().sox_unit_runner_waves(self.h)

    def _window(self, fn, unit: int) -> np.ndarray:
        p = ctypes.POINTER(N.c_float)()
        n = N.c_int64()
        N.check(fn(self.h, unit, ctypes.byref(p), ctypes.byref(n)), "UnitRunner window")
        return np.ctypeslib.as_array(p, shape=(n.value,))

    def input(self, unit: int) -> np.ndarray:
        return self._window(N.backend().sox_unit_runner_input, unit)

    def output(self, unit: int) -> np.ndarray:
        g = self._graphs[unit]
        return self._window(N.backend().sox_unit_runner_output, unit).reshape(g.plan.values[g.plan.output].phys)

    def submit(self):
        N.check(N.backend().sox_unit_runner_submit(self.h), "UnitRunner.Submit")

    def wait(self, wave: Optional[int] = None):
        N.check(N.backend().sox_unit_runner_wait(self.h, self.waves - 1 if wave is None else wave), "UnitRunner.Wait")

    def close(self):
        if self.h:
            N.backend().sox_unit_runner_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

