"""ctypes bindings of the two C-ABI libraries (include/sox_hip.h, include/sox_backend.h).

The libraries are built in-tree by ``simdonnx_amd.build`` into ``simdonnx_amd/lib``. Nothing here
falls back to anything else: if a library is missing, loading raises.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(HERE, "lib")
THIN_PATH = os.path.join(LIB_DIR, "libsoxhip.so")
# SIMDONNX_HIP_BACKEND_LIB names another build of the same library: the host-sanitizer build
# (simdonnx_amd.build.build_sanitized_backend) that the device-free lowering checks load
BACKEND_PATH = os.environ.get("SIMDONNX_HIP_BACKEND_LIB") or os.path.join(LIB_DIR, "libsoxbackend.so")

c_int32, c_int64, c_uint32, c_uint64, c_float, c_void_p, c_size_t = (
    ctypes.c_int32, ctypes.c_int64, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_float, ctypes.c_void_p,
    ctypes.c_size_t)

SOX_OK, SOX_E_INVALID, SOX_E_NOT_FOUND, SOX_E_LOST, SOX_E_UNSUPPORTED = 0, -1, -2, -3, -4

# ExecOp numbering (Engine/ExecPlan.cs:4-40)
OP = dict(Conv=0, MaxPool=1, Elementwise=2, Relu=3, Sigmoid=4, Erf=5, Gelu=6, LayerNorm=7, Gemm=8,
          ResizeBilinear=9, Pad=10, Transpose=11, Slice=12, Concat=13, Copy=14, HardSigmoid=15, GlobalAvgPool=16,
          ConvTranspose=17, ResizeNearest=18, MatMul=19, Softmax=20, ReduceMean=21, Sqrt=22, AvgPool=23,
          HardSwish=24, Swish=25, Ext=26, ChannelGate=27, Attention=28, LeakyRelu=29, Tanh=30, Clip=31,
          DepthToSpace=32, SpaceToDepth=33)
ACT = dict(none=0, relu=1, sigmoid=2, gelu=3, hardswish=4, swish=5)
CK = dict(raw=0, f32=1, convwt=2, gemmnk=3, dww=4, convtw=5, f32t=7)
SLOT_ARENA, SLOT_CONSTS, SLOT_DUMMY, SLOT_SYNC = 0, 1, 2, 3
PIX = dict(Bgr24=0, Rgb24=1, Bgra32=2, Rgba32=3)  # PixelFormat (Imaging/ImageTensor.cs:8-20)
RUN_STAGING, RUN_DISPATCHES = 1, 2


class DeviceInfo(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 256), ("arch", ctypes.c_char * 64), ("device", c_int32),
                ("compute_units", c_int32), ("lds_per_cu", c_int32), ("clock_khz", c_int32), ("warp_size", c_int32),
                ("vendor_id", c_int32), ("hbm_bytes", c_uint64), ("xcds", c_int32), ("pad_", c_int32)]


class ConvP(ctypes.Structure):
    _fields_ = [("pads", c_int32 * 4), ("strides", c_int32 * 2), ("dilations", c_int32 * 2), ("kernel", c_int32 * 2),
                ("group", c_int32), ("act", c_int32), ("pad_mode", c_int32), ("pad_value", c_float),
                ("bias_value", c_int32), ("add_value", c_int32), ("has_pool", c_int32), ("pool_kernel", c_int32 * 2),
                ("pool_strides", c_int32 * 2), ("pool_pads", c_int32 * 4), ("pool_relu", c_int32)]


class PoolP(ctypes.Structure):
    _fields_ = [("kernel", c_int32 * 2), ("strides", c_int32 * 2), ("pads", c_int32 * 4), ("fuse_relu", c_int32),
                ("count_include_pad", c_int32)]


class EwP(ctypes.Structure):
    _fields_ = [("op", c_int32), ("act", c_int32)]


class LnP(ctypes.Structure):
    _fields_ = [("eps", c_float)]


class GemmP(ctypes.Structure):
    _fields_ = [("trans_b", c_int32), ("bias_value", c_int32), ("act", c_int32)]


class HardSigmoidP(ctypes.Structure):
    _fields_ = [("alpha", c_float), ("beta", c_float)]


class ConvTP(ctypes.Structure):
    _fields_ = [("kernel", c_int32 * 2), ("bias_value", c_int32), ("act", c_int32)]


class ResizeNearestP(ctypes.Structure):
    _fields_ = [("scales", c_float * 4), ("add_relu", c_int32)]


class ConcatP(ctypes.Structure):
    _fields_ = [("axis", c_int32)]


class ChannelGateP(ctypes.Structure):
    _fields_ = [("b1", c_int32), ("b2", c_int32), ("act1", c_int32), ("hard", c_int32), ("alpha", c_float),
                ("beta", c_float), ("offset", c_float)]


class AttentionP(ctypes.Structure):
    _fields_ = [("scale", c_float), ("dims", (c_int32 * 4) * 3), ("fix_axis", c_int32 * 3), ("fix_index", c_int32 * 3),
                ("out_layout", c_int32 * 4)]


class ResizeP(ctypes.Structure):
    _fields_ = [("scales", c_float * 4), ("fuse_relu", c_int32), ("add_relu", c_int32)]


class PadP(ctypes.Structure):
    _fields_ = [("rank", c_int32), ("pads", c_int32 * 12), ("mode", c_int32), ("value", c_float)]


class TransposeP(ctypes.Structure):
    _fields_ = [("rank", c_int32), ("perm", c_int32 * 6)]


class SliceP(ctypes.Structure):
    _fields_ = [("naxes", c_int32), ("starts", c_int32 * 6), ("ends", c_int32 * 6), ("axes", c_int32 * 6),
                ("steps", c_int32 * 6)]


class LeakyReluP(ctypes.Structure):
    _fields_ = [("alpha", c_float)]


class TanhP(ctypes.Structure):
    _fields_ = [("in_scale", c_float), ("out_scale", c_float)]


class ClipP(ctypes.Structure):
    _fields_ = [("min", c_float), ("max", c_float)]


class DepthToSpaceP(ctypes.Structure):
    _fields_ = [("block", c_int32), ("crd", c_int32)]


class SafeDivP(ctypes.Structure):
    _fields_ = [("eps", c_float), ("lo", c_float), ("hi", c_float)]


class ShiftP(ctypes.Structure):
    _fields_ = [("axis", c_int32), ("ngroups", c_int32), ("group_ends", c_int32 * 5), ("offsets", c_int32 * 5)]


class UpHeadP(ctypes.Structure):
    _fields_ = [("scales", c_float * 4), ("resize_relu", c_int32), ("skip_relu", c_int32), ("act", c_int32),
                ("has_skip_conv", c_int32), ("skip_conv", ConvP), ("skip_w", c_int32), ("skip_b", c_int32)]


class Bind(ctypes.Structure):
    _fields_ = [("slot", c_int32), ("pad_", c_int32), ("offset", c_uint64), ("size", c_uint64)]


EXT_EMIT_FN = ctypes.CFUNCTYPE(c_int32, c_void_p, c_void_p, c_int32)
EXT_CONSTS_FN = ctypes.CFUNCTYPE(c_int32, c_void_p, c_void_p, c_int32, ctypes.POINTER(c_int32),
                                 ctypes.POINTER(c_int32), c_int32)

# Every function each header declares, with its ctypes signature: (restype, argtypes).
THIN_API = {
    "sox_init": (c_int32, [c_int32, ctypes.POINTER(DeviceInfo)]),
    "sox_error_string": (ctypes.c_char_p, [c_int32]),
    "sox_device_lost": (c_int32, []),
    "sox_device_reset_lost": (None, []),
    "sox_device_mark_lost": (None, []),
    "sox_device_sync": (c_int32, []),
    "sox_malloc": (c_int32, [ctypes.POINTER(c_void_p), c_size_t]),
    "sox_alloc_count": (c_uint64, []),
    "sox_free": (c_int32, [c_void_p]),
    "sox_host_alloc": (c_int32, [ctypes.POINTER(c_void_p), c_size_t]),
    "sox_host_free": (c_int32, [c_void_p]),
    "sox_memcpy_h2d": (c_int32, [c_void_p, c_void_p, c_size_t, c_void_p]),
    "sox_memcpy_d2h": (c_int32, [c_void_p, c_void_p, c_size_t, c_void_p]),
    "sox_memcpy_d2d": (c_int32, [c_void_p, c_void_p, c_size_t, c_void_p]),
    "sox_module_load": (c_int32, [ctypes.POINTER(c_void_p), c_void_p, c_size_t]),
    "sox_module_unload": (c_int32, [c_void_p]),
    "sox_module_function": (c_int32, [ctypes.POINTER(c_void_p), c_void_p, ctypes.c_char_p]),
    "sox_launch": (c_int32, [c_void_p, ctypes.POINTER(c_uint32), ctypes.POINTER(c_uint32), c_uint32, c_void_p,
                             c_void_p, c_size_t]),
    "sox_stream_create": (c_int32, [ctypes.POINTER(c_void_p)]),
    "sox_stream_destroy": (c_int32, [c_void_p]),
    "sox_stream_sync": (c_int32, [c_void_p]),
    "sox_stream_wait_event": (c_int32, [c_void_p, c_void_p]),
    "sox_stream_is_capturing": (c_int32, [c_void_p, ctypes.POINTER(c_int32)]),
    "sox_event_create": (c_int32, [ctypes.POINTER(c_void_p)]),
    "sox_event_destroy": (c_int32, [c_void_p]),
    "sox_event_record": (c_int32, [c_void_p, c_void_p]),
    "sox_event_sync": (c_int32, [c_void_p]),
    "sox_event_elapsed_ms": (c_int32, [ctypes.POINTER(c_float), c_void_p, c_void_p]),
    "sox_graph_begin": (c_int32, [c_void_p]),
    "sox_graph_end": (c_int32, [c_void_p, ctypes.POINTER(c_void_p)]),
    "sox_graph_launch": (c_int32, [c_void_p, c_void_p]),
    "sox_graph_destroy": (c_int32, [c_void_p]),
    "sox_scratch": (c_int32, [c_int32, ctypes.POINTER(c_void_p), ctypes.POINTER(c_size_t)]),
}

BACKEND_API = {
    "sox_plan_create": (c_int32, [ctypes.POINTER(c_void_p)]),
    "sox_plan_destroy": (None, [c_void_p]),
    "sox_plan_add_value": (c_int32, [c_void_p, ctypes.POINTER(c_int32), c_int32, ctypes.POINTER(c_int32), c_int32,
                                     c_void_p, c_int64, ctypes.c_char_p, ctypes.POINTER(c_int32)]),
    "sox_plan_add_node": (c_int32, [c_void_p, c_int32, ctypes.POINTER(c_int32), c_int32, ctypes.POINTER(c_int32),
                                    c_int32, c_void_p, c_size_t, ctypes.c_char_p, ctypes.POINTER(c_int32)]),
    "sox_plan_set_arena": (c_int32, [c_void_p, ctypes.POINTER(c_int64), c_int32, c_int64]),
    "sox_plan_set_io": (c_int32, [c_void_p, ctypes.POINTER(c_int32), c_int32, c_int32]),
    "sox_backend_default": (c_int32, [ctypes.POINTER(c_void_p)]),
    "sox_backend_create_offline": (c_int32, [c_void_p, ctypes.POINTER(c_void_p)]),
    "sox_backend_destroy": (None, [c_void_p]),
    "sox_backend_info": (c_int32, [c_void_p, ctypes.POINTER(DeviceInfo)]),
    "sox_backend_is_lost": (c_int32, [c_void_p]),
    "sox_backend_load_module": (c_int32, [c_void_p, c_void_p, c_size_t, ctypes.POINTER(c_void_p)]),
    "sox_backend_register_ext": (c_int32, [c_void_p, ctypes.c_char_p, EXT_EMIT_FN, EXT_CONSTS_FN, c_void_p]),
    "sox_graph_bind": (c_int32, [c_void_p, c_int32, c_int32, ctypes.POINTER(Bind)]),
    "sox_graph_scratch": (c_int32, [c_void_p, c_uint64, ctypes.POINTER(Bind)]),
    "sox_graph_dispatch": (c_int32, [c_void_p, c_int32, c_void_p, ctypes.c_char_p, ctypes.POINTER(Bind), c_int32,
                                     c_void_p, c_size_t, ctypes.POINTER(c_uint32), ctypes.POINTER(c_uint32),
                                     c_uint32]),
    "sox_graph_node_info": (c_int32, [c_void_p, c_int32, ctypes.POINTER(c_int32), ctypes.POINTER(c_void_p),
                                      ctypes.POINTER(c_size_t)]),
    "sox_graph_node_values": (c_int32, [c_void_p, c_int32, ctypes.POINTER(c_int32), c_int32, ctypes.POINTER(c_int32),
                                        ctypes.POINTER(c_int32), c_int32, ctypes.POINTER(c_int32)]),
    "sox_graph_value_shape": (c_int32, [c_void_p, c_int32, ctypes.POINTER(c_int32), c_int32,
                                        ctypes.POINTER(c_int32)]),
    "sox_graph_is_f16": (c_int32, [c_void_p]),
    "sox_graph_create": (c_int32, [c_void_p, c_void_p, c_int32, ctypes.POINTER(c_void_p)]),
    "sox_graph_release": (None, [c_void_p]),
    "sox_graph_dispatch_count": (c_int32, [c_void_p]),
    "sox_graph_dispatch_kernel": (c_int32, [c_void_p, c_int32, ctypes.c_char_p, c_size_t]),
    "sox_graph_dispatch_info": (c_int32, [c_void_p, c_int32, ctypes.c_char_p, c_size_t, ctypes.POINTER(c_uint32),
                                          ctypes.POINTER(c_int32)]),
    "sox_graph_dispatch_binds": (c_int32, [c_void_p, c_int32, c_void_p, c_int32, ctypes.POINTER(c_int32)]),
    "sox_graph_value_place": (c_int32, [c_void_p, c_int32, ctypes.POINTER(c_uint64), ctypes.POINTER(c_uint64)]),
    "sox_graph_arena_bytes": (c_uint64, [c_void_p]),
    "sox_graph_const_bytes": (c_uint64, [c_void_p]),
    "sox_graph_sync_bytes": (c_uint64, [c_void_p]),
    "sox_last_error": (ctypes.c_char_p, []),
    "sox_session_create": (c_int32, [c_void_p, ctypes.POINTER(c_void_p)]),
    "sox_session_destroy": (None, [c_void_p]),
    "sox_buffer_pool_create": (c_int32, [c_void_p, ctypes.POINTER(c_void_p)]),
    "sox_buffer_pool_destroy": (None, [c_void_p]),
    "sox_buffer_pool_info": (c_int32, [c_void_p, ctypes.POINTER(c_uint64), ctypes.POINTER(c_int32)]),
    "sox_session_create_pooled": (c_int32, [c_void_p, c_void_p, ctypes.POINTER(c_void_p)]),
    "sox_session_is_stale": (c_int32, [c_void_p]),
    "sox_session_input": (c_int32, [c_void_p, c_int32, ctypes.POINTER(ctypes.POINTER(c_float)),
                                    ctypes.POINTER(c_int64)]),
    "sox_session_output": (c_int32, [c_void_p, ctypes.POINTER(ctypes.POINTER(c_float)), ctypes.POINTER(c_int64)]),
    "sox_session_run": (c_int32, [c_void_p]),
    "sox_session_submit": (c_int32, [c_void_p]),
    "sox_session_wait": (c_int32, [c_void_p]),
    "sox_session_set_replay": (c_int32, [c_void_p, c_int32]),
    "sox_session_is_replaying": (c_int32, [c_void_p]),
    "sox_session_time": (c_int32, [c_void_p, c_int32, c_int32, ctypes.POINTER(c_float)]),
    "sox_session_profile": (c_int32, [c_void_p, c_int32, ctypes.POINTER(c_float), c_int32]),
    "sox_session_read_value": (c_int32, [c_void_p, c_int32, ctypes.POINTER(c_float), c_int64]),
    "sox_session_value_ptr": (c_int32, [c_void_p, c_int32, ctypes.POINTER(c_void_p)]),
    "sox_session_stream": (c_void_p, [c_void_p]),
    "sox_image_session_create": (c_int32, [c_void_p, c_void_p, c_int32, c_float, c_int32, c_int32,
                                           ctypes.POINTER(c_void_p)]),
    "sox_image_session_destroy": (None, [c_void_p]),
    "sox_image_session_tensor_size": (c_int32, [c_void_p, c_int32, c_int32, ctypes.POINTER(c_int32),
                                                ctypes.POINTER(c_int32)]),
    "sox_image_session_run": (c_int32, [c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_int32, c_void_p, c_int32,
                                        c_int32]),
    "sox_unit_runner_create": (c_int32, [c_void_p, c_int32, ctypes.POINTER(c_void_p)]),
    "sox_unit_runner_destroy": (None, [c_void_p]),
    "sox_unit_runner_clear": (c_int32, [c_void_p]),
    "sox_unit_runner_add": (c_int32, [c_void_p, c_void_p, ctypes.POINTER(c_int32)]),
    "sox_unit_runner_cut": (c_int32, [c_void_p]),
    "sox_unit_runner_waves": (c_int32, [c_void_p]),
    "sox_unit_runner_wave_end": (c_int32, [c_void_p, c_int32]),
    "sox_unit_runner_input": (c_int32, [c_void_p, c_int32, ctypes.POINTER(ctypes.POINTER(c_float)),
                                        ctypes.POINTER(c_int64)]),
    "sox_unit_runner_output": (c_int32, [c_void_p, c_int32, ctypes.POINTER(ctypes.POINTER(c_float)),
                                         ctypes.POINTER(c_int64)]),
    "sox_unit_runner_submit": (c_int32, [c_void_p]),
    "sox_unit_runner_wait": (c_int32, [c_void_p, c_int32]),
    "sox_ctc_create": (c_int32, [c_void_p, c_void_p, c_void_p, c_int32, c_int32, ctypes.POINTER(c_void_p)]),
    "sox_ctc_destroy": (None, [c_void_p]),
    "sox_ctc_is_fused": (c_int32, [c_void_p]),
    "sox_ctc_argmax": (c_int32, [c_void_p, c_void_p, c_int32, c_int32, c_int32, c_void_p, c_void_p]),
    "sox_ctc_argmax_noalloc": (c_int32, [c_void_p, c_void_p, c_int32, c_int32, c_int32, c_void_p, c_void_p,
                                         c_void_p]),
}

_thin = None
_backend = None


def _bind(lib, api):
    for name, (res, args) in api.items():
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args
    return lib


def thin():
    """libsoxhip.so (include/sox_hip.h)."""
    global _thin
    if _thin is None:
        if not os.path.exists(THIN_PATH):
            raise RuntimeError(f"{THIN_PATH} is not built: run `python -m simdonnx_amd.build`")
        _thin = _bind(ctypes.CDLL(THIN_PATH), THIN_API)
    return _thin


def backend():
    """libsoxbackend.so (include/sox_backend.h)."""
    global _backend
    if _backend is None:
        thin()
        if not os.path.exists(BACKEND_PATH):
            raise RuntimeError(f"{BACKEND_PATH} is not built: run `python -m simdonnx_amd.build`")
        _backend = _bind(ctypes.CDLL(BACKEND_PATH), BACKEND_API)
    return _backend


class SoxError(RuntimeError):
    def __init__(self, status: int, what: str):
        detail = backend().sox_last_error().decode() if _backend is not None else ""
        msg = thin().sox_error_string(status).decode() if _thin is not None else str(status)
        super().__init__(f"{what}: {msg} ({status}) {detail}".strip())
        self.status = status


class DeviceLostError(SoxError):
    """VkDeviceLostException analogue (Backends/Vulkan/Vk.cs:44-49)."""


class NotSupportedError(SoxError):
    """NotSupportedException analogue: an op / epilogue this backend does not implement."""


def check(status: int, what: str) -> None:
    if status == SOX_OK:
        return
    if status == SOX_E_LOST:
        raise DeviceLostError(status, what)
    if status == SOX_E_UNSUPPORTED:
        raise NotSupportedError(status, what)
    raise SoxError(status, what)
