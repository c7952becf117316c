"""simdonnx_amd: an MI355X-native (gfx950 / CDNA4) HIP backend for SimdOnnx's conv/GEMM hot path.

Layers (top to bottom):
  plan.py      ExecPlan / PlanBuilder: the fused NHWC plan the backend consumes (Engine/ExecPlan.cs)
  backend.py   HipBackend / HipGraphModel / HipInferenceSession (the Vulkan backend surface)
  native.py    ctypes bindings of lib/libsoxbackend.so (include/sox_backend.h) and
               lib/libsoxhip.so (include/sox_hip.h, the thin C ABI over libamdhip64)
  csrc/        hand-written gfx950 kernels (csrc/kernels/*.hip -> embedded code objects) and the
               C++ host side (csrc/host)
  graphs.py    the benchmark workloads as plans; synth.py their seeded inputs
"""
from .plan import ExecPlan, PlanBuilder, NHWC  # noqa: F401

__all__ = ["ExecPlan", "PlanBuilder", "NHWC"]
