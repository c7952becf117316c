"""Builds the HIP backend in-tree: gfx950 code objects + the two C-ABI shared libraries.

  1. every ``csrc/kernels/*.hip`` -> ``_build/<name>.hsaco`` (``hipcc --genco --offload-arch=gfx950``);
  2. the code objects are embedded into the backend library with ``.incbin`` (the resource table
     the backend loads with ``sox_module_load`` = hipModuleLoadData, as the reference embeds its
     shaders, Sdcb.SimdOnnx.Sources.props:21-31);
  3. ``lib/libsoxhip.so``      - the thin C ABI over libamdhip64 (include/sox_hip.h);
     ``lib/libsoxbackend.so``  - HipBackend / HipGraphModel / HipInferenceSession (include/sox_backend.h);
  4. ``csrc/ext_example/*.hip`` -> ``_build/ext/<name>.hsaco``: an extension operator's kernels in a
     code object of their own (not embedded), loaded at run time with ``sox_backend_load_module``.

Run ``python -m simdonnx_amd.build`` (or ``__graft_entry__.build()``). Compiles every time it is called.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
KDIR = os.path.join(HERE, "csrc", "kernels")
EXT_DIR = os.path.join(HERE, "csrc", "ext_example")
HDIR = os.path.join(HERE, "csrc", "host")
BUILD = os.path.join(HERE, "_build")
EXT_BUILD = os.path.join(BUILD, "ext")
LIB = os.path.join(HERE, "lib")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
ARCH = "gfx950"

# All HIP code is built without packed fp32 ops (v_pk_*_f32).
HIP_FLAGS = ["-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def _hipcc() -> str:
    p = shutil.which("hipcc") or os.path.join(ROCM, "bin", "hipcc")
    if not os.path.exists(p):
        raise RuntimeError("hipcc not found: the HIP backend cannot be built")
    return p


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"build step failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return r


def build_code_objects(verbose=False):
    os.makedirs(BUILD, exist_ok=True)
    # the large ring instantiations first, so the parallel build ends with the short files
    srcs = sorted((f for f in os.listdir(KDIR) if f.endswith(".hip")),
                  key=lambda f: (-os.path.getsize(os.path.join(KDIR, f)) if f.startswith(("gemm", "conv_ring")) else 0, f))
    hipcc = _hipcc()

    def one(src):
        name = src[:-4]
        out = os.path.join(BUILD, name + ".hsaco")
        _run([hipcc, "--genco", "--no-gpu-bundle-output", f"--offload-arch={ARCH}", *HIP_FLAGS, "-o", out,
              os.path.join(KDIR, src)])
        if verbose:
            print("built", out, os.path.getsize(out), "bytes", flush=True)
        return name, out

    with ThreadPoolExecutor(max_workers=min(max(2, (os.cpu_count() or 4)), 8, len(srcs))) as ex:
        return sorted(ex.map(one, srcs))


def build_ext_examples(verbose=False):
    """Extension code objects: built like the embedded ones, but left as files for their owner to load."""
    os.makedirs(EXT_BUILD, exist_ok=True)
    outs = []
    for src in sorted(f for f in os.listdir(EXT_DIR) if f.endswith(".hip")):
        out = os.path.join(EXT_BUILD, src[:-4] + ".hsaco")
        _run([_hipcc(), "--genco", "--no-gpu-bundle-output", f"--offload-arch={ARCH}", *HIP_FLAGS, "-o", out,
              os.path.join(EXT_DIR, src)])
        if verbose:
            print("built", out, os.path.getsize(out), "bytes", flush=True)
        outs.append(out)
    return outs


def ext_example_path(name: str) -> str:
    """Path of a built extension code object (``build_ext_examples``)."""
    return os.path.join(EXT_BUILD, name + ".hsaco")


def write_resources(objs):
    asm = [".section .rodata"]
    table = ["static const SoxResource sox_resources[] = {"]
    for name, path in objs:
        sym = f"sox_res_{name}"
        asm += [".balign 4096", f".global {sym}_start", f"{sym}_start:", f'.incbin "{path}"',
                f".global {sym}_end", f"{sym}_end:"]
        table.insert(0, f'extern "C" const unsigned char {sym}_start[], {sym}_end[];')
        table.append(f'    {{"{name}", {sym}_start, {sym}_end}},')
    asm.append('.section .note.GNU-stack,"",@progbits')
    table.append("    {nullptr, nullptr, nullptr},")
    table.append("};")
    with open(os.path.join(BUILD, "resources.S"), "w") as f:
        f.write("\n".join(asm) + "\n")
    with open(os.path.join(BUILD, "resources_table.inc"), "w") as f:
        f.write("\n".join(table) + "\n")


def link_backend(cxx=None):
    """Links libsoxbackend.so from the compiled host code (backend.o) and the code objects that
    resources.S embeds (the .hsaco files under _build as they are now)."""
    cxx = cxx or os.path.join(ROCM, "llvm", "bin", "clang++")
    be = os.path.join(LIB, "libsoxbackend.so")
    _run([cxx, "-fPIC", f"-I{BUILD}", "-shared", "-o", be, os.path.join(BUILD, "backend.o"),
          os.path.join(BUILD, "resources.S"), f"-L{LIB}", "-lsoxhip", "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{ROCM}/lib"])
    return be


def build_libs(verbose=False):
    os.makedirs(LIB, exist_ok=True)
    cxx = os.path.join(ROCM, "llvm", "bin", "clang++")
    if not os.path.exists(cxx):
        cxx = _hipcc()
    common = ["-O2", "-fPIC", "-std=c++17", "-D__HIP_PLATFORM_AMD__", f"-I{ROCM}/include", "-Wall",
              "-Wno-unused-result"]
    thin = os.path.join(LIB, "libsoxhip.so")
    # the static device scratch (sox_scratch.hip) is the one host-library source compiled as HIP: its
    # array needs the device code object the HIP runtime registers with the library
    os.makedirs(BUILD, exist_ok=True)
    scratch_o = os.path.join(BUILD, "sox_scratch.o")
    _run([_hipcc(), "-c", "-fPIC", f"--offload-arch={ARCH}", *HIP_FLAGS, "-o", scratch_o,
          os.path.join(HDIR, "sox_scratch.hip")])
    _run([cxx, *common, "-shared", "-o", thin, os.path.join(HDIR, "sox_hip.cpp"), scratch_o, f"-L{ROCM}/lib",
          "-lamdhip64", f"-Wl,-rpath,{ROCM}/lib"])
    be = os.path.join(LIB, "libsoxbackend.so")
    # the host code and the embedded code objects link separately: a kernel change re-links the
    # library without recompiling backend.cpp (link_backend)
    _run([cxx, *common, f"-I{BUILD}", "-c", "-o", os.path.join(BUILD, "backend.o"), os.path.join(HDIR, "backend.cpp")])
    link_backend(cxx)
    if verbose:
        print("built", thin, be, flush=True)
    return thin, be


SAN_DIR = os.path.join(BUILD, "sanitize")
SAN_BACKEND = os.path.join(SAN_DIR, "libsoxbackend.so")
SAN_FLAGS = ["-fsanitize=address,undefined", "-fno-sanitize-recover=undefined", "-shared-libasan"]


def _host_cxx() -> str:
    cxx = os.path.join(ROCM, "llvm", "bin", "clang++")
    return cxx if os.path.exists(cxx) else _hipcc()


def sanitizer_runtime() -> str:
    """The shared AddressSanitizer runtime (with UndefinedBehaviorSanitizer) of the host compiler that
    builds the sanitizer library: a process must preload it to load that library ("" when absent)."""
    r = subprocess.run([_host_cxx(), "-print-file-name=libclang_rt.asan-x86_64.so"], capture_output=True, text=True)
    path = r.stdout.strip()
    return path if r.returncode == 0 and os.path.isabs(path) and os.path.exists(path) else ""


def build_sanitized_backend(verbose=False):
    """The backend library again with its host code built under AddressSanitizer and
    UndefinedBehaviorSanitizer, into _build/sanitize/ (host code only: it embeds the same code objects
    and links the same libsoxhip.so). Loaded through SIMDONNX_HIP_BACKEND_LIB with the sanitizer
    runtime preloaded, it runs the host lowering (graph-creation rewrites, arena moves, const packing,
    kernel choice) of every workload plan on a backend created without a device
    (tests/test_host_lowering.py)."""
    os.makedirs(SAN_DIR, exist_ok=True)
    _run([_host_cxx(), "-O1", "-g", "-fno-omit-frame-pointer", *SAN_FLAGS, "-fPIC", "-std=c++17", "-Wall",
          "-Wno-unused-result", f"-I{BUILD}", "-shared", "-o", SAN_BACKEND, os.path.join(HDIR, "backend.cpp"),
          os.path.join(BUILD, "resources.S"), f"-L{LIB}", "-lsoxhip", "-Wl,-rpath,$ORIGIN/../../lib",
          f"-Wl,-rpath,{ROCM}/lib"])
    if verbose:
        print("built", SAN_BACKEND, flush=True)
    return SAN_BACKEND


def build(verbose=False):
    objs = build_code_objects(verbose)
    write_resources(objs)
    build_ext_examples(verbose)
    libs = build_libs(verbose)
    build_sanitized_backend(verbose)
    return libs


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
