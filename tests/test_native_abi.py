"""The C-ABI libraries load and export every function their headers declare (no GPU calls)."""
import ctypes
import os
import re
import subprocess

import pytest

from simdonnx_amd import native as N

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared(header):
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"^\s*(?:const\s+)?[A-Za-z_][A-Za-z0-9_ \*]*?\b(sox_[a-z0-9_]+)\s*\(", text, flags=re.M)
    return sorted(set(n for n in names if not n.endswith("_fn")))


def exported(path):
    out = subprocess.run(["nm", "-D", "--defined-only", path], capture_output=True, text=True, check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if " T " in line}


@pytest.mark.parametrize("header,path,api", [("sox_hip.h", N.THIN_PATH, N.THIN_API),
                                             ("sox_backend.h", N.BACKEND_PATH, N.BACKEND_API)])
def test_exports_every_declared_function(header, path, api):
    assert os.path.exists(path), f"{path} not built"
    names = declared(header)
    assert len(names) > 20
    missing = set(names) - exported(path)
    assert not missing, f"{os.path.basename(path)} lacks {sorted(missing)}"
    # and the Python bindings cover the same surface
    assert set(names) == set(api), (set(names) ^ set(api))


def test_libraries_load_without_a_device():
    thin = N.thin()
    N.backend()
    assert thin.sox_error_string(0) == b"ok"
    assert thin.sox_error_string(N.SOX_E_UNSUPPORTED) == b"not supported by the HIP backend"


def test_kernarg_abi_layout():
    """The ctypes mirrors of the param records match the C struct sizes (x86-64 SysV)."""
    assert ctypes.sizeof(N.ConvP) == 4 * 26
    assert ctypes.sizeof(N.GemmP) == 12
    assert ctypes.sizeof(N.AttentionP) == 4 * (1 + 12 + 3 + 3 + 4)
    assert ctypes.sizeof(N.Bind) == 24


def test_code_objects_embedded_for_gfx950():
    """Every kernel source was compiled for gfx950 and embedded in the backend library."""
    build = os.path.join(ROOT, "simdonnx_amd", "_build")
    srcs = [f[:-4] for f in os.listdir(os.path.join(ROOT, "simdonnx_amd", "csrc", "kernels")) if f.endswith(".hip")]
    table = open(os.path.join(build, "resources_table.inc")).read()
    for s in srcs:
        co = os.path.join(build, s + ".hsaco")
        assert os.path.exists(co)
        assert f'"{s}"' in table
        head = open(co, "rb").read(4)
        assert head == b"\x7fELF"
    syms = subprocess.run(["nm", "-D", N.BACKEND_PATH], capture_output=True, text=True).stdout
    for s in srcs:
        assert f"sox_res_{s}_start" in syms
