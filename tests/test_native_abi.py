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
    assert ctypes.sizeof(N.ResizeP) == 4 * 6 and ctypes.sizeof(N.PadP) == 4 * 15
    assert ctypes.sizeof(N.TransposeP) == 4 * 7 and ctypes.sizeof(N.SliceP) == 4 * 25
    assert ctypes.sizeof(N.DepthToSpaceP) == 8 and ctypes.sizeof(N.TanhP) == 8 and ctypes.sizeof(N.ClipP) == 8


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


def _kernel_descriptors(path):
    """(name, 64-byte kernel descriptor) of every `<kernel>.kd` symbol in a gfx950 code object (ELF64)."""
    import struct
    data = open(path, "rb").read()
    shoff = struct.unpack_from("<Q", data, 0x28)[0]
    shentsize, shnum = struct.unpack_from("<HH", data, 0x3A)
    secs = [struct.unpack_from("<IIQQQQIIQQ", data, shoff + i * shentsize) for i in range(shnum)]
    out = {}
    for sec in secs:
        if sec[1] != 2:  # SHT_SYMTAB
            continue
        strtab = secs[sec[6]]
        for i in range(sec[5] // 24):
            st_name, _, _, st_shndx, st_value, _ = struct.unpack_from("<IBBHQQ", data, sec[4] + i * 24)
            end = data.index(b"\0", strtab[4] + st_name)
            name = data[strtab[4] + st_name:end].decode()
            if name.endswith(".kd") and st_shndx < len(secs):
                home = secs[st_shndx]
                off = home[4] + (st_value - home[3])
                out[name[:-3]] = data[off:off + 64]
    return out


def test_kernels_use_no_scratch():
    """No built kernel spills to scratch (private segment 0): the ring kernels index their accumulators
    with constants only, and a spill there costs ~15% (it happened once when a lambda was not inlined)."""
    import glob
    import struct
    build = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "simdonnx_amd", "_build")
    objs = sorted(glob.glob(os.path.join(build, "*.hsaco")))
    if not objs:
        pytest.skip("code objects not built")
    spills = {}
    count = 0
    for path in objs:
        for name, kd in _kernel_descriptors(path).items():
            count += 1
            private = struct.unpack_from("<I", kd, 4)[0]  # private_segment_fixed_size
            if private:
                spills[name] = private
    assert count > 50
    assert not spills, spills
