"""Mutation guard of the CPU oracle: a copy of oracle/src/oracle.cpp with one planted mistake of the
kinds a restatement gets wrong (a shifted tap index, a transposed operand, a sign, a dropped term,
swapped operands) is compiled with the oracle's own flags, and the pinning checks of
tests/test_oracle.py (golden closed forms, tier and Winograd invariants, numpy-exact ops) run against
it in a child process: each mutant must fail them. The unmutated copy, built the same way, must pass
(so a failure comes from the mistake, not from the harness).
"""
import os
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "oracle", "src", "oracle.cpp")
FLAGS = ["-O3", "-fPIC", "-fopenmp", "-ffp-contract=off", "-fno-fast-math", "-std=c++17", "-shared"]

# name: (text in oracle.cpp, its replacement, the checks of tests/test_oracle.py that must catch it)
MUTANTS = {
    "conv tap index shifted": ("int s = o * stride + kk - pad;", "int s = o * stride + kk - pad + 1;",
                               "conv_matches_golden"),
    "dense tile drops the bias (scalar tier)": ("float acc = bias[h * Ob + l];", "float acc = 0.0f;",
                                                "conv_tiers_bitwise or gemm_matches"),
    "Winograd input transform sign": ("o[3 * vstride] = r4 - r2 + 2.0f * (r3 - r1);",
                                      "o[3 * vstride] = r4 - r2 + 2.0f * (r1 - r3);", "winograd_vs_direct"),
    "depthwise weight taps transposed": ("acc = fmaf(xv, pw[(size_t)(ky * kw + kx) * c + ch], acc);",
                                         "acc = fmaf(xv, pw[(size_t)(kx * kw + ky) * c + ch], acc);",
                                         "depthwise_matches_golden"),
    "Gemm operand transposed": ("trans_b ? b[(size_t)o * k + c] : b[(size_t)c * n + o]",
                                "trans_b ? b[(size_t)c * n + o] : b[(size_t)o * k + c]", "gemm_matches"),
    "GELU sign": ("(0.5f * x) * (1.0f + erf_core(x * 0.70710678118654752f))",
                  "(0.5f * x) * (1.0f - erf_core(x * 0.70710678118654752f))", "math_cores or activation_kinds"),
    "Sub operands swapped": ("op == 1 ? a[i] - b[i]", "op == 1 ? b[i] - a[i]", "elementwise_broadcast"),
}


def _build(tmp, name, text):
    d = os.path.join(tmp, name.replace(" ", "_").replace("(", "").replace(")", ""))
    os.makedirs(os.path.join(d, "src"))
    with open(os.path.join(d, "src", "oracle.cpp"), "w") as f:
        f.write(text)
    with open(os.path.join(ROOT, "oracle", "oracle.h")) as f, open(os.path.join(d, "oracle.h"), "w") as g:
        g.write(f.read())
    lib = os.path.join(d, "liboracle.so")
    r = subprocess.run(["g++", *FLAGS, "-o", lib, os.path.join(d, "src", "oracle.cpp")], capture_output=True,
                       text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    return lib


def _checks(lib, select):
    env = dict(os.environ, SIMDONNX_ORACLE_LIB=lib, OMP_NUM_THREADS="2")
    r = subprocess.run([sys.executable, "-m", "pytest", "-x", "-q", "-p", "no:cacheprovider",
                        os.path.join(ROOT, "tests", "test_oracle.py"), "-k", select], cwd=ROOT, env=env,
                       capture_output=True, text=True, timeout=600)
    return r.returncode, (r.stdout + r.stderr)[-1500:]


def test_planted_mistakes_fail_the_pinning_checks():
    with open(SRC) as f:
        src = f.read()
    for name, (old, new, _) in MUTANTS.items():
        assert src.count(old) == 1, f"mutation site of '{name}' not found once in oracle.cpp"
    with tempfile.TemporaryDirectory() as tmp:
        with ThreadPoolExecutor(max_workers=4) as ex:
            libs = dict(zip(["control", *MUTANTS],
                            ex.map(lambda kv: _build(tmp, kv[0], kv[1]),
                                   [("control", src)] + [(n, src.replace(o, r)) for n, (o, r, _) in MUTANTS.items()])))
            selects = {n: s for n, (_, _, s) in MUTANTS.items()}
            every = " or ".join(f"({s})" for s in selects.values())
            jobs = {"control": ex.submit(_checks, libs["control"], every)}
            jobs.update({n: ex.submit(_checks, libs[n], s) for n, s in selects.items()})
            results = {n: j.result() for n, j in jobs.items()}
    rc, out = results.pop("control")
    assert rc == 0, f"the unmutated copy fails its checks:\n{out}"
    survived = [n for n, (rc, _) in results.items() if rc == 0]
    assert not survived, f"planted mistakes the checks did not catch: {survived}"
    for n, (rc, out) in results.items():
        assert rc == 1, f"{n}: the checks did not run to a failure (exit {rc}):\n{out}"
