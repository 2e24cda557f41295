"""The CPU-side code under AddressSanitizer and UndefinedBehaviorSanitizer.

Two builds, each loaded by a child pytest process with its sanitizer
runtime preloaded (errors abort the child, so a report fails the test):
  * the oracle (oracle.c, gcc) from `make -C oracle sanitize`, running the
    oracle's pinning suites;
  * the C ABI's host code (api.hip host pass: validation, shape planners,
    batch offsets, status and error strings) from build.py's sanitized
    build, running the ABI and planner suites and a null-argument call of
    every entry point.
No GPU is used: the host-side checks all run before any device work."""
import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT / "onnx_runtime_dart_amd" / "csrc"))


def _gcc_runtime(name):
    r = subprocess.run(["gcc", f"-print-file-name={name}"], capture_output=True, text=True)
    p = Path(r.stdout.strip())
    if r.returncode != 0 or not p.is_absolute() or not p.exists():
        pytest.skip(f"gcc's {name} is not installed")
    return p


def _child(env_extra, tests):
    env = dict(os.environ)
    env.update(env_extra)
    env["ASAN_OPTIONS"] = "detect_leaks=0:abort_on_error=1"
    env["UBSAN_OPTIONS"] = "print_stacktrace=1:halt_on_error=1"
    code = ("import ctypes, sys, pytest\n"
            "ctypes.CDLL(None).__asan_init  # the sanitizer runtime is loaded\n"
            "sys.exit(pytest.main(['-q', '-p', 'no:cacheprovider', '-m', 'not gpu', "
            + ", ".join(repr(str(ROOT / "tests" / t)) for t in tests) + "]))\n")
    r = subprocess.run([sys.executable, "-c", code], cwd=ROOT, env=env, capture_output=True,
                       text=True, timeout=600)
    tail = (r.stdout + r.stderr)[-4000:]
    assert r.returncode == 0, tail
    assert "ERROR: AddressSanitizer" not in tail and "runtime error" not in tail, tail
    return tail


def test_oracle_under_asan_and_ubsan():
    subprocess.run(["make", "-s", "-C", str(ROOT / "oracle"), "sanitize"], check=True)
    lib = ROOT / "oracle" / "lib" / "liboracle_san.so"
    out = _child({"LD_PRELOAD": str(_gcc_runtime("libasan.so")), "ORACLE_LIBRARY": str(lib)},
                 ["test_oracle.py", "test_oracle_elem.py"])
    assert " passed" in out


def test_host_abi_under_asan_and_ubsan():
    import build as B  # onnx_runtime_dart_amd/csrc/build.py
    lib = B.SAN_LIB
    if not lib.exists() or lib.stat().st_mtime < (B.CSRC / "api.hip").stat().st_mtime:
        B.build_sanitized()
    out = _child({"LD_PRELOAD": str(B.asan_runtime()), "MIGEMM_LIBRARY": str(lib)},
                 ["test_abi.py", "test_f32_plan.py"])
    assert " passed" in out
