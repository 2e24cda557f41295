"""Builds libmigemm.so (HIP kernels + C ABI) for gfx950 with hipcc.

    python onnx_runtime_dart_amd/csrc/build.py [--jobs N] [--sanitize]

Objects go to onnx_runtime_dart_amd/csrc/_build/, the library to
onnx_runtime_dart_amd/lib/libmigemm.so.  Every source is recompiled on each
call (the build is a few seconds per file).

--sanitize (build_sanitized) also writes lib/libmigemm_san.so: the same
kernels with the C ABI's host code (api.hip: validation, planners, staging)
compiled with AddressSanitizer and UndefinedBehaviorSanitizer (host pass
only; errors abort).  It is loaded through MIGEMM_LIBRARY with clang's ASan
runtime preloaded, for CPU tests of the host side (tests/test_sanitizers.py).
"""
from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

CSRC = Path(__file__).resolve().parent
PKG = CSRC.parent
ROOT = PKG.parent
BUILD = CSRC / "_build"
LIB = PKG / "lib" / "libmigemm.so"

SOURCES = ["api.hip", "nbits.hip", "nbits_f8.hip", "int8.hip", "f32.hip", "dql.hip", "attn.hip", "conv.hip",
           "elem.hip"]

# Packed fp32 VALU forms are disabled (-packed-fp32-ops); the compiler still
# schedules plain fp32 and the MFMA units.
HIPFLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Werror=shadow",  # a local shadowing a kernel argument has written the wrong buffer
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{ROOT / 'include'}",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libmigemm)")


def _compile(src: str) -> Path:
    obj = BUILD / (Path(src).stem + ".o")
    cmd = [hipcc(), *HIPFLAGS, "-Rpass-analysis=kernel-resource-usage", "-c", str(CSRC / src),
           "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr}")
    # Per-kernel resource report (registers, scratch, LDS, occupancy).
    usage = [ln.split("remark: ", 1)[1].replace(" [-Rpass-analysis=kernel-resource-usage]", "")
             for ln in r.stderr.splitlines() if "remark: " in ln and "kernel-resource-usage" in ln]
    (BUILD / (Path(src).stem + ".usage.txt")).write_text("\n".join(usage) + "\n")
    warn = [ln for ln in r.stderr.splitlines() if "warning" in ln and "packed-fp32-ops" not in ln]
    if warn:
        print("\n".join(warn), file=sys.stderr)
    return obj


def kernels_with_scratch() -> list[str]:
    """Kernels of the last build that use scratch (per-lane stack) memory."""
    out = []
    for f in sorted(BUILD.glob("*.usage.txt")):
        name = None
        for ln in f.read_text().splitlines():
            ln = ln.strip()
            if ln.startswith("Function Name:"):
                name = ln.split(":", 1)[1].strip()
            elif ln.startswith("ScratchSize") and not ln.endswith(": 0"):
                out.append(f"{f.stem}: {name} ({ln})")
    return out


def build(jobs: int | None = None) -> Path:
    BUILD.mkdir(parents=True, exist_ok=True)
    LIB.parent.mkdir(parents=True, exist_ok=True)
    jobs = jobs or min(len(SOURCES), os.cpu_count() or 4)
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB.with_suffix(".so.tmp")
    # --no-undefined: a declared but missing definition fails here, not at load.
    cmd = [hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", "-Wl,--no-undefined", "-o",
           str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    for k in kernels_with_scratch():
        print(f"warning: kernel uses scratch memory: {k}", file=sys.stderr)
    return LIB


SAN_LIB = PKG / "lib" / "libmigemm_san.so"
# Sanitizers on the host pass only: each flag behind -Xarch_host.
SAN_HOST = ["-Xarch_host", "-fsanitize=address",
            "-Xarch_host", "-fsanitize=undefined",
            "-Xarch_host", "-fno-sanitize-recover=undefined",
            "-Xarch_host", "-fno-omit-frame-pointer",
            "-Xarch_host", "-g"]


def asan_runtime() -> Path:
    """clang's shared ASan runtime (preloaded before the sanitized library)."""
    hits = sorted(Path(hipcc()).resolve().parent.parent.glob(
        "llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
    if not hits:
        hits = sorted(Path("/opt/rocm/llvm/lib/clang").glob("*/lib/linux/libclang_rt.asan-x86_64.so"))
    if not hits:
        raise RuntimeError("clang ASan runtime not found")
    return hits[-1]


def build_sanitized() -> Path:
    """api.hip with host ASan/UBSan, linked with the other objects of the last
    build(), into SAN_LIB."""
    objs = [BUILD / (Path(src).stem + ".o") for src in SOURCES if src != "api.hip"]
    if not all(o.exists() for o in objs):
        build()
    san_obj = BUILD / "api_san.o"
    flags = [f for f in HIPFLAGS if f != "-O3"] + ["-O1"]
    r = subprocess.run([hipcc(), *flags, *SAN_HOST, "-c", str(CSRC / "api.hip"), "-o",
                        str(san_obj)], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc (sanitized api.hip) failed:\n{r.stderr}")
    tmp = SAN_LIB.with_suffix(".so.tmp")
    link_san = ["-Xarch_host", "-fsanitize=address",
                "-Xarch_host", "-fsanitize=undefined",
                "-Xarch_host", "-shared-libasan"]
    r = subprocess.run([hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", *link_san, "-o",
                        str(tmp), str(san_obj), *map(str, objs)], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link (sanitized) failed:\n{r.stderr}")
    os.replace(tmp, SAN_LIB)
    return SAN_LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--sanitize", action="store_true")
    a = ap.parse_args()
    print(build(a.jobs))
    if a.sanitize:
        print(build_sanitized())
