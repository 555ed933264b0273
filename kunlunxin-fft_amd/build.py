"""Build libmfft.so in-tree with hipcc for gfx950.

Each ``csrc/*.hip`` file is compiled to an object in ``_build/`` (in
parallel) and the objects are linked into ``libmfft.so`` next to this file,
which the ctypes layer (``native.py``) loads.  Run ``python build.py`` from
anywhere, or call :func:`build`.
"""
from __future__ import annotations

import concurrent.futures as cf
import hashlib
import json
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libmfft.so")
# what the library was built from, written beside it: a run on a copy of the
# tree without its git metadata can still name the commit and the sources
BUILD_INFO = os.path.join(HERE, "libmfft.build.json")
ARCH = "gfx950"

# Packed-FP32 instructions are disabled on purpose: hipcc must not emit
# v_pk_{add,mul,fma}_f32, some forms of which have given wrong results, now
# and then and with no error, on the gfx950 machines this library is
# measured on (hipcc's host pass warns that it does not know the feature).
HIP_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]


def _hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(exe):
        raise RuntimeError("hipcc not found: cannot build the gfx950 library")
    return exe


def _compile(src: str, hipcc: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    cmd = [hipcc, *HIP_FLAGS, "-c", src, "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{res.stdout}\n{res.stderr}")
    return obj


def sources_sha16(paths) -> str | None:
    """sha256 (first 16 hex digits) over each file's name and bytes, in the
    order given; None when none of them can be read."""
    h = hashlib.sha256()
    seen = False
    for p in paths:
        try:
            with open(p, "rb") as f:
                h.update(os.path.basename(p).encode() + b"\0" + f.read())
            seen = True
        except OSError:
            continue
    return h.hexdigest()[:16] if seen else None


def _git(*args) -> str | None:
    try:
        r = subprocess.run(["git", *args], cwd=HERE, capture_output=True, text=True, timeout=10)
    except (OSError, subprocess.SubprocessError):
        return None
    return r.stdout.strip() if r.returncode == 0 else None


def _write_build_info() -> None:
    status = _git("status", "--porcelain", "--untracked-files=no")
    info = {"commit": _git("rev-parse", "--short=12", "HEAD") or None,
            "dirty": bool(status) if status is not None else None,
            "csrc_sha16": sources_sha16(sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC))),
            "arch": ARCH, "hip_flags": HIP_FLAGS}
    tmp = BUILD_INFO + ".tmp"
    with open(tmp, "w") as f:
        json.dump(info, f, indent=1)
    os.replace(tmp, BUILD_INFO)


def build(jobs: int | None = None, verbose: bool = False) -> str:
    """Compile every csrc/*.hip for gfx950 and link libmfft.so; returns its path."""
    hipcc = _hipcc()
    os.makedirs(BUILD, exist_ok=True)
    srcs = sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))
    jobs = jobs or min(len(srcs), os.cpu_count() or 4, 8)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, hipcc), srcs))
    tmp = LIB + ".tmp"
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB)
    _write_build_info()
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
