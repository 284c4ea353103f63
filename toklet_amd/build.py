"""Build libtokhip.so (the gfx950 session attention library) in-tree with hipcc.

    python -m toklet_amd.build [--incremental]

Each source compiles to an object under toklet_amd/_build/ in parallel, then
links into toklet_amd/libtokhip.so next to this file.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libtokhip.so")
# The decode kernel's builds are spread over one unit per (dtype, head_dim) so
# they compile in parallel; the largest units are listed first.
DECODE_UNITS = [f"decode_{dt}_{d}.hip" for dt in ("bf16", "f16", "f32") for d in (128, 64, 256)]
SOURCES = DECODE_UNITS + ["prefill.hip", "decode.hip", "api.cpp", "session.cpp", "attention.hip",
                          "kv.hip", "produce.hip", "project.hip"]
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # No packed FP32 (v_pk_*_f32) instructions anywhere in the device code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-result",
    f"-I{os.path.join(ROOT, 'include')}",
    f"-I{CSRC}",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found: the ROCm toolchain is required to build libtokhip")
    return path


def _stale(src: str, obj: str) -> bool:
    if not os.path.exists(obj):
        return True
    deps = [os.path.join(CSRC, src)] + [os.path.join(CSRC, h) for h in os.listdir(CSRC)
                                        if h.endswith(".hpp")]
    deps.append(os.path.join(ROOT, "include", "tokhip.h"))
    return os.path.getmtime(obj) < max(os.path.getmtime(d) for d in deps)


def _compile(src: str, incremental: bool = False) -> str:
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    if incremental and not _stale(src, obj):
        return obj
    cmd = [hipcc(), *HIPCC_FLAGS, "-x", "hip", "-c", os.path.join(CSRC, src), "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stderr}")
    return obj


def build(verbose: bool = False, incremental: bool = False) -> str:
    """Compile every source (or, with `incremental`, those older than a source
    or header) and link the library."""
    os.makedirs(BUILD, exist_ok=True)
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 8)) as pool:
        objs = list(pool.map(lambda s: _compile(s, incremental), SOURCES))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True, incremental="--incremental" in sys.argv)
    sys.exit(0)
