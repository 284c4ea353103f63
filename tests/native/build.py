"""Build the native test programs next to this file (test infrastructure).

    python tests/native/build.py

session_allocations: a host program (g++) over libtokhip's C ABI that counts
the library's host allocations and the device's free memory across a session's
steady state.  It links toklet_amd/libtokhip.so, found at run time through an
rpath relative to the program, and the HIP runtime.
"""

from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")


def build(verbose: bool = False) -> str:
    out = os.path.join(HERE, "session_allocations")
    cmd = ["g++", "-O1", "-std=c++17", "-D__HIP_PLATFORM_AMD__", f"-I{os.path.join(ROOT, 'include')}",
           f"-I{ROCM}/include", os.path.join(HERE, "session_allocations.cpp"), "-o", out,
           f"-L{os.path.join(ROOT, 'toklet_amd')}", "-ltokhip", f"-L{ROCM}/lib", "-lamdhip64", "-ldl",
           "-Wl,-rpath,$ORIGIN/../../toklet_amd", f"-Wl,-rpath,{ROCM}/lib"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"native test build failed:\n{res.stderr}")
    if verbose:
        print(f"built {out}")
    return out


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
