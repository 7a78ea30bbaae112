"""Build libkvint4.so in-tree with hipcc for gfx950.

    python -m kvint4.build            # from kv-cache-triton_amd/
    python kv-cache-triton_amd/kvint4/build.py

The library is written next to this file (kvint4/libkvint4.so) so it ships
with the source tree; nothing is installed into site-packages.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile

_HERE = os.path.dirname(os.path.abspath(__file__))
PKG_ROOT = os.path.dirname(_HERE)  # kv-cache-triton_amd/
CSRC = os.path.join(PKG_ROOT, "csrc")
OUT = os.path.join(_HERE, "libkvint4.so")

SOURCES = ("kvq_capi.hip", "kvq_quant.hip", "kvq_attn.hip", "kvq_prefill.hip")
ARCH = os.environ.get("KVQ_OFFLOAD_ARCH", "gfx950")

# Packed-FP32 VALU forms are kept out of the generated code (the value path is
# written in scalar fp32 and v_dot2); -O3 and IEEE division are the defaults.
HIPCC_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def build(verbose: bool = False) -> str:
    """Compile every HIP source into kvint4/libkvint4.so; return its path."""
    srcs = [os.path.join(CSRC, s) for s in SOURCES]
    fd, tmp = tempfile.mkstemp(prefix="libkvint4.", suffix=".so.tmp", dir=_HERE)
    os.close(fd)
    cmd = [hipcc(), *HIPCC_FLAGS, *srcs, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        os.unlink(tmp)
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, OUT)  # atomic: a reader never sees a half-written library
    return OUT


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
