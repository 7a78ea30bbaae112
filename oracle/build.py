"""Build the C restatement (oracle/kvq_ref.c) into oracle/libkvqref.so with gcc.

Test infrastructure only (the checker and the CPU baseline). The reference
itself is Python + Triton, so there is nothing of it to compile; there is no
oracle/_ref build.
"""

from __future__ import annotations

import os
import subprocess
import sys
import tempfile

_HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(_HERE, "kvq_ref.c")
OUT = os.path.join(_HERE, "libkvqref.so")

# x86-64-v3 (AVX2/FMA) runs on this container and on the GPU hosts alike;
# no -ffast-math: division, nearbyintf and expf keep their IEEE meaning.
CFLAGS = ["-O3", "-march=x86-64-v3", "-fPIC", "-shared", "-fopenmp", "-std=c11"]


def build(verbose: bool = False) -> str:
    fd, tmp = tempfile.mkstemp(prefix="libkvqref.", suffix=".so.tmp", dir=_HERE)
    os.close(fd)
    cmd = ["gcc", *CFLAGS, SRC, "-o", tmp, "-lm"]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        os.unlink(tmp)
        raise RuntimeError(f"gcc failed ({proc.returncode}):\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
