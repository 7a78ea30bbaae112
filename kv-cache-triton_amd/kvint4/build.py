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
# Per-source flags. The decode kernels keep their MFMA accumulators in VGPRs:
# the compiler's default puts the PV accumulators in AGPRs, and the two-row-set
# kernel then copies about 72 values between AGPRs and VGPRs on every tile
# (its VALU uses them, for the lazy rescale), with ~100 registers held twice.
# The prefill kernel's one-row-block variant likewise drops its 32 AGPRs
# (176 copies) and runs four waves per SIMD instead of three.
SOURCE_FLAGS = {"kvq_attn.hip": ("-mllvm", "-amdgpu-mfma-vgpr-form=true"),
                "kvq_prefill.hip": ("-mllvm", "-amdgpu-mfma-vgpr-form=true")}
# gfx950 only: the decode kernels assume its wave64 MFMA forms and its
# round-robin workgroup-to-XCD dispatch (checked again at run time).
ARCH = "gfx950"

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


# The measurement library behind bench.py --stream-probe: the streaming-read
# probe kernels and the decode kernels built with phase stamps.
PROBE_OUT = os.path.join(_HERE, "libkvq_probe.so")
# The probe kernels take plain scalar arguments, which the hardware can load
# into SGPRs at wave launch (kernarg preload): a wave then starts its loads
# without first waiting for the argument block to come from memory. Measured
# on the decode step's 18.9 MB, 4.60 -> 4.22 us per launch; the smallest
# launches lose about 0.1 us. So the probe is built both ways and the
# ceiling takes the better. The decode kernels take one 456-byte argument
# struct, which preload (at most 14 SGPRs, and never an aggregate) cannot
# carry, so the flag is for the probe only. A third build adds the
# nontemporal hint to the read's loads (4.18 -> 4.13 us at 18.9 MB, 51 -> 47
# us at 267 MB).
_PRELOAD = ("-DKVQ_PROBE_PRELOAD=1", "-mllvm", "-amdgpu-kernarg-preload-count=16")
PROBE_SOURCES = (("probe/kvq_probe.hip", ()),
                 ("probe/kvq_probe.hip", _PRELOAD),
                 ("probe/kvq_probe.hip", _PRELOAD + ("-DKVQ_PROBE_NT=1",)),
                 ("kvq_attn.hip", SOURCE_FLAGS["kvq_attn.hip"] + ("-DKVQ_PHASE_STAMPS=1",)),
                 ("kvq_capi.hip", ()))


def _build_libs(libs, verbose: bool) -> None:
    """libs: [(output path, [(source under csrc, extra flags)])]. Every
    object compiles in parallel, then each library links."""
    from concurrent.futures import ThreadPoolExecutor

    tmpdir = tempfile.mkdtemp(prefix="kvint4-build.", dir=_HERE)
    try:
        compile_flags = [f for f in HIPCC_FLAGS if f != "-shared"]
        jobs = []
        for li, (_, srcs) in enumerate(libs):
            for si, (s, extra) in enumerate(srcs):
                jobs.append((os.path.join(CSRC, s), list(extra), os.path.join(tmpdir, f"{li}_{si}.o")))

        def compile_one(job) -> None:
            src, extra, obj = job
            cmd = [hipcc(), *compile_flags, *extra, "-c", src, "-o", obj]
            if verbose:
                print(" ".join(cmd), flush=True)
            proc = subprocess.run(cmd, capture_output=True, text=True)
            if proc.returncode != 0:
                raise RuntimeError(f"hipcc failed ({proc.returncode}) on {src}:\n{proc.stdout}\n{proc.stderr}")

        with ThreadPoolExecutor(max_workers=min(8, len(jobs))) as ex:
            list(ex.map(compile_one, jobs))
        for li, (out, srcs) in enumerate(libs):
            objs = [os.path.join(tmpdir, f"{li}_{si}.o") for si in range(len(srcs))]
            tmp = os.path.join(tmpdir, os.path.basename(out))
            cmd = [hipcc(), *HIPCC_FLAGS, *objs, "-o", tmp]
            if verbose:
                print(" ".join(cmd), flush=True)
            proc = subprocess.run(cmd, capture_output=True, text=True)
            if proc.returncode != 0:
                raise RuntimeError(f"hipcc link failed ({proc.returncode}):\n{proc.stdout}\n{proc.stderr}")
            os.replace(tmp, out)  # atomic: a reader never sees a half-written library
    finally:
        shutil.rmtree(tmpdir, ignore_errors=True)


def build(verbose: bool = False) -> str:
    """Compile every HIP source into kvint4/libkvint4.so (the product) and
    kvint4/libkvq_probe.so (measurement only); return the product's path."""
    _build_libs([(OUT, [(s, SOURCE_FLAGS.get(s, ())) for s in SOURCES]), (PROBE_OUT, list(PROBE_SOURCES))],
                verbose)
    return OUT
