"""The cross-split merge of the decode kernel assumes that every split of a
unit (batch x KV head x row chunk) runs on one XCD, so that the partials the
splits store and the merging workgroup reads share that XCD's L2
(kv-cache-triton_amd/csrc/kvq_attn.hip, unit_and_split and the merge's
ordering comment). This checks the assumption on the hardware: the phase-
stamped build of the decode kernels (libkvq_probe.so, measurement only)
records each wave's HW_REG_XCC_ID at entry, and for the split plans of the
north-star (Llama-3.1-8B, 16K), C2 (4K), C4 (Llama-3.1-70B shape, batch 8,
32K) and C5 (GPT-2-xl MHA, batch 16, 1K) launches every workgroup of a unit
must report the same XCC (C5's own plan does not split; it runs with four
splits here). The reference has no counterpart (its Triton
kernel merges nothing across programs: kernels/llama3/attention_quant.py:104-152
walks the whole sequence in one program)."""

from __future__ import annotations

import ctypes
import os

import numpy as np
import pytest
import torch

from kvint4 import _native as nat
from kvint4 import ops

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
PROBE = os.path.join(os.path.dirname(nat.LIB_PATH), "libkvq_probe.so")
SLOTS, XCC_SLOT = 16, 12


def _probe_lib():
    if not os.path.exists(PROBE):
        raise RuntimeError(f"{PROBE} is missing: build it first (python -m kvint4.build)")
    lib = ctypes.CDLL(PROBE)
    prod = nat.lib()
    for name in ("kvq_decode_attn", "kvq_decode_attn_num_splits", "kvq_decode_attn_workspace_bytes",
                 "kvq_last_error"):
        getattr(lib, name).restype = getattr(prod, name).restype
        getattr(lib, name).argtypes = getattr(prod, name).argtypes
    lib.kvq_probe_set_phase_stamps.restype = ctypes.c_int
    lib.kvq_probe_set_phase_stamps.argtypes = [ctypes.c_void_p]
    return lib


# name: (B, Hq, Hkv, D, ctx, dtype)
PLANS = {
    "north-star": (1, 32, 8, 128, 16384, torch.bfloat16),
    "c2": (1, 32, 8, 128, 4096, torch.bfloat16),
    "c4": (8, 64, 8, 128, 32768, torch.bfloat16),
    "c5": (16, 25, 25, 64, 1024, torch.float16),
}


@pytest.mark.parametrize("name", sorted(PLANS))
def test_every_split_of_a_unit_runs_on_one_xcc(name):
    B, Hq, Hkv, D, L, dt = PLANS[name]
    print(f"xcd mapping: {name} B={B} Hq={Hq} Hkv={Hkv} D={D} ctx={L}", flush=True)
    lib = _probe_lib()
    G = 32
    gen = torch.Generator(device=DEV).manual_seed(3)
    kp, ks = ops.quantize(torch.randn(B, Hkv, L, D, device=DEV, generator=gen).to(dt), G, dt)
    vp, vs = ops.quantize(torch.randn(B, Hkv, L, D, device=DEV, generator=gen).to(dt), G, dt)
    q = torch.randn(B, Hq, 1, D, device=DEV, generator=gen).to(dt)
    out = torch.empty_like(q)
    qd, sd = nat.DTYPE_CODE[dt], nat.DTYPE_CODE[ks.dtype]
    planned = lib.kvq_decode_attn_num_splits(B, Hq, Hkv, 1, D, L, qd, sd, ops._num_cus(DEV))
    # C5 fills the chip without splitting (400 units); a caller may still ask
    # for splits, and the merge must then hold too
    ns = planned if planned > 1 else 4
    ws = torch.zeros(max(lib.kvq_decode_attn_workspace_bytes(B, Hq, Hkv, 1, D, qd, sd, ns), 1),
                     dtype=torch.uint8, device=DEV)
    # upper bound on the launched workgroups: 8 n_split x ceil(units / 8),
    # units <= B Hkv (rows per KV head) (one row chunk per row at most)
    units_max = B * Hkv * (Hq // Hkv)
    wg_max = 8 * ns * -(-units_max // 8)
    stamps = torch.full((wg_max * 16 * SLOTS,), -1, dtype=torch.int64, device=DEV)
    stream = torch.cuda.current_stream(DEV)
    arr = nat.i64_array
    assert lib.kvq_probe_set_phase_stamps(stamps.data_ptr()) == 0
    try:
        rc = lib.kvq_decode_attn(q.data_ptr(), qd, arr(q.stride()),
                                 kp.data_ptr(), arr(kp.stride()[:3]), ks.data_ptr(), arr(ks.stride()[:3]),
                                 vp.data_ptr(), arr(vp.stride()[:3]), vs.data_ptr(), arr(vs.stride()[:3]), sd,
                                 out.data_ptr(), arr(out.stride()), B, Hq, Hkv, 1, D, G, L,
                                 None, 0, D ** -0.5, ns, ws.data_ptr(), ws.numel(), stream.cuda_stream)
        torch.cuda.synchronize()
    finally:
        lib.kvq_probe_set_phase_stamps(None)
    assert rc == 0, lib.kvq_last_error().decode()
    a = stamps.view(wg_max, 16, SLOTS).cpu().numpy()
    launched = a[:, 0, 0] != -1
    n_wg = int(launched.sum())
    X = 8 * ns
    # the launched workgroups are a prefix of the buffer, whole rows of X
    assert n_wg > 0 and n_wg % X == 0 and launched[:n_wg].all() and not launched[n_wg:].any()
    xcc = a[:n_wg, :, XCC_SLOT]
    waves = a[:n_wg, :, 0] != -1
    # every stamped wave of a workgroup reports its workgroup's XCC
    for w in range(n_wg):
        ids = np.unique(xcc[w][waves[w]])
        assert ids.size == 1, (w, ids)
    wg_xcc = xcc[:, 0]
    idx = np.arange(n_wg)
    x, y = idx % X, idx // X  # grid (8 n_split, groups, 1): no z at these sizes
    unit = (x & 7) + 8 * y
    split = x >> 3
    bad = []
    for u in np.unique(unit):
        ids = np.unique(wg_xcc[unit == u])
        assert np.array_equal(np.sort(split[unit == u]), np.arange(ns))
        if ids.size != 1:
            bad.append((int(u), ids.tolist()))
    print(f"xcd mapping: {name}: n_split {ns} (planned {planned}), {n_wg} workgroups, {np.unique(unit).size} units, "
          f"XCCs seen {np.unique(wg_xcc).tolist()}, units on more than one XCC: {len(bad)}", flush=True)
    assert not bad, bad[:8]
