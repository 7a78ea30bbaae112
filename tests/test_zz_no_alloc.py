"""GPU, through the C ABI: kvq_decode_step_noalloc (the decode step whose
split workspace is the library's static per-GPU scratch) against
kvq_decode_step with a caller workspace. Same cache bytes written and the
same output bits (one kernel, one split plan), on calls in a row whose plans
differ: a 4096-key context (32 splits), then a smaller input (1000 keys,
7 splits), then the first size again."""

from __future__ import annotations

import pytest
import torch

from kvint4 import _native as nat
from kvint4 import ops

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _case(B, Hq, Hkv, D, G, ctx, seed, xdt=torch.bfloat16, sdt=torch.bfloat16):
    g = torch.Generator(device=DEV).manual_seed(seed)
    cap = ctx + 1
    W, NG = ops.packed_width(D, G), ops.num_groups(D, G)
    c = {}
    for name in ("k", "v"):
        packed = torch.zeros(B, Hkv, cap, W, dtype=torch.uint8, device=DEV)
        scales = torch.zeros(B, Hkv, cap, NG, dtype=sdt, device=DEV)
        x = torch.randn(B, Hkv, ctx, D, generator=g, device=DEV).to(xdt)
        ops.quantize_into(x, packed, scales, G, 0)
        c[name + "p"], c[name + "s"] = packed, scales
    c["q"] = torch.randn(B, Hq, 1, D, generator=g, device=DEV).to(xdt)
    c["kn"] = torch.randn(B, Hkv, 1, D, generator=g, device=DEV).to(xdt)
    c["vn"] = torch.randn(B, Hkv, 1, D, generator=g, device=DEV).to(xdt)
    torch.cuda.synchronize()
    return c


def _args(c, out, B, Hq, Hkv, D, G, ctx):
    i64 = nat.i64_array
    return [
        c["q"].data_ptr(), nat.DTYPE_CODE[c["q"].dtype], i64(c["q"].stride()),
        c["kn"].data_ptr(), i64(c["kn"].stride()), c["vn"].data_ptr(), i64(c["vn"].stride()),
        c["kp"].data_ptr(), i64(c["kp"].stride()[:3]), c["ks"].data_ptr(), i64(c["ks"].stride()[:3]),
        c["vp"].data_ptr(), i64(c["vp"].stride()[:3]), c["vs"].data_ptr(), i64(c["vs"].stride()[:3]),
        nat.DTYPE_CODE[c["ks"].dtype], out.data_ptr(), i64(out.stride()),
        B, Hq, Hkv, D, G, ctx + 1, None, ctx, float(D ** -0.5),
    ]


def test_noalloc_step_matches_workspace_step_on_calls_in_a_row():
    lib = nat.lib()
    B, Hq, Hkv, D, G = 1, 32, 8, 128, 32
    cus = torch.cuda.get_device_properties(DEV).multi_processor_count
    stream = torch.cuda.current_stream(DEV).cuda_stream
    for call, (ctx, seed) in enumerate(((4096, 11), (1000, 12), (4096, 13))):
        print(f"[no-alloc] call {call}: B={B} Hq={Hq} Hkv={Hkv} D={D} ctx={ctx}", flush=True)
        ref = _case(B, Hq, Hkv, D, G, ctx, seed)
        mine = {k: v.clone() for k, v in ref.items()}
        ns = lib.kvq_decode_attn_num_splits(B, Hq, Hkv, 1, D, ctx + 1, nat.KVQ_BF16, nat.KVQ_BF16, cus)
        assert ns > 1, "the plan must split, so that the static scratch is used"
        ws = torch.zeros(lib.kvq_decode_attn_workspace_bytes(B, Hq, Hkv, 1, D, nat.KVQ_BF16, nat.KVQ_BF16, ns),
                         dtype=torch.uint8, device=DEV)
        out_ref = torch.empty(B, Hq, 1, D, dtype=torch.bfloat16, device=DEV)
        out_mine = torch.full_like(out_ref, float("nan"))
        rc = lib.kvq_decode_step(*_args(ref, out_ref, B, Hq, Hkv, D, G, ctx), ns, ws.data_ptr(), ws.numel(), stream)
        nat.check(rc, "kvq_decode_step")
        rc = lib.kvq_decode_step_noalloc(*_args(mine, out_mine, B, Hq, Hkv, D, G, ctx), ns, stream)
        nat.check(rc, "kvq_decode_step_noalloc")
        torch.cuda.synchronize()
        assert torch.equal(out_mine, out_ref), f"call {call}: outputs differ"
        for k in ("kp", "ks", "vp", "vs"):
            assert torch.equal(mine[k], ref[k]), f"call {call}: cache tensor {k} differs"


def test_noalloc_fp32_step_matches_workspace_step():
    """The same comparison on the fp32 kernel's decode step (fp32 queries and
    rows, fp32 scales; GPT-2-small shape), a 1024-key context then 300 keys."""
    lib = nat.lib()
    B, Hq, Hkv, D, G = 1, 12, 12, 64, 32
    F32 = nat.DTYPE_CODE[torch.float32]
    cus = torch.cuda.get_device_properties(DEV).multi_processor_count
    stream = torch.cuda.current_stream(DEV).cuda_stream
    for call, (ctx, seed) in enumerate(((1024, 21), (300, 22))):
        print(f"[no-alloc fp32] call {call}: B={B} Hq={Hq} Hkv={Hkv} D={D} ctx={ctx}", flush=True)
        ref = _case(B, Hq, Hkv, D, G, ctx, seed, torch.float32, torch.float32)
        mine = {k: v.clone() for k, v in ref.items()}
        ns = lib.kvq_decode_attn_num_splits(B, Hq, Hkv, 1, D, ctx + 1, F32, F32, cus)
        assert ns > 1, "the plan must split, so that the static scratch is used"
        ws = torch.zeros(lib.kvq_decode_attn_workspace_bytes(B, Hq, Hkv, 1, D, F32, F32, ns),
                         dtype=torch.uint8, device=DEV)
        out_ref = torch.empty(B, Hq, 1, D, dtype=torch.float32, device=DEV)
        out_mine = torch.full_like(out_ref, float("nan"))
        rc = lib.kvq_decode_step(*_args(ref, out_ref, B, Hq, Hkv, D, G, ctx), ns, ws.data_ptr(), ws.numel(), stream)
        nat.check(rc, "kvq_decode_step")
        rc = lib.kvq_decode_step_noalloc(*_args(mine, out_mine, B, Hq, Hkv, D, G, ctx), ns, stream)
        nat.check(rc, "kvq_decode_step_noalloc")
        torch.cuda.synchronize()
        assert torch.equal(out_mine, out_ref), f"call {call}: outputs differ"
        for k in ("kp", "ks", "vp", "vs"):
            assert torch.equal(mine[k], ref[k]), f"call {call}: cache tensor {k} differs"
