"""The C-ABI library: it loads, exports every symbol include/kvint4.h declares,
and its host-only entry points (planning, argument validation) behave. No
kernel is launched here (no GPU needed)."""

from __future__ import annotations

import ctypes
import os
import re

import pytest

from kvint4 import _native as nat

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_symbols() -> set[str]:
    text = open(os.path.join(ROOT, "include", "kvint4.h")).read()
    return set(re.findall(r"^\s*(?:int64_t|int|const char\*)\s+(kvq_\w+)\s*\(", text, re.M))


def test_header_and_binding_agree():
    assert _declared_symbols() == set(nat.EXPORTED_SYMBOLS)


def test_library_exports_every_declared_symbol():
    lib = nat.lib()
    for name in _declared_symbols():
        assert hasattr(lib, name), name
        assert ctypes.cast(getattr(lib, name), ctypes.c_void_p).value


def test_version_and_error_slot():
    lib = nat.lib()
    assert lib.kvq_version() // 10000 == nat.KVQ_MAJOR
    assert isinstance(nat.last_error(), str)


def test_num_splits_planning():
    lib = nat.lib()
    B16, F16, F32 = nat.KVQ_BF16, nat.KVQ_F16, nat.KVQ_F32
    # Llama-3.1-8B decode at 16K on 256 CUs: 8 KV heads x 32 splits (512 tokens each)
    assert lib.kvq_decode_attn_num_splits(1, 32, 8, 1, 128, 16384, B16, B16, 256) == 32
    # no split shorter than two 64-token tiles
    assert lib.kvq_decode_attn_num_splits(1, 32, 8, 1, 128, 600, B16, B16, 256) == 4
    assert lib.kvq_decode_attn_num_splits(1, 32, 8, 1, 128, 100, B16, B16, 256) == 1
    # plenty of units already -> one split
    assert lib.kvq_decode_attn_num_splits(16, 25, 25, 1, 64, 1024, F16, F16, 256) == 1
    # fp32 queries plan for the VALU kernel the same way: no split shorter than
    # 128 keys (1K keys: 8 splits), otherwise enough splits to cover the CUs
    assert lib.kvq_decode_attn_num_splits(1, 12, 12, 1, 64, 1024, F32, F16, 256) == 8
    assert lib.kvq_decode_attn_num_splits(1, 12, 12, 1, 64, 16384, F32, F16, 256) == 22
    assert lib.kvq_decode_attn_num_splits(1, 32, 8, 1, 96, 1024, B16, B16, 256) == nat.KVQ_EUNSUP
    assert lib.kvq_decode_attn_num_splits(1, 30, 8, 1, 128, 1024, B16, B16, 256) == nat.KVQ_EINVAL
    # an empty batch or query block launches nothing: one split, no workspace
    assert lib.kvq_decode_attn_num_splits(0, 32, 8, 1, 128, 1024, B16, B16, 256) == 1
    assert lib.kvq_decode_attn_num_splits(2, 32, 8, 0, 128, 1024, B16, B16, 256) == 1
    assert lib.kvq_decode_attn_workspace_bytes(0, 32, 8, 1, 128, B16, B16, 1) == 0
    assert lib.kvq_decode_attn_num_splits(-1, 32, 8, 1, 128, 1024, B16, B16, 256) == nat.KVQ_EINVAL


def test_workspace_bytes():
    lib = nat.lib()
    B16 = nat.KVQ_BF16
    # a requested split count is kept whatever the kernel's minimum split
    # length (the VALU kernel's is 1024 keys): 12 units x 3 splits of partials
    ws3 = lib.kvq_decode_attn_workspace_bytes(1, 12, 12, 1, 64, nat.KVQ_F32, nat.KVQ_F16, 3)
    assert ws3 == 1024 * 64 + 512 + 12 * 3 * 64 * 4  # counters, (max, sum) pairs padded to 256 B, partials
    assert lib.kvq_decode_attn_workspace_bytes(1, 32, 8, 1, 128, B16, B16, 1) == 0
    ws = lib.kvq_decode_attn_workspace_bytes(1, 32, 8, 1, 128, B16, B16, 32)
    # counter block (1024 units x one counter x 64 bytes), then 8 units x 32 splits x 4 rows x (128 + 2) floats
    assert ws == 1024 * 64 + 8 * 32 * 4 * 130 * 4
    assert lib.kvq_decode_attn_workspace_bytes(1, 32, 8, 1, 128, 7, B16, 4) == nat.KVQ_EINVAL


def test_invalid_arguments_rejected_before_any_launch():
    lib = nat.lib()
    s4 = nat.i64_array([0, 0, 0, 1])
    s3 = nat.i64_array([0, 0, 0])
    rc = lib.kvq_quantize(None, nat.KVQ_BF16, s4, 1, 1, 1, 128, 0, None, s3, None, nat.KVQ_BF16, s3,
                          None, 0, 1, None)
    assert rc == nat.KVQ_EINVAL and "group_size" in nat.last_error()
    rc = lib.kvq_quantize(None, 9, s4, 1, 1, 1, 128, 32, None, s3, None, nat.KVQ_BF16, s3, None, 0, 1, None)
    assert rc == nat.KVQ_EINVAL and "dtype" in nat.last_error()
    rc = lib.kvq_quantize(None, nat.KVQ_BF16, s4, 1, 1, 1, 128, 32, None, s3, None, nat.KVQ_BF16, s3,
                          None, 0, 1, None)
    assert rc == nat.KVQ_EINVAL and "null" in nat.last_error()
    # a scalar position whose rows do not fit the destination, and a negative capacity
    rc = lib.kvq_quantize(None, nat.KVQ_BF16, s4, 1, 1, 3, 128, 32, None, s3, None, nat.KVQ_BF16, s3,
                          None, 8, 10, None)
    assert rc == nat.KVQ_EINVAL and "outside the destination" in nat.last_error()
    rc = lib.kvq_quantize(None, nat.KVQ_BF16, s4, 1, 1, 1, 128, 32, None, s3, None, nat.KVQ_BF16, s3,
                          None, 0, -1, None)
    assert rc == nat.KVQ_EINVAL and "capacity" in nat.last_error()
    rc = lib.kvq_dequantize(None, s3, None, nat.KVQ_BF16, s3, 1, 1, 1, 32, 4, None, nat.KVQ_BF16, s4,
                            200, None)
    assert rc == nat.KVQ_EINVAL and "d_out" in nat.last_error()
    rc = lib.kvq_decode_attn(None, nat.KVQ_BF16, s4, None, s3, None, s3, None, s3, None, s3,
                             nat.KVQ_BF16, None, s4, 1, 6, 4, 1, 128, 32, 16, None, 0, 1.0, 1,
                             None, 0, None)
    assert rc == nat.KVQ_EINVAL and "multiple" in nat.last_error()
    rc = lib.kvq_decode_attn(None, nat.KVQ_BF16, s4, None, s3, None, s3, None, s3, None, s3,
                             nat.KVQ_BF16, None, s4, 1, 8, 4, 1, 96, 32, 16, None, 0, 1.0, 1,
                             None, 0, None)
    assert rc == nat.KVQ_EUNSUP


def test_check_maps_status_to_exceptions():
    with pytest.raises(ValueError):
        nat.check(nat.KVQ_EINVAL, "x")
    with pytest.raises(nat.KVQUnsupported):
        nat.check(nat.KVQ_EUNSUP, "x")
    with pytest.raises(RuntimeError):
        nat.check(nat.KVQ_EHIP, "x")


def test_prefill_entry_points_validate_before_any_launch():
    """kvq_prefill_attn(_paged): shape, dtype and geometry checks, and the
    split plan's workspace figures, all host arithmetic (no device call)."""
    lib = nat.lib()
    B16, F32 = nat.KVQ_BF16, nat.KVQ_F32
    q4 = nat.i64_array([32 * 64 * 128, 64 * 128, 128, 1])
    c3 = nat.i64_array([8 * 1000 * 64, 1000 * 64, 64])
    s3 = nat.i64_array([8 * 1000 * 4, 1000 * 4, 4])

    def call(q_dtype=B16, s_dtype=B16, B=1, Hq=32, Hkv=8, Sq=64, D=128, G=32, Sk=1000, q_str=q4):
        return lib.kvq_prefill_attn(None, q_dtype, q_str, None, c3, None, s3, None, c3, None, s3, s_dtype,
                                    None, q4, B, Hq, Hkv, Sq, D, G, Sk, 1, 0.1, None, 0, None)

    assert call(Hq=30) == nat.KVQ_EINVAL                      # Hq not a multiple of Hkv
    assert call(q_dtype=F32) == nat.KVQ_EUNSUP and "bf16/fp16" in nat.last_error()
    assert call(D=96) == nat.KVQ_EUNSUP
    assert call(Hq=8 * 5) == nat.KVQ_EUNSUP                   # GQA ratio 5 does not divide 64
    assert call(q_str=nat.i64_array([0, 0, 256, 2])) == nat.KVQ_EUNSUP and "contiguous" in nat.last_error()
    assert call(B=0) == nat.KVQ_OK and call(Sq=0) == nat.KVQ_OK    # nothing to launch, no pointer read
    assert call() == nat.KVQ_EINVAL and "null" in nat.last_error()
    # paged: page size and table geometry
    p2 = nat.i64_array([4096 * 64, 64])
    p2s = nat.i64_array([4096 * 4, 4])

    def paged(page_size=64, cols=16, n_blocks=64, Sk=1000):
        return lib.kvq_prefill_attn_paged(None, B16, q4, None, p2, None, p2s, None, p2, None, p2s, B16,
                                          None, 16, cols, n_blocks, page_size, None, q4,
                                          1, 32, 8, 64, 128, 32, Sk, 1, 0.1, None, 0, None)

    assert paged(page_size=32) == nat.KVQ_EINVAL and "page_size" in nat.last_error()
    assert paged(Sk=16 * 64 + 1) == nat.KVQ_EINVAL            # Sk past the table's capacity
    assert paged() == nat.KVQ_EINVAL and "null" in nat.last_error()
    # split plan: a launch too small for the device splits over keys and needs
    # (D + 2) floats per row, split and workgroup; one that fills it needs none
    ws = lib.kvq_prefill_attn_workspace_bytes(1, 32, 8, 128, 128, 16384)
    assert ws == 8 * 8 * 8 * 64 * (128 + 2) * 4              # 8 heads x 8 row blocks x 8 splits x 64 rows
    assert lib.kvq_prefill_attn_workspace_bytes(1, 32, 8, 16384, 128, 16384) == 0
    assert lib.kvq_prefill_attn_workspace_bytes(0, 32, 8, 128, 128, 16384) == 0
    assert lib.kvq_prefill_attn_workspace_bytes(1, 32, 8, 128, 96, 16384) == nat.KVQ_EINVAL


def test_noalloc_step_refuses_plans_beyond_its_scratch():
    """kvq_decode_step_noalloc: a split plan whose workspace exceeds the 4 MiB
    static scratch is refused with KVQ_ESPACE before any device call (null
    tensors are never read), and planner errors pass through."""
    lib = nat.lib()
    B16 = nat.KVQ_BF16
    s4 = nat.i64_array([0, 0, 0, 1])
    s3 = nat.i64_array([0, 0, 0])

    def call(B, Hkv, n_split, D=128):
        return lib.kvq_decode_step_noalloc(None, B16, s4, None, s4, None, s4, None, s3, None, s3, None, s3,
                                           None, s3, B16, None, s4, B, 8 * Hkv, Hkv, D, 32, 4097, None, 4096,
                                           0.1, n_split, None)

    need = lib.kvq_decode_attn_workspace_bytes(64, 64, 8, 1, 128, B16, B16, 4)
    assert need > 4 << 20
    assert call(64, 8, 4) == nat.KVQ_ESPACE and "static scratch" in nat.last_error()
    assert call(1, 8, 4, D=96) == nat.KVQ_EUNSUP
