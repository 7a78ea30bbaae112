"""Device operators of the INT4 KV path, on top of the C ABI.

Everything here works on GPU tensors and enqueues HIP kernels on the current
stream. The model-family front-ends (``kvint4.llama3``, ``kvint4.gpt2``) add the
reference's argument contracts and dtype policies on top.

Layouts (bit-identical to the reference's, ``kernels/llama3/quantize.py:7-14``):
  x       [..., d]                        bf16 / fp16 / fp32
  packed  [..., ceil(d/G) * ceil(G/2)]    uint8, element 2i -> low nibble of byte i
  scales  [..., ceil(d/G)]                scale dtype (per family policy)
"""

from __future__ import annotations

import contextlib
import math
import threading

import torch
import torch.nn.functional as F

from . import _native as nat

SUPPORTED_FLOATS = (torch.bfloat16, torch.float16, torch.float32)

# Query rows per KV head (GQA group x query length) above which a multi-token
# query block goes to dequantize + dense SDPA instead of the fused kernel. The
# fused kernel streams the cache once per 8 rows; on one MI355X it is the
# faster route up to 1024 rows and flash SDPA beyond 2048, at 512 to 16K keys
# (e.g. 16K keys, GQA 4: 256 queries 610 vs 652 us, 512 queries 1251 vs 654 us).
MAX_FUSED_ROWS = 1024
# A block of at least PREFILL_MIN_ROWS rows per KV head whose rows x keys
# reach PREFILL_MIN_WORK, over a cache with one length for the batch (a
# prompt, a prompt chunk, a large speculative block), goes to the matrix-core
# prefill kernel instead: it dequantizes each 64-key tile into LDS once for
# 64 or 128 rows and splits the key range when the launch is small. Measured
# crossover with the fused kernel (GQA 4): 64 rows at 16K keys (16 queries
# 48 vs 60 us), 128-256 at 4K, 512-1024 at 1K; a whole 16K prompt takes
# 3.50 ms vs 4.50 ms for dequantize + flash SDPA.
PREFILL_MIN_ROWS = 64
PREFILL_MIN_WORK = 1 << 20


def use_prefill_kernel(rows: int, Sk: int) -> bool:
    return rows >= PREFILL_MIN_ROWS and rows * Sk >= PREFILL_MIN_WORK


def dense_fast_path(q: torch.Tensor, seq_lens: torch.Tensor | None) -> bool:
    """Whether dense_attention runs the fused flash SDPA kernel for this query
    (16-bit queries, one length for the whole batch); otherwise it masks
    explicitly on the fp32 math backend, and the fused kernel is preferred at
    any block length."""
    return q.dtype in (torch.bfloat16, torch.float16) and seq_lens is None


def packed_width(d: int, group_size: int) -> int:
    return math.ceil(d / group_size) * ((group_size + 1) // 2)


def num_groups(d: int, group_size: int) -> int:
    return math.ceil(d / group_size)


def _as_bhs(t: torch.Tensor) -> tuple[torch.Tensor, tuple[int, int, int], tuple[int, int, int]]:
    """View the leading dims of `t` as (B, H, S): returns (tensor, sizes, strides).

    Up to three leading dims are used as they are; more are collapsed with
    `reshape` (a copy only if the strides cannot be merged).
    """
    lead = t.dim() - 1
    if lead > 3:
        t = t.reshape(-1, t.shape[-1])
        lead = 1
    sizes = [1] * (3 - lead) + list(t.shape[:-1])
    strides = [0] * (3 - lead) + list(t.stride()[:-1])
    return t, tuple(sizes), tuple(strides)


def _check_cuda(*ts: torch.Tensor, what: str) -> None:
    for t in ts:
        if not t.is_cuda:
            raise ValueError(f"{what} expects GPU tensors (got a tensor on {t.device})")


# ---------------------------------------------------------------------------
# quantize / dequantize


def quantize_into(
    x: torch.Tensor,
    packed: torch.Tensor,
    scales: torch.Tensor,
    group_size: int,
    write_pos: int | torch.Tensor = 0,
) -> None:
    """Quantize x [B, H, S, D] and write the rows at positions pos_b + s of the
    cache tensors packed [B, H, S_cap, W] / scales [B, H, S_cap, n_groups].

    `write_pos` is an int (same position for every batch row; rows past the
    cache's capacity raise ValueError) or a device int32 tensor [B] of
    per-sequence positions (rows past the capacity are dropped).
    """
    _check_cuda(x, packed, scales, what="quantize_into")
    if x.dim() != 4 or packed.dim() != 4 or scales.dim() != 4:
        raise ValueError("quantize_into expects 4D x, packed and scales")
    B, H, S, D = x.shape
    if packed.shape[:2] != (B, H) or scales.shape[:2] != (B, H):
        raise ValueError("cache leading dims must match x [B, H, ...]")
    if packed.shape[-1] < packed_width(D, group_size) or scales.shape[-1] < num_groups(D, group_size):
        raise ValueError("cache last dims are too small for this head dim / group size")
    if packed.stride(-1) != 1 or scales.stride(-1) != 1:
        raise ValueError("cache last dims must be contiguous")
    if packed.dtype != torch.uint8 or scales.dtype not in SUPPORTED_FLOATS:
        raise ValueError("cache dtypes must be uint8 codes and float scales")
    wp_ptr, wp0 = None, 0
    if isinstance(write_pos, torch.Tensor):
        if write_pos.dtype != torch.int32 or write_pos.numel() != B or not write_pos.is_cuda:
            raise ValueError("write_pos must be a device int32 tensor of shape [B]")
        write_pos = write_pos.contiguous()
        wp_ptr = write_pos.data_ptr()
    else:
        wp0 = int(write_pos)
        if wp0 < 0 or wp0 + S > packed.shape[2] or wp0 + S > scales.shape[2]:
            raise ValueError("write position out of the cache's range")
    lib = nat.lib()
    with nat.device_of(x):
        rc = lib.kvq_quantize(
            x.data_ptr(), nat.DTYPE_CODE[x.dtype], nat.i64_array(x.stride()),
            B, H, S, D, group_size,
            packed.data_ptr(), nat.i64_array(packed.stride()[:3]),
            scales.data_ptr(), nat.DTYPE_CODE[scales.dtype], nat.i64_array(scales.stride()[:3]),
            wp_ptr, wp0, min(int(packed.shape[2]), int(scales.shape[2])), nat.stream_handle(x.device),
        )
    nat.check(rc, "kvq_quantize")


def quantize(x: torch.Tensor, group_size: int, scale_dtype: torch.dtype) -> tuple[torch.Tensor, torch.Tensor]:
    """Fresh (packed, scales) for x [..., d]; scales stored in `scale_dtype`."""
    _check_cuda(x, what="quantize_int4")
    lead_shape = x.shape[:-1]
    d = x.shape[-1]
    w, ng = packed_width(d, group_size), num_groups(d, group_size)
    packed = torch.empty((*lead_shape, w), dtype=torch.uint8, device=x.device)
    scales = torch.empty((*lead_shape, ng), dtype=scale_dtype, device=x.device)
    if x.numel() == 0 or ng == 0:
        return packed, scales
    xv, sizes, strides = _as_bhs(x)
    pv = packed.reshape(*sizes, w)
    sv = scales.reshape(*sizes, ng)
    lib = nat.lib()
    with nat.device_of(x):
        rc = lib.kvq_quantize(
            xv.data_ptr(), nat.DTYPE_CODE[x.dtype], nat.i64_array((*strides, xv.stride(-1))),
            sizes[0], sizes[1], sizes[2], d, group_size,
            pv.data_ptr(), nat.i64_array(pv.stride()[:3]),
            sv.data_ptr(), nat.DTYPE_CODE[scale_dtype], nat.i64_array(sv.stride()[:3]),
            None, 0, sizes[2], nat.stream_handle(x.device),
        )
    nat.check(rc, "kvq_quantize")
    return packed, scales


def dequantize(
    packed: torch.Tensor,
    scales: torch.Tensor,
    group_size: int,
    d_out: int,
    out_dtype: torch.dtype,
) -> torch.Tensor:
    """(nibble - 8) * fp32(scale) -> out_dtype, first `d_out` columns."""
    _check_cuda(packed, scales, what="dequantize_int4")
    ng = scales.shape[-1]
    width = packed.shape[-1]
    if width * 2 < ng * group_size and ng > 0:
        raise ValueError("packed has insufficient width for the provided group_size")
    d_out = min(int(d_out), ng * group_size)
    lead_shape = packed.shape[:-1]
    out = torch.empty((*lead_shape, d_out), dtype=out_dtype, device=packed.device)
    if out.numel() == 0:
        return out
    if packed.stride(-1) != 1:
        packed = packed.contiguous()
    if scales.stride(-1) != 1:
        scales = scales.contiguous()
    pv, sizes, pstr = _as_bhs(packed)
    sv, ssz, sstr = _as_bhs(scales)
    if ssz != sizes:
        sv = scales.reshape(*sizes, ng)
        sstr = sv.stride()[:3]
    ov = out.reshape(*sizes, d_out)
    lib = nat.lib()
    with nat.device_of(packed):
        rc = lib.kvq_dequantize(
            pv.data_ptr(), nat.i64_array(pstr),
            sv.data_ptr(), nat.DTYPE_CODE[scales.dtype], nat.i64_array(sstr),
            sizes[0], sizes[1], sizes[2], group_size, ng,
            ov.data_ptr(), nat.DTYPE_CODE[out_dtype], nat.i64_array(ov.stride()), d_out,
            nat.stream_handle(packed.device),
        )
    nat.check(rc, "kvq_dequantize")
    return out


# ---------------------------------------------------------------------------
# decode attention


class _Workspaces:
    """Zero-initialised split-K workspaces, one per (device, stream).

    The kernel returns its counters to zero, so a workspace is reused across
    calls issued on the same stream (which are ordered). A HIP graph captured
    on a stream keeps the address of the workspace it was captured with, so a
    buffer is never freed once handed out: when a later call needs more bytes
    the key gets a new, larger buffer and the old one stays allocated (the
    retired buffers together are at most the size of the current one, since
    sizes at least double). Inside ``using_workspace(buf)`` calls on this
    thread take ``buf`` instead (a graph that owns its workspace: two graphs
    replayed concurrently then share no counters).
    """

    def __init__(self) -> None:
        self._lock = threading.Lock()
        self._bufs: dict[tuple[int, int], torch.Tensor] = {}
        self._retired: list[torch.Tensor] = []
        self._local = threading.local()

    def get(self, device: torch.device, stream: int, nbytes: int) -> torch.Tensor:
        own = getattr(self._local, "buf", None)
        if own is not None:
            if own.device != device or own.numel() < nbytes:
                raise ValueError(f"the workspace given to using_workspace ({own.numel()} bytes on {own.device}) "
                                 f"is too small or on another device: {nbytes} bytes needed on {device}")
            return own
        idx = device.index
        if idx is None:
            idx = torch.cuda.current_device() if device.type == "cuda" else -1
        key = (idx, stream)
        with self._lock:
            buf = self._bufs.get(key)
            if buf is None or buf.numel() < nbytes:
                size = max(nbytes, 1 << 20)
                if buf is not None:
                    size = max(size, 2 * buf.numel())
                    self._retired.append(buf)
                buf = torch.zeros(size, dtype=torch.uint8, device=device)
                self._bufs[key] = buf
            return buf

    @contextlib.contextmanager
    def using(self, buf: torch.Tensor):
        if buf.dtype != torch.uint8 or buf.dim() != 1:
            raise ValueError("a workspace is a 1-D uint8 tensor")
        prev = getattr(self._local, "buf", None)
        self._local.buf = buf
        try:
            yield buf
        finally:
            self._local.buf = prev


_workspaces = _Workspaces()
# prefill split partials: a separate buffer, so that they never overwrite the
# decode kernels' arrival counters
_prefill_workspaces = _Workspaces()


def decode_workspace_bytes(B: int, Hq: int, Hkv: int, D: int, q_dtype: torch.dtype,
                           scale_dtype: torch.dtype, Sq: int = 1, n_split: int = 64) -> int:
    """Workspace bytes that cover every decode launch of this shape with up to
    `n_split` splits (64 is the library's largest split count)."""
    lib = nat.lib()
    n = lib.kvq_decode_attn_workspace_bytes(B, Hq, Hkv, Sq, D, nat.DTYPE_CODE[q_dtype],
                                            nat.DTYPE_CODE[scale_dtype], n_split)
    if n < 0:
        nat.check(int(n), "kvq_decode_attn_workspace_bytes")
    return int(n)


def using_workspace(buf: torch.Tensor):
    """Context manager: decode launches made on this thread inside it use the
    zero-filled uint8 device tensor `buf` as their split-K workspace (size it
    with decode_workspace_bytes). Launches that overlap in time must not share
    one workspace."""
    return _workspaces.using(buf)


def _prefill_ws(q: torch.Tensor, Hkv: int, Sk: int, stream: int) -> tuple:
    B, Hq, Sq, D = q.shape
    n = nat.lib().kvq_prefill_attn_workspace_bytes(B, Hq, Hkv, Sq, D, Sk)
    if n < 0:
        nat.check(int(n), "kvq_prefill_attn_workspace_bytes")
    if n == 0:
        return None, 0
    ws = _prefill_workspaces.get(q.device, stream, n)
    return ws.data_ptr(), ws.numel()
_cu_count: dict[int, int] = {}


def _num_cus(device: torch.device) -> int:
    idx = device.index if device.index is not None else torch.cuda.current_device()
    n = _cu_count.get(idx)
    if n is None:
        n = torch.cuda.get_device_properties(idx).multi_processor_count
        _cu_count[idx] = n
    return n


def fused_decode_attention(
    q: torch.Tensor,
    k_packed: torch.Tensor,
    k_scales: torch.Tensor,
    v_packed: torch.Tensor,
    v_scales: torch.Tensor,
    *,
    n_kv_heads: int,
    group_size: int,
    is_causal: bool,
    sm_scale: float,
    seq_lens: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
    n_split: int | None = None,
) -> torch.Tensor:
    """Launch the fused split-K decode kernel; raises KVQUnsupported for shapes
    it does not handle. q [B, Hq, Sq, D]; K/V codes [B, Hkv, Sk, W] (strided views
    of a larger cache are fine as long as the last dim is contiguous).
    `n_split` overrides the planner's sequence-split count (tuning)."""
    B, Hq, Sq, D = q.shape
    Sk = k_packed.shape[2]
    if out is None:
        out = torch.empty_like(q)
    if k_packed.stride(-1) != 1 or v_packed.stride(-1) != 1:
        raise nat.KVQUnsupported("packed K/V last dim must be contiguous")
    if k_scales.stride(-1) != 1:
        k_scales = k_scales.contiguous()
    if v_scales.stride(-1) != 1:
        v_scales = v_scales.contiguous()
    if v_scales.dtype != k_scales.dtype:
        v_scales = v_scales.to(k_scales.dtype)
    sl_ptr = None
    if seq_lens is not None:
        if seq_lens.dtype != torch.int32 or not seq_lens.is_cuda or seq_lens.numel() != B:
            raise ValueError("seq_lens must be a device int32 tensor of shape [B]")
        seq_lens = seq_lens.contiguous()
        sl_ptr = seq_lens.data_ptr()
    lib = nat.lib()
    qd = nat.DTYPE_CODE[q.dtype]
    sd = nat.DTYPE_CODE[k_scales.dtype]
    if n_split is None:
        n_split = lib.kvq_decode_attn_num_splits(B, Hq, n_kv_heads, Sq, D, Sk, qd, sd, _num_cus(q.device))
        if n_split < 0:
            nat.check(int(n_split), "kvq_decode_attn_num_splits")
    elif n_split < 1:
        raise ValueError("n_split must be >= 1")
    ws_bytes = lib.kvq_decode_attn_workspace_bytes(B, Hq, n_kv_heads, Sq, D, qd, sd, n_split)
    if ws_bytes < 0:
        nat.check(int(ws_bytes), "kvq_decode_attn_workspace_bytes")
    with nat.device_of(q):
        stream = nat.stream_handle(q.device)
        ws_ptr, ws_len = None, 0
        if ws_bytes > 0:
            ws = _workspaces.get(q.device, stream, ws_bytes)
            ws_ptr, ws_len = ws.data_ptr(), ws.numel()
        rc = lib.kvq_decode_attn(
            q.data_ptr(), qd, nat.i64_array(q.stride()),
            k_packed.data_ptr(), nat.i64_array(k_packed.stride()[:3]),
            k_scales.data_ptr(), nat.i64_array(k_scales.stride()[:3]),
            v_packed.data_ptr(), nat.i64_array(v_packed.stride()[:3]),
            v_scales.data_ptr(), nat.i64_array(v_scales.stride()[:3]),
            sd,
            out.data_ptr(), nat.i64_array(out.stride()),
            B, Hq, n_kv_heads, Sq, D, group_size, Sk,
            sl_ptr, 1 if is_causal else 0, float(sm_scale),
            n_split, ws_ptr, ws_len, stream,
        )
    nat.check(rc, "kvq_decode_attn")
    return out


def prefill_attention(
    q: torch.Tensor,
    k_packed: torch.Tensor,
    k_scales: torch.Tensor,
    v_packed: torch.Tensor,
    v_scales: torch.Tensor,
    *,
    n_kv_heads: int,
    group_size: int,
    is_causal: bool,
    sm_scale: float,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Long query blocks (prefill, prompt chunks) over the INT4 cache on the
    matrix cores (kvq_prefill_attn); raises KVQUnsupported for shapes or
    dtypes it does not handle. q [B, Hq, Sq, D]; K/V codes [B, Hkv, Sk, W],
    one length Sk for the batch; causal masking aligned bottom-right."""
    B, Hq, Sq, D = q.shape
    Sk = k_packed.shape[2]
    if q.stride(-1) != 1:
        q = q.contiguous()
    if out is None:
        out = torch.empty_like(q)
    if k_packed.stride(-1) != 1 or v_packed.stride(-1) != 1:
        raise nat.KVQUnsupported("packed K/V last dim must be contiguous")
    if k_scales.stride(-1) != 1:
        k_scales = k_scales.contiguous()
    if v_scales.stride(-1) != 1:
        v_scales = v_scales.contiguous()
    if v_scales.dtype != k_scales.dtype:
        v_scales = v_scales.to(k_scales.dtype)
    lib = nat.lib()
    with nat.device_of(q):
        stream = nat.stream_handle(q.device)
        ws_ptr, ws_len = _prefill_ws(q, n_kv_heads, Sk, stream)
        rc = lib.kvq_prefill_attn(
            q.data_ptr(), nat.DTYPE_CODE[q.dtype], nat.i64_array(q.stride()),
            k_packed.data_ptr(), nat.i64_array(k_packed.stride()[:3]),
            k_scales.data_ptr(), nat.i64_array(k_scales.stride()[:3]),
            v_packed.data_ptr(), nat.i64_array(v_packed.stride()[:3]),
            v_scales.data_ptr(), nat.i64_array(v_scales.stride()[:3]),
            nat.DTYPE_CODE[k_scales.dtype],
            out.data_ptr(), nat.i64_array(out.stride()),
            B, Hq, n_kv_heads, Sq, D, group_size, Sk,
            1 if is_causal else 0, float(sm_scale), ws_ptr, ws_len, stream,
        )
    nat.check(rc, "kvq_prefill_attn")
    return out


def decode_step(
    q: torch.Tensor,
    k_new: torch.Tensor,
    v_new: torch.Tensor,
    k_packed: torch.Tensor,
    k_scales: torch.Tensor,
    v_packed: torch.Tensor,
    v_scales: torch.Tensor,
    position,
    *,
    n_kv_heads: int,
    group_size: int,
    sm_scale: float,
    out: torch.Tensor | None = None,
    n_split: int | None = None,
) -> torch.Tensor:
    """One decode token in one launch: quantize k_new / v_new [B, Hkv, 1, D]
    into row `position` of the capacity buffers (an int for every sequence, or
    a device int32 [B] of per-sequence old lengths) and attend q [B, Hq, 1, D]
    over the cache including the new row. The buffers are the cache's
    [B, Hkv, capacity, .] tensors, written in place; the caller advances its
    lengths. Raises KVQUnsupported for dtype/group combinations the fused
    step does not handle (the caller then quantizes and attends separately)."""
    B, Hq, Sq, D = q.shape
    if Sq != 1:
        raise nat.KVQUnsupported("decode_step handles one query position")
    cap = int(k_packed.shape[2])
    if out is None:
        out = torch.empty_like(q)
    if k_new.dtype != q.dtype or v_new.dtype != q.dtype:
        raise nat.KVQUnsupported("decode_step needs K/V rows in q's dtype")
    if k_new.stride(-1) != 1:
        k_new = k_new.contiguous()
    if v_new.stride(-1) != 1:
        v_new = v_new.contiguous()
    lib = nat.lib()
    qd = nat.DTYPE_CODE[q.dtype]
    sd = nat.DTYPE_CODE[k_scales.dtype]
    if isinstance(position, torch.Tensor):
        if position.dtype != torch.int32 or not position.is_cuda or position.numel() != B:
            raise ValueError("position must be an int or a device int32 tensor of shape [B]")
        pos_ptr, pos0, s_max = position.contiguous().data_ptr(), 0, cap
    else:
        pos_ptr, pos0 = None, int(position)
        if not 0 <= pos0 < cap:
            raise ValueError(f"write position {pos0} outside the cache capacity {cap}")
        s_max = pos0 + 1
    if n_split is None:
        n_split = lib.kvq_decode_attn_num_splits(B, Hq, n_kv_heads, 1, D, s_max, qd, sd, _num_cus(q.device))
        if n_split < 0:
            nat.check(int(n_split), "kvq_decode_attn_num_splits")
    ws_bytes = lib.kvq_decode_attn_workspace_bytes(B, Hq, n_kv_heads, 1, D, qd, sd, n_split)
    if ws_bytes < 0:
        nat.check(int(ws_bytes), "kvq_decode_attn_workspace_bytes")
    with nat.device_of(q):
        stream = nat.stream_handle(q.device)
        ws_ptr, ws_len = None, 0
        if ws_bytes > 0:
            ws = _workspaces.get(q.device, stream, ws_bytes)
            ws_ptr, ws_len = ws.data_ptr(), ws.numel()
        rc = lib.kvq_decode_step(
            q.data_ptr(), qd, nat.i64_array(q.stride()),
            k_new.data_ptr(), nat.i64_array(k_new.stride()),
            v_new.data_ptr(), nat.i64_array(v_new.stride()),
            k_packed.data_ptr(), nat.i64_array(k_packed.stride()[:3]),
            k_scales.data_ptr(), nat.i64_array(k_scales.stride()[:3]),
            v_packed.data_ptr(), nat.i64_array(v_packed.stride()[:3]),
            v_scales.data_ptr(), nat.i64_array(v_scales.stride()[:3]),
            sd,
            out.data_ptr(), nat.i64_array(out.stride()),
            B, Hq, n_kv_heads, D, group_size, cap,
            pos_ptr, pos0, float(sm_scale),
            n_split, ws_ptr, ws_len, stream,
        )
    nat.check(rc, "kvq_decode_step")
    return out


def _sdpa_dense(q, k, v, *, is_causal: bool, sm_scale: float, attn_mask=None) -> torch.Tensor:
    """Dense attention on already-dequantized, GQA-expanded K/V.

    bf16/fp16 run on the fused flash / memory-efficient SDPA backends only (the
    math backend would issue batched GEMMs on transposed half-precision views);
    fp32 uses the math backend.
    """
    from torch.nn.attention import SDPBackend, sdpa_kernel

    if q.dtype in (torch.bfloat16, torch.float16) and attn_mask is None:
        try:
            with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
                return F.scaled_dot_product_attention(q, k, v, is_causal=is_causal, scale=sm_scale)
        except RuntimeError:
            pass
    qf, kf, vf = q.float(), k.float(), v.float()
    with sdpa_kernel([SDPBackend.MATH]):
        o = F.scaled_dot_product_attention(
            qf, kf, vf, attn_mask=attn_mask, is_causal=is_causal and attn_mask is None, scale=sm_scale
        )
    return o.to(q.dtype)


def dense_attention_over_quantized(
    q: torch.Tensor,
    k_packed: torch.Tensor,
    k_scales: torch.Tensor,
    v_packed: torch.Tensor,
    v_scales: torch.Tensor,
    *,
    n_kv_heads: int,
    group_size: int,
    is_causal: bool,
    sm_scale: float,
    seq_lens: torch.Tensor | None = None,
) -> torch.Tensor:
    """Long query blocks (prefill) and shapes outside the fused kernel: HIP
    dequantize of the INT4 cache, then dense SDPA. Causal masking is aligned to
    the bottom-right corner (query i sees keys j <= Sk - Sq + i), as in the
    reference kernel (kernels/llama3/attention_quant.py:91-97,123)."""
    D = q.shape[-1]
    k = dequantize(k_packed, k_scales, group_size, D, q.dtype)
    v = dequantize(v_packed, v_scales, group_size, D, q.dtype)
    return dense_attention(q, k, v, n_kv_heads=n_kv_heads, is_causal=is_causal, sm_scale=sm_scale,
                           seq_lens=seq_lens)


def dense_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    n_kv_heads: int,
    is_causal: bool,
    sm_scale: float,
    seq_lens: torch.Tensor | None = None,
) -> torch.Tensor:
    """Dense SDPA of q [B, Hq, Sq, D] over dequantized k, v [B, Hkv, Sk, D]
    with the fused kernel's conventions: GQA head map h // (Hq / Hkv), keys
    past seq_lens[b] masked, causal aligned bottom-right, rows with no
    admissible key zero."""
    B, Hq, Sq, D = q.shape
    Sk = k.shape[2]
    ratio = Hq // n_kv_heads
    if dense_fast_path(q, seq_lens) and is_causal and 0 < Sq < Sk:
        # bottom-right causal block (a prompt chunk after cached tokens): the
        # flash kernel with its lower-right causal variant and native GQA
        from torch.nn.attention import SDPBackend, sdpa_kernel
        from torch.nn.attention.bias import causal_lower_right

        try:
            with sdpa_kernel([SDPBackend.FLASH_ATTENTION]):
                return F.scaled_dot_product_attention(q, k, v, attn_mask=causal_lower_right(Sq, Sk),
                                                      scale=sm_scale, enable_gqa=True)
        except RuntimeError:
            pass
    if (ratio > 1 and seq_lens is None and not (is_causal and Sq != Sk)
            and q.dtype in (torch.bfloat16, torch.float16)):
        # the fused SDPA kernels read each KV head for its whole query group
        # (no GQA-expanded copy of K/V)
        from torch.nn.attention import SDPBackend, sdpa_kernel

        try:
            with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
                return F.scaled_dot_product_attention(q, k, v, is_causal=is_causal, scale=sm_scale,
                                                      enable_gqa=True)
        except RuntimeError:
            pass
    if ratio > 1:
        k = k.repeat_interleave(ratio, dim=1)
        v = v.repeat_interleave(ratio, dim=1)
    mask = None
    if seq_lens is not None or (is_causal and Sq != Sk):
        jj = torch.arange(Sk, device=q.device)
        ii = torch.arange(Sq, device=q.device)
        lens = (seq_lens.to(torch.int64) if seq_lens is not None
                else torch.full((B,), Sk, dtype=torch.int64, device=q.device))
        allowed = jj[None, None, :] < lens[:, None, None]  # [B, 1, Sk]
        if is_causal:
            allowed = allowed & (jj[None, None, :] <= (lens[:, None, None] - Sq + ii[None, :, None]))
        mask = allowed[:, None, :, :]  # [B, 1, Sq, Sk]
        out = _sdpa_dense(q, k, v, is_causal=False, sm_scale=sm_scale, attn_mask=mask)
        # rows with no admissible key: zeros (the fused kernel's convention)
        empty = ~allowed.any(dim=-1)  # [B, Sq]
        if bool(empty.any()):
            out = out.masked_fill(empty[:, None, :, None], 0)
        return out
    return _sdpa_dense(q, k, v, is_causal=is_causal, sm_scale=sm_scale)


def attention_over_quantized(
    q: torch.Tensor,
    k_packed: torch.Tensor,
    k_scales: torch.Tensor,
    v_packed: torch.Tensor,
    v_scales: torch.Tensor,
    *,
    n_kv_heads: int,
    group_size: int,
    is_causal: bool,
    sm_scale: float,
    seq_lens: torch.Tensor | None = None,
) -> torch.Tensor:
    """Route by query rows per KV head: the matrix-core prefill kernel for
    long blocks with one length for the batch (whole prompts and prompt
    chunks, use_prefill_kernel), the fused decode kernel for blocks of at
    most MAX_FUSED_ROWS rows (decode, speculative blocks) and for causal
    blocks after cached tokens that the dense route would mask explicitly
    (fp32 queries or per-sequence lengths), and dequantize + dense SDPA for
    the rest (KVQ_EUNSUP shapes, long blocks the prefill kernel does not
    take)."""
    B, Hq, Sq, D = q.shape
    Sk = k_packed.shape[2]
    rows = (Hq // n_kv_heads) * Sq
    if seq_lens is None and use_prefill_kernel(rows, Sk):
        try:
            return prefill_attention(q, k_packed, k_scales, v_packed, v_scales, n_kv_heads=n_kv_heads,
                                     group_size=group_size, is_causal=is_causal, sm_scale=sm_scale)
        except nat.KVQUnsupported:
            pass
    use_fused = rows <= MAX_FUSED_ROWS or (is_causal and Sq != Sk and not dense_fast_path(q, seq_lens))
    if use_fused:
        try:
            return fused_decode_attention(
                q, k_packed, k_scales, v_packed, v_scales,
                n_kv_heads=n_kv_heads, group_size=group_size, is_causal=is_causal,
                sm_scale=sm_scale, seq_lens=seq_lens,
            )
        except nat.KVQUnsupported:
            pass
    return dense_attention_over_quantized(
        q, k_packed, k_scales, v_packed, v_scales,
        n_kv_heads=n_kv_heads, group_size=group_size, is_causal=is_causal,
        sm_scale=sm_scale, seq_lens=seq_lens,
    )


# ---------------------------------------------------------------------------
# paged caches


class PageTable:
    """A block table for paged caches: device int32 [B, cols] of block ids
    (-1: no block) for pages of `page_size` rows (a power of two) in pools of
    `num_blocks` blocks. Token t of sequence b lives in pool row
    table[b, t // page_size] * page_size + t % page_size."""

    __slots__ = ("table", "page_size", "num_blocks")

    def __init__(self, table: torch.Tensor, page_size: int, num_blocks: int) -> None:
        if table.dtype != torch.int32 or table.dim() != 2 or not table.is_cuda or table.stride(-1) != 1:
            raise ValueError("block table must be a device int32 [B, cols] tensor with contiguous rows")
        if page_size < 1 or page_size & (page_size - 1):
            raise ValueError("page_size must be a power of two")
        self.table, self.page_size, self.num_blocks = table, int(page_size), int(num_blocks)

    def args(self) -> tuple:
        return (self.table.data_ptr(), self.table.stride(0), self.table.shape[1], self.num_blocks, self.page_size)

    @property
    def capacity(self) -> int:
        return self.table.shape[1] * self.page_size


def _check_pool(pool: torch.Tensor, scales: torch.Tensor, pt: PageTable, H: int, D: int, group_size: int) -> None:
    rows = pt.num_blocks * pt.page_size
    if pool.dim() != 3 or scales.dim() != 3 or pool.shape[:2] != (H, rows) or scales.shape[:2] != (H, rows):
        raise ValueError(f"pools must be [H={H}, num_blocks*page_size={rows}, .] (got {tuple(pool.shape)}, "
                         f"{tuple(scales.shape)})")
    if pool.dtype != torch.uint8 or scales.dtype not in SUPPORTED_FLOATS:
        raise ValueError("pool dtypes must be uint8 codes and float scales")
    if pool.shape[-1] < packed_width(D, group_size) or scales.shape[-1] < num_groups(D, group_size):
        raise ValueError("pool rows are too small for this head dim / group size")
    if pool.stride(-1) != 1 or scales.stride(-1) != 1:
        raise ValueError("pool rows must be contiguous")


def quantize_into_paged(
    x: torch.Tensor,
    pool: torch.Tensor,
    scales: torch.Tensor,
    pt: PageTable,
    group_size: int,
    write_pos: int | torch.Tensor = 0,
) -> None:
    """quantize_into for a paged cache: row (b, h, s) of x [B, H, S, D] goes to
    sequence b's position pos_b + s, i.e. its page's pool row; positions whose
    page has no block are dropped."""
    _check_cuda(x, pool, scales, pt.table, what="quantize_into_paged")
    if x.dim() != 4:
        raise ValueError("quantize_into_paged expects 4D x")
    B, H, S, D = x.shape
    if pt.table.shape[0] < B:
        raise ValueError("block table has fewer rows than the batch")
    _check_pool(pool, scales, pt, H, D, group_size)
    wp_ptr, wp0 = None, 0
    if isinstance(write_pos, torch.Tensor):
        if write_pos.dtype != torch.int32 or write_pos.numel() != B or not write_pos.is_cuda:
            raise ValueError("write_pos must be a device int32 tensor of shape [B]")
        write_pos = write_pos.contiguous()
        wp_ptr = write_pos.data_ptr()
    else:
        wp0 = int(write_pos)
        if wp0 < 0:
            raise ValueError("write position must be >= 0")
    lib = nat.lib()
    with nat.device_of(x):
        rc = lib.kvq_quantize_paged(
            x.data_ptr(), nat.DTYPE_CODE[x.dtype], nat.i64_array(x.stride()),
            B, H, S, D, group_size,
            pool.data_ptr(), nat.i64_array(pool.stride()[:2]),
            scales.data_ptr(), nat.DTYPE_CODE[scales.dtype], nat.i64_array(scales.stride()[:2]),
            *pt.args(), wp_ptr, wp0, nat.stream_handle(x.device),
        )
    nat.check(rc, "kvq_quantize_paged")


def dequantize_paged(
    pool: torch.Tensor,
    scales: torch.Tensor,
    pt: PageTable,
    B: int,
    S: int,
    group_size: int,
    d_out: int,
    out_dtype: torch.dtype,
) -> torch.Tensor:
    """[B, H, S, d_out] of the first S positions of every sequence (positions
    whose page has no block come out as zeros)."""
    _check_cuda(pool, scales, pt.table, what="dequantize_paged")
    if pt.table.shape[0] < B:
        raise ValueError("block table has fewer rows than the batch")
    H, ng = pool.shape[0], scales.shape[-1]
    d_out = min(int(d_out), ng * group_size)
    out = torch.empty((B, H, S, d_out), dtype=out_dtype, device=pool.device)
    if out.numel() == 0:
        return out
    lib = nat.lib()
    with nat.device_of(pool):
        rc = lib.kvq_dequantize_paged(
            pool.data_ptr(), nat.i64_array(pool.stride()[:2]),
            scales.data_ptr(), nat.DTYPE_CODE[scales.dtype], nat.i64_array(scales.stride()[:2]),
            *pt.args(), B, H, S, group_size, ng,
            out.data_ptr(), nat.DTYPE_CODE[out_dtype], nat.i64_array(out.stride()), d_out,
            nat.stream_handle(pool.device),
        )
    nat.check(rc, "kvq_dequantize_paged")
    return out


def _plan(lib, q: torch.Tensor, B: int, Hq: int, n_kv_heads: int, Sq: int, D: int, s_max: int,
          sd: int, n_split: int | None) -> tuple[int, int]:
    qd = nat.DTYPE_CODE[q.dtype]
    if n_split is None:
        n_split = lib.kvq_decode_attn_num_splits(B, Hq, n_kv_heads, Sq, D, s_max, qd, sd, _num_cus(q.device))
        if n_split < 0:
            nat.check(int(n_split), "kvq_decode_attn_num_splits")
    elif n_split < 1:
        raise ValueError("n_split must be >= 1")
    ws_bytes = lib.kvq_decode_attn_workspace_bytes(B, Hq, n_kv_heads, Sq, D, qd, sd, n_split)
    if ws_bytes < 0:
        nat.check(int(ws_bytes), "kvq_decode_attn_workspace_bytes")
    return int(n_split), int(ws_bytes)


def fused_decode_attention_paged(
    q: torch.Tensor,
    k_pool: torch.Tensor,
    k_scales: torch.Tensor,
    v_pool: torch.Tensor,
    v_scales: torch.Tensor,
    pt: PageTable,
    *,
    n_kv_heads: int,
    group_size: int,
    is_causal: bool,
    sm_scale: float,
    seq_lens: torch.Tensor | None = None,
    seq_len: int | None = None,
    out: torch.Tensor | None = None,
    n_split: int | None = None,
) -> torch.Tensor:
    """fused_decode_attention over a paged cache. Sequence b attends its first
    seq_lens[b] tokens (device int32 [B]) or `seq_len` tokens. bf16/fp16
    queries with 16-bit scales run on the matrix cores, fp32 queries or scales
    on the exact-fp32 kernel. Raises KVQUnsupported where neither applies
    (page_size < 64)."""
    _check_cuda(q, k_pool, k_scales, v_pool, v_scales, pt.table, what="fused_decode_attention_paged")
    B, Hq, Sq, D = q.shape
    if pt.table.shape[0] < B:
        raise ValueError("block table has fewer rows than the batch")
    for pool, sc in ((k_pool, k_scales), (v_pool, v_scales)):
        _check_pool(pool, sc, pt, n_kv_heads, D, group_size)
    if out is None:
        out = torch.empty_like(q)
    if v_scales.dtype != k_scales.dtype:
        raise ValueError("K and V scale pools must share a dtype")
    sl_ptr, s_max = None, pt.capacity
    if seq_lens is not None:
        if seq_lens.dtype != torch.int32 or not seq_lens.is_cuda or seq_lens.numel() != B:
            raise ValueError("seq_lens must be a device int32 tensor of shape [B]")
        seq_lens = seq_lens.contiguous()
        sl_ptr, seq_len = seq_lens.data_ptr(), 0
    else:
        if seq_len is None or not 0 <= int(seq_len) <= pt.capacity:
            raise ValueError(f"seq_len must be in [0, {pt.capacity}] when seq_lens is not given")
        seq_len = int(seq_len)
        s_max = seq_len
    lib = nat.lib()
    sd = nat.DTYPE_CODE[k_scales.dtype]
    n_split, ws_bytes = _plan(lib, q, B, Hq, n_kv_heads, Sq, D, s_max, sd, n_split)
    with nat.device_of(q):
        stream = nat.stream_handle(q.device)
        ws_ptr, ws_len = None, 0
        if ws_bytes > 0:
            ws = _workspaces.get(q.device, stream, ws_bytes)
            ws_ptr, ws_len = ws.data_ptr(), ws.numel()
        rc = lib.kvq_decode_attn_paged(
            q.data_ptr(), nat.DTYPE_CODE[q.dtype], nat.i64_array(q.stride()),
            k_pool.data_ptr(), nat.i64_array(k_pool.stride()[:2]),
            k_scales.data_ptr(), nat.i64_array(k_scales.stride()[:2]),
            v_pool.data_ptr(), nat.i64_array(v_pool.stride()[:2]),
            v_scales.data_ptr(), nat.i64_array(v_scales.stride()[:2]),
            sd, *pt.args(),
            out.data_ptr(), nat.i64_array(out.stride()),
            B, Hq, n_kv_heads, Sq, D, group_size,
            sl_ptr, seq_len, 1 if is_causal else 0, float(sm_scale),
            n_split, ws_ptr, ws_len, stream,
        )
    nat.check(rc, "kvq_decode_attn_paged")
    return out


def prefill_attention_paged(
    q: torch.Tensor,
    k_pool: torch.Tensor,
    k_scales: torch.Tensor,
    v_pool: torch.Tensor,
    v_scales: torch.Tensor,
    pt: PageTable,
    seq_len: int,
    *,
    n_kv_heads: int,
    group_size: int,
    is_causal: bool,
    sm_scale: float,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """prefill_attention over a paged cache: every sequence attends its first
    seq_len tokens through the block table (pages of >= 64 rows); raises
    KVQUnsupported for shapes or dtypes the kernel does not handle."""
    _check_cuda(q, k_pool, v_pool, pt.table, what="prefill_attention_paged")
    B, Hq, Sq, D = q.shape
    if pt.table.shape[0] < B:
        raise ValueError("block table has fewer rows than the batch")
    _check_pool(k_pool, k_scales, pt, n_kv_heads, D, group_size)
    _check_pool(v_pool, v_scales, pt, n_kv_heads, D, group_size)
    if not 0 <= seq_len <= pt.capacity:
        raise ValueError(f"seq_len {seq_len} outside [0, {pt.capacity}]")
    if q.stride(-1) != 1:
        q = q.contiguous()
    if out is None:
        out = torch.empty_like(q)
    if v_scales.dtype != k_scales.dtype:
        raise nat.KVQUnsupported("K and V scales must share a dtype")
    lib = nat.lib()
    with nat.device_of(q):
        stream = nat.stream_handle(q.device)
        ws_ptr, ws_len = _prefill_ws(q, n_kv_heads, seq_len, stream)
        rc = lib.kvq_prefill_attn_paged(
            q.data_ptr(), nat.DTYPE_CODE[q.dtype], nat.i64_array(q.stride()),
            k_pool.data_ptr(), nat.i64_array(k_pool.stride()[:2]),
            k_scales.data_ptr(), nat.i64_array(k_scales.stride()[:2]),
            v_pool.data_ptr(), nat.i64_array(v_pool.stride()[:2]),
            v_scales.data_ptr(), nat.i64_array(v_scales.stride()[:2]),
            nat.DTYPE_CODE[k_scales.dtype], *pt.args(),
            out.data_ptr(), nat.i64_array(out.stride()),
            B, Hq, n_kv_heads, Sq, D, group_size, seq_len,
            1 if is_causal else 0, float(sm_scale), ws_ptr, ws_len, stream,
        )
    nat.check(rc, "kvq_prefill_attn_paged")
    return out


def decode_step_paged(
    q: torch.Tensor,
    k_new: torch.Tensor,
    v_new: torch.Tensor,
    k_pool: torch.Tensor,
    k_scales: torch.Tensor,
    v_pool: torch.Tensor,
    v_scales: torch.Tensor,
    pt: PageTable,
    position,
    *,
    n_kv_heads: int,
    group_size: int,
    sm_scale: float,
    out: torch.Tensor | None = None,
    n_split: int | None = None,
) -> torch.Tensor:
    """decode_step over a paged cache: the new token of sequence b goes to its
    position (int, or device int32 [B] of old lengths) through the block table;
    a position whose page has no block is neither written nor attended."""
    _check_cuda(q, k_new, v_new, k_pool, pt.table, what="decode_step_paged")
    B, Hq, Sq, D = q.shape
    if pt.table.shape[0] < B:
        raise ValueError("block table has fewer rows than the batch")
    for pool, sc in ((k_pool, k_scales), (v_pool, v_scales)):
        _check_pool(pool, sc, pt, n_kv_heads, D, group_size)
    if Sq != 1:
        raise nat.KVQUnsupported("decode_step_paged handles one query position")
    if out is None:
        out = torch.empty_like(q)
    if k_new.dtype != q.dtype or v_new.dtype != q.dtype:
        raise nat.KVQUnsupported("decode_step_paged needs K/V rows in q's dtype")
    if k_new.stride(-1) != 1:
        k_new = k_new.contiguous()
    if v_new.stride(-1) != 1:
        v_new = v_new.contiguous()
    cap = pt.capacity
    if isinstance(position, torch.Tensor):
        if position.dtype != torch.int32 or not position.is_cuda or position.numel() != B:
            raise ValueError("position must be an int or a device int32 tensor of shape [B]")
        pos_ptr, pos0, s_max = position.contiguous().data_ptr(), 0, cap
    else:
        pos_ptr, pos0 = None, int(position)
        if not 0 <= pos0 < cap:
            raise ValueError(f"write position {pos0} outside the table's capacity {cap}")
        s_max = pos0 + 1
    lib = nat.lib()
    sd = nat.DTYPE_CODE[k_scales.dtype]
    n_split, ws_bytes = _plan(lib, q, B, Hq, n_kv_heads, 1, D, s_max, sd, n_split)
    with nat.device_of(q):
        stream = nat.stream_handle(q.device)
        ws_ptr, ws_len = None, 0
        if ws_bytes > 0:
            ws = _workspaces.get(q.device, stream, ws_bytes)
            ws_ptr, ws_len = ws.data_ptr(), ws.numel()
        rc = lib.kvq_decode_step_paged(
            q.data_ptr(), nat.DTYPE_CODE[q.dtype], nat.i64_array(q.stride()),
            k_new.data_ptr(), nat.i64_array(k_new.stride()),
            v_new.data_ptr(), nat.i64_array(v_new.stride()),
            k_pool.data_ptr(), nat.i64_array(k_pool.stride()[:2]),
            k_scales.data_ptr(), nat.i64_array(k_scales.stride()[:2]),
            v_pool.data_ptr(), nat.i64_array(v_pool.stride()[:2]),
            v_scales.data_ptr(), nat.i64_array(v_scales.stride()[:2]),
            sd, *pt.args(),
            out.data_ptr(), nat.i64_array(out.stride()),
            B, Hq, n_kv_heads, D, group_size,
            pos_ptr, pos0, float(sm_scale),
            n_split, ws_ptr, ws_len, stream,
        )
    nat.check(rc, "kvq_decode_step_paged")
    return out
