"""Fused decode step (kvq_decode_step): quantize-append of the new token and
decode attention in one launch, against the two-launch path it replaces
(quantize_into + fused attention over the appended cache; reference
models/llama3/kv_cache.py:76-105 then kernels/llama3/attention_quant.py:159-286)
and against the float64 oracle."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from kvint4 import ops
from oracle import kvq_oracle as O

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
TDT = {"bf16": torch.bfloat16, "f16": torch.float16}


def _cache(B, Hkv, cap, D, G, dtype, n_fill, seed):
    g = torch.Generator().manual_seed(seed)
    t, sdt = TDT[dtype], TDT[dtype]
    W, NG = ops.packed_width(D, G), ops.num_groups(D, G)
    kp = torch.zeros(B, Hkv, cap, W, dtype=torch.uint8, device=DEV)
    vp = torch.zeros_like(kp)
    ks = torch.zeros(B, Hkv, cap, NG, dtype=sdt, device=DEV)
    vs = torch.zeros_like(ks)
    if n_fill:
        k = torch.randn(B, Hkv, n_fill, D, generator=g).to(t).to(DEV)
        v = torch.randn(B, Hkv, n_fill, D, generator=g).to(t).to(DEV)
        ops.quantize_into(k, kp, ks, G, 0)
        ops.quantize_into(v, vp, vs, G, 0)
    return [kp, ks, vp, vs]


def _close(got, want):
    """Same attention, the new key folded in fp32 instead of through the
    matrix-core PV product, whose softmax weights are rounded to bf16 (2^-9
    relative). With few keys the weighted values can cancel, so the bound is
    absolute: 2^-6 (about 2^-9 times the largest |v| of these inputs, 8
    times) plus one bf16 unit in the last place of the output."""
    g, w = got.float().cpu().numpy(), want.float().cpu().numpy()
    assert np.all(np.abs(g - w) <= 2.0 ** -6 + 2.0 ** -7 * np.abs(w)), np.abs(g - w).max()


def _new(B, Hq, Hkv, D, dtype, seed):
    g = torch.Generator().manual_seed(seed + 1000)
    t = TDT[dtype]
    q = torch.randn(B, Hq, 1, D, generator=g).to(t).to(DEV)
    kn = (3.0 * torch.randn(B, Hkv, 1, D, generator=g)).to(t).to(DEV)
    vn = torch.randn(B, Hkv, 1, D, generator=g).to(t).to(DEV)
    return q, kn, vn


CASES = [
    # B, Hq, Hkv, D, G, pos, dtype
    (1, 32, 8, 128, 32, 16384, "bf16"),  # north-star shape
    (1, 32, 8, 128, 32, 4096, "bf16"),
    (1, 32, 8, 128, 32, 1, "bf16"),
    (1, 32, 8, 128, 32, 300, "bf16"),
    (2, 64, 8, 128, 32, 2000, "bf16"),   # 8 query rows per KV head
    (1, 8, 2, 128, 64, 777, "bf16"),
    (1, 8, 2, 128, 128, 513, "bf16"),
    (2, 12, 12, 64, 32, 1023, "f16"),    # GPT-2 shape (MHA, fp16 scales)
    (1, 16, 4, 64, 64, 100, "f16"),
    (1, 4, 4, 64, 128, 65, "f16"),       # G > D: padded group
]


@pytest.mark.parametrize("B,Hq,Hkv,D,G,pos,dtype", CASES)
def test_decode_step_matches_append_then_attend(B, Hq, Hkv, D, G, pos, dtype):
    cap = pos + 8
    a = _cache(B, Hkv, cap, D, G, dtype, pos, seed=pos + D)
    b = [t.clone() for t in a]
    q, kn, vn = _new(B, Hq, Hkv, D, dtype, seed=pos)
    sm = D ** -0.5
    # two-launch path
    ops.quantize_into(kn, a[0], a[1], G, pos)
    ops.quantize_into(vn, a[2], a[3], G, pos)
    n = pos + 1
    want = ops.fused_decode_attention(q, a[0][:, :, :n], a[1][:, :, :n], a[2][:, :, :n], a[3][:, :, :n],
                                      n_kv_heads=Hkv, group_size=G, is_causal=False, sm_scale=sm)
    # one launch
    got = ops.decode_step(q, kn, vn, b[0], b[1], b[2], b[3], pos, n_kv_heads=Hkv, group_size=G, sm_scale=sm)
    torch.cuda.synchronize()
    for x, y in zip(a, b):  # the whole buffers: new row bit-identical, nothing else touched
        assert torch.equal(x, y)
    exact = O.attention_over_quantized(
        q.float().cpu().numpy(), a[0][:, :, :n].cpu().numpy(), a[1][:, :, :n].float().cpu().numpy(),
        a[2][:, :, :n].cpu().numpy(), a[3][:, :, :n].float().cpu().numpy(), group_size=G, scale=sm)
    assert np.abs(got.float().cpu().numpy() - exact).max() <= 2e-2
    _close(got, want)


def test_decode_step_ragged_positions():
    B, Hq, Hkv, D, G = 4, 32, 8, 128, 32
    cap = 1200
    a = _cache(B, Hkv, cap, D, G, "bf16", 1100, seed=7)
    b = [t.clone() for t in a]
    pos = torch.tensor([1100, 0, 517, 1], dtype=torch.int32, device=DEV)
    q, kn, vn = _new(B, Hq, Hkv, D, "bf16", seed=7)
    sm = D ** -0.5
    ops.quantize_into(kn, a[0], a[1], G, pos)
    ops.quantize_into(vn, a[2], a[3], G, pos)
    want = ops.fused_decode_attention(q, a[0], a[1], a[2], a[3], n_kv_heads=Hkv, group_size=G,
                                      is_causal=False, sm_scale=sm, seq_lens=pos + 1)
    got = ops.decode_step(q, kn, vn, b[0], b[1], b[2], b[3], pos, n_kv_heads=Hkv, group_size=G, sm_scale=sm)
    torch.cuda.synchronize()
    for x, y in zip(a, b):
        assert torch.equal(x, y)
    _close(got, want)


def test_decode_step_position_past_capacity_leaves_row():
    """A sequence whose old length already fills the buffers is not written
    and attends the keys it has."""
    B, Hq, Hkv, D, G = 2, 32, 8, 128, 32
    cap = 600
    a = _cache(B, Hkv, cap, D, G, "bf16", cap, seed=11)
    before = [t.clone() for t in a]
    pos = torch.tensor([cap, 300], dtype=torch.int32, device=DEV)
    q, kn, vn = _new(B, Hq, Hkv, D, "bf16", seed=11)
    sm = D ** -0.5
    got = ops.decode_step(q, kn, vn, a[0], a[1], a[2], a[3], pos, n_kv_heads=Hkv, group_size=G, sm_scale=sm)
    torch.cuda.synchronize()
    for x, y in zip(a, before):
        assert torch.equal(x[0], y[0])          # sequence 0 untouched
        assert torch.equal(x[1, :, :300], y[1, :, :300])
        assert torch.equal(x[1, :, 301:], y[1, :, 301:])
    want0 = ops.fused_decode_attention(q[:1], a[0][:1], a[1][:1], a[2][:1], a[3][:1], n_kv_heads=Hkv,
                                       group_size=G, is_causal=False, sm_scale=sm)
    _close(got[:1], want0)


def test_decode_step_rejects_bad_position_and_unsupported():
    B, Hq, Hkv, D, G = 1, 8, 2, 128, 32
    a = _cache(B, Hkv, 64, D, G, "bf16", 10, seed=3)
    q, kn, vn = _new(B, Hq, Hkv, D, "bf16", seed=3)
    with pytest.raises(ValueError):
        ops.decode_step(q, kn, vn, *a, 64, n_kv_heads=Hkv, group_size=G, sm_scale=1.0)
    with pytest.raises(ops.nat.KVQUnsupported):  # new rows in another dtype than q
        ops.decode_step(q, kn.float(), vn.float(), *a, 10, n_kv_heads=Hkv, group_size=G, sm_scale=1.0)


# The fp32 VALU kernel's decode step: fp32 queries (exact fp32 arithmetic) or
# fp32 scales. Codes and scales bit-identical to kvq_quantize's; attention
# within 1e-4 of the two-launch path and of the float64 oracle for fp32
# queries (the new key is folded in exact fp32 in both), and within the
# 16-bit bound for bf16/fp16 queries (outputs rounded to the query dtype).
TDT32 = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}


def _cache_dt(B, Hkv, cap, D, G, xdt, sdt, n_fill, seed):
    g = torch.Generator().manual_seed(seed)
    W, NG = ops.packed_width(D, G), ops.num_groups(D, G)
    kp = torch.zeros(B, Hkv, cap, W, dtype=torch.uint8, device=DEV)
    vp = torch.zeros_like(kp)
    ks = torch.zeros(B, Hkv, cap, NG, dtype=TDT32[sdt], device=DEV)
    vs = torch.zeros_like(ks)
    if n_fill:
        k = torch.randn(B, Hkv, n_fill, D, generator=g).to(TDT32[xdt]).to(DEV)
        v = torch.randn(B, Hkv, n_fill, D, generator=g).to(TDT32[xdt]).to(DEV)
        ops.quantize_into(k, kp, ks, G, 0)
        ops.quantize_into(v, vp, vs, G, 0)
    return [kp, ks, vp, vs]


def _new_dt(B, Hq, Hkv, D, xdt, seed):
    g = torch.Generator().manual_seed(seed + 1000)
    t = TDT32[xdt]
    q = torch.randn(B, Hq, 1, D, generator=g).to(t).to(DEV)
    kn = (3.0 * torch.randn(B, Hkv, 1, D, generator=g)).to(t).to(DEV)
    vn = torch.randn(B, Hkv, 1, D, generator=g).to(t).to(DEV)
    return q, kn, vn


def _close_dt(got, want, xdt):
    if xdt != "f32":
        _close(got, want)
        return
    g, w = got.cpu().numpy(), want.cpu().numpy()
    assert np.all(np.abs(g - w) <= 1e-4 + 1e-4 * np.abs(w)), np.abs(g - w).max()


VALU_CASES = [
    # B, Hq, Hkv, D, G, pos, query/new-row dtype, scale dtype
    (1, 12, 12, 64, 32, 1023, "f32", "f32"),   # GPT-2 small decode shape
    (2, 12, 12, 64, 64, 300, "f32", "f32"),
    (1, 32, 8, 128, 32, 4096, "f32", "f32"),   # 4 query heads per KV head: 2 rows per workgroup
    (1, 32, 8, 128, 32, 1, "f32", "f32"),
    (1, 8, 2, 128, 128, 513, "f32", "bf16"),
    (1, 8, 2, 128, 32, 70, "f32", "f16"),
    (1, 4, 4, 64, 128, 65, "f32", "f32"),      # G > D: padded group
    (2, 32, 8, 128, 32, 2000, "bf16", "f32"),  # 16-bit queries with fp32 scales
    (1, 16, 4, 64, 64, 100, "f16", "f32"),
]


@pytest.mark.parametrize("B,Hq,Hkv,D,G,pos,xdt,sdt", VALU_CASES)
def test_valu_decode_step_matches_append_then_attend(B, Hq, Hkv, D, G, pos, xdt, sdt):
    print(f"valu decode step: B {B} Hq {Hq} Hkv {Hkv} D {D} G {G} pos {pos} {xdt}/{sdt}", flush=True)
    cap = pos + 8
    a = _cache_dt(B, Hkv, cap, D, G, xdt, sdt, pos, seed=pos + D + 5)
    b = [t.clone() for t in a]
    q, kn, vn = _new_dt(B, Hq, Hkv, D, xdt, seed=pos + 3)
    sm = D ** -0.5
    ops.quantize_into(kn, a[0], a[1], G, pos)
    ops.quantize_into(vn, a[2], a[3], G, pos)
    n = pos + 1
    want = ops.fused_decode_attention(q, a[0][:, :, :n], a[1][:, :, :n], a[2][:, :, :n], a[3][:, :, :n],
                                      n_kv_heads=Hkv, group_size=G, is_causal=False, sm_scale=sm)
    got = ops.decode_step(q, kn, vn, b[0], b[1], b[2], b[3], pos, n_kv_heads=Hkv, group_size=G, sm_scale=sm)
    torch.cuda.synchronize()
    for x, y in zip(a, b):  # the whole buffers: new row bit-identical, nothing else touched
        assert torch.equal(x, y)
    exact = O.attention_over_quantized(
        q.float().cpu().numpy(), a[0][:, :, :n].cpu().numpy(), a[1][:, :, :n].float().cpu().numpy(),
        a[2][:, :, :n].cpu().numpy(), a[3][:, :, :n].float().cpu().numpy(), group_size=G, scale=sm)
    tol = 1e-4 if xdt == "f32" else 2e-2
    assert np.abs(got.float().cpu().numpy() - exact).max() <= tol
    _close_dt(got, want, xdt)


def test_valu_decode_step_ragged_positions_and_full_sequence():
    """Per-sequence positions on the fp32 kernel, one of them at capacity
    (not written; attends the keys it has), with the split count forced up so
    the new token lands in the last of several splits."""
    print("valu decode step: ragged positions", flush=True)
    B, Hq, Hkv, D, G, cap = 4, 12, 12, 64, 32, 1100
    b = _cache_dt(B, Hkv, cap, D, G, "f32", "f32", cap, seed=17)
    pos = torch.tensor([1000, 0, cap, 517], dtype=torch.int32, device=DEV)
    q, kn, vn = _new_dt(B, Hq, Hkv, D, "f32", seed=17)
    sm = D ** -0.5
    ref = [t.clone() for t in b]
    for i, p in enumerate(pos.tolist()):
        if p < cap:  # the two-launch path writes in bounds only (views of one sequence)
            ops.quantize_into(kn[i:i + 1], ref[0][i:i + 1], ref[1][i:i + 1], G, p)
            ops.quantize_into(vn[i:i + 1], ref[2][i:i + 1], ref[3][i:i + 1], G, p)
    lens = torch.clamp(pos + 1, max=cap)
    want = ops.fused_decode_attention(q, ref[0], ref[1], ref[2], ref[3], n_kv_heads=Hkv, group_size=G,
                                      is_causal=False, sm_scale=sm, seq_lens=lens)
    got = ops.decode_step(q, kn, vn, b[0], b[1], b[2], b[3], pos, n_kv_heads=Hkv, group_size=G, sm_scale=sm,
                          n_split=4)
    torch.cuda.synchronize()
    for x, y in zip(ref, b):
        assert torch.equal(x, y)
    _close_dt(got, want, "f32")


def test_valu_decode_step_in_hip_graph_replays():
    """The fp32 kernel's decode step captured in a HIP graph: every replay
    (eager work and synchronisation between them) gives the eager result and
    the same cache bytes (its split counters re-armed by the kernel)."""
    print("valu decode step in a HIP graph", flush=True)
    B, Hq, Hkv, D, G, pos = 1, 12, 12, 64, 32, 1000
    a = _cache_dt(B, Hkv, pos + 8, D, G, "f32", "f32", pos, seed=23)
    q, kn, vn = _new_dt(B, Hq, Hkv, D, "f32", seed=23)
    sm = D ** -0.5
    out = torch.empty_like(q)
    ops.decode_step(q, kn, vn, *a, pos, n_kv_heads=Hkv, group_size=G, sm_scale=sm, out=out)  # warm-up
    torch.cuda.synchronize()
    want = out.clone()
    cache_want = [t.clone() for t in a]
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        ops.decode_step(q, kn, vn, *a, pos, n_kv_heads=Hkv, group_size=G, sm_scale=sm, out=out)
    torch.cuda.synchronize()
    for _ in range(4):
        out.zero_()
        (torch.randn(256, 256, device=DEV) @ torch.randn(256, 256, device=DEV)).sum().item()  # eager work
        with torch.cuda.stream(stream):
            graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want)
        for x, y in zip(a, cache_want):
            assert torch.equal(x, y)


def test_decode_step_in_hip_graph_replays():
    """The decode step captured in a HIP graph: every replay (with eager work
    and synchronisation between them) gives the eager result and the same
    cache bytes; the split-merge counters are re-armed by the kernel itself
    (no memset node in the graph)."""
    B, Hq, Hkv, D, G, pos = 1, 32, 8, 128, 32, 5000
    a = _cache(B, Hkv, pos + 64, D, G, "bf16", pos, seed=21)
    q, kn, vn = _new(B, Hq, Hkv, D, "bf16", seed=21)
    sm = D ** -0.5
    out = torch.empty_like(q)
    ops.decode_step(q, kn, vn, *a, pos, n_kv_heads=Hkv, group_size=G, sm_scale=sm, out=out)  # warm-up
    torch.cuda.synchronize()
    want = out.clone()
    cache_want = [t.clone() for t in a]
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        ops.decode_step(q, kn, vn, *a, pos, n_kv_heads=Hkv, group_size=G, sm_scale=sm, out=out)
    torch.cuda.synchronize()
    for _ in range(4):
        out.zero_()
        (torch.randn(256, 256, device=DEV) @ torch.randn(256, 256, device=DEV)).sum().item()  # eager work
        with torch.cuda.stream(stream):
            graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want)
        for x, y in zip(a, cache_want):
            assert torch.equal(x, y)


@pytest.mark.parametrize("D,n_split", [(64, None), (128, None), (128, 1)])
def test_decode_steps_of_several_layers_in_one_graph_advance_device_positions(D, n_split):
    """Four layers' decode steps captured in one HIP graph, each advancing its
    layer's device positions in place (the shape of a captured model step and
    of the bench's timed step), replayed with new inputs copied in between:
    every replay's outputs and the caches equal the same launches made
    eagerly, bit for bit."""
    print(f"graph of 4 decode steps: D {D}, n_split {n_split}", flush=True)
    B, Hq, Hkv, G, cap, fill, steps, nl = 2, 8, 2, 32, 512, 70, 6, 4
    sm = D ** -0.5
    g = torch.Generator(device=DEV).manual_seed(30 + D)
    caches_e = [_cache(B, Hkv, cap, D, G, "bf16", fill, seed=40 + l) for l in range(nl)]
    caches_g = [_cache(B, Hkv, cap, D, G, "bf16", fill, seed=40 + l) for l in range(nl)]
    inp = [[tuple(torch.randn(B, h, 1, D, device=DEV, generator=g).to(torch.bfloat16) for h in (Hq, Hkv, Hkv))
            for _ in range(nl)] for _ in range(steps)]
    kw = dict(n_kv_heads=Hkv, group_size=G, sm_scale=sm, n_split=n_split)
    pos_e = [torch.full((B,), fill, dtype=torch.int32, device=DEV) for _ in range(nl)]
    eager = []
    for i in range(steps):
        row = []
        for l in range(nl):
            row.append(ops.decode_step(*inp[i][l], *caches_e[l], pos_e[l], **kw).clone())
            pos_e[l].add_(1)
        eager.append(row)
    pos_g = [torch.full((B,), fill, dtype=torch.int32, device=DEV) for _ in range(nl)]
    static = [tuple(t.clone() for t in inp[0][l]) for l in range(nl)]
    side = torch.cuda.Stream(DEV)
    side.wait_stream(torch.cuda.current_stream(DEV))
    first = []
    with torch.cuda.stream(side):  # step 0 eagerly on the capture stream (its workspace)
        for l in range(nl):
            first.append(ops.decode_step(*static[l], *caches_g[l], pos_g[l], **kw).clone())
            pos_g[l].add_(1)
    torch.cuda.current_stream(DEV).wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        outs = []
        for l in range(nl):
            outs.append(ops.decode_step(*static[l], *caches_g[l], pos_g[l], **kw))
            pos_g[l].add_(1)
    got = [first]
    junk = torch.randn(256, 256, device=DEV)
    for i in range(1, steps):
        for l in range(nl):
            for dst, src in zip(static[l], inp[i][l]):
                dst.copy_(src)
        graph.replay()
        junk = (junk @ junk).tanh_()
        torch.cuda.synchronize()
        got.append([o.clone() for o in outs])
    for i in range(steps):
        for l in range(nl):
            assert torch.equal(got[i][l], eager[i][l]), (i, l)
    for l in range(nl):
        assert torch.equal(pos_g[l], pos_e[l])
        for a, b in zip(caches_e[l], caches_g[l]):
            assert torch.equal(a, b)


def _random_step_case(seed):
    r = np.random.default_rng(seed)
    xdt = ["bf16", "f16", "f32"][r.integers(3)]
    sdt = ["bf16", "f16", "f32"][r.integers(3)]
    B = int(r.integers(1, 4))
    Hkv = int(r.choice([1, 2, 4, 8]))
    ratio = int(r.choice([1, 2, 4, 8]))
    D = int(r.choice([64, 128]))
    G = int(r.choice([32, 64, 128]))
    cap = int(r.integers(40, 2500))
    pos = [int(r.integers(0, cap)) for _ in range(B)]
    if B > 1 and r.random() < 0.5:
        pos[int(r.integers(B))] = cap  # a full sequence: not written, attends its cap keys
    n_split = None if r.random() < 0.5 else int(r.integers(1, 9))
    return xdt, sdt, B, Hkv, ratio, D, G, cap, pos, n_split


@pytest.mark.parametrize("seed", range(24))
def test_decode_step_random_shapes(seed):
    """Seeded random decode steps over both kernels (query and scale dtypes),
    GQA ratios, head dims, group sizes, per-sequence positions (one may be at
    the capacity) and forced split counts: cache bytes bit-identical to the
    two-launch route, output within its bar, and within the oracle's bar."""
    xdt, sdt, B, Hkv, ratio, D, G, cap, pos, n_split = _random_step_case(seed)
    Hq = Hkv * ratio
    print(f"random decode step {seed}: {xdt}/{sdt} B {B} Hq {Hq} Hkv {Hkv} D {D} G {G} cap {cap} "
          f"pos {pos} n_split {n_split}", flush=True)
    b = _cache_dt(B, Hkv, cap, D, G, xdt, sdt, cap, seed=300 + seed)
    q, kn, vn = _new_dt(B, Hq, Hkv, D, xdt, seed=300 + seed)
    sm = D ** -0.5
    ref = [t.clone() for t in b]
    for i, p in enumerate(pos):
        if p < cap:
            ops.quantize_into(kn[i:i + 1], ref[0][i:i + 1], ref[1][i:i + 1], G, p)
            ops.quantize_into(vn[i:i + 1], ref[2][i:i + 1], ref[3][i:i + 1], G, p)
    pos_t = torch.tensor(pos, dtype=torch.int32, device=DEV)
    lens = torch.clamp(pos_t + 1, max=cap)
    want = ops.fused_decode_attention(q, ref[0], ref[1], ref[2], ref[3], n_kv_heads=Hkv, group_size=G,
                                      is_causal=False, sm_scale=sm, seq_lens=lens)
    if n_split is not None:
        n_split = max(1, min(n_split, cap // 128))
    got = ops.decode_step(q, kn, vn, b[0], b[1], b[2], b[3], pos_t, n_kv_heads=Hkv, group_size=G,
                          sm_scale=sm, n_split=n_split)
    torch.cuda.synchronize()
    for x, y in zip(ref, b):
        assert torch.equal(x, y)
    _close_dt(got, want, xdt)
    tol = 1e-4 if xdt == "f32" else 2e-2
    g = got.float().cpu().numpy()
    for i, n in enumerate(lens.tolist()):
        exact = O.attention_over_quantized(
            q[i:i + 1].float().cpu().numpy(), ref[0][i:i + 1, :, :n].cpu().numpy(),
            ref[1][i:i + 1, :, :n].float().cpu().numpy(), ref[2][i:i + 1, :, :n].cpu().numpy(),
            ref[3][i:i + 1, :, :n].float().cpu().numpy(), group_size=G, scale=sm)
        assert np.abs(g[i:i + 1] - exact).max() <= tol, (i, np.abs(g[i:i + 1] - exact).max())


@pytest.mark.parametrize("xdt,sdt", [("bf16", "bf16"), ("f32", "f32")])
def test_decode_step_negative_position_writes_nothing(xdt, sdt):
    """A negative old length (invalid input from a caller's device state)
    leaves that sequence's cache untouched and yields zeros; the other
    sequences step as usual. Both kernels."""
    print(f"decode step with a negative position: {xdt}/{sdt}", flush=True)
    B, Hq, Hkv, D, G, cap = 2, 8, 2, 128, 32, 300
    b = _cache_dt(B, Hkv, cap, D, G, xdt, sdt, 200, seed=31)
    before = [t.clone() for t in b]
    q, kn, vn = _new_dt(B, Hq, Hkv, D, xdt, seed=31)
    sm = D ** -0.5
    pos = torch.tensor([-3, 150], dtype=torch.int32, device=DEV)
    got = ops.decode_step(q, kn, vn, *b, pos, n_kv_heads=Hkv, group_size=G, sm_scale=sm)
    torch.cuda.synchronize()
    for x, y in zip(b, before):
        assert torch.equal(x[0], y[0])  # sequence 0 untouched
    assert torch.all(got[0] == 0)
    ref = [t[1:].clone() for t in before]
    ops.quantize_into(kn[1:], ref[0], ref[1], G, 150)
    ops.quantize_into(vn[1:], ref[2], ref[3], G, 150)
    for x, y in zip(b, ref):
        assert torch.equal(x[1:], y)
    want = ops.fused_decode_attention(q[1:], *(t[:, :, :151] for t in ref), n_kv_heads=Hkv, group_size=G,
                                      is_causal=False, sm_scale=sm)
    _close_dt(got[1:], want, xdt)
