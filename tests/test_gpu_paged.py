"""GPU: the paged INT4 cache (block pools + block table) against the
contiguous one and the oracle.

The reference has no paged layout (models/llama3/kv_cache.py:30-166 keeps one
tensor per layer); the paged entry points must therefore reproduce exactly
what the contiguous path stores and computes:
  * quantize_into_paged: every row's codes and scales, gathered back through
    the table, equal the oracle's (bit for bit); positions whose page has no
    block are dropped and leave the pool untouched;
  * dequantize_paged: equal to dequantize of the gathered rows (absent pages
    give zeros);
  * fused_decode_attention_paged / decode_step_paged: against the float64
    oracle (max-abs <= 2e-2 after rounding to the output dtype) and against
    the contiguous kernel on the same rows (the paged kernel splits the
    sequence at multiples of 64 keys, so outputs may differ in the last bf16
    bit only);
  * PagedQuantizedKVCache in a tiny Llama: the same logits as QuantizedKVCache,
    ragged sequences, freeing a sequence and reusing its blocks.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
from transformers import LlamaConfig, LlamaForCausalLM

from kvint4 import ops
from kvint4.llama3.kv_cache import QuantizedKVCache
from kvint4.llama3.llama3_quant import replace_llama_attention_with_quantized
from kvint4.paged_cache import PagedQuantizedKVCache
from oracle import kvq_oracle as O

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
TDT = {"bf16": torch.bfloat16, "f16": torch.float16}


def _table(lens, page_size, n_blocks, seed, extra_cols=1):
    """Random distinct blocks for each sequence's pages, -1 past them."""
    rng = np.random.default_rng(seed)
    need = [-(-n // page_size) for n in lens]
    perm = rng.permutation(n_blocks)
    cols = max(need) + extra_cols
    t = np.full((len(lens), cols), -1, dtype=np.int32)
    k = 0
    for b, n in enumerate(need):
        t[b, :n] = perm[k:k + n]
        k += n
    assert k <= n_blocks
    return torch.from_numpy(t).to(DEV)


def _pools(H, n_blocks, page_size, D, G, sdt):
    rows = n_blocks * page_size
    w, ng = ops.packed_width(D, G), ops.num_groups(D, G)
    fill = torch.Generator(device=DEV).manual_seed(123)
    kp = torch.randint(0, 256, (H, rows, w), dtype=torch.uint8, device=DEV, generator=fill)
    vp = torch.randint(0, 256, (H, rows, w), dtype=torch.uint8, device=DEV, generator=fill)
    ks = torch.rand(H, rows, ng, device=DEV, generator=fill).to(sdt)
    vs = torch.rand(H, rows, ng, device=DEV, generator=fill).to(sdt)
    return [kp, ks, vp, vs]


def _gather(pool, table, page_size, S):
    """[B, H, S, .] rows of each sequence's first S positions (absent -> row 0)."""
    t = torch.arange(S, device=DEV)
    page = table[:, t // page_size].to(torch.int64)
    rows = page.clamp(min=0) * page_size + (t % page_size)[None, :]
    return pool[:, rows].permute(1, 0, 2, 3)


def _close_splits(got, want):
    """Same attention computed with different sequence splits (the paged
    kernel splits at multiples of 64 keys and plans on the table's capacity):
    the partials' bf16 weight rounding differs, so a couple of output ulps."""
    g, w = got.float().cpu().numpy(), want.float().cpu().numpy()
    assert np.all(np.abs(g - w) <= 2.0 ** -7 * np.abs(w) + 2.0 ** -7), np.abs(g - w).max()


@pytest.mark.parametrize("page_size", [16, 64, 128])
@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_quantize_paged_matches_oracle_and_drops_unmapped(page_size, dtype):
    B, H, S, D, G = 3, 4, 200, 128, 32
    lens = [150, 200, 37]
    n_blocks = sum(-(-n // page_size) for n in lens) + 5
    table = _table(lens, page_size, n_blocks, seed=page_size)
    pt = ops.PageTable(table, page_size, n_blocks)
    pools = _pools(H, n_blocks, page_size, D, G, TDT[dtype])
    before = [p.clone() for p in pools]
    g = torch.Generator().manual_seed(7)
    x = torch.randn(B, H, S, D, generator=g).to(TDT[dtype])
    # sequence 1 writes at position 10 (rows past 200 - 10 ... beyond its pages are dropped)
    pos = torch.tensor([0, 10, 0], dtype=torch.int32, device=DEV)
    ops.quantize_into_paged(x.to(DEV), pools[0], pools[1], pt, G, pos)
    want_p, want_s = O.quantize_int4(x.float().numpy(), G, dtype)
    got_p = _gather(pools[0], table, page_size, S + 10).cpu().numpy()
    got_s = _gather(pools[1], table, page_size, S + 10).float().cpu().numpy()
    for b, (p0, n) in enumerate([(0, lens[0]), (10, lens[1]), (0, lens[2])]):
        cap = -(-n // page_size) * page_size  # rows with a block
        m = min(S, cap - p0)
        assert np.array_equal(got_p[b, :, p0:p0 + m], want_p[b, :, :m]), b
        assert np.array_equal(O.bits(got_s[b, :, p0:p0 + m], dtype), O.bits(want_s[b, :, :m], dtype)), b
    # blocks no sequence maps are untouched
    mapped = set(table[table >= 0].tolist())
    free = [i for i in range(n_blocks) if i not in mapped]
    for i in free:
        r = slice(i * page_size, (i + 1) * page_size)
        for x_now, x_was in zip(pools, before):
            assert torch.equal(x_now[:, r], x_was[:, r])


def test_dequantize_paged_matches_contiguous():
    B, H, S, D, G, P = 2, 4, 300, 128, 32, 64
    lens = [300, 130]
    n_blocks = 12
    table = _table(lens, P, n_blocks, seed=3)
    pt = ops.PageTable(table, P, n_blocks)
    pools = _pools(H, n_blocks, P, D, G, torch.bfloat16)
    out = ops.dequantize_paged(pools[0], pools[1], pt, B, S, G, D, torch.float32)
    want = ops.dequantize(_gather(pools[0], table, P, S).contiguous(), _gather(pools[1], table, P, S).contiguous(),
                          G, D, torch.float32)
    for b, n in enumerate(lens):
        cap = -(-n // P) * P
        assert torch.equal(out[b, :, :cap], want[b, :, :cap])
        assert torch.all(out[b, :, cap:] == 0)


def test_quantize_dequantize_paged_large_launch():
    """Launches above 256K 8-element chunks take four rows per lane: codes
    through the table against the oracle, dequantize_paged against the
    contiguous dequantize of the gathered rows."""
    B, H, S, D, G, P = 3, 8, 1400, 128, 32, 64
    lens = [1400, 1100, 333]
    assert B * H * S * D // 8 > 256 * 1024
    n_blocks = sum(-(-n // P) for n in lens) + 3
    table = _table(lens, P, n_blocks, seed=41)
    pt = ops.PageTable(table, P, n_blocks)
    pools = _pools(H, n_blocks, P, D, G, torch.bfloat16)
    x = torch.randn(B, H, S, D, generator=torch.Generator().manual_seed(41)).to(torch.bfloat16)
    ops.quantize_into_paged(x.to(DEV), pools[0], pools[1], pt, G, 0)
    want_p, want_s = O.quantize_int4(x.float().numpy(), G, "bf16")
    got_p = _gather(pools[0], table, P, S).cpu().numpy()
    got_s = _gather(pools[1], table, P, S).float().cpu().numpy()
    for b, n in enumerate(lens):
        assert np.array_equal(got_p[b, :, :n], want_p[b, :, :n]), b
        assert np.array_equal(O.bits(got_s[b, :, :n], "bf16"), O.bits(want_s[b, :, :n], "bf16")), b
    out = ops.dequantize_paged(pools[0], pools[1], pt, B, S, G, D, torch.bfloat16)
    want = ops.dequantize(_gather(pools[0], table, P, S).contiguous(), _gather(pools[1], table, P, S).contiguous(),
                          G, D, torch.bfloat16)
    for b, n in enumerate(lens):
        cap = -(-n // P) * P
        assert torch.equal(out[b, :, :cap], want[b, :, :cap]), b
        assert torch.all(out[b, :, cap:] == 0), b


@pytest.mark.parametrize("S", [20, 1100])
def test_table_without_columns_maps_nothing(S):
    """A block table with no columns places no position: the quantizer writes
    nothing and the dequantizer returns zeros (at one and four rows per lane)."""
    B, H, D, G, P, n_blocks = 2, 8, 128, 32, 16, 4
    table = torch.empty((B, 0), dtype=torch.int32, device=DEV)
    pt = ops.PageTable(table, P, n_blocks)
    pools = _pools(H, n_blocks, P, D, G, torch.bfloat16)
    before = [t.clone() for t in pools]
    x = torch.randn(B, H, S, D, generator=torch.Generator().manual_seed(S)).to(torch.bfloat16)
    ops.quantize_into_paged(x.to(DEV), pools[0], pools[1], pt, G, 0)
    torch.cuda.synchronize()
    for now, was in zip(pools, before):
        assert torch.equal(now, was)
    out = ops.dequantize_paged(pools[0], pools[1], pt, B, S, G, D, torch.bfloat16)
    assert out.shape == (B, H, S, D) and torch.all(out == 0)


ATTN_CASES = [
    # B, Hq, Hkv, D, G, page, lens, dtype
    (1, 32, 8, 128, 32, 64, [16385], "bf16"),
    (2, 32, 8, 128, 32, 128, [5000, 777], "bf16"),
    (3, 64, 8, 128, 32, 256, [2048, 1, 999], "bf16"),
    (4, 16, 4, 64, 64, 64, [300, 64, 65, 1024], "f16"),
    (2, 12, 12, 64, 32, 64, [1023, 500], "f16"),
]


@pytest.mark.parametrize("B,Hq,Hkv,D,G,P,lens,dtype", ATTN_CASES)
def test_decode_attention_paged(B, Hq, Hkv, D, G, P, lens, dtype):
    t = TDT[dtype]
    n_blocks = sum(-(-n // P) for n in lens) + 3
    table = _table(lens, P, n_blocks, seed=len(lens) + P)
    pt = ops.PageTable(table, P, n_blocks)
    pools = _pools(Hkv, n_blocks, P, D, G, t)
    S = max(lens)
    g = torch.Generator().manual_seed(S)
    k = torch.randn(B, Hkv, S, D, generator=g).to(t)
    v = torch.randn(B, Hkv, S, D, generator=g).to(t)
    ops.quantize_into_paged(k.to(DEV), pools[0], pools[1], pt, G, 0)
    ops.quantize_into_paged(v.to(DEV), pools[2], pools[3], pt, G, 0)
    q = torch.randn(B, Hq, 1, D, generator=g).to(t).to(DEV)
    sl = torch.tensor(lens, dtype=torch.int32, device=DEV)
    sm = D ** -0.5
    got = ops.fused_decode_attention_paged(q, *pools, pt, n_kv_heads=Hkv, group_size=G, is_causal=False,
                                           sm_scale=sm, seq_lens=sl)
    cont = [_gather(p, table, P, S).contiguous() for p in pools]
    exact = O.attention_over_quantized(q.float().cpu().numpy(), *(c.cpu().numpy() if c.dtype == torch.uint8
                                       else c.float().cpu().numpy() for c in cont),
                                       group_size=G, scale=sm, seq_lens=lens)
    err = np.abs(got.float().cpu().numpy() - O.round_to(exact.astype(np.float32), dtype)).max()
    assert err <= 2e-2, err
    # One split: the paged and contiguous kernels then take the same tiles in
    # the same order, so only the addressing differs and the bits must agree.
    got1 = ops.fused_decode_attention_paged(q, *pools, pt, n_kv_heads=Hkv, group_size=G, is_causal=False,
                                            sm_scale=sm, seq_lens=sl, n_split=1)
    want1 = ops.fused_decode_attention(q, *cont, n_kv_heads=Hkv, group_size=G, is_causal=False, sm_scale=sm,
                                       seq_lens=sl, n_split=1)
    assert torch.equal(got1, want1)
    # uniform length form
    n = min(lens)
    got_u = ops.fused_decode_attention_paged(q, *pools, pt, n_kv_heads=Hkv, group_size=G, is_causal=False,
                                             sm_scale=sm, seq_len=n, n_split=1)
    want_u = ops.fused_decode_attention(q, *(c[:, :, :n] for c in cont), n_kv_heads=Hkv, group_size=G,
                                        is_causal=False, sm_scale=sm, n_split=1)
    assert torch.equal(got_u, want_u)


def test_causal_query_block_paged():
    B, Hq, Hkv, D, G, P, Sq = 2, 8, 2, 128, 32, 64, 5
    lens = [400, 130]
    n_blocks = 12
    table = _table(lens, P, n_blocks, seed=9)
    pt = ops.PageTable(table, P, n_blocks)
    pools = _pools(Hkv, n_blocks, P, D, G, torch.bfloat16)
    g = torch.Generator().manual_seed(1)
    k = torch.randn(B, Hkv, 400, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, Hkv, 400, D, generator=g).to(torch.bfloat16)
    ops.quantize_into_paged(k.to(DEV), pools[0], pools[1], pt, G, 0)
    ops.quantize_into_paged(v.to(DEV), pools[2], pools[3], pt, G, 0)
    q = torch.randn(B, Hq, Sq, D, generator=g).to(torch.bfloat16).to(DEV)
    sl = torch.tensor(lens, dtype=torch.int32, device=DEV)
    got = ops.fused_decode_attention_paged(q, *pools, pt, n_kv_heads=Hkv, group_size=G, is_causal=True,
                                           sm_scale=D ** -0.5, seq_lens=sl)
    cont = [_gather(p, table, P, 400).contiguous() for p in pools]
    exact = O.attention_over_quantized(q.float().cpu().numpy(), cont[0].cpu().numpy(), cont[1].float().cpu().numpy(),
                                       cont[2].cpu().numpy(), cont[3].float().cpu().numpy(), group_size=G,
                                       is_causal=True, seq_lens=lens)
    err = np.abs(got.float().cpu().numpy() - O.round_to(exact.astype(np.float32), "bf16")).max()
    assert err <= 2e-2, err


@pytest.mark.parametrize("P", [64, 128])
def test_decode_step_paged_matches_contiguous(P):
    B, Hq, Hkv, D, G = 3, 32, 8, 128, 32
    lens = [1000, 63, 4097]
    n_blocks = sum(-(-(n + 1) // P) for n in lens) + 2
    table = _table([n + 1 for n in lens], P, n_blocks, seed=P)
    pt = ops.PageTable(table, P, n_blocks)
    pools = _pools(Hkv, n_blocks, P, D, G, torch.bfloat16)
    S = max(lens)
    g = torch.Generator().manual_seed(11)
    k = torch.randn(B, Hkv, S, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, Hkv, S, D, generator=g).to(torch.bfloat16)
    ops.quantize_into_paged(k.to(DEV), pools[0], pools[1], pt, G, 0)
    ops.quantize_into_paged(v.to(DEV), pools[2], pools[3], pt, G, 0)
    q = torch.randn(B, Hq, 1, D, generator=g).to(torch.bfloat16).to(DEV)
    kn = (3 * torch.randn(B, Hkv, 1, D, generator=g)).to(torch.bfloat16).to(DEV)
    vn = torch.randn(B, Hkv, 1, D, generator=g).to(torch.bfloat16).to(DEV)
    pos = torch.tensor(lens, dtype=torch.int32, device=DEV)
    got = ops.decode_step_paged(q, kn, vn, *pools, pt, pos, n_kv_heads=Hkv, group_size=G, sm_scale=D ** -0.5)
    # the new rows, gathered back, are the quantizer's
    want_kp, want_ks = O.quantize_int4(kn.float().cpu().numpy(), G, "bf16")
    want_vp, want_vs = O.quantize_int4(vn.float().cpu().numpy(), G, "bf16")
    cont = [_gather(p, table, P, S + 1).contiguous() for p in pools]
    for b, n in enumerate(lens):
        assert np.array_equal(cont[0][b, :, n].cpu().numpy(), want_kp[b, :, 0])
        assert np.array_equal(cont[2][b, :, n].cpu().numpy(), want_vp[b, :, 0])
        assert np.array_equal(O.bits(cont[1][b, :, n].float().cpu().numpy(), "bf16"), O.bits(want_ks[b, :, 0], "bf16"))
        assert np.array_equal(O.bits(cont[3][b, :, n].float().cpu().numpy(), "bf16"), O.bits(want_vs[b, :, 0], "bf16"))
    new_lens = [n + 1 for n in lens]
    want = ops.fused_decode_attention(q, *cont, n_kv_heads=Hkv, group_size=G, is_causal=False,
                                      sm_scale=D ** -0.5, seq_lens=torch.tensor(new_lens, dtype=torch.int32, device=DEV))
    g_np, w_np = got.float().cpu().numpy(), want.float().cpu().numpy()
    # the new key is folded in fp32, the cached ones through bf16 weights
    assert np.all(np.abs(g_np - w_np) <= 2.0 ** -6 + 2.0 ** -7 * np.abs(w_np)), np.abs(g_np - w_np).max()


def _tiny_llama():
    cfg = LlamaConfig(vocab_size=256, hidden_size=128, intermediate_size=256, num_hidden_layers=2,
                      num_attention_heads=8, num_key_value_heads=2, head_dim=64,
                      max_position_embeddings=1024, rms_norm_eps=1e-5, tie_word_embeddings=False)
    torch.manual_seed(0)
    m = LlamaForCausalLM(cfg).to(dtype=torch.bfloat16).eval()
    replace_llama_attention_with_quantized(m, group_size=32)
    return m.to(DEV)


def test_paged_cache_in_llama_matches_contiguous_cache():
    model = _tiny_llama()
    torch.manual_seed(5)
    prompt = torch.randint(0, 256, (2, 150), device=DEV)
    with torch.no_grad():
        cc, pc = QuantizedKVCache(group_size=32), PagedQuantizedKVCache(group_size=32, page_size=64)
        lc = model(input_ids=prompt, past_key_values=cc, use_cache=True).logits[:, -1].float()
        lp = model(input_ids=prompt, past_key_values=pc, use_cache=True).logits[:, -1].float()
        assert (lc - lp).abs().max().item() < 2e-2
        for _ in range(70):  # crosses page boundaries (block allocation mid-run)
            nid = lc.argmax(-1, keepdim=True)
            lc = model(input_ids=nid, past_key_values=cc, use_cache=True).logits[:, -1].float()
            lp = model(input_ids=nid, past_key_values=pc, use_cache=True).logits[:, -1].float()
            assert (lc - lp).abs().max().item() < 5e-2
    assert pc.get_seq_length(0) == cc.get_seq_length(0) == 220
    # layer 0's K/V come from the embeddings alone: the same codes in both caches
    for x, y in zip(pc.get_quantized(0), cc.get_quantized(0)):
        assert torch.equal(x, y)
    assert pc.nbytes() == cc.nbytes()


def test_paged_cache_ragged_free_and_reuse():
    B, Hq, Hkv, D, G = 3, 16, 4, 128, 32
    g = torch.Generator().manual_seed(2)
    k0 = torch.randn(B, Hkv, 300, D, generator=g).to(torch.bfloat16).to(DEV)
    v0 = torch.randn(B, Hkv, 300, D, generator=g).to(torch.bfloat16).to(DEV)
    lens = torch.tensor([300, 70, 129], dtype=torch.int32)
    pc = PagedQuantizedKVCache(group_size=G, page_size=64)
    pc.load_ragged(k0, v0, 0, lens)
    cc = QuantizedKVCache(group_size=G)
    cc.load_ragged(k0, v0, 0, lens)
    for step in range(3):
        q = torch.randn(B, Hq, 1, D, generator=g).to(torch.bfloat16).to(DEV)
        kn = torch.randn(B, Hkv, 1, D, generator=g).to(torch.bfloat16).to(DEV)
        vn = torch.randn(B, Hkv, 1, D, generator=g).to(torch.bfloat16).to(DEV)
        got = pc.append_and_attend(q, kn, vn, 0, n_kv_heads=Hkv, scale=D ** -0.5)
        want = cc.append_and_attend(q, kn, vn, 0, n_kv_heads=Hkv, scale=D ** -0.5)
        assert got is not None and want is not None
        _close_splits(got, want)
        parts = [t.cpu() for t in pc.get_quantized(0)]
        exact = O.attention_over_quantized(q.float().cpu().numpy(), parts[0].numpy(), parts[1].float().numpy(),
                                           parts[2].numpy(), parts[3].float().numpy(), group_size=G,
                                           scale=D ** -0.5, seq_lens=pc.get_seq_lens(0).tolist())
        assert np.abs(got.float().cpu().numpy() - exact).max() <= 2e-2
    assert pc.get_seq_lens(0).tolist() == [303, 73, 132]
    # free sequence 1 and start a new one in its slot: its blocks are reused
    used_before = pc._num_blocks - len(pc._free)
    pc.free_sequence(1)
    assert pc._num_blocks - len(pc._free) == used_before - 2
    kx = torch.randn(B, Hkv, 1, D, generator=g).to(torch.bfloat16).to(DEV)
    pc.append(kx, kx, 0)
    assert pc.get_seq_lens(0).tolist() == [304, 1, 133]
    kp, ks, _, _ = pc.get_quantized(0)
    want_p, _ = O.quantize_int4(kx[1:2].float().cpu().numpy(), G, "bf16")
    assert np.array_equal(kp[1, :, 0].cpu().numpy(), want_p[0, :, 0])
    # attention of the fresh sequence sees only its one key: the output is that value
    q = torch.randn(B, Hq, 1, D, generator=g).to(torch.bfloat16).to(DEV)
    out = pc.attend(q, 0, n_kv_heads=Hkv, scale=D ** -0.5, is_causal=False)
    deq = ops.dequantize(kp[1:2, :, :1].contiguous(), ks[1:2, :, :1].contiguous(), G, D, torch.float32)
    want_v = deq.repeat_interleave(Hq // Hkv, dim=1)[0, :, 0]
    assert (out[1, :, 0].float() - want_v).abs().max().item() <= 2e-2


def test_paged_attend_small_pages_use_dense_route():
    """Pages below 64 rows take dequantize + dense SDPA (the fused kernel needs
    a 64-key tile inside one page); the result is the same attention."""
    B, Hq, Hkv, D, G = 2, 8, 2, 128, 32
    g = torch.Generator().manual_seed(4)
    k = torch.randn(B, Hkv, 90, D, generator=g).to(torch.bfloat16).to(DEV)
    v = torch.randn(B, Hkv, 90, D, generator=g).to(torch.bfloat16).to(DEV)
    pc = PagedQuantizedKVCache(group_size=G, page_size=16)
    pc.append(k, v, 0)
    q = torch.randn(B, Hq, 1, D, generator=g).to(torch.bfloat16).to(DEV)
    out = pc.attend(q, 0, n_kv_heads=Hkv, scale=D ** -0.5, is_causal=False)
    kp, ks, vp, vs = pc.get_quantized(0)
    exact = O.attention_over_quantized(q.float().cpu().numpy(), kp.cpu().numpy(), ks.float().cpu().numpy(),
                                       vp.cpu().numpy(), vs.float().cpu().numpy(), group_size=G)
    assert np.abs(out.float().cpu().numpy() - exact).max() <= 2e-2


@pytest.mark.parametrize("B,Hq,Hkv,Sq,S,P", [(2, 8, 2, 300, 700, 64), (2, 32, 8, 2048, 2500, 128),
                                             (1, 8, 2, 100, 2000, 64)])
def test_prefill_kernel_paged_matches_contiguous(B, Hq, Hkv, Sq, S, P):
    """The matrix-core prefill kernel through a block table (one and two row
    blocks per wave; the second case takes eight waves per workgroup) reads
    the same keys in the same 64-key tiles as on the contiguous cache:
    bit-identical outputs."""
    D, G = 128, 32
    lens = [S] * B
    n_blocks = sum(-(-n // P) for n in lens) + 3
    table = _table(lens, P, n_blocks, seed=P + Sq)
    pt = ops.PageTable(table, P, n_blocks)
    pools = _pools(Hkv, n_blocks, P, D, G, torch.bfloat16)
    g = torch.Generator().manual_seed(Sq)
    k = torch.randn(B, Hkv, S, D, generator=g).to(torch.bfloat16).to(DEV)
    v = torch.randn(B, Hkv, S, D, generator=g).to(torch.bfloat16).to(DEV)
    ops.quantize_into_paged(k, pools[0], pools[1], pt, G, 0)
    ops.quantize_into_paged(v, pools[2], pools[3], pt, G, 0)
    q = torch.randn(B, Hq, Sq, D, generator=g).to(torch.bfloat16).to(DEV)
    got = ops.prefill_attention_paged(q, *pools, pt, S, n_kv_heads=Hkv, group_size=G, is_causal=True,
                                      sm_scale=D ** -0.5)
    kp, ks, vp, vs = (_gather(p, table, P, S).contiguous() for p in pools)
    want = ops.prefill_attention(q, kp, ks, vp, vs, n_kv_heads=Hkv, group_size=G, is_causal=True,
                                 sm_scale=D ** -0.5)
    assert torch.equal(got, want)
    # and the paged cache routes a long block of one length to it
    cache = PagedQuantizedKVCache(group_size=G, page_size=P)
    cache.append(k, v, 0)
    out = cache.attend(q, 0, n_kv_heads=Hkv, scale=D ** -0.5, is_causal=True)
    assert (out.float() - want.float()).abs().max().item() <= 2e-2


def _random_paged_case(seed):
    r = np.random.default_rng(3000 + seed)
    dtype = ["bf16", "f16"][r.integers(2)]
    B = int(r.integers(1, 4))
    Hkv = int(r.choice([1, 2, 4, 8]))
    ratio = int(r.choice([1, 2, 4, 8]))
    D = int(r.choice([64, 128]))
    G = int(r.choice([32, 64, 128]))
    P = int(r.choice([64, 128, 256]))
    lens = [int(r.integers(1, 1500)) for _ in range(B)]
    Sq = int(r.choice([1, 1, 2, 4]))
    causal = Sq > 1 and bool(r.random() < 0.5)
    return dtype, B, Hkv, ratio, D, G, P, lens, Sq, causal


@pytest.mark.parametrize("seed", range(16))
def test_paged_random_shapes(seed):
    """Seeded random paged caches (page sizes 64-256, permuted block tables,
    ragged lengths, GQA ratios, D, G, query blocks with and without the causal
    mask): attention within 2e-2 of the oracle; at one split bit-identical to
    the contiguous kernel over the gathered rows; for one-token queries the
    paged decode step writes the quantizer's bytes and matches the
    contiguous step."""
    dtype, B, Hkv, ratio, D, G, P, lens, Sq, causal = _random_paged_case(seed)
    Hq = Hkv * ratio
    print(f"random paged {seed}: {dtype} B {B} Hq {Hq} Hkv {Hkv} D {D} G {G} P {P} lens {lens} Sq {Sq} "
          f"causal {causal}", flush=True)
    t = TDT[dtype]
    n_blocks = sum(-(-(n + 1) // P) for n in lens) + 2
    table = _table([n + 1 for n in lens], P, n_blocks, seed=4000 + seed)
    pt = ops.PageTable(table, P, n_blocks)
    pools = _pools(Hkv, n_blocks, P, D, G, t)
    S = max(lens)
    g = torch.Generator().manual_seed(5000 + seed)
    k = torch.randn(B, Hkv, S, D, generator=g).to(t)
    v = torch.randn(B, Hkv, S, D, generator=g).to(t)
    ops.quantize_into_paged(k.to(DEV), pools[0], pools[1], pt, G, 0)
    ops.quantize_into_paged(v.to(DEV), pools[2], pools[3], pt, G, 0)
    q = torch.randn(B, Hq, Sq, D, generator=g).to(t).to(DEV)
    sl = torch.tensor(lens, dtype=torch.int32, device=DEV)
    sm = D ** -0.5
    got = ops.fused_decode_attention_paged(q, *pools, pt, n_kv_heads=Hkv, group_size=G, is_causal=causal,
                                           sm_scale=sm, seq_lens=sl)
    cont = [_gather(p, table, P, S).contiguous() for p in pools]
    exact = O.attention_over_quantized(q.float().cpu().numpy(), *(c.cpu().numpy() if c.dtype == torch.uint8
                                       else c.float().cpu().numpy() for c in cont),
                                       group_size=G, scale=sm, is_causal=causal, seq_lens=lens)
    err = np.abs(got.float().cpu().numpy() - O.round_to(exact.astype(np.float32), dtype)).max()
    assert err <= 2e-2, err
    got1 = ops.fused_decode_attention_paged(q, *pools, pt, n_kv_heads=Hkv, group_size=G, is_causal=causal,
                                            sm_scale=sm, seq_lens=sl, n_split=1)
    want1 = ops.fused_decode_attention(q, *cont, n_kv_heads=Hkv, group_size=G, is_causal=causal, sm_scale=sm,
                                       seq_lens=sl, n_split=1)
    assert torch.equal(got1, want1)
    if Sq != 1:
        return
    kn = (3 * torch.randn(B, Hkv, 1, D, generator=g)).to(t).to(DEV)
    vn = torch.randn(B, Hkv, 1, D, generator=g).to(t).to(DEV)
    got_s = ops.decode_step_paged(q, kn, vn, *pools, pt, sl, n_kv_heads=Hkv, group_size=G, sm_scale=sm)
    want_kp, want_ks = O.quantize_int4(kn.float().cpu().numpy(), G, dtype)
    want_vp, want_vs = O.quantize_int4(vn.float().cpu().numpy(), G, dtype)
    cont = [_gather(p, table, P, S + 1).contiguous() for p in pools]
    for b, n in enumerate(lens):
        assert np.array_equal(cont[0][b, :, n].cpu().numpy(), want_kp[b, :, 0])
        assert np.array_equal(cont[2][b, :, n].cpu().numpy(), want_vp[b, :, 0])
        assert np.array_equal(O.bits(cont[1][b, :, n].float().cpu().numpy(), dtype), O.bits(want_ks[b, :, 0], dtype))
        assert np.array_equal(O.bits(cont[3][b, :, n].float().cpu().numpy(), dtype), O.bits(want_vs[b, :, 0], dtype))
    want_s = ops.fused_decode_attention(q, *cont, n_kv_heads=Hkv, group_size=G, is_causal=False, sm_scale=sm,
                                        seq_lens=sl + 1)
    g_np, w_np = got_s.float().cpu().numpy(), want_s.float().cpu().numpy()
    assert np.all(np.abs(g_np - w_np) <= 2.0 ** -6 + 2.0 ** -7 * np.abs(w_np)), np.abs(g_np - w_np).max()


def test_paged_cache_fp32_matches_contiguous_cache():
    """fp32 activations (GPT-2-style exact path) in the paged cache: ragged
    sequences, three fused decode steps, each within 1e-4 of the contiguous
    cache's fused fp32 step and of the float64 oracle."""
    print("paged cache, fp32 activations", flush=True)
    B, Hq, Hkv, D, G = 3, 12, 12, 64, 32
    g = torch.Generator().manual_seed(6)
    k0 = torch.randn(B, Hkv, 400, D, generator=g).to(DEV)
    v0 = torch.randn(B, Hkv, 400, D, generator=g).to(DEV)
    lens = torch.tensor([400, 90, 257], dtype=torch.int32)
    pc = PagedQuantizedKVCache(group_size=G, page_size=64)
    pc.load_ragged(k0, v0, 0, lens)
    cc = QuantizedKVCache(group_size=G)
    cc.load_ragged(k0, v0, 0, lens)
    sm = D ** -0.5
    for step in range(3):
        q = torch.randn(B, Hq, 1, D, generator=g).to(DEV)
        kn = torch.randn(B, Hkv, 1, D, generator=g).to(DEV)
        vn = torch.randn(B, Hkv, 1, D, generator=g).to(DEV)
        got = pc.append_and_attend(q, kn, vn, 0, n_kv_heads=Hkv, scale=sm)
        assert got is not None  # the paged fp32 decode step (one launch)
        want = cc.append_and_attend(q, kn, vn, 0, n_kv_heads=Hkv, scale=sm)
        assert want is not None
        g_np, w_np = got.cpu().numpy(), want.cpu().numpy()
        assert np.abs(g_np - w_np).max() <= 1e-4
        parts = [t.cpu() for t in pc.get_quantized(0)]
        exact = O.attention_over_quantized(q.cpu().numpy(), parts[0].numpy(), parts[1].numpy(), parts[2].numpy(),
                                           parts[3].numpy(), group_size=G, scale=sm,
                                           seq_lens=pc.get_seq_lens(0).tolist())
        assert np.abs(g_np - exact).max() <= 1e-4
    assert pc.get_seq_lens(0).tolist() == [403, 93, 260]



TDT32 = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}


@pytest.mark.parametrize("xdt,sdt,B,Hq,Hkv,D,G,P,lens", [
    ("f32", "f32", 2, 12, 12, 64, 32, 64, [1000, 130]),
    ("f32", "f16", 3, 32, 8, 128, 64, 128, [700, 1, 2049]),
    ("bf16", "f32", 2, 16, 4, 128, 32, 64, [333, 900]),
    ("f32", "bf16", 1, 8, 2, 64, 128, 256, [600]),
])
def test_fp32_kernel_paged_matches_contiguous(xdt, sdt, B, Hq, Hkv, D, G, P, lens):
    """The exact-fp32 kernel over a paged cache (fp32 queries or fp32
    scales): at one split bit-identical to the contiguous kernel over the
    gathered rows, at the planner's splits within its bar of the oracle; the
    paged decode step writes the quantizer's bytes through the table and
    matches the contiguous step."""
    print(f"fp32 kernel, paged: {xdt}/{sdt} B {B} Hq {Hq} Hkv {Hkv} D {D} G {G} P {P} lens {lens}", flush=True)
    t, st = TDT32[xdt], TDT32[sdt]
    n_blocks = sum(-(-(n + 1) // P) for n in lens) + 2
    table = _table([n + 1 for n in lens], P, n_blocks, seed=P + len(lens))
    pt = ops.PageTable(table, P, n_blocks)
    pools = _pools(Hkv, n_blocks, P, D, G, st)
    S = max(lens)
    g = torch.Generator().manual_seed(S + D)
    k = torch.randn(B, Hkv, S, D, generator=g).to(t)
    v = torch.randn(B, Hkv, S, D, generator=g).to(t)
    ops.quantize_into_paged(k.to(DEV), pools[0], pools[1], pt, G, 0)
    ops.quantize_into_paged(v.to(DEV), pools[2], pools[3], pt, G, 0)
    q = torch.randn(B, Hq, 1, D, generator=g).to(t).to(DEV)
    sl = torch.tensor(lens, dtype=torch.int32, device=DEV)
    sm = D ** -0.5
    cont = [_gather(p, table, P, S).contiguous() for p in pools]
    got1 = ops.fused_decode_attention_paged(q, *pools, pt, n_kv_heads=Hkv, group_size=G, is_causal=False,
                                            sm_scale=sm, seq_lens=sl, n_split=1)
    want1 = ops.fused_decode_attention(q, *cont, n_kv_heads=Hkv, group_size=G, is_causal=False, sm_scale=sm,
                                       seq_lens=sl, n_split=1)
    assert torch.equal(got1, want1)
    got = ops.fused_decode_attention_paged(q, *pools, pt, n_kv_heads=Hkv, group_size=G, is_causal=False,
                                           sm_scale=sm, seq_lens=sl)
    exact = O.attention_over_quantized(q.float().cpu().numpy(), *(c.cpu().numpy() if c.dtype == torch.uint8
                                       else c.float().cpu().numpy() for c in cont),
                                       group_size=G, scale=sm, seq_lens=lens)
    tol = 1e-4 if xdt == "f32" else 2e-2
    assert np.abs(got.float().cpu().numpy() - exact).max() <= tol
    # the paged decode step
    kn = (3 * torch.randn(B, Hkv, 1, D, generator=g)).to(t).to(DEV)
    vn = torch.randn(B, Hkv, 1, D, generator=g).to(t).to(DEV)
    got_s = ops.decode_step_paged(q, kn, vn, *pools, pt, sl, n_kv_heads=Hkv, group_size=G, sm_scale=sm)
    want_kp, want_ks = O.quantize_int4(kn.float().cpu().numpy(), G, sdt)
    want_vp, want_vs = O.quantize_int4(vn.float().cpu().numpy(), G, sdt)
    cont = [_gather(p, table, P, S + 1).contiguous() for p in pools]
    for b, n in enumerate(lens):
        assert np.array_equal(cont[0][b, :, n].cpu().numpy(), want_kp[b, :, 0])
        assert np.array_equal(cont[2][b, :, n].cpu().numpy(), want_vp[b, :, 0])
        assert np.array_equal(O.bits(cont[1][b, :, n].float().cpu().numpy(), sdt), O.bits(want_ks[b, :, 0], sdt))
        assert np.array_equal(O.bits(cont[3][b, :, n].float().cpu().numpy(), sdt), O.bits(want_vs[b, :, 0], sdt))
    want_s = ops.fused_decode_attention(q, *cont, n_kv_heads=Hkv, group_size=G, is_causal=False, sm_scale=sm,
                                        seq_lens=sl + 1)
    g_np, w_np = got_s.float().cpu().numpy(), want_s.float().cpu().numpy()
    if xdt == "f32":
        assert np.abs(g_np - w_np).max() <= 1e-4 + 1e-4 * np.abs(w_np).max()
    else:
        assert np.all(np.abs(g_np - w_np) <= 2.0 ** -6 + 2.0 ** -7 * np.abs(w_np)), np.abs(g_np - w_np).max()
