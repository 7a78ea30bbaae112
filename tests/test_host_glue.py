"""Host logic of the cache and the HF glue, on the CPU.

The native ops are replaced, inside this test only, by fakes built on the CPU
oracle (a fake backend, as the reference's tests mock kernel calls with
unittest.mock — tests/gpt2/test_gpt2_triton_routing.py:33-37). This checks
that transformers 5.x drives the cache protocol and the swapped attention
modules as expected (call counts, routing, shapes, positions) without a GPU.
The product path itself has no CPU implementation: without the fakes, CPU
tensors raise ValueError.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
from transformers import GPT2Config, GPT2LMHeadModel, LlamaConfig, LlamaForCausalLM
from transformers.cache_utils import DynamicCache

import kvint4.gpt2.gpt2_quant as g2q
import kvint4.llama3.llama3_quant as l3q
from kvint4 import cache_base, ops
from kvint4.gpt2.kv_cache import QuantizedKVCache as GPT2Cache
from kvint4.llama3.attention_quant import attention_forward_quant_gqa
from kvint4.llama3.kv_cache import QuantizedKVCache, _LayerQuantizedKV
from oracle import kvq_oracle as O

_NP = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}


class FakeBackend:
    def __init__(self):
        self.calls = {"quantize_into": 0, "attention": 0, "dequantize": 0}

    def quantize_into(self, x, packed, scales, group_size, write_pos=0):
        self.calls["quantize_into"] += 1
        p, s = O.quantize_int4(x.float().numpy(), group_size, _NP[scales.dtype])
        S = x.shape[2]
        if isinstance(write_pos, torch.Tensor):
            for b, p0 in enumerate(write_pos.tolist()):
                packed[b, :, p0:p0 + S] = torch.from_numpy(p[b])
                scales[b, :, p0:p0 + S] = torch.from_numpy(s[b]).to(scales.dtype)
        else:
            packed[:, :, write_pos:write_pos + S] = torch.from_numpy(p)
            scales[:, :, write_pos:write_pos + S] = torch.from_numpy(s).to(scales.dtype)

    def dequantize(self, packed, scales, group_size, d_out, out_dtype):
        self.calls["dequantize"] += 1
        out = O.dequantize_int4(packed.numpy(), scales.float().numpy(), group_size, d_out, _NP[out_dtype])
        return torch.from_numpy(out).to(out_dtype)

    def attention(self, q, kp, ks, vp, vs, *, n_q_heads, n_kv_heads, group_size=32, is_causal=False,
                  scale=None, seq_lens=None):
        self.calls["attention"] += 1
        out = O.attention_over_quantized(q.float().numpy(), kp.numpy(), ks.float().numpy(), vp.numpy(),
                                         vs.float().numpy(), group_size=group_size, scale=scale,
                                         is_causal=is_causal,
                                         seq_lens=None if seq_lens is None else seq_lens.tolist())
        return torch.from_numpy(out.astype(np.float32)).to(q.dtype)


@pytest.fixture
def fake(monkeypatch):
    fb = FakeBackend()
    monkeypatch.setattr(ops, "quantize_into", fb.quantize_into)
    monkeypatch.setattr(ops, "dequantize", fb.dequantize)
    monkeypatch.setattr(l3q, "attention_forward_quant_gqa", fb.attention)

    def gpt2_attn(q, kp, ks, vp, vs, *, group_size=32, is_causal=False, scale=None, seq_lens=None):
        return fb.attention(q, kp, ks, vp, vs, n_q_heads=q.shape[1], n_kv_heads=q.shape[1],
                            group_size=group_size, is_causal=is_causal, scale=scale, seq_lens=seq_lens)

    monkeypatch.setattr(g2q, "attention_forward_quant", gpt2_attn)
    return fb


def _tiny_llama():
    cfg = LlamaConfig(vocab_size=256, hidden_size=128, intermediate_size=256, num_hidden_layers=2,
                      num_attention_heads=8, num_key_value_heads=2, head_dim=64,
                      max_position_embeddings=512, tie_word_embeddings=False)
    torch.manual_seed(0)
    return LlamaForCausalLM(cfg).eval()


def test_llama_glue_routing_and_logits(fake):
    ref = _tiny_llama()
    quant = _tiny_llama()
    quant.load_state_dict(ref.state_dict())
    l3q.replace_llama_attention_with_quantized(quant, group_size=32)
    l3q.replace_llama_attention_with_quantized(quant, group_size=64)  # idempotent: only updates G
    assert all(l.self_attn.quant_group_size == 64 for l in quant.model.layers)
    l3q.replace_llama_attention_with_quantized(quant, group_size=32)
    assert quant.model.layers[0].self_attn.q_proj.weight is not None
    prompt = torch.randint(0, 256, (1, 12), generator=torch.Generator().manual_seed(1))
    with torch.no_grad():
        cr, cq = DynamicCache(), QuantizedKVCache()
        lr = ref(input_ids=prompt, past_key_values=cr, use_cache=True).logits[:, -1]
        lq = quant(input_ids=prompt, past_key_values=cq, use_cache=True).logits[:, -1]
        assert fake.calls["attention"] == 2 and fake.calls["quantize_into"] == 4
        assert (lr - lq).abs().max() < 1.0
        for _ in range(3):
            nid = torch.randint(0, 256, (1, 1))
            ref(input_ids=nid, past_key_values=cr, use_cache=True)
            quant(input_ids=nid, past_key_values=cq, use_cache=True)
    assert fake.calls["attention"] == 8
    assert cq.get_seq_length(0) == 15 and cq.get_seq_length(1) == 15


def test_llama_masked_input_takes_dequant_path(fake):
    model = _tiny_llama()
    l3q.replace_llama_attention_with_quantized(model)
    ids = torch.randint(0, 256, (2, 6), generator=torch.Generator().manual_seed(2))
    mask = torch.ones(2, 6, dtype=torch.long)
    mask[0, :2] = 0  # left padding -> a real mask reaches attention
    with torch.no_grad():
        model(input_ids=ids, attention_mask=mask, past_key_values=QuantizedKVCache(), use_cache=True)
    assert fake.calls["attention"] == 0 and fake.calls["dequantize"] == 4


def test_gpt2_glue_routing(fake):
    cfg = GPT2Config(n_layer=2, n_head=4, n_embd=64, vocab_size=128, n_positions=64)
    torch.manual_seed(0)
    ref = GPT2LMHeadModel(cfg).eval()
    quant = GPT2LMHeadModel(cfg).eval()
    quant.load_state_dict(ref.state_dict())
    g2q.replace_gpt2_attention_with_quantized(quant)
    prompt = torch.randint(0, 128, (1, 9), generator=torch.Generator().manual_seed(3))
    with torch.no_grad():
        cr, cq = DynamicCache(), GPT2Cache()
        lr = ref(input_ids=prompt, past_key_values=cr, use_cache=True).logits[:, -1]
        lq = quant(input_ids=prompt, past_key_values=cq, use_cache=True).logits[:, -1]
        assert (lr - lq).abs().max() < 1.0
        nid = torch.randint(0, 128, (1, 1))
        ref(input_ids=nid, past_key_values=cr, use_cache=True)
        quant(input_ids=nid, past_key_values=cq, use_cache=True)
    assert fake.calls["attention"] == 4
    assert cq.get_seq_length(1) == 10
    assert cq.get_quantized(0)[1].dtype == torch.float16


def test_cache_storage_accounting_matches_reference():
    # tests/gpt2/test_kv_cache_metrics.py:26-41
    cache = GPT2Cache(group_size=32)
    k_p = torch.zeros(1, 2, 3, 8, dtype=torch.uint8)
    k_s = torch.zeros(1, 2, 3, 2, dtype=torch.float16)
    v_p = torch.ones(1, 2, 3, 8, dtype=torch.uint8)
    v_s = torch.ones(1, 2, 3, 2, dtype=torch.float16)
    cache._layers[0] = _LayerQuantizedKV(k_packed=k_p, k_scales=k_s, v_packed=v_p, v_scales=v_s, seq_len=3)
    assert cache.nbytes() == sum(t.element_size() * t.numel() for t in (k_p, k_s, v_p, v_s))


def test_cache_protocol_without_kernels():
    c = QuantizedKVCache()
    assert c.get_seq_length() == 0 and c.get_query_offset() == 0
    assert c.get_mask_sizes(4, 0) == (4, 0) and c.get_mask_sizes(torch.tensor(4), 0) == (4, 0)
    assert c.is_sliding == [] and not c.is_initialized and c.is_compileable is False
    with pytest.raises(ValueError):
        QuantizedKVCache(group_size=0)
    with pytest.raises(KeyError):
        c.get_quantized(0)


def test_cpu_tensors_are_rejected_by_the_product_path():
    q = torch.randn(1, 8, 1, 128)
    kp = torch.zeros(1, 2, 4, 64, dtype=torch.uint8)
    ks = torch.ones(1, 2, 4, 4)
    with pytest.raises(ValueError, match="CUDA"):
        attention_forward_quant_gqa(q, kp, ks, kp, ks, n_q_heads=8, n_kv_heads=2)
    with pytest.raises(ValueError, match="GPU"):
        ops.quantize(torch.randn(2, 64), 32, torch.float32)
    with pytest.raises(ValueError):
        cache_base.QuantizedKVCacheBase(group_size=-1)


def test_make_static_reserves_room_and_moves_lengths_to_device_tensors():
    c = QuantizedKVCache()
    with pytest.raises(ValueError):
        c.make_static(4)
    for i, n in ((0, 5), (1, 5)):
        c._layers[i] = _LayerQuantizedKV(
            k_packed=torch.arange(2 * 2 * 8 * 4, dtype=torch.uint8).view(2, 2, 8, 4),
            k_scales=torch.ones(2, 2, 8, 1, dtype=torch.bfloat16),
            v_packed=torch.full((2, 2, 8, 4), 7, dtype=torch.uint8),
            v_scales=torch.ones(2, 2, 8, 1, dtype=torch.bfloat16), seq_len=n)
    before = c.get_quantized(0)
    before = [t.clone() for t in before]
    assert c.room() == 3
    c.make_static(300)
    assert c.room() >= 300 and c._layers[0].capacity % 256 == 0
    for a, b in zip(before, c.get_quantized(0)):  # the stored rows moved with the growth
        assert torch.equal(a, b)
    assert c.get_seq_lens(1).dtype == torch.int32 and c.get_seq_lens(1).tolist() == [5, 5]
    base = c.host_lengths()
    c.advance_host_lengths(base, 3)
    assert c.get_seq_length(0) == 8 and c.get_seq_length(1) == 8
    with pytest.raises(ValueError):
        c.make_static(-1)


def test_graph_decoder_rejects_unswapped_models_and_other_caches():
    from kvint4.llama3.graph_decode import GraphedGreedyDecoder
    from kvint4.paged_cache import PagedQuantizedKVCache

    cfg = LlamaConfig(vocab_size=64, hidden_size=64, intermediate_size=128, num_hidden_layers=1,
                      num_attention_heads=2, num_key_value_heads=1)
    model = LlamaForCausalLM(cfg)
    tok = torch.zeros(1, 1, dtype=torch.int64)
    with pytest.raises(ValueError, match="replace_llama_attention_with_quantized"):
        GraphedGreedyDecoder(model, QuantizedKVCache(), tok, max_new_tokens=4)
    with pytest.raises(TypeError):
        GraphedGreedyDecoder(model, object(), tok, max_new_tokens=4)
    del PagedQuantizedKVCache


def test_graph_decoder_replay_checks_buffers_and_lengths():
    """step() replays only while the cache holds the captured buffers and the
    lengths the previous replays left; a crop keeps the buffers but moves the
    lengths and must stop the replay before it runs."""
    from kvint4.llama3.graph_decode import GraphedGreedyDecoder

    class Cache:
        def __init__(self):
            self.lengths = {0: 40, 1: 40}
            self.sig = ("bufs",)

        def buffer_signature(self):
            return self.sig

        def host_lengths(self):
            return dict(self.lengths)

        def advance_host_lengths(self, base, n):
            self.lengths = {i: b + n for i, b in base.items()}

        def crop(self, max_length):
            self.lengths = {i: min(n, max_length) for i, n in self.lengths.items()}

    class Graph:
        replays = 0

        def replay(self):
            Graph.replays += 1

    def decoder(cache):
        d = object.__new__(GraphedGreedyDecoder)
        d.cache, d.graph, d.max_new_tokens = cache, Graph(), 8
        d.done, d._base_done, d._base = 1, 1, cache.host_lengths()
        d._signature = cache.buffer_signature()
        return d

    c = Cache()
    d = decoder(c)
    d.step()
    d.step()
    assert Graph.replays == 2 and c.lengths == {0: 42, 1: 42} and d.done == 3
    c.crop(41)
    with pytest.raises(RuntimeError, match="lengths changed"):
        d.step()
    assert Graph.replays == 2 and d.done == 3
    c.lengths = {0: 42, 1: 42}
    c.sig = ("other bufs",)
    with pytest.raises(RuntimeError, match="buffers changed"):
        d.step()
    assert Graph.replays == 2


def test_paged_make_static_takes_blocks_unshares_them_and_fixes_the_table(monkeypatch):
    """PagedQuantizedKVCache.make_static (host bookkeeping, CPU pools; the
    table holder's device check is lifted for the test): the blocks for the
    extra positions are taken now, a block two sequences share inside that
    range gets a private copy, the table is uploaded once, and later
    decode-step bookkeeping finds nothing to allocate or copy."""
    from kvint4.paged_cache import PagedQuantizedKVCache

    class HostTable:
        def __init__(self, table, page_size, num_blocks):
            self.table, self.page_size, self.num_blocks = table, page_size, num_blocks

    monkeypatch.setattr(ops, "PageTable", HostTable)

    c = PagedQuantizedKVCache(group_size=32, page_size=64)
    with pytest.raises(ValueError):
        c.make_static(4)
    c._setup(torch.zeros(1, 2, 1, 64, dtype=torch.bfloat16))  # B=1, 2 KV heads, d_head 64
    for i in (0, 1):
        c._layer(i)
    c._ensure_pages([100])                                     # 2 blocks
    c._lens = {0: [100], 1: [100]}
    for i in (0, 1):
        c._seq_lens[i].fill_(100)
        for t in c._pools[i]:
            t.copy_(torch.arange(t.numel()).view(t.shape).to(t.dtype))
    c.batch_repeat_interleave(2)                               # both sequences share both blocks
    assert c._pages[0] == c._pages[1] and all(c._ref[b] == 2 for b in c._pages[0])
    shared_last = c._pages[0][1]
    before = [t.clone() for t in c.get_quantized(0)]
    c.make_static(60)                                          # positions 100..159: pages 1 and 2
    assert len(c._pages[0]) == 3 and len(c._pages[1]) == 3
    assert c._pages[0][0] == c._pages[1][0]                   # page 0 is not written: still shared
    assert c._pages[0][1] != c._pages[1][1]                   # page 1 is written: copied apart
    assert all(c._ref[c._pages[b][i]] == 1 for b in (0, 1) for i in (1, 2))
    assert shared_last in (c._pages[0][1], c._pages[1][1])
    for a, b in zip(before, c.get_quantized(0)):               # the stored rows are unchanged
        assert torch.equal(a, b)
    sig = c.buffer_signature()
    table = c.block_table()
    # what a captured decode step does on the host: nothing to allocate, copy or upload
    lens = c._lens[0]
    c._ensure_pages([n + 1 for n in lens])
    c._make_writable(lens, 1)
    assert not c._table_dirty and c.block_table() is table and c.buffer_signature() == sig
    base = c.host_lengths()
    assert base == {0: 100, 1: 100}
    c.advance_host_lengths(base, 7)
    assert c.get_seq_length(0) == 107 and c._lens[1] == [107, 107]
    c._lens[1] = [107, 106]
    with pytest.raises(ValueError, match="differ"):
        c.host_lengths()
    with pytest.raises(ValueError):
        c.make_static(-1)


def test_workspace_growth_keeps_captured_buffers_alive():
    """A HIP graph keeps the address of the split-K workspace it was captured
    with. When a later call on the same (device, stream) needs a larger one,
    the old buffer must stay allocated (retired, not freed), and a private
    workspace given with using_workspace takes precedence on this thread."""
    ws = ops._Workspaces()
    dev = torch.device("cpu")
    small = ws.get(dev, 7, 1000)
    ptr = small.data_ptr()
    assert ws.get(dev, 7, 500) is small  # large enough: reused
    big = ws.get(dev, 7, 3 << 20)
    assert big is not small and big.numel() >= 3 << 20
    assert any(t.data_ptr() == ptr for t in ws._retired), "the replaced buffer was dropped"
    assert ws.get(dev, 8, 10) is not big  # another stream, another buffer
    own = torch.zeros(4096, dtype=torch.uint8)
    with ws.using(own):
        assert ws.get(dev, 7, 4096) is own
        with pytest.raises(ValueError):
            ws.get(dev, 7, 8192)
    assert ws.get(dev, 7, 10) is big
    with pytest.raises(ValueError):
        with ws.using(torch.zeros(4, dtype=torch.float32)):
            pass
