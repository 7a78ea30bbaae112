"""GPU: QuantizedKVCache storage and the HF attention glue.

Cache: chunked appends (and capacity growth) equal one-shot quantization of
the concatenation bit for bit — the reference's append is quantize + torch.cat
(models/llama3/kv_cache.py:76-102); views, nbytes, the transformers 5.x cache
protocol, ragged appends.

Model glue (tests/llama3/test_llama3_quant_decode.py:21-122,
tests/llama3/test_llama3_generate_parity.py:52-74): a tiny random-init Llama
(and GPT-2) swapped to the INT4 path vs the same stock model with a
DynamicCache, both on the GPU. The stock model attends through an fp32
reference attention (tests/_hf_ref.py) so that no half-precision batched GEMM
runs on the GPU; everything else is the same kernels, so the comparison
isolates the INT4 KV. Bars are the reference's own: prefill last-logit
max-abs < 1.0 and same argmax, 8 decode steps < 2.0, greedy prefix agreement
>= 4 of 16.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
from transformers import GPT2Config, GPT2LMHeadModel, LlamaConfig, LlamaForCausalLM
from transformers.cache_utils import DynamicCache

from kvint4.gpt2.gpt2_quant import replace_gpt2_attention_with_quantized
from kvint4.gpt2.kv_cache import QuantizedKVCache as GPT2Cache
from kvint4.llama3.attention_quant import attention_forward_quant_gqa
from kvint4.llama3.kv_cache import QuantizedKVCache
from kvint4.llama3.llama3_quant import LlamaAttentionQuantized, replace_llama_attention_with_quantized
from oracle import kvq_oracle as O

from _hf_ref import use_fp32_reference_attention

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def test_chunked_append_equals_one_shot_and_growth():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(2, 4, 700, 128, generator=g).to(torch.bfloat16)
    y = torch.randn(2, 4, 700, 128, generator=g).to(torch.bfloat16)
    cache = QuantizedKVCache(group_size=32)
    bounds = [0, 37, 38, 300, 301, 302, 700]  # first allocation is 256 + 37 rounded; forces growth
    for a, b in zip(bounds[:-1], bounds[1:]):
        cache.append(x[:, :, a:b].to(DEV), y[:, :, a:b].to(DEV), 3)
    assert cache.get_seq_length(3) == 700 and cache.get_seq_length(0) == 0
    kp, ks, vp, vs = cache.get_quantized(3)
    assert kp.shape == (2, 4, 700, 64) and ks.shape == (2, 4, 700, 4) and ks.dtype == torch.bfloat16
    okp, oks = O.quantize_int4(x.float().numpy(), 32, "bf16")
    ovp, ovs = O.quantize_int4(y.float().numpy(), 32, "bf16")
    assert np.array_equal(kp.cpu().numpy(), okp) and np.array_equal(vp.cpu().numpy(), ovp)
    assert np.array_equal(ks.float().cpu().numpy(), oks) and np.array_equal(vs.float().cpu().numpy(), ovs)
    assert cache.nbytes() == 2 * (2 * 4 * 700 * 64) + 2 * (2 * 4 * 700 * 4 * 2)
    assert cache.capacity_nbytes() >= cache.nbytes()
    k_deq, v_deq = cache.get_dequantized(3, out_dtype=torch.float32)
    assert np.array_equal(k_deq.cpu().numpy(), O.dequantize_int4(okp, oks, 32, 128, "f32"))


def test_protocol_and_update_path():
    cache = QuantizedKVCache()
    k = torch.randn(1, 2, 5, 64, device=DEV, dtype=torch.float32)
    kd, vd = cache.update(k, k, 0)
    assert kd.dtype == torch.float32 and kd.shape == (1, 2, 5, 64)
    assert cache.get_mask_sizes(3, 0) == (8, 0)
    assert cache.get_mask_sizes(torch.arange(3), 0) == (8, 0)
    assert cache.get_query_offset(0) == 5
    assert cache.is_sliding == [False] and cache.is_initialized and len(cache) == 1
    assert cache.get_max_cache_shape() == -1
    gc = GPT2Cache()
    kd, _ = gc.update(k, k, 0)
    assert kd.dtype == torch.float16 and gc.get_max_cache_shape() is None
    cache.reset()
    assert not cache.is_initialized


def test_ragged_append_positions():
    cache = GPT2Cache(group_size=32)
    g = torch.Generator().manual_seed(1)
    x = torch.randn(3, 2, 40, 64, generator=g).half()
    lens = torch.tensor([5, 40, 17])
    cache.load_ragged(x.to(DEV), x.to(DEV), 0, lens)
    new = torch.randn(3, 2, 1, 64, generator=g).half()
    cache.append(new.to(DEV), new.to(DEV), 0)
    assert cache.get_seq_lens(0).tolist() == [6, 41, 18]
    kp, ks, _, _ = cache.get_quantized(0)
    want_p, _ = O.quantize_int4(new.float().numpy(), 32, "f16")
    for b, p in enumerate([5, 40, 17]):
        assert np.array_equal(kp[b, :, p].cpu().numpy(), want_p[b, :, 0])


def _tiny_llama(dtype=torch.bfloat16):
    cfg = LlamaConfig(vocab_size=256, hidden_size=128, intermediate_size=256, num_hidden_layers=2,
                      num_attention_heads=8, num_key_value_heads=2, head_dim=64,
                      max_position_embeddings=512, rms_norm_eps=1e-5, tie_word_embeddings=False,
                      attention_bias=False, mlp_bias=False)
    torch.manual_seed(0)
    return LlamaForCausalLM(cfg).to(dtype=dtype).eval()


def _pair():
    """(stock reference, INT4-swapped) tiny Llamas with identical weights, on the GPU."""
    ref = _tiny_llama()
    quant = _tiny_llama()
    quant.load_state_dict(ref.state_dict())
    use_fp32_reference_attention(ref)
    replace_llama_attention_with_quantized(quant, group_size=32)
    return ref.to(DEV), quant.to(DEV)


def test_llama_prefill_decode_matches_reference():
    ref, quant = _pair()
    assert all(isinstance(l.self_attn, LlamaAttentionQuantized) for l in quant.model.layers)
    torch.manual_seed(123)
    prompt = torch.randint(0, 256, (1, 32), device=DEV)
    with torch.no_grad():
        cache_ref, cache_q = DynamicCache(), QuantizedKVCache(group_size=32)
        out_r = ref(input_ids=prompt, past_key_values=cache_ref, use_cache=True)
        out_q = quant(input_ids=prompt, past_key_values=cache_q, use_cache=True)
        lr, lq = out_r.logits[:, -1].float(), out_q.logits[:, -1].float()
        d0 = (lr - lq).abs().max().item()
        print(f"prefill last-logit max-abs diff {d0:.4f}")
        assert d0 < 1.0
        assert lr.argmax(-1).item() == lq.argmax(-1).item()
        for step in range(8):
            nid = torch.randint(0, 256, (1, 1), device=DEV)
            out_r = ref(input_ids=nid, past_key_values=cache_ref, use_cache=True)
            out_q = quant(input_ids=nid, past_key_values=cache_q, use_cache=True)
            d = (out_r.logits[:, -1].float() - out_q.logits[:, -1].float()).abs().max().item()
            print(f"decode step {step} last-logit max-abs diff {d:.4f}")
            assert d < 2.0, f"decode step {step}: {d}"
    assert cache_q.get_seq_length(0) == 40
    seq = 40
    assert cache_q.nbytes() < (2 * 2 * 1 * 2 * seq * 64 * 2) / 2


def test_llama_greedy_prefix_agreement():
    ref, quant = _pair()
    torch.manual_seed(321)
    prompt = torch.randint(0, 256, (1, 24), device=DEV)

    def greedy(model, dev, cache, n):
        toks = []
        with torch.no_grad():
            out = model(input_ids=prompt, past_key_values=cache, use_cache=True)
            top2 = out.logits[0, -1].float().topk(2).values
            print(f"first-token top-2 logit gap {float(top2[0] - top2[1]):.4f}")
            nid = out.logits[:, -1].argmax(-1, keepdim=True)
            toks.append(int(nid.item()))
            for _ in range(n - 1):
                out = model(input_ids=nid, past_key_values=cache, use_cache=True)
                nid = out.logits[:, -1].argmax(-1, keepdim=True)
                toks.append(int(nid.item()))
        return toks

    a = greedy(ref, DEV, DynamicCache(), 16)
    b = greedy(quant, DEV, QuantizedKVCache(), 16)
    agree = next((i for i, (x, y) in enumerate(zip(a, b)) if x != y), 16)
    assert agree >= 4, (a, b)


def test_gpt2_random_init_decode_matches_reference():
    cfg = GPT2Config(n_layer=2, n_head=4, n_embd=128, vocab_size=256, n_positions=256)
    torch.manual_seed(0)
    ref = GPT2LMHeadModel(cfg).eval()                       # fp32, DynamicCache
    quant = GPT2LMHeadModel(cfg).eval()
    quant.load_state_dict(ref.state_dict())
    use_fp32_reference_attention(ref)
    replace_gpt2_attention_with_quantized(quant)
    ref, quant = ref.to(DEV), quant.to(DEV)
    torch.manual_seed(7)
    prompt = torch.randint(0, 256, (1, 20), device=DEV)
    with torch.no_grad():
        cr, cq = DynamicCache(), GPT2Cache()
        lr = ref(input_ids=prompt, past_key_values=cr, use_cache=True).logits[:, -1]
        lq = quant(input_ids=prompt, past_key_values=cq, use_cache=True).logits[:, -1]
        assert (lr - lq).abs().max().item() < 1.0 and lr.argmax().item() == lq.argmax().item()
        for _ in range(6):
            nid = torch.randint(0, 256, (1, 1), device=DEV)
            lr = ref(input_ids=nid, past_key_values=cr, use_cache=True).logits[:, -1]
            lq = quant(input_ids=nid, past_key_values=cq, use_cache=True).logits[:, -1]
            assert (lr - lq).abs().max().item() < 2.0
    assert cq.get_seq_length(0) == 26


def test_gpt2_eager_reorder_and_upcast_path():
    """GPT-2 with reorder_and_upcast_attn under eager attention: the quantized
    module attends over the dequantized cache through the model's own
    _upcast_and_reordered_attn (transformers 5.x signature: query, key, value,
    attention_mask; reference models/gpt2/gpt2_quant.py:104-106 passes the
    4.x arguments). Stock eager model with a DynamicCache as the reference, fp32."""
    cfg = GPT2Config(n_layer=2, n_head=4, n_embd=128, vocab_size=256, n_positions=256,
                     reorder_and_upcast_attn=True)
    torch.manual_seed(1)
    ref = GPT2LMHeadModel(cfg).eval()
    quant = GPT2LMHeadModel(cfg).eval()
    quant.load_state_dict(ref.state_dict())
    ref.set_attn_implementation("eager")
    quant.set_attn_implementation("eager")
    replace_gpt2_attention_with_quantized(quant)
    ref, quant = ref.to(DEV), quant.to(DEV)
    torch.manual_seed(8)
    prompt = torch.randint(0, 256, (1, 20), device=DEV)
    with torch.no_grad():
        cr, cq = DynamicCache(), GPT2Cache()
        lr = ref(input_ids=prompt, past_key_values=cr, use_cache=True).logits[:, -1]
        lq = quant(input_ids=prompt, past_key_values=cq, use_cache=True).logits[:, -1]
        assert (lr - lq).abs().max().item() < 1.0 and lr.argmax().item() == lq.argmax().item()
        for _ in range(4):
            nid = torch.randint(0, 256, (1, 1), device=DEV)
            lr = ref(input_ids=nid, past_key_values=cr, use_cache=True).logits[:, -1]
            lq = quant(input_ids=nid, past_key_values=cq, use_cache=True).logits[:, -1]
            assert (lr - lq).abs().max().item() < 2.0
    assert cq.get_seq_length(0) == 24


def test_cache_append_and_attend_matches_append_then_attend():
    """QuantizedKVCache.append_and_attend (one launch) leaves the same cache
    as append and gives the attention over it, for a uniform and a ragged layer."""
    g = torch.Generator().manual_seed(5)
    B, Hq, Hkv, D = 2, 16, 4, 128
    k0 = torch.randn(B, Hkv, 300, D, generator=g).to(torch.bfloat16).to(DEV)
    v0 = torch.randn(B, Hkv, 300, D, generator=g).to(torch.bfloat16).to(DEV)
    lens = torch.tensor([300, 123], dtype=torch.int32)
    for ragged in (False, True):
        ca, cb = QuantizedKVCache(group_size=32), QuantizedKVCache(group_size=32)
        for c in (ca, cb):
            if ragged:
                c.load_ragged(k0, v0, 0, lens)
            else:
                c.append(k0, v0, 0)
        for step in range(3):
            q = torch.randn(B, Hq, 1, D, generator=g).to(torch.bfloat16).to(DEV)
            kn = torch.randn(B, Hkv, 1, D, generator=g).to(torch.bfloat16).to(DEV)
            vn = torch.randn(B, Hkv, 1, D, generator=g).to(torch.bfloat16).to(DEV)
            got = cb.append_and_attend(q, kn, vn, 0, n_kv_heads=Hkv, scale=D ** -0.5)
            assert got is not None
            ca.append(kn, vn, 0)
            kp, ks, vp, vs = ca.get_quantized(0)
            want = attention_forward_quant_gqa(q, kp, ks, vp, vs, n_q_heads=Hq, n_kv_heads=Hkv,
                                               scale=D ** -0.5, seq_lens=ca.get_seq_lens(0))
            # Rows a ragged sequence has not written yet are uninitialised
            # capacity in both caches: compare each sequence's own rows.
            valid = [int(n) + step + 1 for n in lens] if ragged else [301 + step] * B
            for i, (x, y) in enumerate(zip(ca.get_quantized(0), cb.get_quantized(0))):
                for b in range(B):
                    assert torch.equal(x[b, :, :valid[b]], y[b, :, :valid[b]]), (ragged, step, i, b)
            assert ca.get_seq_length(0) == cb.get_seq_length(0) == 301 + step
            if ragged:
                assert torch.equal(ca.get_seq_lens(0), cb.get_seq_lens(0))
            err = (got.float() - want.float()).abs().max().item()
            assert err <= 2.0 ** -5, err


def test_gpt2_fp16_decode_through_fused_step_matches_reference():
    cfg = GPT2Config(n_layer=2, n_head=4, n_embd=256, vocab_size=256, n_positions=256)
    torch.manual_seed(0)
    ref = GPT2LMHeadModel(cfg).eval()                       # fp32, DynamicCache
    quant = GPT2LMHeadModel(cfg).eval()
    quant.load_state_dict(ref.state_dict())
    use_fp32_reference_attention(ref)
    replace_gpt2_attention_with_quantized(quant)
    ref, quant = ref.to(DEV), quant.to(DEV).half()
    torch.manual_seed(9)
    prompt = torch.randint(0, 256, (1, 30), device=DEV)
    with torch.no_grad():
        cr, cq = DynamicCache(), GPT2Cache()
        lr = ref(input_ids=prompt, past_key_values=cr, use_cache=True).logits[:, -1]
        lq = quant(input_ids=prompt, past_key_values=cq, use_cache=True).logits[:, -1].float()
        assert (lr - lq).abs().max().item() < 1.0 and lr.argmax().item() == lq.argmax().item()
        for _ in range(6):
            nid = torch.randint(0, 256, (1, 1), device=DEV)
            lr = ref(input_ids=nid, past_key_values=cr, use_cache=True).logits[:, -1]
            lq = quant(input_ids=nid, past_key_values=cq, use_cache=True).logits[:, -1].float()
            assert (lr - lq).abs().max().item() < 2.0
    assert cq.get_seq_length(0) == 36 and cq.get_quantized(0)[1].dtype == torch.float16
