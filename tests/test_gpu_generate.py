"""GPU: the caches under transformers' generate() — beam search and assisted
decoding — and the batch / length edits those use.

The reference's cache has no reorder_cache or crop (models/llama3/kv_cache.py:
30-166), so beam search and assisted decoding do not run with it; transformers
5.x calls ``reorder_cache(beam_idx)`` after every beam step and ``crop(-n)``
after a rejected draft (generation/utils.py). Parity here:

  * edits: after reorder / select / repeat / crop (and appends after them)
    every sequence's stored codes and scales are byte-equal to a fresh cache
    fed that sequence's own K/V history, for the contiguous cache and the
    paged one (whose children share their parent's blocks until they write);
  * beam search: a tiny fp32 Llama swapped to the INT4 path, with either
    cache, returns the same beams as the stock model with a DynamicCache and
    the INT4 dense reference attention (the reference's quantize ->
    dequantize -> attention, tests/_hf_ref.py);
  * assisted decoding: greedy generation with a draft model returns the same
    tokens as plain greedy generation with the same cache type (crop and
    multi-token verification steps in between).
"""

from __future__ import annotations

import pytest
import torch
from transformers import LlamaConfig, LlamaForCausalLM
from transformers.cache_utils import DynamicCache

from kvint4 import ops
from kvint4.llama3.kv_cache import QuantizedKVCache
from kvint4.llama3.llama3_quant import replace_llama_attention_with_quantized
from kvint4.paged_cache import PagedQuantizedKVCache

from _hf_ref import use_int4_dense_reference_attention

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
H, D, LAYERS = 2, 64, 2


def _make(kind: str):
    if kind == "contiguous":
        return QuantizedKVCache(group_size=32)
    return PagedQuantizedKVCache(group_size=32, page_size=int(kind.split("-")[1]))


class _History:
    """Per-sequence K/V history of every layer, kept on the CPU."""

    def __init__(self, B: int, seed: int):
        self.g = torch.Generator().manual_seed(seed)
        self.seqs = [[[[], []] for _ in range(LAYERS)] for _ in range(B)]

    def step(self, cache, S: int) -> None:
        B = len(self.seqs)
        for layer in range(LAYERS):
            k = torch.randn(B, H, S, D, generator=self.g).to(torch.bfloat16)
            v = torch.randn(B, H, S, D, generator=self.g).to(torch.bfloat16)
            cache.append(k.to(DEV), v.to(DEV), layer)
            for b in range(B):
                self.seqs[b][layer][0].append(k[b])
                self.seqs[b][layer][1].append(v[b])

    def remap(self, src: list[int]) -> None:
        self.seqs = [[[list(kv[0]), list(kv[1])] for kv in self.seqs[s]] for s in src]

    def crop(self, n: int) -> None:
        for seq in self.seqs:
            for kv in seq:
                for i in range(2):
                    rows = torch.cat(kv[i], dim=1)
                    keep = max(rows.shape[1] + n, 0) if n < 0 else min(rows.shape[1], n)
                    kv[i] = [rows[:, :keep]]


def _attention_check(cache, hist: _History, kind: str) -> None:
    """Decode attention over the edited cache (the fused kernel reading
    shared and copied blocks) against fp32 attention over each sequence's
    dequantized rows, within the bf16 attention bar."""
    B, Hq = len(hist.seqs), 2 * H
    q = torch.randn(B, Hq, 1, D, generator=torch.Generator().manual_seed(B)).to(torch.bfloat16).to(DEV)
    for layer in range(LAYERS):
        if kind == "contiguous":
            got = ops.fused_decode_attention(q, *cache.get_quantized(layer), n_kv_heads=H, group_size=32,
                                             is_causal=False, sm_scale=D ** -0.5)
        else:
            got = cache.attend(q, layer, n_kv_heads=H, scale=D ** -0.5, is_causal=False)
        k, v = cache.get_dequantized(layer, out_dtype=torch.float32)
        for b, seq in enumerate(hist.seqs):
            n = torch.cat(seq[layer][0], dim=1).shape[1]
            kk = k[b, :, :n].repeat_interleave(Hq // H, dim=0)
            vv = v[b, :, :n].repeat_interleave(Hq // H, dim=0)
            p = torch.softmax((q[b].float() @ kk.transpose(1, 2)) * D ** -0.5, dim=-1)
            want = p @ vv
            assert (got[b].float() - want).abs().max().item() < 2e-2, (b, layer)


def _check(cache, hist: _History, kind: str) -> None:
    """Each sequence's valid rows equal a fresh cache of its own history."""
    _attention_check(cache, hist, kind)
    for b, seq in enumerate(hist.seqs):
        fresh = _make(kind)
        for layer, (ks, vs) in enumerate(seq):
            fresh.append(torch.cat(ks, dim=1)[None].to(DEV), torch.cat(vs, dim=1)[None].to(DEV), layer)
        for layer in range(LAYERS):
            n = torch.cat(seq[layer][0], dim=1).shape[1]
            if kind == "contiguous":
                assert cache.get_seq_length(layer) == n
            else:
                assert int(cache.get_seq_lens(layer)[b]) == n
            got = cache.get_quantized(layer)
            want = fresh.get_quantized(layer)
            for g_t, w_t in zip(got, want):
                assert torch.equal(g_t[b, :, :n], w_t[0, :, :n]), (b, layer)


@pytest.mark.parametrize("kind", ["contiguous", "paged-16", "paged-64"])
def test_batch_edits_and_crop_match_rebuilt_history(kind):
    cache = _make(kind)
    hist = _History(B=3, seed=5)
    hist.step(cache, 70)          # prompt
    hist.step(cache, 1)
    _check(cache, hist, kind)
    # beam step: sequence 0 gets two children, sequence 1 is dropped
    src = [2, 0, 0]
    cache.reorder_cache(torch.tensor(src, device=DEV))
    hist.remap(src)
    _check(cache, hist, kind)
    for _ in range(3):            # the two children write different tokens into the shared page
        hist.step(cache, 1)
    _check(cache, hist, kind)
    cache.crop(-2)                # a rejected draft of 2 tokens
    hist.crop(-2)
    _check(cache, hist, kind)
    hist.step(cache, 5)           # verification block after the crop
    _check(cache, hist, kind)
    cache.crop(60)                # legacy absolute length; cuts into the prompt's pages
    hist.crop(60)
    _check(cache, hist, kind)
    cache.batch_repeat_interleave(2)
    hist.remap([0, 0, 1, 1, 2, 2])
    hist.step(cache, 1)
    _check(cache, hist, kind)
    keep = torch.tensor([True, False, False, True, True, False], device=DEV)
    cache.batch_select_indices(keep)
    hist.remap([0, 3, 4])
    hist.step(cache, 2)
    _check(cache, hist, kind)
    cache.crop(0)                 # no-op
    _check(cache, hist, kind)


def test_paged_children_share_blocks_until_they_write():
    cache = PagedQuantizedKVCache(group_size=32, page_size=16)
    hist = _History(B=2, seed=9)
    hist.step(cache, 40)          # 3 pages per sequence, the last one partly filled
    used = cache._num_blocks - len(cache._free)
    cache.reorder_cache(torch.tensor([0, 0, 0, 1], device=DEV))
    hist.remap([0, 0, 0, 1])
    assert cache._num_blocks - len(cache._free) == used   # nothing copied yet
    hist.step(cache, 1)           # three children write into sequence 0's shared last page
    # two of them copy that page; the third ends up as its only holder
    assert cache._num_blocks - len(cache._free) == used + 2
    _check(cache, hist, "paged-16")
    cache.reorder_cache(torch.tensor([3], device=DEV))
    hist.remap([3])
    assert cache._num_blocks - len(cache._free) == 3    # everything else released
    _check(cache, hist, "paged-16")


def _llama_pair():
    cfg = LlamaConfig(vocab_size=256, hidden_size=128, intermediate_size=256, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=256,
                      rms_norm_eps=1e-5, tie_word_embeddings=False)
    torch.manual_seed(0)
    ref = LlamaForCausalLM(cfg).eval()
    quant = LlamaForCausalLM(cfg).eval()
    quant.load_state_dict(ref.state_dict())
    use_int4_dense_reference_attention(ref)
    replace_llama_attention_with_quantized(quant)
    return ref.to(DEV), quant.to(DEV)


@pytest.mark.parametrize("kind", ["contiguous", "paged-16", "paged-64"])
def test_beam_search_matches_reference(kind):
    ref, quant = _llama_pair()
    torch.manual_seed(11)
    prompt = torch.randint(0, 256, (2, 12), device=DEV)
    args = dict(num_beams=3, num_return_sequences=3, do_sample=False, max_new_tokens=8,
                attention_mask=torch.ones_like(prompt), pad_token_id=0)
    with torch.no_grad():
        want = ref.generate(prompt, past_key_values=DynamicCache(), **args)
        got = quant.generate(prompt, past_key_values=_make(kind), **args)
    assert torch.equal(got, want), (got, want)


@pytest.mark.parametrize("kind", ["contiguous", "paged-64"])
def test_assisted_decoding_matches_greedy(kind):
    _, quant = _llama_pair()
    draft_cfg = LlamaConfig(vocab_size=256, hidden_size=64, intermediate_size=128, num_hidden_layers=1,
                            num_attention_heads=2, num_key_value_heads=1, max_position_embeddings=256,
                            tie_word_embeddings=False)
    torch.manual_seed(1)
    draft = LlamaForCausalLM(draft_cfg).eval().to(DEV)
    torch.manual_seed(12)
    prompt = torch.randint(0, 256, (1, 10), device=DEV)
    args = dict(do_sample=False, max_new_tokens=16, attention_mask=torch.ones_like(prompt), pad_token_id=0)
    with torch.no_grad():
        plain = quant.generate(prompt, past_key_values=_make(kind), **args)
        assisted = quant.generate(prompt, past_key_values=_make(kind), assistant_model=draft, **args)
    assert torch.equal(plain, assisted), (plain, assisted)
