"""Graph-captured greedy decoding (kvint4.llama3.graph_decode): a small
random-init Llama with the attention modules swapped
(replace_llama_attention_with_quantized, reference
models/llama3/llama3_quant.py:171-204) decodes from a prefilled INT4 cache,
one HIP graph replay per token. Every replay must give what the same step
gives eagerly: the test feeds the graph's tokens to eager steps over a cache
in the same device-length mode (make_static; the attention launches and
their split plans are then the same) and compares logits step by step. On
the MI355X the replays give the eager logits and cache bytes exactly; the
bar allows bf16 rounding in case a library GEMM picks another algorithm
under capture: logits within 5e-2, each replay's token a best token of the
eager logits to within twice that step's difference, and 99 % of the cache
bytes equal (a code moves where the projected K/V round differently). The replays are interleaved with unrelated eager work and host
synchronisations. Plain eager decoding (host write positions, a split plan
sized to the context) is compared on the logits of the first step, within
the attention bar. Caches: contiguous; paged (pages of 64, the table grown
and uploaded by make_static before capture); and paged with the batch's
sequences sharing their prompt blocks (batch_repeat_interleave), which
make_static copies apart before capture."""

from __future__ import annotations

import pytest
import torch
from transformers import LlamaConfig, LlamaForCausalLM

from kvint4.llama3.graph_decode import GraphedGreedyDecoder
from kvint4.llama3.kv_cache import QuantizedKVCache
from kvint4.llama3.llama3_quant import replace_llama_attention_with_quantized
from kvint4.paged_cache import PagedQuantizedKVCache

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _model(head_dim: int):
    cfg = LlamaConfig(vocab_size=512, hidden_size=8 * head_dim, intermediate_size=1024, num_hidden_layers=2,
                      num_attention_heads=8, num_key_value_heads=2, rope_theta=500000.0,
                      max_position_embeddings=4096, rms_norm_eps=1e-5, initializer_range=0.05,
                      tie_word_embeddings=False)
    torch.manual_seed(11)
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device(DEV):
            model = LlamaForCausalLM(cfg).eval()
    finally:
        torch.set_default_dtype(prev)
    model.set_attn_implementation("sdpa")
    replace_llama_attention_with_quantized(model, group_size=32)
    return model


def _prefill(model, prompt, kind="contiguous"):
    """Prefill a fresh cache. kind: "contiguous", "paged" (pages of 64), or
    "shared" (paged; the batch's first prompt prefilled once and repeated
    with batch_repeat_interleave, so the sequences share their blocks)."""
    if kind == "contiguous":
        cache = QuantizedKVCache(group_size=32)
    else:
        cache = PagedQuantizedKVCache(group_size=32, page_size=64)
    B = prompt.shape[0]
    with torch.no_grad():
        if kind == "shared":
            out = model(input_ids=prompt[:1], past_key_values=cache, use_cache=True, logits_to_keep=1)
            cache.batch_repeat_interleave(B)
            logits = out.logits[:, -1].repeat(B, 1)
        else:
            out = model(input_ids=prompt, past_key_values=cache, use_cache=True, logits_to_keep=1)
            logits = out.logits[:, -1]
    return cache, logits.float(), logits.argmax(-1, keepdim=True)


@pytest.mark.parametrize("head_dim,B,prompt_len,steps,kind", [
    (64, 2, 70, 12, "contiguous"), (128, 1, 300, 10, "contiguous"),
    (128, 2, 300, 40, "paged"), (64, 2, 100, 12, "shared"),
])
def test_graph_replays_match_eager_steps(head_dim, B, prompt_len, steps, kind):
    print(f"graph decode: head_dim {head_dim}, batch {B}, prompt {prompt_len}, steps {steps}, {kind} cache",
          flush=True)
    model = _model(head_dim)
    prompt = torch.randint(0, 512, (B, prompt_len), generator=torch.Generator().manual_seed(5)).to(DEV)

    # graph replays, with unrelated eager work between them
    cache_g, _, nxt_g = _prefill(model, prompt, kind)
    warm = 2
    dec = GraphedGreedyDecoder(model, cache_g, nxt_g, max_new_tokens=steps, warmup_steps=warm)
    junk = torch.randn(256, 256, device=DEV)
    graph_logits = {}
    while dec.done < steps:
        dec.step()
        graph_logits[dec.done - 1] = dec.last_logits.clone()
        junk = (junk @ junk).tanh_()
        torch.cuda.synchronize()
        assert cache_g.get_seq_length() == prompt_len + dec.done
    with pytest.raises(RuntimeError):
        dec.step()
    toks = dec.tokens

    # eager steps over a cache in the same device-length mode, fed the graph's
    # tokens (teacher forcing)
    cache_e, _, nxt = _prefill(model, prompt, kind)
    assert torch.equal(nxt, nxt_g)
    cache_e.make_static(steps)
    pos = torch.full((B, 1), prompt_len, dtype=torch.int64, device=DEV)
    worst = 0.0
    with torch.no_grad():
        for i in range(steps):
            feed = nxt_g if i == 0 else toks[:, i - 1:i]
            out = model(input_ids=feed, position_ids=pos, past_key_values=cache_e, use_cache=True,
                        logits_to_keep=1)
            pos += 1
            lg = out.logits[:, -1].float()
            if i in graph_logits:
                gl = graph_logits[i]
                d = (gl - lg).abs().max().item()
                worst = max(worst, d)
                # the replay's token is its own argmax, and a near-best token
                # of the eager logits
                assert torch.equal(gl.argmax(-1), toks[:, i])
                best = lg.max(-1).values
                got = lg.gather(1, toks[:, i:i + 1]).squeeze(1)
                assert bool((got >= best - 2 * d - 1e-6).all()), (i, best, got)
            else:  # eager warmup steps of the decoder: the same launches
                assert torch.equal(lg.argmax(-1), toks[:, i])
    print(f"graph decode: replay vs eager logits max-abs {worst:.3e} over {steps - warm} replays")
    assert worst < 5e-2
    same = 0
    total = 0
    for layer in range(len(cache_e)):
        assert torch.equal(cache_e.get_seq_lens(layer), cache_g.get_seq_lens(layer))
        for a, b in zip(cache_e.get_quantized(layer), cache_g.get_quantized(layer)):
            assert a.shape == b.shape
            same += int((a == b).sum().item())
            total += a.numel()
    print(f"graph decode: cache elements equal {same}/{total}")
    assert same >= 0.99 * total

    # plain eager decoding (host write positions): its split plan is sized to
    # the context, not to the capacity, so the attention rounds differently
    # (each within the attention bar of the oracle, tests/test_gpu_decode_step.py);
    # the two layers carry that to the first step's logits
    cache_p, _, nxt_p = _prefill(model, prompt, kind)
    with torch.no_grad():
        out = model(input_ids=nxt_p, past_key_values=cache_p, use_cache=True, logits_to_keep=1)
        cache_s, _, _ = _prefill(model, prompt, kind)
        cache_s.make_static(1)
        ref = model(input_ids=nxt_p, position_ids=torch.full((B, 1), prompt_len, device=DEV),
                    past_key_values=cache_s, use_cache=True, logits_to_keep=1)
    diff = (out.logits[:, -1].float() - ref.logits[:, -1].float()).abs().max().item()
    print(f"graph decode: first-step logits, device-length mode vs host positions: max-abs {diff:.3e}")
    assert diff < 0.1


def test_decoder_rejects_what_it_cannot_capture():
    model = _model(64)
    prompt = torch.randint(0, 512, (1, 40), generator=torch.Generator().manual_seed(6)).to(DEV)
    cache, _, nxt = _prefill(model, prompt)
    with pytest.raises(ValueError):
        GraphedGreedyDecoder(model, cache, nxt.view(-1), max_new_tokens=4)
    with pytest.raises(ValueError):
        GraphedGreedyDecoder(model, cache, nxt, max_new_tokens=2, warmup_steps=2)
    with pytest.raises(ValueError):
        QuantizedKVCache(group_size=32).make_static(4)


def test_crop_between_replays_stops_the_decoder():
    """A crop keeps the cache's buffers and moves its lengths: the captured
    step would append at the uncropped positions, so step() must refuse."""
    model = _model(64)
    prompt = torch.randint(0, 512, (1, 40), generator=torch.Generator().manual_seed(7)).to(DEV)
    cache, _, nxt = _prefill(model, prompt)
    dec = GraphedGreedyDecoder(model, cache, nxt, max_new_tokens=6, warmup_steps=1)
    dec.step()
    torch.cuda.synchronize()
    n = cache.get_seq_length()
    cache.crop(n - 1)
    assert cache.get_seq_length() == n - 1
    with pytest.raises(RuntimeError, match="lengths changed"):
        dec.step()
