"""The attention swap shared by the Llama and GPT-2 glue (kvint4.module_swap),
on the CPU: the replacement owns the original's Parameters (no copies), an
accelerate hook on a submodule moves to the submodule of the same name and
still runs, and a replacement whose tensors do not match the original raises
instead of leaving meta tensors behind. The reference's swap
(models/llama3/llama3_quant.py:146-204) rebinds the projection Parameters and
moves hooks; its hook move swallows every exception, which this one does not.
"""

from __future__ import annotations

import pytest
import torch
from accelerate.hooks import ModelHook, add_hook_to_module
from transformers import GPT2Config, GPT2LMHeadModel, LlamaConfig, LlamaForCausalLM

import kvint4.gpt2.gpt2_quant as g2q
import kvint4.llama3.llama3_quant as l3q
from kvint4.module_swap import swap_attention_modules


def _llama():
    cfg = LlamaConfig(vocab_size=64, hidden_size=64, intermediate_size=128, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, head_dim=16)
    torch.manual_seed(0)
    return LlamaForCausalLM(cfg).eval()


class CountingHook(ModelHook):
    def __init__(self):
        super().__init__()
        self.calls = 0

    def pre_forward(self, module, *args, **kwargs):
        self.calls += 1
        return args, kwargs


def test_llama_swap_rebinds_parameters_without_copies():
    model = _llama()
    before = {n: p for n, p in model.named_parameters()}
    l3q.replace_llama_attention_with_quantized(model, group_size=32)
    after = dict(model.named_parameters())
    assert before.keys() == after.keys()
    assert all(after[n] is before[n] for n in before), "a Parameter was copied instead of rebound"
    assert all(isinstance(l.self_attn, l3q.LlamaAttentionQuantized) for l in model.model.layers)
    assert not any(p.is_meta for p in model.parameters())


def test_gpt2_swap_keeps_weights_and_device():
    cfg = GPT2Config(n_layer=2, n_head=4, n_embd=64, vocab_size=128, n_positions=64)
    torch.manual_seed(0)
    model = GPT2LMHeadModel(cfg).eval()
    ref = {n: p.detach().clone() for n, p in model.named_parameters()}
    g2q.replace_gpt2_attention_with_quantized(model)
    assert all(isinstance(b.attn, g2q.GPT2AttentionQuantized) for b in model.transformer.h)
    for n, p in model.named_parameters():
        assert not p.is_meta and torch.equal(p, ref[n]), n
    assert model.transformer.h[0].attn.layer_idx == 0 and model.transformer.h[1].attn.layer_idx == 1


def test_accelerate_hook_moves_with_its_projection():
    model = _llama()
    hook = CountingHook()
    old_q = model.model.layers[0].self_attn.q_proj
    add_hook_to_module(old_q, hook)
    l3q.replace_llama_attention_with_quantized(model, group_size=32)
    new_q = model.model.layers[0].self_attn.q_proj
    assert new_q is not old_q
    assert getattr(new_q, "_hf_hook", None) is hook
    assert getattr(old_q, "_hf_hook", None) is None
    with torch.no_grad():
        model(input_ids=torch.zeros(1, 3, dtype=torch.int64))  # no cache: the stock route
    assert hook.calls == 1


def test_hook_on_the_attention_module_itself_moves():
    model = _llama()
    hook = CountingHook()
    add_hook_to_module(model.model.layers[1].self_attn, hook)
    l3q.replace_llama_attention_with_quantized(model)
    assert getattr(model.model.layers[1].self_attn, "_hf_hook", None) is hook


def test_mismatched_replacement_raises():
    model = _llama()

    class Extra(l3q.LlamaAttentionQuantized):
        def __init__(self, config, layer_idx):
            super().__init__(config, layer_idx)
            self.extra = torch.nn.Parameter(torch.zeros(3))

    with pytest.raises(RuntimeError, match="extra"):
        swap_attention_modules(model.model.layers, "self_attn", Extra,
                               lambda old: Extra(old.config, old.layer_idx), 32)


def test_repeated_swap_only_updates_group_size():
    model = _llama()
    l3q.replace_llama_attention_with_quantized(model, group_size=32)
    mods = [l.self_attn for l in model.model.layers]
    l3q.replace_llama_attention_with_quantized(model, group_size=128)
    assert [l.self_attn for l in model.model.layers] == mods
    assert all(m.quant_group_size == 128 for m in mods)
