"""Greedy decoding of a Llama model over the INT4 cache, one HIP graph replay
per token.

The reference decodes eagerly through Hugging Face's forward
(models/llama3/llama3_quant.py:36-143 per layer, driven by
benchmarks/llama3/run_llama3_benchmark.py). At batch 1 that costs more host
time per token than the GPU spends on it. Here one decode step of the whole
model (embedding, 32 decoder layers with one fused append + attention launch
each, norm, LM head, argmax) is captured once into a HIP graph and replayed:

  * the cache keeps its write positions in device memory (``make_static``),
    and the captured step advances them in place; a paged cache also takes
    the blocks of every step and uploads its block table before capture;
  * position ids, the input token and the step counter are device tensors
    that the step also updates in place, so each replay feeds the next;
  * generated tokens are written into a device [B, max_new_tokens] buffer;
  * the decoder owns the split-K workspace its attention launches use, so no
    later call that grows or reuses the library's shared workspace can move it
    under the graph, and two decoders share no arrival counters;
  * every replay first checks that the cache still has the buffers the graph
    was captured with (reorder, batch select, crop-and-regrow or a load
    replace them) and the lengths the previous steps left (a crop changes
    them in place), and raises otherwise.

Batches with padding are not supported: the step runs without an attention
mask, so every sequence of the batch must hold the same number of tokens.

A replay runs the kernels of one eager step on the same buffers. The
attention launches are the same; the library GEMMs of the projections may
pick other algorithms under capture, so logits can differ from eager
decoding by bf16 rounding, and greedy tokens can differ where two logits
tie to within it.
"""

from __future__ import annotations

import contextlib

import torch
from transformers import AttentionInterface
from transformers.integrations.sdpa_attention import sdpa_attention_forward

from .. import ops
from ..cache_base import QuantizedKVCacheBase
from ..paged_cache import PagedQuantizedKVCache
from .llama3_quant import LlamaAttentionQuantized


# An attention implementation name with no mask function registered for it.
# transformers builds no mask for such a name (masking_utils
# _preprocess_mask_arguments returns None early). It is in force only while
# the decode step is run for warm-up and for capture: the sdpa mask path would
# otherwise build a causal mask under stream capture (its tracing check counts
# capture as tracing), and the swapped attention modules take the dense
# fallback whenever a mask is given. A one-token decode step of sequences of
# one length needs no mask: every cached key is visible to it.
_NO_MASK_IMPL = "kvint4_no_mask"
AttentionInterface.register(_NO_MASK_IMPL, sdpa_attention_forward)


@contextlib.contextmanager
def _no_mask_creation(model):
    configs = {id(m.config): m.config for m in model.modules() if hasattr(m, "config")}
    configs.setdefault(id(model.config), model.config)
    old = {k: c._attn_implementation for k, c in configs.items()}
    try:
        for c in configs.values():
            c._attn_implementation = _NO_MASK_IMPL
        yield
    finally:
        for k, c in configs.items():
            c._attn_implementation = old[k]


class GraphedGreedyDecoder:
    """Greedy decoding of `max_new_tokens` tokens from a prefilled cache.

    model          a Llama causal LM whose attention modules were swapped by
                   ``replace_llama_attention_with_quantized``.
    cache          the ``QuantizedKVCache`` or ``PagedQuantizedKVCache`` the
                   prompt was prefilled into (every sequence of the batch the
                   same length: the decode step runs without a mask). A paged
                   cache gets its blocks for every step now (``make_static``),
                   so the captured step allocates and copies nothing.
    next_token     [B, 1] int64 device tensor: the token after the prompt
                   (argmax of the prefill's last logits), fed to step 0.
    warmup_steps   eager steps run before capture (they are real steps: their
                   tokens are the first ones generated). They initialise the
                   libraries' per-stream state that capture may not create.

    ``run()`` replays the graph for the remaining steps and returns the
    [B, max_new_tokens] tokens. ``step()`` replays one step; ``last_logits``
    (fp32 [B, vocab]) then holds that step's logits.
    """

    def __init__(self, model, cache: QuantizedKVCacheBase, next_token: torch.Tensor,
                 max_new_tokens: int, warmup_steps: int = 2):
        if not isinstance(cache, (QuantizedKVCacheBase, PagedQuantizedKVCache)):
            raise TypeError("GraphedGreedyDecoder needs a QuantizedKVCache or a PagedQuantizedKVCache")
        attn = [m for m in model.modules() if isinstance(m, LlamaAttentionQuantized)]
        if not attn:
            raise ValueError("the model's attention modules are not LlamaAttentionQuantized "
                             "(call replace_llama_attention_with_quantized first)")
        if next_token.dim() != 2 or next_token.shape[1] != 1 or not next_token.is_cuda:
            raise ValueError("next_token must be a [B, 1] device tensor")
        max_new_tokens = int(max_new_tokens)
        warmup_steps = int(warmup_steps)
        if max_new_tokens < 1 or not 0 <= warmup_steps < max_new_tokens:
            raise ValueError("need max_new_tokens >= 1 and 0 <= warmup_steps < max_new_tokens")
        lengths = set(cache.host_lengths().values())
        if len(lengths) != 1:
            raise ValueError("every cache layer must hold the same number of tokens")
        for idx in range(len(cache)):
            sl = cache.get_seq_lens(idx)
            if sl is not None and bool((sl != sl[0]).any()):
                raise ValueError("GraphedGreedyDecoder decodes batches whose sequences have one length")
        self.model = model
        self.cache = cache
        self.max_new_tokens = max_new_tokens
        dev = next_token.device
        B = int(next_token.shape[0])
        L0 = lengths.pop()
        cache.make_static(max_new_tokens)
        self._ids = next_token.to(torch.int64).clone()
        self._pos = torch.full((B, 1), L0, dtype=torch.int64, device=dev)
        self._step_idx = torch.zeros(1, dtype=torch.int64, device=dev)
        self.tokens = torch.zeros((B, max_new_tokens), dtype=torch.int64, device=dev)
        self.last_logits = torch.zeros((B, model.config.vocab_size), dtype=torch.float32, device=dev)
        self.done = 0
        self.graph = None
        cfg = model.config
        head_dim = getattr(cfg, "head_dim", None) or cfg.hidden_size // cfg.num_attention_heads
        self._workspace = torch.zeros(
            max(1, ops.decode_workspace_bytes(B, cfg.num_attention_heads, cfg.num_key_value_heads, head_dim,
                                              torch.bfloat16, torch.bfloat16)),
            dtype=torch.uint8, device=dev)
        self._stream = torch.cuda.Stream(device=dev)
        self._stream.wait_stream(torch.cuda.current_stream(dev))
        with torch.no_grad(), torch.cuda.stream(self._stream), _no_mask_creation(model), \
                ops.using_workspace(self._workspace):
            for _ in range(warmup_steps):
                self._body()
                self.done += 1
        # capture: a replay runs the kernels; the Python side effects of the
        # captured call (each layer's host length + 1) are undone and later
        # advanced per replay
        base = cache.host_lengths()
        fused0 = cache.fused_steps
        self.graph = torch.cuda.CUDAGraph()
        with torch.no_grad(), _no_mask_creation(model), ops.using_workspace(self._workspace), \
                torch.cuda.graph(self.graph, stream=self._stream):
            self._body()
        cache.advance_host_lengths(base, 0)
        if cache.fused_steps - fused0 != len(base):
            # some layer took another route (a mask, an unsupported dtype):
            # its launches would replay with the capture's host lengths
            raise RuntimeError(f"captured step ran {cache.fused_steps - fused0} fused decode steps for "
                               f"{len(base)} cache layers; the graph would not advance every layer")
        self._base = base
        self._base_done = self.done
        self._signature = cache.buffer_signature()
        torch.cuda.current_stream(dev).wait_stream(self._stream)

    def _body(self) -> None:
        out = self.model(input_ids=self._ids, position_ids=self._pos, past_key_values=self.cache,
                         use_cache=True, logits_to_keep=1)
        self.last_logits.copy_(out.logits[:, -1])
        nxt = out.logits[:, -1].argmax(-1, keepdim=True)
        self.tokens.index_copy_(1, self._step_idx, nxt)
        self._ids.copy_(nxt)
        self._pos.add_(1)
        self._step_idx.add_(1)

    def step(self) -> None:
        """Replay one decode step on the current stream."""
        if self.done >= self.max_new_tokens:
            raise RuntimeError(f"all {self.max_new_tokens} steps have run")
        if self.cache.buffer_signature() != self._signature:
            raise RuntimeError("the cache's buffers changed since the decode step was captured (a reorder, "
                               "batch select, growth or load); capture a new GraphedGreedyDecoder")
        # an in-place edit keeps the buffers but moves the lengths (a crop):
        # the replay would append at the device positions of the uncropped
        # cache while the host reports the cropped ones
        want = {i: int(b) + (self.done - self._base_done) for i, b in self._base.items()}
        if self.cache.host_lengths() != want:
            raise RuntimeError("the cache's lengths changed since the last decode step (a crop, or tokens "
                               "appended outside the decoder); capture a new GraphedGreedyDecoder")
        self.graph.replay()
        self.done += 1
        self.cache.advance_host_lengths(self._base, self.done - self._base_done)

    def run(self) -> torch.Tensor:
        """Replay the remaining steps; returns the [B, max_new_tokens] tokens."""
        while self.done < self.max_new_tokens:
            self.step()
        return self.tokens
