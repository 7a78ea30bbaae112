"""kvint4 — MI355X-native (gfx950) INT4 KV-cache decode path.

Drop-in for the hot path of johnchmura/kv-cache-triton:

    reference module                    this package
    kernels.llama3.quantize         ->  kvint4.llama3.quantize
    kernels.llama3.attention_quant  ->  kvint4.llama3.attention_quant
    models.llama3.kv_cache          ->  kvint4.llama3.kv_cache
    models.llama3.llama3_quant      ->  kvint4.llama3.llama3_quant
    kernels.gpt2.quantize           ->  kvint4.gpt2.quantize
    kernels.gpt2.attention_quant    ->  kvint4.gpt2.attention_quant
    models.gpt2.kv_cache            ->  kvint4.gpt2.kv_cache
    models.gpt2.gpt2_quant          ->  kvint4.gpt2.gpt2_quant

All compute runs in hand-written HIP kernels (libkvint4.so, C ABI in
include/kvint4.h) on GPU tensors; there is no CPU path.
"""

__version__ = "0.1.0"
