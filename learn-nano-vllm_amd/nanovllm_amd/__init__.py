"""nanovllm_amd — the KV-cache hot path of nano-vLLM on MI355X (gfx950).

Drop-in replacements for the reference's nanovllm/layers/attention.py
(``store_kvcache``, ``Attention``), nanovllm/utils/context.py (``Context`` and
its accessors) and the two flash-attn entry points it imports
(``flash_attn_varlen_func``, ``flash_attn_with_kvcache``), plus the fused
q/k RMSNorm + RoPE + KV-store prologue of qwen3.py:79-86
(``qk_norm_rope_store``), all running on the HIP kernels of libnvk.so through
its C ABI (include/nvk.h).
"""
from nanovllm_amd.utils.context import Context, get_context, set_context, reset_context
from nanovllm_amd.layers.attention import Attention, store_kvcache
from nanovllm_amd.flash_api import (flash_attn_varlen_func, flash_attn_with_kvcache,
                                    varlen_prefill, paged_decode)
from nanovllm_amd.layers.prologue import (qk_norm_rope_store, attention_with_prologue,
                                          paged_decode_with_prologue, rope_cos_sin_cache)

__all__ = ["Context", "get_context", "set_context", "reset_context", "Attention",
           "store_kvcache", "flash_attn_varlen_func", "flash_attn_with_kvcache",
           "varlen_prefill", "paged_decode", "qk_norm_rope_store", "attention_with_prologue",
           "paged_decode_with_prologue", "rope_cos_sin_cache"]
