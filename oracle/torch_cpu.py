"""The reference's KV-cache path on the host CPU, in PyTorch.

TEST INFRASTRUCTURE ONLY.  Only tests/ and the cpu_baseline leg of bench.py
may import this module: it is the timed CPU baseline (PyTorch CPU index_put +
block-table gather + scaled_dot_product_attention, on as many host threads as
torch is given), never part of the product.

  store_kvcache_cpu     store_kvcache_kernel, nanovllm/layers/attention.py:10-30:
                        k_cache.view(-1, D)[slot] = key[t] for slot != -1
                        (index_put on the flat cache views).
  paged_attention_cpu   flash_attn_varlen_func / flash_attn_with_kvcache as
                        called at attention.py:64-74: per sequence, gather the
                        keys through the block table (index_select), then
                        scaled_dot_product_attention in float32 with GQA and the
                        bottom-right aligned causal mask (key j visible to query
                        row i iff j <= i + Lk - Lq); rows that see no key are 0.
  qk_norm_rope_store_cpu  the attention prologue of Qwen3Attention.forward,
                        nanovllm/models/qwen3.py:79-86 (split, RMSNorm.rms_forward
                        layernorm.py:16-26, apply_rotary_emb rotary_embedding.py:6-14
                        as eager tensor operations) and the store of
                        attention.py:62-63 (store_kvcache_cpu).

Pinned by tests/test_oracle_torch_cpu.py against oracle/kv_oracle.py (store
bit for bit, attention to float32 rounding, the prologue to the rounding of
the norm's sum of squares), which the golden vectors and closed forms pin in
turn.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def store_kvcache_cpu(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor,
                      v_cache: torch.Tensor, slot_mapping: torch.Tensor) -> None:
    """key/value [N, Hkv, D]; caches [NB, bs, Hkv, D] (updated in place);
    slot_mapping [N] int32 with -1 = skip."""
    n = key.shape[0]
    d = key.shape[1] * key.shape[2]
    keep = slot_mapping >= 0
    rows = slot_mapping[keep].long()
    k_cache.view(-1, d).index_put_((rows,), key.reshape(n, d)[keep])
    v_cache.view(-1, d).index_put_((rows,), value.reshape(n, d)[keep])


def _gather(cache: torch.Tensor, table: torch.Tensor, n: int) -> torch.Tensor:
    """The first n key rows [n, Hkv, D] of a sequence whose pages are `table`."""
    bs = cache.shape[1]
    pos = torch.arange(n)
    rows = table[pos // bs].long() * bs + pos % bs
    return cache.view(-1, cache.shape[2], cache.shape[3]).index_select(0, rows)


def paged_attention_cpu(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                        cu_seqlens_q, seqlens_k, scale: float,
                        block_tables: torch.Tensor) -> torch.Tensor:
    """q [Tq, Hq, D]; caches [NB, bs, Hkv, D]; block_tables [B, W] int32.
    Sequence s owns query rows cu_seqlens_q[s]:cu_seqlens_q[s+1] and has
    seqlens_k[s] keys.  Returns float32 [Tq, Hq, D]."""
    out = torch.zeros(q.shape, dtype=torch.float32)
    cu_q = [int(x) for x in cu_seqlens_q]
    for s in range(len(cu_q) - 1):
        q0, q1 = cu_q[s], cu_q[s + 1]
        lq, lk = q1 - q0, int(seqlens_k[s])
        if lq == 0 or lk == 0:
            continue
        k = _gather(k_cache, block_tables[s], lk).float().transpose(0, 1)   # [Hkv, Lk, D]
        v = _gather(v_cache, block_tables[s], lk).float().transpose(0, 1)
        qs = q[q0:q1].float().transpose(0, 1)                              # [Hq, Lq, D]
        vis = (torch.arange(lk)[None, :] <= torch.arange(lq)[:, None] + (lk - lq))
        mask = None if bool(vis.all()) else vis
        o = F.scaled_dot_product_attention(qs, k, v, attn_mask=mask, scale=scale,
                                           enable_gqa=True)
        o = o.transpose(0, 1)                                              # [Lq, Hq, D]
        seen = vis.any(dim=1)
        if not bool(seen.all()):
            o = torch.where(seen[:, None, None], o, torch.zeros((), dtype=o.dtype))
        out[q0:q1] = o
    return out


def qk_norm_rope_store_cpu(positions: torch.Tensor, qkv: torch.Tensor, num_q_heads: int,
                           num_kv_heads: int, head_dim: int, q_weight: torch.Tensor,
                           k_weight: torch.Tensor, eps: float, cos_sin: torch.Tensor,
                           k_cache: torch.Tensor, v_cache: torch.Tensor,
                           slot_mapping: torch.Tensor):
    """qkv [T, (Hq + 2 Hkv) D] bf16, positions int64 [T], cos_sin float32
    [max_position, D] (cos | sin halves).  Returns (q, k, v) [T, H, D] bf16
    and stores k, v at slot_mapping (-1 skipped)."""
    t = qkv.shape[0]
    qs, ks = num_q_heads * head_dim, num_kv_heads * head_dim
    q, k, v = qkv.split([qs, ks, ks], dim=-1)
    q, k, v = (q.reshape(t, num_q_heads, head_dim), k.reshape(t, num_kv_heads, head_dim),
               v.reshape(t, num_kv_heads, head_dim))

    def rms(x, w):                                   # layernorm.py:16-26
        dt = x.dtype
        x = x.float()
        var = x.pow(2).mean(dim=-1, keepdim=True)
        x.mul_(torch.rsqrt(var + eps))
        return x.to(dt).mul_(w)

    def rope(x, cos, sin):                           # rotary_embedding.py:6-14
        x1, x2 = torch.chunk(x.float(), 2, dim=-1)
        return torch.cat((x1 * cos - x2 * sin, x2 * cos + x1 * sin), dim=-1).to(x.dtype)

    q, k = rms(q, q_weight), rms(k, k_weight)
    cos, sin = cos_sin[positions].unsqueeze(1).chunk(2, dim=-1)
    q, k = rope(q, cos, sin), rope(k, cos, sin)
    store_kvcache_cpu(k, v, k_cache, v_cache, slot_mapping)
    return q, k, v
