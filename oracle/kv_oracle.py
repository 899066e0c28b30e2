"""CPU oracle of the nano-vLLM KV-cache hot path.

TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py may import this module, and only as the parity
reference or the timed CPU baseline.  The product (learn-nano-vllm_amd/nanovllm_amd and
libnvk.so) never calls it: there is no CPU fallback.

What it restates (numpy, bf16 carried as uint16 bit patterns):

  kv_store          store_kvcache_kernel, nanovllm/layers/attention.py:10-30
                    (k_cache.view(-1, D)[slot] = key[t], slot == -1 skipped)
  paged_attention   flash_attn_varlen_func / flash_attn_with_kvcache as called
                    at attention.py:64-74: per sequence, gather the keys through
                    the block table (or take the dense rows), then
                    softmax(scale * q k^T + M) v in float32, GQA kv head = h // G,
                    M the bottom-right aligned causal mask (key j visible to
                    query row i iff j <= i + Lk - Lq); rows that see no key are 0.
  slots_for         the slot formula slot = bt[p // bs] * bs + p % bs used by
                    model_runner.py:151-161, 181.
  rms_norm          RMSNorm.rms_forward, nanovllm/layers/layernorm.py:16-26
                    (bf16 or f16 elements, the model's dtype, model_runner.py:29)
  apply_rotary_emb  rotary_embedding.py:6-14 (x.float(), halves, separately
                    rounded f32 products, bf16 result)
  qk_norm_rope_store  the prologue of Qwen3Attention.forward,
                    nanovllm/models/qwen3.py:79-86, followed by the store of
                    attention.py:62-63
  last_token_rows   ParallelLMHead's prefill selection, embed_head.py:57-59
  sample_tokens     Sampler.forward, nanovllm/layers/sampler.py:7-12, for a
                    given noise tensor (softmax in float32, probs / noise
                    clamped at 1e-10, first maximal index)

How each function is pinned (tests/test_oracle.py):
  kv_store          the guide's worked store example and test matrix
                    (master_nano-vllm-v2.md:2807-2921) and a per-token
                    brute-force loop; invariants (untouched cells, -1 rows, no
                    K/V swap, inputs unmodified, store->gather round trip).
  paged_attention   scalar brute force with math.exp on small cases, torch's
                    CPU scaled_dot_product_attention where the two conventions
                    coincide (Lq == Lk, and Lq == 1), closed forms (one key ->
                    v; constant V -> V; q = 0 -> mean of the visible V rows,
                    which fixes the causal alignment), block-table permutation
                    invariance and the committed golden fixtures.  A planted
                    mistake (top-left mask, h % Hkv head map, missing scale,
                    off-by-one limit) fails at least one of these checks.
  slots_for         the guide's known answer [14,15,0,3,20,21]
                    (master_nano-vllm-v2.md:2766-2776).
  rms_norm          transformers' Qwen3RMSNorm (an independent library routine
                    of the same definition) and closed forms: exact invariance
                    under scaling the row by a power of two (eps = 0), unit
                    mean square for unit weights, sign symmetry.
  apply_rotary_emb  transformers' apply_rotary_pos_emb (rotate-half form) with
                    its own Qwen3 cos/sin, bit for bit in float32; identity at
                    position 0; the relative-position property
                    <R(m)q, R(n)k> = <R(m+s)q, R(n+s)k>; pair norms preserved.
                    A planted mistake (swapped halves, sign flip, interleaved
                    pairs) fails these checks.
  qk_norm_rope_store  composition of the two above plus kv_store, checked
                    against a per-token loop of them.
  last_token_rows   the guide's LM-head example (query lengths [2, 1, 4],
                    cu_seqlens_q [0, 2, 3, 7], last indices [1, 2, 6],
                    master_nano-vllm-v2.md:1222; tests/golden fixture).
  sample_tokens     the exponential-race theorem (P[token = i] = softmax_i,
                    chi-square over numpy Exp(1) draws), unit noise -> argmax
                    of the logits, temperature scaling of the distribution;
                    planted mistakes (noise multiplied, temperature
                    multiplied) fail the chi-square.
"""
from __future__ import annotations

import numpy as np

__all__ = ["bf16_to_f32", "f32_to_bf16", "kv_store", "slots_for", "gather_rows",
           "paged_attention", "rms_norm",
           "apply_rotary_emb", "qk_norm_rope_store", "last_token_rows",
           "sample_tokens"]


# ---------------------------------------------------------------------------
# bf16 helpers (bf16 = upper 16 bits of an IEEE float32)
# ---------------------------------------------------------------------------
def bf16_to_f32(u16: np.ndarray) -> np.ndarray:
    return (np.asarray(u16, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even float32 -> bf16 bits (NaN kept quiet)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    out = rounded.astype(np.uint16)
    nan = np.isnan(x)
    out[nan] = 0x7FC0
    return out


# ---------------------------------------------------------------------------
# KV-store scatter
# ---------------------------------------------------------------------------
def kv_store(key: np.ndarray, value: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray,
             slot_mapping: np.ndarray) -> None:
    """In place: k_cache.reshape(-1, D)[slot] = key.reshape(N, D)[t] for slot != -1.

    attention.py:21-30: one program per token, ``if slot == -1: return``, then a
    contiguous D-element copy to ``slot * D``.  key/value: [N, ...] (any row
    shape of D elements); caches: any shape whose trailing dims hold D per slot.
    """
    n = key.shape[0]
    slots = np.asarray(slot_mapping).astype(np.int64).reshape(-1)
    assert slots.shape[0] == n
    d = int(np.prod(key.shape[1:])) if key.ndim > 1 else 1
    kc = k_cache.reshape(-1, d)
    vc = v_cache.reshape(-1, d)
    valid = slots != -1
    if np.any(slots[valid] < 0) or np.any(slots[valid] >= kc.shape[0]):
        raise ValueError("slot outside the cache (undefined in the reference)")
    kc[slots[valid]] = key.reshape(n, d)[valid]
    vc[slots[valid]] = value.reshape(n, d)[valid]


def slots_for(block_table, positions, block_size: int) -> list[int]:
    """slot = block_table[p // bs] * bs + p % bs (model_runner.py:151-161, 181)."""
    return [int(block_table[p // block_size]) * block_size + p % block_size for p in positions]


def gather_rows(cache: np.ndarray, block_table, length: int, block_size: int) -> np.ndarray:
    """Rows of one sequence's first ``length`` positions from a paged cache
    [NB, bs, ...] (the guide's gather reference, master_nano-vllm-v2.md:2923-2944)."""
    flat = cache.reshape(cache.shape[0] * cache.shape[1], *cache.shape[2:])
    idx = np.asarray(slots_for(block_table, range(length), block_size), dtype=np.int64)
    return flat[idx]


# ---------------------------------------------------------------------------
# Attention
# ---------------------------------------------------------------------------
def _attend(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float, diag: int,
            _mutation: str | None) -> np.ndarray:
    """One sequence.  q [Lq, Hq, D], k/v [Lk, Hkv, D] float32 -> [Lq, Hq, D]."""
    lq, hq, d = q.shape
    lk, hkv = k.shape[0], k.shape[1]
    g = hq // hkv
    out = np.zeros((lq, hq, d), dtype=np.float32)
    if lq == 0 or lk == 0:
        return out
    i = np.arange(lq)[:, None]
    j = np.arange(lk)[None, :]
    if _mutation == "top_left":
        visible = j <= i
    elif _mutation == "strict":
        visible = j < i + diag
    else:
        visible = j <= i + diag                     # bottom-right aligned causal
    eff_scale = 1.0 if _mutation == "no_scale" else scale
    for h in range(hq):
        kvh = h % hkv if _mutation == "gqa_mod" else h // g
        s = (q[:, h, :] @ k[:, kvh, :].T) * np.float32(eff_scale)      # [Lq, Lk]
        s = np.where(visible, s, -np.inf)
        m = s.max(axis=1, keepdims=True)
        has = np.isfinite(m[:, 0])
        p = np.exp(s - np.where(np.isfinite(m), m, 0.0))
        l = p.sum(axis=1, keepdims=True)
        o = (p @ v[:, kvh, :]) / np.where(l > 0, l, 1.0)
        out[:, h, :] = np.where(has[:, None], o, 0.0)
    return out


def _as_f32(x: np.ndarray) -> np.ndarray:
    """float arrays as float32; uint16 arrays are bf16 bit patterns."""
    return bf16_to_f32(x) if x.dtype == np.uint16 else x.astype(np.float32)


def paged_attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, cu_seqlens_q, seqlens_k,
                    scale: float, block_tables: np.ndarray | None = None, block_size: int = 0,
                    cu_seqlens_k=None, _mutation: str | None = None) -> np.ndarray:
    """Varlen causal attention, float32.

    q, k, v: float arrays, or uint16 arrays holding bf16 bit patterns (only the
    rows a sequence reads are widened).
    q: [Tq, Hq, D].  Sequence s owns query rows cu_seqlens_q[s]:cu_seqlens_q[s+1]
    and has seqlens_k[s] keys.  Paged (block_tables given): k/v are caches
    [NB, bs, Hkv, D] and key p of sequence s is at page block_tables[s][p // bs].
    Dense: k/v are [Tk, Hkv, D] and sequence s's keys are rows
    cu_seqlens_k[s]:cu_seqlens_k[s+1].  Decode is the case Lq == 1.
    ``_mutation`` plants a known mistake; only the oracle's own tests use it.
    """
    cu_q = np.asarray(cu_seqlens_q, dtype=np.int64)
    lens_k = np.asarray(seqlens_k, dtype=np.int64)
    out = np.zeros(q.shape, dtype=np.float32)
    for s in range(cu_q.shape[0] - 1):
        q0, q1 = int(cu_q[s]), int(cu_q[s + 1])
        lk = int(lens_k[s])
        if block_tables is not None:
            ks = gather_rows(k, block_tables[s], lk, block_size)
            vs = gather_rows(v, block_tables[s], lk, block_size)
        else:
            k0 = int(cu_seqlens_k[s])
            ks, vs = k[k0:k0 + lk], v[k0:k0 + lk]
        lq = q1 - q0
        out[q0:q1] = _attend(_as_f32(q[q0:q1]), _as_f32(ks), _as_f32(vs), scale, lk - lq,
                             _mutation)
    return out


# ---------------------------------------------------------------------------
# Attention prologue: q/k RMSNorm + RoPE (+ the KV store)
# ---------------------------------------------------------------------------
def f16_to_f32(u16: np.ndarray) -> np.ndarray:
    """float16 bit patterns (uint16) -> float32 (exact)."""
    return np.asarray(u16, dtype=np.uint16).view(np.float16).astype(np.float32)


def f32_to_f16(x: np.ndarray) -> np.ndarray:
    """float32 -> float16 bit patterns, round to nearest even."""
    return np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


# 16-bit element types of the model (model_runner.py:29): widen, round
_ELT = {"bf16": (bf16_to_f32, f32_to_bf16), "f16": (f16_to_f32, f32_to_f16)}


def rms_norm(x_bits: np.ndarray, weight_bits: np.ndarray, eps: float,
             _mutation: str | None = None, elt: str = "bf16") -> np.ndarray:
    """RMSNorm over the last dim, T in / T out (layernorm.py:16-26), T the
    element type `elt` ("bf16" or "f16", bit patterns as uint16):
    x = x.float(); x *= rsqrt(mean(x^2) + eps); x = T(x) * weight -> T.
    rsqrt is evaluated in float64 and rounded once to float32."""
    widen, narrow = _ELT[elt]
    x = widen(x_bits)
    var = np.mean(x * x, axis=-1, keepdims=True, dtype=np.float32)
    if _mutation == "sum":
        var = np.sum(x * x, axis=-1, keepdims=True, dtype=np.float32)
    rstd = (1.0 / np.sqrt((var + np.float32(eps)).astype(np.float64))).astype(np.float32)
    normed = narrow(x * rstd)
    w = widen(weight_bits)
    return narrow(widen(normed) * w)


def apply_rotary_emb(x_bits: np.ndarray, cos: np.ndarray, sin: np.ndarray,
                     _mutation: str | None = None, elt: str = "bf16") -> np.ndarray:
    """rotary_embedding.py:6-14: x1, x2 = halves of x.float();
    y1 = x1*cos - x2*sin, y2 = x2*cos + x1*sin (each product and sum rounded to
    float32), cat -> T (`elt`).  cos/sin broadcast against x's halves."""
    widen, narrow = _ELT[elt]
    x = widen(x_bits)
    h = x.shape[-1] // 2
    if _mutation == "interleaved":
        x1, x2 = x[..., 0::2], x[..., 1::2]
    else:
        x1, x2 = x[..., :h], x[..., h:]
    c = np.asarray(cos, dtype=np.float32)
    s = np.asarray(sin, dtype=np.float32)
    if _mutation == "sign":
        s = -s
    y1 = (x1 * c).astype(np.float32) - (x2 * s).astype(np.float32)
    y2 = (x2 * c).astype(np.float32) + (x1 * s).astype(np.float32)
    if _mutation == "swap":
        y1, y2 = y2, y1
    if _mutation == "interleaved":
        y = np.empty_like(x)
        y[..., 0::2], y[..., 1::2] = y1, y2
        return narrow(y)
    return narrow(np.concatenate([y1, y2], axis=-1))


def qk_norm_rope_store(qkv_bits: np.ndarray, positions, q_weight_bits: np.ndarray,
                       k_weight_bits: np.ndarray, eps: float, cos_sin: np.ndarray,
                       num_q_heads: int, num_kv_heads: int, head_dim: int,
                       k_cache: np.ndarray | None = None, v_cache: np.ndarray | None = None,
                       slot_mapping=None, elt: str = "bf16"):
    """qwen3.py:79-86 + attention.py:62-63 on bit patterns of the element type
    `elt` ("bf16" or "f16").

    qkv_bits [T, (Hq + 2*Hkv)*D]; cos_sin float32 [max_position, D] (cos | sin
    halves).  Returns (q [T,Hq,D], k [T,Hkv,D], v [T,Hkv,D]) as uint16; with
    caches and slot_mapping given, k and v are stored as kv_store does."""
    t = qkv_bits.shape[0]
    qs, ks = num_q_heads * head_dim, num_kv_heads * head_dim
    q = qkv_bits[:, :qs].reshape(t, num_q_heads, head_dim)
    k = qkv_bits[:, qs:qs + ks].reshape(t, num_kv_heads, head_dim)
    v = np.ascontiguousarray(qkv_bits[:, qs + ks:qs + 2 * ks]).reshape(t, num_kv_heads, head_dim)
    q = rms_norm(q, q_weight_bits, eps, elt=elt)
    k = rms_norm(k, k_weight_bits, eps, elt=elt)
    cs = np.asarray(cos_sin, dtype=np.float32)[np.asarray(positions, dtype=np.int64)]
    cos, sin = cs[:, None, :head_dim // 2], cs[:, None, head_dim // 2:]
    q = apply_rotary_emb(q, cos, sin, elt=elt)
    k = apply_rotary_emb(k, cos, sin, elt=elt)
    if k_cache is not None and slot_mapping is not None:
        kv_store(k, v, k_cache, v_cache, slot_mapping)
    return q, k, v


# ---------------------------------------------------------------------------
# LM-head last-token selection and the sampler
# ---------------------------------------------------------------------------
def last_token_rows(x: np.ndarray, cu_seqlens_q) -> np.ndarray:
    """x[cu_seqlens_q[1:] - 1] (embed_head.py:57-59)."""
    cu = np.asarray(cu_seqlens_q, dtype=np.int64)
    return x[cu[1:] - 1]


def sample_tokens(logits: np.ndarray, temperatures, noise: np.ndarray,
                  _mutation: str | None = None) -> np.ndarray:
    """sampler.py:7-12 with the Exp(1) draw given: probs = softmax(logits.float()
    / T) in float32, probs / max(noise, 1e-10), argmax (first maximal index).
    logits: float array or uint16 bf16 bit patterns [B, V]."""
    x = bf16_to_f32(logits) if logits.dtype == np.uint16 else logits.astype(np.float32)
    t = np.asarray(temperatures, dtype=np.float32)[:, None]
    x = x * t if _mutation == "temp_mul" else x / t
    m = x.max(axis=1, keepdims=True)
    p = np.exp(x - m)
    p = (p / p.sum(axis=1, keepdims=True)).astype(np.float32)
    e = np.maximum(np.asarray(noise, dtype=np.float32), np.float32(1e-10))
    q = p * e if _mutation == "noise_mul" else p / e
    return np.argmax(q, axis=1).astype(np.int64)
