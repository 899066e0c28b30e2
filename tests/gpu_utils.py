"""Helpers shared by the GPU parity tests (not collected by pytest)."""
import os
import sys

import numpy as np
import torch

from oracle import kv_oracle as orc

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
# Attention tolerance: bf16 inputs/outputs, f32 accumulation, against the f32 oracle.
ATOL, RTOL = 2e-2, 1e-2


def say(msg: str) -> None:
    """Name the case on stdout before a GPU step (so a fault is attributable)."""
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def bits(t: torch.Tensor) -> np.ndarray:
    """bf16 tensor -> uint16 bit pattern array (CPU)."""
    return t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def f32(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def from_bits(a: np.ndarray, device="cuda") -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).to(device)


def assert_attn_close(out: torch.Tensor, ref: np.ndarray, what: str = "") -> None:
    got = out.detach().float().cpu()
    exp = torch.from_numpy(np.asarray(ref, dtype=np.float32)).reshape(got.shape)
    assert torch.isfinite(got).all(), f"{what}: non-finite output"
    torch.testing.assert_close(got, exp, atol=ATOL, rtol=RTOL, msg=lambda m: f"{what}: {m}")


def assert_rotated_close(got_bits: np.ndarray, ref_bits: np.ndarray, what: str = "",
                         elt: str = "bf16") -> None:
    """Normed + rotated rows (last dim D) of element type `elt` against the
    oracle: bit-exact but for < 0.1 % of elements where sum-of-squares / rsqrt
    rounding moved a normed value across a rounding boundary of the type,
    which stay within 2 ulps of the rotated pair, |diff| <= 2^-6 (bf16) or
    2^-9 (f16) * (|x1| + |x2|)."""
    widen = orc.bf16_to_f32 if elt == "bf16" else orc.f16_to_f32
    got = widen(got_bits).astype(np.float64)
    ref = widen(ref_bits).astype(np.float64)
    same = got_bits == ref_bits
    assert same.mean() > 0.999, f"{what}: {(~same).sum()} of {same.size} differ"
    h = ref.shape[-1] // 2
    scale = np.abs(ref[..., :h]) + np.abs(ref[..., h:])
    scale = np.concatenate([scale, scale], axis=-1)
    bad = np.abs(got - ref) > (2.0 ** -6 if elt == "bf16" else 2.0 ** -9) * scale + 1e-30
    assert not bad.any(), f"{what}: {bad.sum()} elements beyond 2 bf16 ulps"


def oracle_decode(q, k_cache, v_cache, block_tables, context_lens, block_size, scale):
    """Oracle for one query per sequence; all args CPU tensors."""
    b = q.shape[0]
    return orc.paged_attention(f32(q), f32(k_cache), f32(v_cache), np.arange(b + 1),
                               context_lens.numpy(), scale, block_tables=block_tables.numpy(),
                               block_size=block_size)


def oracle_paged_bits(q, k_cache, v_cache, block_tables, cu_q, lens_k, block_size, scale):
    """Oracle over bf16 tensors passed as bit patterns, so that only the rows a
    sequence reads are widened (large caches); any device."""
    return orc.paged_attention(bits(q), bits(k_cache), bits(v_cache),
                               np.asarray(cu_q.cpu() if hasattr(cu_q, "cpu") else cu_q),
                               np.asarray(lens_k.cpu() if hasattr(lens_k, "cpu") else lens_k),
                               scale, block_tables=block_tables.cpu().numpy(),
                               block_size=block_size)


def oracle_prefill_paged(q, k_cache, v_cache, block_tables, cu_q, cu_k, block_size, scale):
    lens_k = np.diff(cu_k.numpy())
    return orc.paged_attention(f32(q), f32(k_cache), f32(v_cache), cu_q.numpy(), lens_k, scale,
                               block_tables=block_tables.numpy(), block_size=block_size)


def oracle_prefill_dense(q, k, v, cu_q, cu_k, scale):
    lens_k = np.diff(cu_k.numpy())
    return orc.paged_attention(f32(q), f32(k), f32(v), cu_q.numpy(), lens_k, scale,
                               cu_seqlens_k=cu_k.numpy())


def oracle_store(key, value, k_cache, v_cache, slot_mapping):
    """Returns the expected caches as uint16 bit arrays (inputs untouched)."""
    kc, vc = bits(k_cache).copy(), bits(v_cache).copy()
    orc.kv_store(bits(key), bits(value), kc, vc, slot_mapping.cpu().numpy())
    return kc, vc
