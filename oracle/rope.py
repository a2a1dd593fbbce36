"""CPU oracle for the fused rotary + cache write -- TEST INFRASTRUCTURE ONLY.

  rope_table_ref        reference nanoserve/layers.py:65-73 (cos/sin table)
  rope_cos_sin_ref      reference nanoserve/layers.py:75-79 (per-forward lookup)
  rotate_half_ref       reference nanoserve/layers.py:81-84
  rope_apply_ref        reference nanoserve/layers.py:86-90 (tensor arithmetic)
  rope_apply_bits       independent numpy restatement of rope_apply_ref with
                        one explicit rounding per tensor op
  rope_reshape_and_cache_ref
                        reference nanoserve/qwen2.py:53-57: rope_apply_ref,
                        then PagedKVCache.write (kv_cache.py:73-81)

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this
module, and only as the checker.

Parity pinning (tests/test_oracle_rope.py):
  rope_apply_ref  bit-exact against rope_apply_bits (numpy's own float16
                  arithmetic, an integer bfloat16 rounding, numpy float32) on
                  random and special values; closed forms cos=1/sin=0
                  (identity) and cos=0/sin=1 (rotate_half); in float64 the
                  rotation preserves each (x[i], x[i+D/2]) pair's norm and
                  composes (position a then b == position a+b).
  rope_table_ref  against math.cos/math.sin of pos * base**(-2i/D) in float64.
  rotate_half_ref against a per-index loop.
The reference ships no rotary tests or vectors; tests/golden/rope_*.npz are
fixtures written by this oracle (tests/golden/make_golden.py).
"""

from __future__ import annotations

import numpy as np
import torch

from .paged_attention import bf16_bits_ref, reshape_and_cache_ref


def rope_table_ref(head_dim: int, max_position: int, base: float = 10000.0):
    """float32 cos/sin tables [max_position, head_dim] (layers.py:65-73)."""
    inv_freq = 1.0 / (base ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
    t = torch.arange(max_position, dtype=torch.float32)
    freqs = torch.outer(t, inv_freq)
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos(), emb.sin()


def rope_cos_sin_ref(cos_cached, sin_cached, positions, dtype):
    """[T, 1, D] cos/sin for `positions`, cast to `dtype` (layers.py:75-79)."""
    pos = positions.detach().cpu().to(torch.int64)
    cos = cos_cached.index_select(0, pos).unsqueeze(1).to(dtype)
    sin = sin_cached.index_select(0, pos).unsqueeze(1).to(dtype)
    return cos, sin


def rotate_half_ref(x: torch.Tensor) -> torch.Tensor:
    """cat(-x[..., D/2:], x[..., :D/2]) (layers.py:81-84)."""
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


@torch.inference_mode()
def rope_apply_ref(q, k, cos, sin):
    """q*cos + rotate_half(q)*sin and the same for k, on CPU copies (layers.py:86-90)."""
    q, k = q.detach().cpu(), k.detach().cpu()
    cos, sin = cos.detach().cpu(), sin.detach().cpu()
    return q * cos + rotate_half_ref(q) * sin, k * cos + rotate_half_ref(k) * sin


def _round(x: np.ndarray, dtype: str) -> np.ndarray:
    """float32 values rounded to `dtype` and returned as float32."""
    if dtype == "float32":
        return x.astype(np.float32)
    if dtype == "float16":
        return x.astype(np.float32).astype(np.float16).astype(np.float32)
    bits = bf16_bits_ref(x).astype(np.uint32) << 16
    return bits.view(np.float32)


def rope_apply_bits(x: np.ndarray, cos: np.ndarray, sin: np.ndarray, dtype: str) -> np.ndarray:
    """Rotate x ([..., D], values exact in `dtype`, given as float32) with one rounding per op.

    Each tensor op of the reference on float16/bfloat16 tensors computes in
    float32 and rounds to the tensor dtype:
        out[:h] = R(R(x[:h]*cos[:h]) + R(-x[h:]*sin[:h]))
        out[h:] = R(R(x[h:]*cos[h:]) + R( x[:h]*sin[h:]))
    Written with numpy and explicit rounding only, sharing no code with torch.
    """
    x = np.asarray(x, np.float32)
    cos = np.broadcast_to(np.asarray(cos, np.float32), x.shape)
    sin = np.broadcast_to(np.asarray(sin, np.float32), x.shape)
    h = x.shape[-1] // 2
    x1, x2 = x[..., :h], x[..., h:]
    lo = _round(_round(x1 * cos[..., :h], dtype) + _round(-x2 * sin[..., :h], dtype), dtype)
    hi = _round(_round(x2 * cos[..., h:], dtype) + _round(x1 * sin[..., h:], dtype), dtype)
    return np.concatenate([lo, hi], axis=-1)


@torch.inference_mode()
def rope_reshape_and_cache_ref(q, k, v, cos, sin, k_cache, v_cache, slot_mapping):
    """Rotated q plus the caches after writing rotated k and v (qwen2.py:53-57).

    Slots outside the cache are dropped before the write, as the HIP path skips
    them (the reference never produces such slots for real tokens).
    """
    qr, kr = rope_apply_ref(q, k, cos, sin)
    slots = slot_mapping.detach().cpu().to(torch.int64)
    NB, BS = k_cache.shape[:2]
    keep = (slots >= 0) & (slots < NB * BS)
    kc, vc = reshape_and_cache_ref(kr[keep], v.detach().cpu()[keep], k_cache, v_cache, slots[keep])
    return qr, kc, vc
