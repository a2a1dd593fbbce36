"""Rotary embedding fused with the paged-cache write.

The reference applies RoPE to Q and K with tensor arithmetic and then writes
K and V into the cache (reference nanoserve/qwen2.py:52-57):

    q, k = rotary.apply(q, k, cos, sin)          # layers.py:86-90
    kv_cache.write(layer, k, v, md.slot_mapping)  # kv_cache.py:73-81

`RotaryEmbedding.apply_and_cache` does both in one HIP launch
(`ns_rope_reshape_and_cache`) and returns the rotated Q; the rotated K only
ever exists in its cache slots.  Results are bit-identical to the two-step
reference on the same inputs: the kernel rounds after every multiply and add
exactly as the reference's f16/bf16 tensor ops do.

The cos/sin table and its per-forward lookup keep the reference's definition
(layers.py:65-80): cos/sin are looked up once per forward pass for all layers.
"""

from __future__ import annotations

import torch

from . import _lib


class RotaryEmbedding:
    """RoPE, NeoX/HF convention: rotate_half over the two contiguous halves.

    Same table as the reference (layers.py:65-73): inv_freq[i] =
    1 / base**(2i/head_dim), emb = cat(freqs, freqs), cos/sin in float32 for
    max_position positions.
    """

    def __init__(self, head_dim: int, max_position: int, base: float = 10000.0, device="cpu") -> None:
        if head_dim % 2:
            raise ValueError("head_dim must be even")
        self.head_dim = head_dim
        self.max_position = max_position
        inv_freq = 1.0 / (base ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
        t = torch.arange(max_position, dtype=torch.float32)
        freqs = torch.outer(t, inv_freq)
        emb = torch.cat((freqs, freqs), dim=-1)
        self.cos_cached = emb.cos().to(device)
        self.sin_cached = emb.sin().to(device)
        self._stack_tables()

    def _stack_tables(self) -> None:
        # cos and sin side by side, [max_position, 2, head_dim], once per
        # dtype: the float32 values rounded once, as the reference's per-step
        # `.to(dtype)` rounds them, so one gather per forward pass yields both.
        both = torch.stack((self.cos_cached, self.sin_cached), dim=1)
        self._tables = {dt: both.to(dt) for dt in (torch.float16, torch.bfloat16)}
        self._tables[torch.float32] = both

    def to(self, device) -> "RotaryEmbedding":
        self.cos_cached = self.cos_cached.to(device)
        self.sin_cached = self.sin_cached.to(device)
        self._stack_tables()
        return self

    def cos_sin(self, positions: torch.Tensor, dtype: torch.dtype):
        """Once per forward pass: cos, sin as [T, 1, head_dim] in `dtype` (layers.py:75-79).

        Both are views of one gathered [T, 2, head_dim] tensor (row stride
        2 * head_dim), the values of the reference's gather-then-convert."""
        table = self._tables.get(dtype)
        if table is None:
            both = torch.stack((self.cos_cached, self.sin_cached), dim=1)
            table = both.to(dtype)
        cs = table.index_select(0, positions)
        return cs[:, 0:1, :], cs[:, 1:2, :]

    @staticmethod
    def apply_and_cache(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                        cos: torch.Tensor, sin: torch.Tensor,
                        k_cache: torch.Tensor, v_cache: torch.Tensor,
                        slot_mapping: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
        """Rotate q and k, write rotated k and v into their slots, return rotated q."""
        return rope_reshape_and_cache(q, k, v, cos, sin, k_cache, v_cache, slot_mapping, out=out)


def _rows(x: torch.Tensor, heads: int, head_dim: int, name: str) -> torch.Tensor:
    if x.dim() != 3 or tuple(x.shape[1:]) != (heads, head_dim):
        raise ValueError(f"{name} must be [T, {heads}, {head_dim}], got {tuple(x.shape)}")
    return x if x.stride(2) == 1 else x.contiguous()


def _table(x: torch.Tensor, T: int, head_dim: int, name: str) -> torch.Tensor:
    """cos/sin as [T, head_dim] rows with a unit element stride (accepts [T,1,D] or [T,D])."""
    if x.dim() == 3 and x.shape[1] == 1:
        x = x[:, 0, :]
    if x.dim() != 2 or tuple(x.shape) != (T, head_dim):
        raise ValueError(f"{name} must be [T, 1, {head_dim}] or [T, {head_dim}], got {tuple(x.shape)}")
    return x if x.stride(1) == 1 else x.contiguous()


@torch.inference_mode()
def rope_reshape_and_cache(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                           cos: torch.Tensor, sin: torch.Tensor,
                           k_cache: torch.Tensor, v_cache: torch.Tensor,
                           slot_mapping: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """Fused `rotary.apply` + `PagedKVCache.write` (reference qwen2.py:53-57).

    q: [T, Hq, D]; k, v: [T, Hkv, D] (any token/head strides with a unit
    head_dim stride, e.g. views of one fused QKV projection); cos, sin:
    [T, 1, D] in q's dtype; caches [num_blocks, block_size, Hkv, D].  Slots
    outside the cache (e.g. -1 padding) are skipped.  Returns rotated q as a
    contiguous [T, Hq, D] tensor: `out` when given (it may be q itself when q
    is contiguous), else a new tensor.
    """
    lib = _lib.load()
    if k_cache.dim() != 4 or v_cache.shape != k_cache.shape:
        raise ValueError("caches must be [num_blocks, block_size, num_kv_heads, head_dim]")
    num_blocks, block_size, Hkv, D = k_cache.shape
    if q.dim() != 3 or q.shape[2] != D:
        raise ValueError(f"q must be [T, Hq, {D}], got {tuple(q.shape)}")
    T, Hq = q.shape[0], q.shape[1]
    q = _rows(q, Hq, D, "q")
    k = _rows(k, Hkv, D, "k")
    v = _rows(v, Hkv, D, "v")
    if k.shape[0] != T or v.shape[0] != T or slot_mapping.shape[0] != T:
        raise ValueError("q, k, v and slot_mapping must have the same number of tokens")
    if not (q.dtype == k.dtype == v.dtype == cos.dtype == sin.dtype):
        raise TypeError("q, k, v, cos and sin must share one dtype")
    if k_cache.dtype != v_cache.dtype:
        raise TypeError("K and V caches must share one dtype")
    if q.dtype not in _lib.DTYPE_CODES or k_cache.dtype not in _lib.DTYPE_CODES:
        raise TypeError(f"unsupported dtypes {q.dtype} -> {k_cache.dtype}")
    tensors = (q, k, v, cos, sin, k_cache, v_cache, slot_mapping)
    if not all(t.is_cuda for t in tensors):
        raise ValueError("rope_reshape_and_cache needs GPU tensors (the HIP path has no CPU fallback)")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("caches must be contiguous")
    if out is None:
        out = torch.empty((T, Hq, D), dtype=q.dtype, device=q.device)
    elif out.shape != (T, Hq, D) or out.dtype != q.dtype or not out.is_contiguous():
        raise ValueError(f"out must be a contiguous [{T}, {Hq}, {D}] {q.dtype} tensor")
    elif out.data_ptr() == q.data_ptr() and not q.is_contiguous():
        raise ValueError("out may alias q only when q is contiguous")
    if T == 0:
        return out
    cos = _table(cos, T, D, "cos")
    sin = _table(sin, T, D, "sin")
    if cos.stride(0) != sin.stride(0):
        sin = sin.contiguous()
        cos = cos.contiguous()
    slots = slot_mapping
    if slots.dtype not in (torch.int32, torch.int64):
        slots = slots.to(torch.int64)
    slots = slots.contiguous()
    stream = torch.cuda.current_stream(q.device).cuda_stream
    rc = lib.ns_rope_reshape_and_cache(
        out.data_ptr(), q.data_ptr(), q.stride(0), q.stride(1),
        k.data_ptr(), k.stride(0), k.stride(1),
        v.data_ptr(), v.stride(0), v.stride(1),
        cos.data_ptr(), sin.data_ptr(), cos.stride(0),
        k_cache.data_ptr(), v_cache.data_ptr(),
        slots.data_ptr(), int(slots.dtype == torch.int64),
        T, Hq, Hkv, D, block_size, num_blocks,
        _lib.DTYPE_CODES[q.dtype], _lib.DTYPE_CODES[k_cache.dtype], stream)
    _lib.check(rc, "ns_rope_reshape_and_cache")
    return out
