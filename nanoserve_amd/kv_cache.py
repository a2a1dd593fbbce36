"""Paged KV cache tensors and the HIP cache write.

Layout per layer, K and V held separately (reference kv_cache.py:49-55):

    [num_blocks, block_size, num_kv_heads, head_dim]

`PagedKVCache.write` keeps the reference contract (kv_cache.py:73-81): row t
of key/value lands in slot slot_mapping[t] of the [num_blocks*block_size,
Hkv, D] view, converted to the cache dtype.  The scatter is one HIP launch
covering K and V (`reshape_and_cache`).
"""

from __future__ import annotations

import torch

from . import _lib


def kv_bytes_per_token(num_layers: int, num_kv_heads: int, head_dim: int, dtype: torch.dtype) -> int:
    """K and V bytes one token occupies across all layers (reference kv_cache.py:20-27)."""
    itemsize = torch.tensor([], dtype=dtype).element_size()
    return 2 * num_layers * num_kv_heads * head_dim * itemsize


@torch.inference_mode()
def reshape_and_cache(key: torch.Tensor, value: torch.Tensor,
                      k_cache: torch.Tensor, v_cache: torch.Tensor,
                      slot_mapping: torch.Tensor) -> None:
    """k_cache.view(-1,Hkv,D)[slot_mapping[t]] = key[t].to(cache dtype), same for V.

    key/value: [num_tokens, num_kv_heads, head_dim] (any token/head strides,
    unit head_dim stride); slot_mapping: [num_tokens] int32 or int64 on the
    cache's device.  Slots outside the cache (e.g. -1 padding) are skipped.
    """
    lib = _lib.load()
    if k_cache.dim() != 4 or v_cache.shape != k_cache.shape:
        raise ValueError("caches must be [num_blocks, block_size, num_kv_heads, head_dim]")
    num_blocks, block_size, num_kv_heads, head_dim = k_cache.shape
    if key.dim() != 3 or tuple(key.shape[1:]) != (num_kv_heads, head_dim) or value.shape != key.shape:
        raise ValueError(
            f"key/value must be [T, {num_kv_heads}, {head_dim}], got {tuple(key.shape)}, {tuple(value.shape)}")
    if key.shape[0] != slot_mapping.shape[0]:
        raise ValueError("slot_mapping length differs from the number of tokens")
    if not (k_cache.is_cuda and v_cache.is_cuda and key.is_cuda and value.is_cuda and slot_mapping.is_cuda):
        raise ValueError("reshape_and_cache needs GPU tensors (the HIP path has no CPU fallback)")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("caches must be contiguous")
    if k_cache.dtype != v_cache.dtype or key.dtype != value.dtype:
        raise TypeError("K/V dtypes must match pairwise")
    if key.dtype not in _lib.DTYPE_CODES or k_cache.dtype not in _lib.DTYPE_CODES:
        raise TypeError(f"unsupported dtypes {key.dtype} -> {k_cache.dtype}")
    if key.shape[0] == 0:
        return
    if key.stride(2) != 1:
        key = key.contiguous()
    if value.stride(2) != 1:
        value = value.contiguous()
    slots = slot_mapping
    if slots.dtype not in (torch.int32, torch.int64):
        slots = slots.to(torch.int64)
    slots = slots.contiguous()
    stream = torch.cuda.current_stream(k_cache.device).cuda_stream
    rc = lib.ns_reshape_and_cache(
        key.data_ptr(), value.data_ptr(),
        key.stride(0), key.stride(1), value.stride(0), value.stride(1),
        k_cache.data_ptr(), v_cache.data_ptr(),
        slots.data_ptr(), int(slots.dtype == torch.int64),
        key.shape[0], num_kv_heads, head_dim, block_size, num_blocks,
        _lib.DTYPE_CODES[key.dtype], _lib.DTYPE_CODES[k_cache.dtype], stream)
    _lib.check(rc, "ns_reshape_and_cache")


class PagedKVCache:
    """Per-layer K and V cache tensors (reference kv_cache.py:30-85)."""

    def __init__(
        self,
        num_blocks: int,
        block_size: int,
        num_layers: int,
        num_kv_heads: int,
        head_dim: int,
        dtype: torch.dtype,
        device: str,
    ) -> None:
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.num_layers = num_layers
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.dtype = dtype
        self.device = device

        shape = (num_blocks, block_size, num_kv_heads, head_dim)
        self.k_cache = [torch.zeros(shape, dtype=dtype, device=device) for _ in range(num_layers)]
        self.v_cache = [torch.zeros(shape, dtype=dtype, device=device) for _ in range(num_layers)]

    @property
    def num_bytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in self.k_cache + self.v_cache)

    @property
    def capacity_tokens(self) -> int:
        return self.num_blocks * self.block_size

    def flat(self, layer: int):
        """Views [num_blocks * block_size, Hkv, D] of one layer's K and V."""
        n = self.num_blocks * self.block_size
        return (
            self.k_cache[layer].view(n, self.num_kv_heads, self.head_dim),
            self.v_cache[layer].view(n, self.num_kv_heads, self.head_dim),
        )

    def write(self, layer: int, key: torch.Tensor, value: torch.Tensor, slot_mapping: torch.Tensor) -> None:
        """Scatter this step's K/V rows ([T, Hkv, D]) into their slots."""
        reshape_and_cache(key, value, self.k_cache[layer], self.v_cache[layer], slot_mapping)

    def zero_(self) -> None:
        for t in self.k_cache + self.v_cache:
            t.zero_()
