"""nanoserve_amd: MI355X-native paged attention for nanoserve.

The package replaces the GPU side of nanoserve's attention op and KV-cache
write with hand-written gfx950 HIP kernels behind a C ABI
(include/nanoserve_paged.h), keeping the reference's call contract:

  attn_fn(query, k_cache, v_cache, md, scale) -> out   (paged_attention_hip)
  PagedKVCache.write(layer, key, value, slot_mapping)  (reshape_and_cache)
  BlockSpaceManager.slot_mapping(seq, start, end)      (addressing contract)
  rotary.apply + PagedKVCache.write fused              (rope_reshape_and_cache)
"""

from .attention import AttentionMetadata, get_attention_backend, paged_attention_hip
from .block_manager import BlockSpaceManager
from .kv_cache import PagedKVCache, kv_bytes_per_token, reshape_and_cache
from .rotary import RotaryEmbedding, rope_reshape_and_cache

__version__ = "0.1.0"

__all__ = [
    "AttentionMetadata",
    "BlockSpaceManager",
    "PagedKVCache",
    "get_attention_backend",
    "kv_bytes_per_token",
    "paged_attention_hip",
    "reshape_and_cache",
    "RotaryEmbedding",
    "rope_reshape_and_cache",
]
