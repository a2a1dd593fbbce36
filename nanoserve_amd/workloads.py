"""Seeded synthetic paged-attention workloads (the benchmark configurations).

Each config describes one attention call over a paged cache:

  c1  decode, B=8, context U[64,512], Hq14/Hkv2/D64, block 16, fp16,
      block tables a random permutation of exactly 256 physical blocks.
  c2  decode at serving load, B=32, context lognormal(median 1024, sigma 0.8)
      clipped to [16, 8192], same heads, fp16, tables shuffled over a pool of
      1.25x the blocks needed.  (The headline benchmark.)
  c3  mixed batch: 28 decode rows with c2's context law, then 4 sequences
      each prefilling a 512-token chunk on top of a context U[0,2048], causal
      inside the chunk, flattened without padding (T = 2076).
  c4  larger-GQA long-context decode, B=64, Hq28/Hkv4/D128, bf16, context
      lognormal(median 4096, sigma 1.0) clipped to [128, 32768], block 16 or 32.
  c5  the engine's request mix (c5_requests): 32 requests, prompt lengths
      lognormal(median 256, sigma 0.7) clipped to [16, 2048], output lengths
      lognormal(median 128, sigma 0.7) clipped to [8, 1024], random token ids.

Lengths use numpy's lognormal with mu = log(median) truncated to int then
clipped, the convention of the reference workload generator
(nanoserve/workload.py:68-73).  Cache, query values are N(0,1); tables follow
the reference's permuted-pool builders (tests/test_paged_attention.py:39-65,
bench/bench_attention.py:83-121).  Every slot of the pool holds random data,
so slots a sequence does not own behave like stale KV.
"""

from __future__ import annotations

import dataclasses
import math
from dataclasses import dataclass

import numpy as np
import torch

from .attention import AttentionMetadata


@dataclass(frozen=True)
class ConfigSpec:
    name: str
    num_heads: int
    num_kv_heads: int
    head_dim: int
    block_size: int
    dtype: torch.dtype


SPECS = {
    "c1": ConfigSpec("c1", 14, 2, 64, 16, torch.float16),
    "c2": ConfigSpec("c2", 14, 2, 64, 16, torch.float16),
    "c3": ConfigSpec("c3", 14, 2, 64, 16, torch.float16),
    "c4": ConfigSpec("c4", 28, 4, 128, 16, torch.bfloat16),
}


def _lognormal_lengths(rng: np.random.Generator, n: int, median: float, sigma: float,
                       lo: int, hi: int) -> list[int]:
    x = rng.lognormal(np.log(median), sigma, n).astype(int)
    return [int(v) for v in np.clip(x, lo, hi)]


def sample_lengths(config: str, seed: int) -> tuple[list[int], list[int]]:
    """(seq_lens, query_lens) of one call of `config` with `seed`."""
    rng = np.random.default_rng(seed)
    if config == "c1":
        sl = [int(v) for v in rng.integers(64, 512, size=8, endpoint=True)]
        return sl, [1] * 8
    if config == "c2":
        return _lognormal_lengths(rng, 32, 1024, 0.8, 16, 8192), [1] * 32
    if config == "c3":
        dec = _lognormal_lengths(rng, 28, 1024, 0.8, 16, 8192)
        ctx = [int(v) for v in rng.integers(0, 2048, size=4, endpoint=True)]
        return dec + [c + 512 for c in ctx], [1] * 28 + [512] * 4
    if config == "c4":
        return _lognormal_lengths(rng, 64, 4096, 1.0, 128, 32768), [1] * 64
    raise ValueError(f"unknown config {config!r}")


@dataclass
class PagedCase:
    """Inputs of one paged-attention call plus the host-side description."""

    config: str
    seed: int
    query: torch.Tensor
    k_cache: torch.Tensor
    v_cache: torch.Tensor
    md: AttentionMetadata
    scale: float
    seq_lens: list[int]
    query_lens: list[int]
    tables: list[list[int]]

    @property
    def num_kv_heads(self) -> int:
        return self.k_cache.shape[2]

    @property
    def head_dim(self) -> int:
        return self.k_cache.shape[3]

    def kv_bytes(self) -> int:
        """K+V bytes any correct kernel must read: sum_i 2 * L_i * Hkv * D * itemsize."""
        isz = self.k_cache.element_size()
        return sum(2 * L * self.num_kv_heads * self.head_dim * isz for L in self.seq_lens)

    def decode_kv_bytes(self) -> int:
        isz = self.k_cache.element_size()
        return sum(2 * L * self.num_kv_heads * self.head_dim * isz
                   for L, q in zip(self.seq_lens, self.query_lens) if q == 1)

    def prefill_flops(self) -> int:
        """QK^T + PV flops of the causal prefill rows: 4*Hq*D*(ql*ctx + ql(ql+1)/2)."""
        hq = self.query.shape[1]
        tot = 0
        for L, q in zip(self.seq_lens, self.query_lens):
            if q > 1:
                tot += q * (L - q) + q * (q + 1) // 2
        return 4 * hq * self.head_dim * tot


def make_case(config: str, seed: int = 0, device="cpu", block_size: int | None = None,
              dtype: torch.dtype | None = None, gen_device="cpu",
              seq_lens: list[int] | None = None, query_lens: list[int] | None = None,
              pool_factor: float | None = None, num_heads: int | None = None,
              num_kv_heads: int | None = None, head_dim: int | None = None,
              index_dtype: torch.dtype = torch.int64) -> PagedCase:
    """Materialise one call of `config`.

    `gen_device` is where random values are drawn: "cpu" gives values that are
    identical on every machine for a seed (used by parity tests); a GPU device
    is much faster for large replicated benchmark inputs.  Lengths, tables and
    head counts may be overridden for small test variants of a config.
    """
    spec = SPECS[config]
    bs = block_size or spec.block_size
    dt = dtype or spec.dtype
    hq = num_heads or spec.num_heads
    hkv = num_kv_heads or spec.num_kv_heads
    d = head_dim or spec.head_dim
    if seq_lens is None:
        seq_lens, query_lens = sample_lengths(config, seed)
    elif query_lens is None:
        query_lens = [1] * len(seq_lens)

    rng = np.random.default_rng(seed + 7919)
    need = [max(1, -(-L // bs)) for L in seq_lens]
    if config == "c1" and pool_factor is None:
        pool = max(256, sum(need))
    else:
        pool = int(math.ceil((pool_factor or 1.25) * sum(need)))
    perm = rng.permutation(pool).tolist()
    tables, cur = [], 0
    for n in need:
        tables.append(perm[cur:cur + n])
        cur += n

    g = torch.Generator(device=gen_device).manual_seed(seed)
    shape = (pool, bs, hkv, d)
    k_cache = torch.randn(shape, generator=g, device=gen_device, dtype=torch.float32).to(device=device, dtype=dt)
    v_cache = torch.randn(shape, generator=g, device=gen_device, dtype=torch.float32).to(device=device, dtype=dt)
    T = sum(query_lens)
    query = torch.randn((T, hq, d), generator=g, device=gen_device, dtype=torch.float32).to(device=device, dtype=dt)

    md = metadata_for(seq_lens, query_lens, tables, bs, device, index_dtype)
    return PagedCase(config, seed, query, k_cache, v_cache, md, 1.0 / math.sqrt(d),
                     list(seq_lens), list(query_lens), tables)


def make_layer(case: PagedCase, seed: int, gen_device="cpu") -> PagedCase:
    """Another layer of the same serving step: fresh queries and K/V caches of
    the same shapes, the same metadata (block tables, lengths, slots)."""
    g = torch.Generator(device=gen_device).manual_seed(seed)

    def like(t: torch.Tensor) -> torch.Tensor:
        return torch.randn(t.shape, generator=g, device=gen_device, dtype=torch.float32).to(
            device=t.device, dtype=t.dtype)

    return dataclasses.replace(case, query=like(case.query), k_cache=like(case.k_cache),
                               v_cache=like(case.v_cache))


def metadata_for(seq_lens: list[int], query_lens: list[int], tables: list[list[int]],
                 block_size: int, device, index_dtype: torch.dtype = torch.int64) -> AttentionMetadata:
    """Metadata of a flattened batch; tables truncated to ceil(max_seq_len/bs) and zero-padded."""
    qsl = [0]
    for q in query_lens:
        qsl.append(qsl[-1] + q)
    max_seq = max(seq_lens)
    max_blk = max(1, -(-max_seq // block_size))
    bt = torch.zeros(len(seq_lens), max_blk, dtype=index_dtype)
    for i, t in enumerate(tables):
        n = min(len(t), max_blk)
        if n:
            bt[i, :n] = torch.tensor(t[:n], dtype=index_dtype)
    slots = []
    for L, q, t in zip(seq_lens, query_lens, tables):
        for pos in range(L - q, L):
            slots.append(t[pos // block_size] * block_size + pos % block_size)
    return AttentionMetadata(
        slot_mapping=torch.tensor(slots, dtype=torch.int64, device=device),
        query_start_loc=torch.tensor(qsl, dtype=index_dtype, device=device),
        seq_lens=torch.tensor(seq_lens, dtype=index_dtype, device=device),
        block_tables=bt.to(device),
        max_query_len=max(query_lens),
        max_seq_len=max_seq,
        num_seqs=len(seq_lens),
        num_tokens=sum(query_lens),
        is_decode_only=all(q == 1 for q in query_lens),
        query_lens_cpu=list(query_lens),
        seq_lens_cpu=list(seq_lens),
        query_start_loc_cpu=qsl,
    )


def c5_requests(n: int, seed: int, vocab: int) -> list[tuple[list[int], int]]:
    """(prompt token ids, output length) of config 5's requests, by the reference's
    lognormal rule (nanoserve/workload.py:57-75) with random token ids."""
    rng = np.random.default_rng(seed)
    p_lens = np.clip(rng.lognormal(np.log(256), 0.7, n).astype(int), 16, 2048)
    o_lens = np.clip(rng.lognormal(np.log(128), 0.7, n).astype(int), 8, 1024)
    tok = np.random.default_rng(seed + 1)
    return [(tok.integers(0, vocab, int(p)).tolist(), int(o)) for p, o in zip(p_lens, o_lens)]
