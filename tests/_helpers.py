"""Case builders shared by the CPU and GPU test modules.

`build_paged` lays random per-sequence K/V into a cache at scattered physical
blocks (the reference's `build`, tests/test_paged_attention.py:39-65) and
`make_md` builds metadata with int32 tables (test_paged_attention.py:68-94);
both also take an index dtype so the engine's int64 contract is covered.
"""

from __future__ import annotations

import torch

from nanoserve_amd.attention import AttentionMetadata


def build_paged(seqs, num_blocks, block_size, num_kv_heads, head_dim, dtype=torch.float32,
                seed=1234, shuffle=True, fill=0.0):
    """Return (k_cache, v_cache, tables, truth) on the CPU.

    truth[i] = (K_i, V_i), each [seq_len_i, Hkv, D] in `dtype`.  Slots no
    sequence owns hold `fill`.
    """
    g = torch.Generator().manual_seed(seed)
    gp = torch.Generator().manual_seed(seed + 1)  # placement drawn apart from values
    shape = (num_blocks, block_size, num_kv_heads, head_dim)
    kc = torch.full(shape, fill, dtype=dtype)
    vc = torch.full(shape, fill, dtype=dtype)
    kf = kc.view(num_blocks * block_size, num_kv_heads, head_dim)
    vf = vc.view(num_blocks * block_size, num_kv_heads, head_dim)
    perm = torch.randperm(num_blocks, generator=gp).tolist() if shuffle else list(range(num_blocks))
    cur = 0
    tables, truth = [], []
    for sl in seqs:
        nb = -(-sl // block_size)
        table = perm[cur:cur + nb]
        cur += nb
        K = torch.randn(sl, num_kv_heads, head_dim, generator=g).to(dtype)
        V = torch.randn(sl, num_kv_heads, head_dim, generator=g).to(dtype)
        slots = torch.tensor([table[p // block_size] * block_size + p % block_size for p in range(sl)],
                             dtype=torch.long)
        if sl:
            kf.index_copy_(0, slots, K)
            vf.index_copy_(0, slots, V)
        tables.append(table)
        truth.append((K, V))
    return kc, vc, tables, truth


def make_md(seqs, query_lens, tables, block_size, device="cpu", index_dtype=torch.int32,
            with_cpu_lists=True):
    qsl = [0]
    for q in query_lens:
        qsl.append(qsl[-1] + q)
    max_seq = max(seqs)
    max_blk = max(1, -(-max_seq // block_size))
    bt = torch.zeros(len(seqs), max_blk, dtype=index_dtype)
    for i, t in enumerate(tables):
        n = min(len(t), max_blk)
        if n:
            bt[i, :n] = torch.tensor(t[:n], dtype=index_dtype)
    return AttentionMetadata(
        slot_mapping=torch.zeros(sum(query_lens), dtype=torch.long, device=device),
        query_start_loc=torch.tensor(qsl, dtype=index_dtype, device=device),
        seq_lens=torch.tensor(seqs, dtype=index_dtype, device=device),
        block_tables=bt.to(device),
        max_query_len=max(query_lens),
        max_seq_len=max_seq,
        num_seqs=len(seqs),
        num_tokens=sum(query_lens),
        is_decode_only=all(q == 1 for q in query_lens),
        query_lens_cpu=list(query_lens) if with_cpu_lists else None,
        seq_lens_cpu=list(seqs) if with_cpu_lists else None,
        query_start_loc_cpu=qsl if with_cpu_lists else None,
    )


def md_to(md: AttentionMetadata, device) -> AttentionMetadata:
    """Same metadata with every tensor moved to `device`."""
    return AttentionMetadata(
        slot_mapping=md.slot_mapping.to(device),
        query_start_loc=md.query_start_loc.to(device),
        seq_lens=md.seq_lens.to(device),
        block_tables=md.block_tables.to(device),
        max_query_len=md.max_query_len,
        max_seq_len=md.max_seq_len,
        num_seqs=md.num_seqs,
        num_tokens=md.num_tokens,
        is_decode_only=md.is_decode_only,
        query_lens_cpu=md.query_lens_cpu,
        seq_lens_cpu=md.seq_lens_cpu,
        query_start_loc_cpu=md.query_start_loc_cpu,
    )
