"""CPU restatement of the reference's paged-attention path (test infrastructure only).

Nothing here is a product path: see oracle/__init__.py for who may import it.
"""

from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F


def _sdpa_gqa(q, k, v, mask, scale, n_rep):
    """SDPA with grouped kv heads, as reference attention.py:78-96.

    q [B, Hq, Lq, D], k/v [B, Hkv, Lk, D], mask [B or 1, 1, Lq, Lk] (True = attend).
    """
    if n_rep > 1:
        return F.scaled_dot_product_attention(q, k, v, attn_mask=mask, scale=scale, enable_gqa=True)
    return F.scaled_dot_product_attention(q, k, v, attn_mask=mask, scale=scale)


def _to_cpu_list(t, cpu_list):
    if cpu_list is not None:
        return list(cpu_list)
    return [int(x) for x in t.detach().cpu().tolist()]


@torch.inference_mode()
def paged_attention_ref(query, k_cache, v_cache, md, scale, upcast: bool = True,
                        per_seq_decode: bool = False):
    """Restatement of reference paged_attention_torch (attention.py:99-151).

    Decode-only batches take the padded batched path of _decode_batched
    (attention.py:154-190): gather a [S, ceil(max_seq_len/bs)*bs] window of
    each table row and mask positions >= seq_len.  Other batches loop over
    sequences (attention.py:118-150): gather seq_len tokens and mask key k for
    query row j with k <= seq_len - query_len + j.

    Runs on the CPU.  With `upcast`, inputs are converted to fp32 first and
    the fp32 result is returned (the tolerance reference); otherwise compute
    and output stay in the query dtype (the timed CPU baseline).
    `per_seq_decode` evaluates decode rows one sequence at a time, the same
    arithmetic without the padded window (for very long contexts).
    """
    dt = torch.float32 if upcast else query.dtype
    q_all = query.detach().to("cpu", dt)
    kc = k_cache.detach().to("cpu", dt)
    vc = v_cache.detach().to("cpu", dt)
    T, Hq, D = q_all.shape
    NB, BS, Hkv, _ = kc.shape
    n_rep = Hq // Hkv
    kf = kc.reshape(NB * BS, Hkv, D)
    vf = vc.reshape(NB * BS, Hkv, D)
    bt = md.block_tables.detach().to("cpu", torch.int64)
    seq_lens = _to_cpu_list(md.seq_lens, md.seq_lens_cpu)
    offs = torch.arange(BS)

    if md.is_decode_only and not per_seq_decode:
        S = md.num_seqs
        nblk = -(-md.max_seq_len // BS)
        if bt.shape[1] < nblk:
            raise ValueError("block_tables narrower than max_seq_len needs")
        idx = (bt[:S, :nblk, None] * BS + offs).reshape(S, nblk * BS)
        ctx = idx.shape[1]
        k = kf.index_select(0, idx.reshape(-1)).view(S, ctx, Hkv, D).permute(0, 2, 1, 3)
        v = vf.index_select(0, idx.reshape(-1)).view(S, ctx, Hkv, D).permute(0, 2, 1, 3)
        q = q_all.view(S, 1, Hq, D).permute(0, 2, 1, 3)
        lens = torch.tensor(seq_lens, dtype=torch.int64)
        valid = torch.arange(ctx)[None, :] < lens[:, None]
        o = _sdpa_gqa(q, k, v, valid[:, None, None, :], scale, n_rep)
        return o.permute(0, 2, 1, 3).reshape(S, Hq, D)

    if md.is_decode_only:
        qsl = list(range(md.num_seqs + 1))
    else:
        qsl = _to_cpu_list(md.query_start_loc, md.query_start_loc_cpu)
    out = torch.empty_like(q_all)
    for i in range(md.num_seqs):
        s, e = qsl[i], qsl[i + 1]
        ql = e - s
        if ql == 0:
            continue
        sl = seq_lens[i]
        nb = -(-sl // BS)
        idx = (bt[i, :nb, None] * BS + offs).reshape(-1)[:sl]
        k = kf.index_select(0, idx).transpose(0, 1)[None]     # [1, Hkv, sl, D]
        v = vf.index_select(0, idx).transpose(0, 1)[None]
        q = q_all[s:e].transpose(0, 1)[None]                  # [1, Hq, ql, D]
        q_pos = torch.arange(sl - ql, sl)
        mask = torch.arange(sl)[None, :] <= q_pos[:, None]     # [ql, sl]
        o = _sdpa_gqa(q, k, v, mask[None, None], scale, n_rep)
        out[s:e] = o[0].transpose(0, 1)
    return out


def dense_reference(q, k, v, q_start: int, n_rep: int, scale: float | None = None) -> np.ndarray:
    """Textbook per-head attention in float64, no paging (reference test_paged_attention.py:24-36).

    q [ql, Hq, D], k/v [sl, Hkv, D] (any array-likes); query row j sits at
    absolute position q_start + j and sees keys [0, q_start + j].
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    ql, Hq, D = q.shape
    sl = k.shape[0]
    sc = 1.0 / math.sqrt(D) if scale is None else scale
    out = np.zeros((ql, Hq, D))
    if sl == 0:
        return out
    pos_ok = np.arange(sl)[None, :] <= (q_start + np.arange(ql))[:, None]
    for h in range(Hq):
        kh, vh = k[:, h // n_rep], v[:, h // n_rep]
        s = (q[:, h] @ kh.T) * sc
        s = np.where(pos_ok, s, -np.inf)
        m = s.max(axis=1, keepdims=True)
        m = np.where(np.isfinite(m), m, 0.0)
        p = np.exp(s - m)
        den = p.sum(axis=1, keepdims=True)
        out[:, h] = np.where(den > 0, (p @ vh) / np.where(den > 0, den, 1.0), 0.0)
    return out


@torch.inference_mode()
def reshape_and_cache_ref(key, value, k_cache, v_cache, slot_mapping):
    """Restatement of PagedKVCache.write (reference kv_cache.py:73-81), on CPU copies.

    Returns new (k_cache, v_cache) with row t of key/value converted by
    Tensor.to(cache dtype) and copied into slot slot_mapping[t].
    """
    kc = k_cache.detach().cpu().clone()
    vc = v_cache.detach().cpu().clone()
    NB, BS, Hkv, D = kc.shape
    kf = kc.view(NB * BS, Hkv, D)
    vf = vc.view(NB * BS, Hkv, D)
    slots = slot_mapping.detach().cpu().to(torch.int64)
    kf.index_copy_(0, slots, key.detach().cpu().to(kf.dtype))
    vf.index_copy_(0, slots, value.detach().cpu().to(vf.dtype))
    return kc, vc


def slot_mapping_ref(block_table: list[int], start: int, end: int, block_size: int) -> list[int]:
    """Per-token closed form slot = table[pos // bs] * bs + pos % bs (block_manager.py:131-132)."""
    out = []
    for pos in range(start, end):
        if pos // block_size >= len(block_table):
            raise IndexError(f"position {pos} beyond a {len(block_table)}-block table")
        out.append(block_table[pos // block_size] * block_size + pos % block_size)
    return out


def bf16_bits_ref(x: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 bit patterns, round to nearest even (integer restatement)."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(np.asarray(x, dtype=np.float32))
    r[nan] = 0x7FC0
    return r
