"""Write the golden fixtures under tests/golden/ from this repo's CPU oracle.

    python tests/golden/make_golden.py

The reference (AadityaK21/nanoserve) ships no golden vectors for the paged
attention path: its tests regenerate seeded inputs and compare against a
textbook dense softmax (reference tests/test_paged_attention.py:24-94).  These
fixtures freeze a handful of such cases -- inputs plus the fp32 oracle output
and the fp64 dense reference -- so a regression in the oracle, the metadata
layout or the kernels shows up as a diff against stored data.  Each fixture is
an .npz of plain arrays (no pickles).
"""

from __future__ import annotations

import math
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle.paged_attention import dense_reference, paged_attention_ref, reshape_and_cache_ref  # noqa: E402
from oracle.rope import rope_cos_sin_ref, rope_reshape_and_cache_ref, rope_table_ref  # noqa: E402
from tests._helpers import build_paged, make_md  # noqa: E402

# name: (seq_lens, query_lens, Hq, Hkv, D, block_size, dtype)
ATTN_CASES = {
    "decode_fp16_d64": ([1, 17, 300, 45], [1, 1, 1, 1], 14, 2, 64, 16, torch.float16),
    "prefill_fp16_d64": ([7, 33], [7, 33], 14, 2, 64, 16, torch.float16),
    "mixed_fp16_d64": ([40, 90, 9], [1, 30, 9], 14, 2, 64, 8, torch.float16),
    "decode_bf16_d128": ([5, 150, 64], [1, 1, 1], 28, 4, 128, 32, torch.bfloat16),
}


def _np(t: torch.Tensor) -> np.ndarray:
    """Raw bit patterns for 16-bit floats (numpy has no bfloat16), values otherwise."""
    t = t.detach().cpu().contiguous()
    if t.dtype in (torch.float16, torch.bfloat16):
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def attn_fixture(name):
    seqs, qls, hq, hkv, d, bs, dt = ATTN_CASES[name]
    nb = sum(-(-s // bs) for s in seqs) + 4
    kc, vc, tables, truth = build_paged(seqs, nb, bs, hkv, d, dtype=dt, seed=4242)
    md = make_md(seqs, qls, tables, bs, index_dtype=torch.int32)
    q = torch.randn(sum(qls), hq, d, generator=torch.Generator().manual_seed(99)).to(dt)
    scale = 1.0 / math.sqrt(d)
    out = paged_attention_ref(q, kc, vc, md, scale)
    dense = []
    off = 0
    for i, (sl, ql) in enumerate(zip(seqs, qls)):
        dense.append(dense_reference(q[off:off + ql].float(), truth[i][0].float(), truth[i][1].float(),
                                     sl - ql, hq // hkv, scale))
        off += ql
    return dict(
        dtype=np.array(str(dt).replace("torch.", "")),
        query=_np(q), k_cache=_np(kc), v_cache=_np(vc),
        block_tables=md.block_tables.numpy(), seq_lens=np.array(seqs, np.int32),
        query_lens=np.array(qls, np.int32), query_start_loc=md.query_start_loc.numpy(),
        scale=np.array(scale, np.float64),
        expected=out.numpy().astype(np.float32), dense=np.concatenate(dense).astype(np.float32),
    )


def cache_write_fixture():
    g = torch.Generator().manual_seed(5)
    NB, BS, Hkv, D, T = 12, 16, 2, 64, 40
    key = (torch.randn(T, Hkv, D, generator=g) * 3).float()
    value = (torch.randn(T, Hkv, D, generator=g) * 3).float()
    kc = torch.randn(NB, BS, Hkv, D, generator=g).half()
    vc = torch.randn(NB, BS, Hkv, D, generator=g).half()
    slots = torch.randperm(NB * BS, generator=g)[:T].to(torch.int64)
    ek, ev = reshape_and_cache_ref(key, value, kc, vc, slots)
    return dict(key=key.numpy(), value=value.numpy(), k_cache=_np(kc), v_cache=_np(vc),
                slot_mapping=slots.numpy(), expected_k=_np(ek), expected_v=_np(ev))


# name: (T, Hq, Hkv, D, num_blocks, block_size, base, dtype)
ROPE_CASES = {
    "fp16_d64": (13, 14, 2, 64, 4, 16, 10000.0, torch.float16),
    "bf16_d128": (9, 28, 4, 128, 3, 32, 1000000.0, torch.bfloat16),
}


def rope_fixture(name):
    """Fused rotary + cache write: inputs, positions, slots (one -1) and the oracle's outputs."""
    T, hq, hkv, d, nb, bs, base, dt = ROPE_CASES[name]
    g = torch.Generator().manual_seed(31)
    q = torch.randn(T, hq, d, generator=g).to(dt)
    k = torch.randn(T, hkv, d, generator=g).to(dt)
    v = torch.randn(T, hkv, d, generator=g).to(dt)
    pos = torch.randint(0, 4096, (T,), generator=g)
    cos_t, sin_t = rope_table_ref(d, 4096, base)
    cos, sin = rope_cos_sin_ref(cos_t, sin_t, pos, dt)
    kc = torch.randn(nb, bs, hkv, d, generator=g).to(dt)
    vc = torch.randn(nb, bs, hkv, d, generator=g).to(dt)
    slots = torch.randperm(nb * bs, generator=g)[:T].to(torch.int64)
    slots[T // 2] = -1
    qr, ek, ev = rope_reshape_and_cache_ref(q, k, v, cos, sin, kc, vc, slots)
    return dict(dtype=np.array(str(dt).replace("torch.", "")), base=np.array(base, np.float64),
                positions=pos.numpy(), query=_np(q), key=_np(k), value=_np(v), cos=_np(cos), sin=_np(sin),
                k_cache=_np(kc), v_cache=_np(vc), slot_mapping=slots.numpy(),
                expected_q=_np(qr), expected_k=_np(ek), expected_v=_np(ev))


def main():
    for name in ATTN_CASES:
        np.savez_compressed(os.path.join(HERE, f"attn_{name}.npz"), **attn_fixture(name))
    np.savez_compressed(os.path.join(HERE, "cache_write_f32_to_f16.npz"), **cache_write_fixture())
    for name in ROPE_CASES:
        np.savez_compressed(os.path.join(HERE, f"rope_{name}.npz"), **rope_fixture(name))
    print("wrote", sorted(f for f in os.listdir(HERE) if f.endswith(".npz")))


if __name__ == "__main__":
    main()
