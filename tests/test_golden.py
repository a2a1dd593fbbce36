"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU side: the oracle still reproduces every stored output, and each stored
oracle output agrees with the stored fp64 textbook result at the reference's
own fp32 tolerance (tests/test_paged_attention.py:97-209, atol 2e-5).
GPU side (marked gpu): the HIP kernels reproduce the stored outputs within the
build's tolerances, and the cache write reproduces the stored cache bits.
"""

from __future__ import annotations

import glob
import os

import numpy as np
import pytest
import torch

from nanoserve_amd.attention import AttentionMetadata
from oracle.paged_attention import paged_attention_ref, reshape_and_cache_ref
from oracle.rope import rope_cos_sin_ref, rope_reshape_and_cache_ref, rope_table_ref

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
ATTN = sorted(glob.glob(os.path.join(HERE, "attn_*.npz")))
ROPE = sorted(glob.glob(os.path.join(HERE, "rope_*.npz")))
TOL = {torch.float16: 2e-3, torch.bfloat16: 1e-2}


def _half(a: np.ndarray, dtype: torch.dtype) -> torch.Tensor:
    return torch.from_numpy(a.astype(np.int16)).view(dtype)


def load_attn(path, device="cpu"):
    z = np.load(path, allow_pickle=False)
    dt = {"float16": torch.float16, "bfloat16": torch.bfloat16}[str(z["dtype"])]
    q = _half(z["query"], dt).to(device)
    kc = _half(z["k_cache"], dt).to(device)
    vc = _half(z["v_cache"], dt).to(device)
    seqs, qls = z["seq_lens"].tolist(), z["query_lens"].tolist()
    qsl = z["query_start_loc"].tolist()
    md = AttentionMetadata(
        slot_mapping=torch.zeros(sum(qls), dtype=torch.int64, device=device),
        query_start_loc=torch.tensor(qsl, dtype=torch.int32, device=device),
        seq_lens=torch.tensor(seqs, dtype=torch.int32, device=device),
        block_tables=torch.from_numpy(z["block_tables"]).to(device),
        max_query_len=max(qls), max_seq_len=max(seqs), num_seqs=len(seqs),
        num_tokens=sum(qls), is_decode_only=all(x == 1 for x in qls),
        query_lens_cpu=qls, seq_lens_cpu=seqs, query_start_loc_cpu=qsl)
    return q, kc, vc, md, float(z["scale"]), torch.from_numpy(z["expected"]), z["dense"], dt


def test_fixtures_present():
    assert len(ATTN) >= 4
    assert os.path.exists(os.path.join(HERE, "cache_write_f32_to_f16.npz"))
    assert len(ROPE) >= 2


@pytest.mark.parametrize("path", ATTN, ids=[os.path.basename(p)[5:-4] for p in ATTN])
def test_oracle_reproduces_golden(path):
    q, kc, vc, md, scale, expected, dense, _ = load_attn(path)
    got = paged_attention_ref(q, kc, vc, md, scale)
    torch.testing.assert_close(got, expected, atol=1e-5, rtol=1e-5)
    np.testing.assert_allclose(expected.numpy(), dense, atol=2e-5, rtol=2e-5)


def test_oracle_reproduces_golden_cache_write():
    z = np.load(os.path.join(HERE, "cache_write_f32_to_f16.npz"), allow_pickle=False)
    kc, vc = _half(z["k_cache"], torch.float16), _half(z["v_cache"], torch.float16)
    ek, ev = reshape_and_cache_ref(torch.from_numpy(z["key"]), torch.from_numpy(z["value"]), kc, vc,
                                   torch.from_numpy(z["slot_mapping"]))
    np.testing.assert_array_equal(ek.view(torch.int16).numpy().view(np.uint16), z["expected_k"])
    np.testing.assert_array_equal(ev.view(torch.int16).numpy().view(np.uint16), z["expected_v"])


@pytest.mark.gpu
@pytest.mark.parametrize("path", ATTN, ids=[os.path.basename(p)[5:-4] for p in ATTN])
def test_hip_matches_golden(path):
    from nanoserve_amd import paged_attention_hip

    q, kc, vc, md, scale, expected, _, dt = load_attn(path, "cuda")
    got = paged_attention_hip(q, kc, vc, md, scale).float().cpu()
    err = (got - expected).abs().max().item()
    assert err <= TOL[dt], f"max abs err {err:.3e}"


@pytest.mark.gpu
def test_hip_cache_write_matches_golden():
    from nanoserve_amd import reshape_and_cache

    z = np.load(os.path.join(HERE, "cache_write_f32_to_f16.npz"), allow_pickle=False)
    kc = _half(z["k_cache"], torch.float16).cuda()
    vc = _half(z["v_cache"], torch.float16).cuda()
    reshape_and_cache(torch.from_numpy(z["key"]).cuda(), torch.from_numpy(z["value"]).cuda(), kc, vc,
                      torch.from_numpy(z["slot_mapping"]).cuda())
    np.testing.assert_array_equal(kc.cpu().view(torch.int16).numpy().view(np.uint16), z["expected_k"])
    np.testing.assert_array_equal(vc.cpu().view(torch.int16).numpy().view(np.uint16), z["expected_v"])


def load_rope(path, device="cpu"):
    z = np.load(path, allow_pickle=False)
    dt = {"float16": torch.float16, "bfloat16": torch.bfloat16}[str(z["dtype"])]
    t = {n: _half(z[n], dt).to(device) for n in ("query", "key", "value", "cos", "sin", "k_cache", "v_cache")}
    return z, dt, t, torch.from_numpy(z["slot_mapping"]).to(device)


def _bits16(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("path", ROPE, ids=[os.path.basename(p)[5:-4] for p in ROPE])
def test_oracle_reproduces_golden_rope(path):
    z, dt, t, slots = load_rope(path)
    d = t["query"].shape[-1]
    cos_t, sin_t = rope_table_ref(d, 4096, float(z["base"]))
    cos, sin = rope_cos_sin_ref(cos_t, sin_t, torch.from_numpy(z["positions"]), dt)
    np.testing.assert_array_equal(_bits16(cos), z["cos"])
    np.testing.assert_array_equal(_bits16(sin), z["sin"])
    qr, ek, ev = rope_reshape_and_cache_ref(t["query"], t["key"], t["value"], cos, sin,
                                            t["k_cache"], t["v_cache"], slots)
    for got, name in ((qr, "expected_q"), (ek, "expected_k"), (ev, "expected_v")):
        np.testing.assert_array_equal(_bits16(got), z[name])


@pytest.mark.gpu
@pytest.mark.parametrize("path", ROPE, ids=[os.path.basename(p)[5:-4] for p in ROPE])
def test_hip_rope_matches_golden(path):
    from nanoserve_amd import rope_reshape_and_cache

    z, dt, t, slots = load_rope(path, "cuda")
    qr = rope_reshape_and_cache(t["query"], t["key"], t["value"], t["cos"], t["sin"],
                                t["k_cache"], t["v_cache"], slots)
    torch.cuda.synchronize()
    for got, name in ((qr, "expected_q"), (t["k_cache"], "expected_k"), (t["v_cache"], "expected_v")):
        np.testing.assert_array_equal(_bits16(got), z[name])
