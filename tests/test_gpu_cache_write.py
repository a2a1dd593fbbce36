"""HIP reshape_and_cache against the oracle's index_copy_ restatement (MI355X).

Bit-exact: same-dtype rows are copied unchanged (any bit pattern), and
f32 -> f16 / bf16 and f16 <-> bf16 conversions round exactly like torch's
Tensor.to.  NaN inputs convert to a NaN (torch's CPU path itself emits
different NaN payloads depending on vectorisation, so only NaN-ness is
compared for them).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from nanoserve_amd import PagedKVCache, paged_attention_hip, reshape_and_cache
from nanoserve_amd.workloads import make_case
from oracle.paged_attention import paged_attention_ref, reshape_and_cache_ref
from tests._helpers import md_to

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _bits(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu().contiguous()
    if t.element_size() == 2:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.view(torch.int32).numpy().view(np.uint32)


def _rand_rows(T, Hkv, D, dtype, seed, special=True):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, Hkv, D, generator=g) * torch.exp(torch.randn(T, Hkv, D, generator=g) * 6)
    if special and T * Hkv * D >= 16:
        flat = x.view(-1)
        flat[:14] = torch.tensor([0.0, -0.0, 65504.0, 65520.0, 1e30, -1e30, float("inf"), float("-inf"),
                                  2 ** -24, 2 ** -25, 1.5 * 2 ** -25, 1 + 2 ** -11, 1 + 3 * 2 ** -11, 1e-40])
    return x.to(dtype)


def _caches(NB, BS, Hkv, D, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    k = torch.randn(NB, BS, Hkv, D, generator=g).to(dtype)
    v = torch.randn(NB, BS, Hkv, D, generator=g).to(dtype)
    return k, v


def _slots(T, NB, BS, seed):
    return torch.randperm(NB * BS, generator=torch.Generator().manual_seed(seed))[:T].to(torch.int64)


@pytest.mark.parametrize("src,dst", [
    (torch.float16, torch.float16), (torch.bfloat16, torch.bfloat16), (torch.float32, torch.float32),
    (torch.float32, torch.float16), (torch.float32, torch.bfloat16),
    (torch.float16, torch.bfloat16), (torch.bfloat16, torch.float16), (torch.float16, torch.float32),
])
@pytest.mark.parametrize("D", [64, 128])
def test_cache_write_bit_exact(src, dst, D):
    NB, BS, Hkv, T = 64, 16, 2, 300
    key, val = _rand_rows(T, Hkv, D, src, 1), _rand_rows(T, Hkv, D, src, 2)
    kc, vc = _caches(NB, BS, Hkv, D, dst, 3)
    slots = _slots(T, NB, BS, 4)
    ek, ev = reshape_and_cache_ref(key, val, kc, vc, slots)
    gk, gv = kc.to(DEV), vc.to(DEV)
    reshape_and_cache(key.to(DEV), val.to(DEV), gk, gv, slots.to(DEV))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_bits(gk), _bits(ek))
    np.testing.assert_array_equal(_bits(gv), _bits(ev))


def test_same_dtype_copy_preserves_arbitrary_bits():
    """Raw fp16 patterns, NaN payloads included, are moved unchanged."""
    NB, BS, Hkv, D, T = 16, 16, 2, 64, 100
    g = torch.Generator().manual_seed(0)
    raw = torch.randint(-32768, 32767, (T, Hkv, D), generator=g, dtype=torch.int16)
    key = raw.view(torch.float16)
    val = raw.flip(0).contiguous().view(torch.float16)
    kc, vc = _caches(NB, BS, Hkv, D, torch.float16, 1)
    slots = _slots(T, NB, BS, 2)
    ek, ev = reshape_and_cache_ref(key, val, kc, vc, slots)
    gk, gv = kc.to(DEV), vc.to(DEV)
    reshape_and_cache(key.to(DEV), val.to(DEV), gk, gv, slots.to(DEV))
    np.testing.assert_array_equal(_bits(gk), _bits(ek))
    np.testing.assert_array_equal(_bits(gv), _bits(ev))


@pytest.mark.parametrize("dst", [torch.float16, torch.bfloat16])
def test_nan_converts_to_nan(dst):
    key = torch.full((3, 1, 64), float("nan"))
    kc = torch.zeros(4, 16, 1, 64, dtype=dst, device=DEV)
    vc = torch.zeros_like(kc)
    reshape_and_cache(key.to(DEV), key.to(DEV), kc, vc, torch.tensor([0, 17, 63], device=DEV))
    f = kc.view(-1, 1, 64)
    assert torch.isnan(f[[0, 17, 63]].float()).all()
    assert torch.count_nonzero(f[1:17].float()) == 0


def test_strided_key_value_and_int32_slots():
    """Rows read through views (a fused qkv projection) with int32 slots."""
    T, Hkv, D, NB, BS = 77, 2, 64, 32, 16
    qkv = _rand_rows(T, 3 * Hkv, D, torch.float16, 5, special=False)
    key, val = qkv[:, Hkv:2 * Hkv], qkv[:, 2 * Hkv:]
    assert not key.is_contiguous()
    kc, vc = _caches(NB, BS, Hkv, D, torch.float16, 6)
    slots = _slots(T, NB, BS, 7)
    ek, ev = reshape_and_cache_ref(key, val, kc, vc, slots)
    gqkv = qkv.to(DEV)
    gk, gv = kc.to(DEV), vc.to(DEV)
    reshape_and_cache(gqkv[:, Hkv:2 * Hkv], gqkv[:, 2 * Hkv:], gk, gv, slots.to(torch.int32).to(DEV))
    np.testing.assert_array_equal(_bits(gk), _bits(ek))
    np.testing.assert_array_equal(_bits(gv), _bits(ev))


def test_unaligned_head_stride_falls_back_to_element_copy():
    T, Hkv, D, NB, BS = 9, 2, 64, 4, 16
    base = _rand_rows(T, Hkv, D + 1, torch.float16, 8, special=False)
    key = base[:, :, 1:]  # rows start at an odd element: not 16-byte aligned
    kc, vc = _caches(NB, BS, Hkv, D, torch.float16, 9)
    slots = _slots(T, NB, BS, 10)
    ek, ev = reshape_and_cache_ref(key, key, kc, vc, slots)
    gk, gv = kc.to(DEV), vc.to(DEV)
    gkey = base.to(DEV)[:, :, 1:]
    reshape_and_cache(gkey, gkey, gk, gv, slots.to(DEV))
    np.testing.assert_array_equal(_bits(gk), _bits(ek))


def test_negative_and_out_of_range_slots_are_skipped():
    T, Hkv, D, NB, BS = 6, 2, 64, 4, 16
    key = _rand_rows(T, Hkv, D, torch.float16, 11, special=False)
    kc, vc = _caches(NB, BS, Hkv, D, torch.float16, 12)
    slots = torch.tensor([5, -1, 9, NB * BS, 63, -7])
    gk, gv = kc.to(DEV), vc.to(DEV)
    reshape_and_cache(key.to(DEV), key.to(DEV), gk, gv, slots.to(DEV))
    keep = slots[(slots >= 0) & (slots < NB * BS)]
    rows = torch.tensor([0, 2, 4])
    ek, _ = reshape_and_cache_ref(key[rows], key[rows], kc, vc, keep)
    np.testing.assert_array_equal(_bits(gk), _bits(ek))


@pytest.mark.parametrize("config", ["c2", "c3"])
def test_write_then_attend_matches_oracle(config):
    """The call-site order (reference qwen2.py:57-65): write the step's K/V, then attend."""
    case = make_case(config, seed=2)
    T, Hkv, D = case.md.num_tokens, case.num_kv_heads, case.head_dim
    g = torch.Generator().manual_seed(9)
    key = torch.randn(T, Hkv, D, generator=g).half()
    val = torch.randn(T, Hkv, D, generator=g).half()
    ek, ev = reshape_and_cache_ref(key, val, case.k_cache, case.v_cache, case.md.slot_mapping)
    ref = paged_attention_ref(case.query, ek, ev, case.md, case.scale)

    cache = PagedKVCache(case.k_cache.shape[0], case.k_cache.shape[1], 1, Hkv, D, torch.float16, DEV)
    cache.k_cache[0].copy_(case.k_cache)
    cache.v_cache[0].copy_(case.v_cache)
    md = md_to(case.md, DEV)
    cache.write(0, key.to(DEV), val.to(DEV), md.slot_mapping)
    np.testing.assert_array_equal(_bits(cache.k_cache[0]), _bits(ek))
    out = paged_attention_hip(case.query.to(DEV), cache.k_cache[0], cache.v_cache[0], md, 1 / math.sqrt(D))
    err = (out.float().cpu() - ref).abs().max().item()
    assert err <= 2e-3, err
