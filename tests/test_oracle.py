"""Pins the CPU oracle before anything is checked against it.

The oracle restates the reference's gather+SDPA backend; here it is checked
against things that do not share its code: the fp64 textbook reference on the
reference's own test cases (tests/test_paged_attention.py:97-209, fp32,
atol=rtol=2e-5), closed forms, a scalar softmax written with math.exp, and
invariants (permuted tables, poisoned stale slots, chunked == whole).  The
dtype conversions of the cache write are pinned against numpy's float16
rounding, an integer bfloat16 rounding and known bit patterns.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle.paged_attention import (bf16_bits_ref, dense_reference, paged_attention_ref,
                                    reshape_and_cache_ref, slot_mapping_ref)
from tests._helpers import build_paged, make_md


def _check_against_dense(seqs, query_lens, Hq, Hkv, D, block_size, q_seed, num_blocks=128,
                         with_cpu_lists=True):
    kc, vc, tables, truth = build_paged(seqs, num_blocks, block_size, Hkv, D)
    md = make_md(seqs, query_lens, tables, block_size, with_cpu_lists=with_cpu_lists)
    g = torch.Generator().manual_seed(q_seed)
    q = torch.randn(sum(query_lens), Hq, D, generator=g)
    got = paged_attention_ref(q, kc, vc, md, 1.0 / math.sqrt(D))
    off = 0
    for i, (sl, ql) in enumerate(zip(seqs, query_lens)):
        K, V = truth[i]
        ref = dense_reference(q[off:off + ql], K, V, sl - ql, Hq // Hkv)
        np.testing.assert_allclose(got[off:off + ql].numpy(), ref, atol=2e-5, rtol=2e-5)
        off += ql
    return got


# ---- the reference's own cases ------------------------------------------
@pytest.mark.parametrize("block_size", [4, 8, 16])
@pytest.mark.parametrize("seqs", [[7], [16], [5, 13, 1], [1, 1, 1, 1]])
def test_prefill_matches_dense(block_size, seqs):
    _check_against_dense(seqs, seqs, 4, 2, 8, block_size, q_seed=7, num_blocks=64)


@pytest.mark.parametrize("block_size", [4, 16])
@pytest.mark.parametrize("seqs", [[1, 9, 33], [16, 16], [64, 3, 17, 40]])
def test_decode_matches_dense(block_size, seqs):
    _check_against_dense(seqs, [1] * len(seqs), 6, 2, 8, block_size, q_seed=11)


def test_mixed_batch_matches_dense():
    _check_against_dense([12, 30, 5], [12, 1, 5], 4, 2, 8, 8, q_seed=17, num_blocks=64)


def test_qsl_tolist_fallback_matches_cpu_lists():
    """Without *_cpu lists the oracle reads the tensors (reference attention.py:119)."""
    a = _check_against_dense([12, 30, 5], [12, 1, 5], 4, 2, 8, 8, 17, 64, with_cpu_lists=True)
    b = _check_against_dense([12, 30, 5], [12, 1, 5], 4, 2, 8, 8, 17, 64, with_cpu_lists=False)
    assert torch.equal(a, b)


def test_decode_ignores_stale_kv_in_padded_slots():
    Hq, Hkv, D, bs = 4, 2, 8, 8
    seqs = [3, 40]
    kc, vc, tables, truth = build_paged(seqs, 64, bs, Hkv, D)
    kf, vf = kc.view(-1, Hkv, D), vc.view(-1, Hkv, D)
    owned = {tables[0][p // bs] * bs + p % bs for p in range(seqs[0])}
    for b in tables[0]:
        for o in range(bs):
            if b * bs + o not in owned:
                kf[b * bs + o] = 1e3
                vf[b * bs + o] = 1e3
    md = make_md(seqs, [1, 1], tables, bs)
    q = torch.randn(2, Hq, D, generator=torch.Generator().manual_seed(3))
    got = paged_attention_ref(q, kc, vc, md, 1.0 / math.sqrt(D))
    K, V = truth[0]
    ref = dense_reference(q[0:1], K, V, seqs[0] - 1, Hq // Hkv)
    np.testing.assert_allclose(got[0:1].numpy(), ref, atol=2e-5, rtol=2e-5)


def test_chunked_prefill_matches_whole_prefill():
    Hq, Hkv, D, bs, sl = 4, 2, 8, 8, 20
    kc, vc, tables, _ = build_paged([sl], 32, bs, Hkv, D)
    q = torch.randn(sl, Hq, D, generator=torch.Generator().manual_seed(5))
    whole = paged_attention_ref(q, kc, vc, make_md([sl], [sl], tables, bs), 1.0 / math.sqrt(D))
    pieces = [paged_attention_ref(q[a:b], kc, vc, make_md([b], [b - a], tables, bs), 1.0 / math.sqrt(D))
              for a, b in ((0, 7), (7, 13), (13, 20))]
    torch.testing.assert_close(torch.cat(pieces), whole, atol=2e-5, rtol=2e-5)


def test_per_seq_decode_equals_padded_decode():
    seqs = [1, 9, 33, 70]
    kc, vc, tables, _ = build_paged(seqs, 64, 16, 2, 16)
    md = make_md(seqs, [1] * 4, tables, 16)
    q = torch.randn(4, 6, 16, generator=torch.Generator().manual_seed(2))
    a = paged_attention_ref(q, kc, vc, md, 0.25)
    b = paged_attention_ref(q, kc, vc, md, 0.25, per_seq_decode=True)
    torch.testing.assert_close(a, b, atol=1e-6, rtol=1e-6)


def test_table_permutation_invariance():
    seqs = [5, 37, 16]
    ka, va, ta, _ = build_paged(seqs, 48, 8, 2, 16, shuffle=True, seed=99)
    kb, vb, tb, _ = build_paged(seqs, 48, 8, 2, 16, shuffle=False, seed=99)
    q = torch.randn(3, 4, 16, generator=torch.Generator().manual_seed(1))
    a = paged_attention_ref(q, ka, va, make_md(seqs, [1] * 3, ta, 8), 0.25)
    b = paged_attention_ref(q, kb, vb, make_md(seqs, [1] * 3, tb, 8), 0.25)
    assert ta != tb
    torch.testing.assert_close(a, b, atol=1e-6, rtol=1e-6)


# ---- closed forms -----------------------------------------------------------
def test_single_key_returns_its_value():
    kc, vc, tables, truth = build_paged([1, 1], 8, 4, 2, 8)
    q = torch.randn(2, 6, 8, generator=torch.Generator().manual_seed(4)) * 10
    got = paged_attention_ref(q, kc, vc, make_md([1, 1], [1, 1], tables, 4), 0.3)
    for i in range(2):
        V = truth[i][1][0]                                   # [Hkv, D]
        exp = V.repeat_interleave(3, dim=0)                   # head h -> kv head h // 3
        torch.testing.assert_close(got[i], exp, atol=1e-6, rtol=0)
        np.testing.assert_allclose(dense_reference(q[i:i + 1], truth[i][0], truth[i][1], 0, 3)[0],
                                   exp.numpy(), atol=1e-12)


def test_identical_keys_average_values():
    sl, Hkv, D = 13, 2, 8
    kc, vc, tables, truth = build_paged([sl], 8, 4, Hkv, D)
    kf = kc.view(-1, Hkv, D)
    kf[:] = 0.5  # every key identical -> uniform softmax
    q = torch.randn(1, 4, D, generator=torch.Generator().manual_seed(6))
    got = paged_attention_ref(q, kc, vc, make_md([sl], [1], tables, 4), 0.125)
    V = truth[0][1]
    exp = V.mean(0).repeat_interleave(2, dim=0)
    torch.testing.assert_close(got[0], exp, atol=1e-6, rtol=1e-6)


def test_zero_query_is_causal_running_mean():
    sl, Hkv, D = 9, 1, 8
    kc, vc, tables, truth = build_paged([sl], 8, 4, Hkv, D)
    q = torch.zeros(sl, 2, D)
    got = paged_attention_ref(q, kc, vc, make_md([sl], [sl], tables, 4), 1.0)
    V = truth[0][1][:, 0]                                    # [sl, D]
    for j in range(sl):
        exp = V[:j + 1].mean(0)
        torch.testing.assert_close(got[j, 0], exp, atol=1e-6, rtol=1e-6)
        torch.testing.assert_close(got[j, 1], exp, atol=1e-6, rtol=1e-6)


def test_scalar_softmax_tiny_case():
    """Two heads, three keys, written out with math.exp."""
    kc, vc, tables, truth = build_paged([3], 4, 2, 1, 4, seed=21)
    q = torch.randn(1, 2, 4, generator=torch.Generator().manual_seed(8))
    scale = 0.7
    got = paged_attention_ref(q, kc, vc, make_md([3], [1], tables, 2), scale)
    K, V = truth[0]
    for h in range(2):
        s = [scale * sum(float(q[0, h, d]) * float(K[t, 0, d]) for d in range(4)) for t in range(3)]
        m = max(s)
        w = [math.exp(x - m) for x in s]
        z = sum(w)
        exp = [sum(w[t] * float(V[t, 0, d]) for t in range(3)) / z for d in range(4)]
        np.testing.assert_allclose(got[0, h].numpy(), exp, atol=1e-6)
        np.testing.assert_allclose(dense_reference(q, K, V, 2, 2, scale)[0, h], exp, atol=1e-12)


def test_fully_masked_row_is_zero():
    """A sequence with no visible key yields zeros (torch SDPA's masked-row result)."""
    kc, vc, tables, _ = build_paged([4, 1], 8, 4, 1, 8)
    md = make_md([4, 0], [1, 1], [tables[0], tables[1]], 4)
    q = torch.randn(2, 2, 8, generator=torch.Generator().manual_seed(9))
    got = paged_attention_ref(q, kc, vc, md, 0.3)
    assert torch.count_nonzero(got[1]) == 0
    assert np.count_nonzero(dense_reference(q[1:2], kc.view(-1, 1, 8)[:0], vc.view(-1, 1, 8)[:0], -1, 2)) == 0


# ---- cache write ------------------------------------------------------------
SPECIAL = np.array([0.0, -0.0, 1.0, -1.0, 65504.0, 65519.99, 65520.0, 1e9, -1e9, np.inf, -np.inf,
                    6.1e-5, 5.96e-8, 2.98e-8, 2.9802322e-08, 2.98023224e-08, 1e-30, -1e-30,
                    1.0 + 2 ** -11, 1.0 + 3 * 2 ** -11, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8,
                    3.1415927, 1.1754944e-38, 1e-45], dtype=np.float32)


def _f32_samples(n=4096, seed=0):
    rng = np.random.default_rng(seed)
    x = np.concatenate([rng.standard_normal(n).astype(np.float32) * 10.0 ** rng.integers(-9, 6, n),
                        SPECIAL])
    # random bit patterns cover every exponent (NaNs removed)
    bits = rng.integers(0, 2 ** 32, n, dtype=np.uint64).astype(np.uint32).view(np.float32)
    x = np.concatenate([x, bits[~np.isnan(bits)]])
    return x.astype(np.float32)


def test_torch_f16_rounding_matches_numpy():
    x = _f32_samples()
    got = torch.from_numpy(x).to(torch.float16).view(torch.int16).numpy().view(np.uint16)
    exp = x.astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(got, exp)


def test_torch_bf16_rounding_matches_integer_rne():
    x = _f32_samples(seed=1)
    got = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(got, bf16_bits_ref(x))


def test_rounding_known_answers():
    f16 = lambda v: int(np.float32(v).astype(np.float16).view(np.uint16))  # noqa: E731
    assert f16(1.0) == 0x3C00 and f16(-2.0) == 0xC000 and f16(65504.0) == 0x7BFF
    assert f16(65520.0) == 0x7C00                       # halfway above max rounds to inf
    assert f16(1.0 + 2 ** -11) == 0x3C00                # tie -> even
    assert f16(1.0 + 3 * 2 ** -11) == 0x3C02            # tie -> even (up)
    assert f16(2 ** -24) == 0x0001 and f16(2 ** -25) == 0x0000 and f16(1.5 * 2 ** -25) == 0x0001
    bf = lambda v: int(bf16_bits_ref(np.array([v], np.float32))[0])  # noqa: E731
    assert bf(1.0) == 0x3F80 and bf(-1.0) == 0xBF80
    assert bf(1.0 + 2 ** -8) == 0x3F80 and bf(1.0 + 3 * 2 ** -8) == 0x3F82
    assert bf(float("nan")) == 0x7FC0


def test_reshape_and_cache_ref_slots_and_untouched():
    NB, BS, Hkv, D = 6, 4, 2, 8
    kc = torch.full((NB, BS, Hkv, D), 7.0, dtype=torch.float16)
    vc = torch.full((NB, BS, Hkv, D), -7.0, dtype=torch.float16)
    key = torch.randn(5, Hkv, D, generator=torch.Generator().manual_seed(0))
    val = torch.randn(5, Hkv, D, generator=torch.Generator().manual_seed(1))
    slots = torch.tensor(slot_mapping_ref([3, 0, 5], 2, 7, BS))
    nk, nv = reshape_and_cache_ref(key, val, kc, vc, slots)
    fk, fv = nk.view(-1, Hkv, D), nv.view(-1, Hkv, D)
    for t, s in enumerate(slots.tolist()):
        assert torch.equal(fk[s], key[t].to(torch.float16))
        assert torch.equal(fv[s], val[t].to(torch.float16))
    rest = sorted(set(range(NB * BS)) - set(slots.tolist()))
    assert torch.all(fk[rest] == 7.0) and torch.all(fv[rest] == -7.0)


# ---- slot mapping -------------------------------------------------------------
def test_slot_mapping_ref_formula():
    table = [9, 2, 7]
    assert slot_mapping_ref(table, 0, 10, 4) == [36, 37, 38, 39, 8, 9, 10, 11, 28, 29]
    assert slot_mapping_ref(table, 6, 7, 4) == [10]
    with pytest.raises(IndexError):
        slot_mapping_ref(table, 0, 13, 4)
