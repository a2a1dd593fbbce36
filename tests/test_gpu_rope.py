"""HIP fused rotary + cache write against the oracle (MI355X).

ns_rope_reshape_and_cache must equal the reference's two steps -- rotary.apply
(reference nanoserve/layers.py:86-90) then PagedKVCache.write
(kv_cache.py:73-81) -- bit for bit: rotated q, the K cache rows (rotated k
converted to the cache dtype) and the V cache rows, with every slot the batch
does not name left untouched.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from nanoserve_amd import (PagedKVCache, RotaryEmbedding, paged_attention_hip, reshape_and_cache,
                           rope_reshape_and_cache)
from nanoserve_amd.workloads import make_case
from oracle.paged_attention import paged_attention_ref
from oracle.rope import rope_apply_ref, rope_cos_sin_ref, rope_reshape_and_cache_ref, rope_table_ref
from tests._helpers import md_to

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _bits(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu().contiguous()
    if t.element_size() == 2:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.view(torch.int32).numpy().view(np.uint32)


def _assert_bits(got: torch.Tensor, want: torch.Tensor, what: str):
    g, w = got.detach().cpu(), want.detach().cpu()
    assert g.shape == w.shape and g.dtype == w.dtype, what
    gn, wn = torch.isnan(g.float()), torch.isnan(w.float())
    assert torch.equal(gn, wn), f"{what}: NaN positions differ"
    gb, wb = _bits(g)[~gn.numpy()], _bits(w)[~wn.numpy()]
    bad = np.flatnonzero(gb != wb)
    assert bad.size == 0, f"{what}: {bad.size} elements differ, first at {bad[:5]}"


def _case(T, Hq, Hkv, D, NB, BS, dtype, cache_dtype=None, seed=0, max_pos=8192, base=10000.0, wide=False):
    g = torch.Generator().manual_seed(seed)
    cache_dtype = cache_dtype or dtype

    def rnd(*shape):
        x = torch.randn(*shape, generator=g)
        if wide:
            x = x * torch.exp(torch.randn(*shape, generator=g) * 3)
        return x.to(dtype)

    q, k, v = rnd(T, Hq, D), rnd(T, Hkv, D), rnd(T, Hkv, D)
    cos_t, sin_t = rope_table_ref(D, max_pos, base)
    pos = torch.randint(0, max_pos, (T,), generator=g)
    cos, sin = rope_cos_sin_ref(cos_t, sin_t, pos, dtype)
    kc = torch.randn(NB, BS, Hkv, D, generator=g).to(cache_dtype)
    vc = torch.randn(NB, BS, Hkv, D, generator=g).to(cache_dtype)
    slots = torch.randperm(NB * BS, generator=g)[:T].to(torch.int64)
    return q, k, v, cos, sin, kc, vc, slots


def _run_and_check(q, k, v, cos, sin, kc, vc, slots, slot_dtype=torch.int64, **kw):
    eq, ek, ev = rope_reshape_and_cache_ref(q, k, v, cos, sin, kc, vc, slots)
    gk, gv = kc.to(DEV), vc.to(DEV)
    got = rope_reshape_and_cache(q.to(DEV), k.to(DEV), v.to(DEV), cos.to(DEV), sin.to(DEV), gk, gv,
                                 slots.to(slot_dtype).to(DEV), **kw)
    torch.cuda.synchronize()
    _assert_bits(got, eq, "q")
    _assert_bits(gk, ek, "k_cache")
    _assert_bits(gv, ev, "v_cache")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("shape", [(14, 2, 64), (28, 4, 128)], ids=["c2heads", "c4heads"])
@pytest.mark.parametrize("T", [1, 7, 300])
def test_matches_oracle_bit_exact(dtype, shape, T):
    Hq, Hkv, D = shape
    print(f"rope T={T} heads={shape} {dtype}", flush=True)
    _run_and_check(*_case(T, Hq, Hkv, D, -(-T // 16) + 3, 16, dtype, seed=T))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_wide_range_values_and_tables(dtype):
    """Values over a wide exponent range (overflow, subnormals) and arbitrary cos/sin."""
    T, Hq, Hkv, D = 40, 3, 1, 64
    q, k, v, cos, sin, kc, vc, slots = _case(T, Hq, Hkv, D, 4, 16, dtype, seed=11, wide=True)
    g = torch.Generator().manual_seed(12)
    cos = (torch.randn(T, 1, D, generator=g) * 4).to(dtype)
    sin = (torch.randn(T, 1, D, generator=g) * 4).to(dtype)
    q.view(-1)[:8] = torch.tensor([0.0, -0.0, 65504.0, -60000.0, 2 ** -24, 3 * 2 ** -25, float("inf"),
                                   float("nan")]).to(dtype)
    _run_and_check(q, k, v, cos, sin, kc, vc, slots)


@pytest.mark.parametrize("model,cache", [(torch.float32, torch.float16), (torch.float32, torch.bfloat16),
                                         (torch.float16, torch.float32), (torch.bfloat16, torch.float16),
                                         (torch.float16, torch.bfloat16)])
def test_cache_dtype_conversion(model, cache):
    _run_and_check(*_case(33, 14, 2, 64, 5, 16, model, cache_dtype=cache, seed=21))


@pytest.mark.parametrize("block_size", [1, 8, 32])
def test_block_sizes_and_int32_slots(block_size):
    T = 50
    _run_and_check(*_case(T, 14, 2, 64, -(-T // block_size) + 2, block_size, torch.float16, seed=block_size),
                   slot_dtype=torch.int32)


def test_padding_and_out_of_range_slots_are_skipped():
    q, k, v, cos, sin, kc, vc, _ = _case(6, 14, 2, 64, 4, 16, torch.float16, seed=3)
    slots = torch.tensor([5, -1, 9, 64, 63, -7])
    _run_and_check(q, k, v, cos, sin, kc, vc, slots)


def test_in_place_q():
    q, k, v, cos, sin, kc, vc, slots = _case(21, 14, 2, 64, 4, 16, torch.bfloat16, seed=4)
    eq, ek, ev = rope_reshape_and_cache_ref(q, k, v, cos, sin, kc, vc, slots)
    gq, gk, gv = q.to(DEV), kc.to(DEV), vc.to(DEV)
    got = rope_reshape_and_cache(gq, k.to(DEV), v.to(DEV), cos.to(DEV), sin.to(DEV), gk, gv, slots.to(DEV), out=gq)
    torch.cuda.synchronize()
    assert got.data_ptr() == gq.data_ptr()
    _assert_bits(gq, eq, "q in place")
    _assert_bits(gk, ek, "k_cache")
    _assert_bits(gv, ev, "v_cache")


def test_fused_qkv_views():
    """q, k, v read as column slices of one [T, (Hq+2Hkv)*D] projection output."""
    T, Hq, Hkv, D = 45, 14, 2, 64
    q, k, v, cos, sin, kc, vc, slots = _case(T, Hq, Hkv, D, 5, 16, torch.float16, seed=5)
    eq, ek, ev = rope_reshape_and_cache_ref(q, k, v, cos, sin, kc, vc, slots)
    qkv = torch.cat([q.reshape(T, -1), k.reshape(T, -1), v.reshape(T, -1)], dim=1).to(DEV)
    gq = qkv[:, :Hq * D].view(T, Hq, D)
    gk_rows = qkv[:, Hq * D:(Hq + Hkv) * D].view(T, Hkv, D)
    gv_rows = qkv[:, (Hq + Hkv) * D:].view(T, Hkv, D)
    assert not gq.is_contiguous() and gk_rows.stride(0) == (Hq + 2 * Hkv) * D
    gk, gv = kc.to(DEV), vc.to(DEV)
    # cos/sin as [T, D] slices of one [T, 2D] table
    cs = torch.cat([cos[:, 0], sin[:, 0]], dim=1).to(DEV)
    got = rope_reshape_and_cache(gq, gk_rows, gv_rows, cs[:, :D], cs[:, D:], gk, gv, slots.to(DEV))
    torch.cuda.synchronize()
    _assert_bits(got, eq, "q")
    _assert_bits(gk, ek, "k_cache")
    _assert_bits(gv, ev, "v_cache")


def test_prefill_sized_batch_c3_shape():
    """T = 2076 tokens (the mixed-batch configuration's token count)."""
    T = 2076
    _run_and_check(*_case(T, 14, 2, 64, T // 16 + 8, 16, torch.float16, seed=6))


def test_zero_tokens_is_a_no_op():
    _, _, _, _, _, kc, vc, _ = _case(1, 14, 2, 64, 2, 16, torch.float16)
    gk, gv = kc.to(DEV), vc.to(DEV)
    e = torch.empty(0, 14, 64, dtype=torch.float16, device=DEV)
    ekv = torch.empty(0, 2, 64, dtype=torch.float16, device=DEV)
    ecs = torch.empty(0, 1, 64, dtype=torch.float16, device=DEV)
    out = rope_reshape_and_cache(e, ekv, ekv, ecs, ecs, gk, gv, torch.empty(0, dtype=torch.int64, device=DEV))
    torch.cuda.synchronize()
    assert out.shape == (0, 14, 64)
    _assert_bits(gk, kc, "k_cache")


def test_host_rejects_misaligned_rows():
    q, k, v, cos, sin, kc, vc, slots = _case(4, 14, 2, 64, 2, 16, torch.float16)
    buf = torch.zeros(q.numel() + 1, dtype=torch.float16, device=DEV)
    qm = buf[1:].view(4, 14, 64)  # 2-byte offset: rows are not 16-byte aligned
    with pytest.raises(RuntimeError):
        rope_reshape_and_cache(qm, k.to(DEV), v.to(DEV), cos.to(DEV), sin.to(DEV), kc.to(DEV), vc.to(DEV),
                               slots.to(DEV))


def test_rotary_embedding_table_and_lookup_match_oracle():
    rot = RotaryEmbedding(128, 4096, base=1000000.0, device=DEV)
    ct, st = rope_table_ref(128, 4096, 1000000.0)
    _assert_bits(rot.cos_cached, ct, "cos table")
    _assert_bits(rot.sin_cached, st, "sin table")
    pos = torch.tensor([0, 4095, 17, 17, 1000])
    cos, sin = rot.cos_sin(pos.to(DEV), torch.bfloat16)
    ec, es = rope_cos_sin_ref(ct, st, pos, torch.bfloat16)
    _assert_bits(cos, ec, "cos")
    _assert_bits(sin, es, "sin")


def test_fused_then_attention_matches_reference_layer_step():
    """A layer's attention step on the mixed-batch shape: fused rotary + write, then paged attention.

    Reference order (qwen2.py:53-64): rotary.apply, kv_cache.write, attn_fn.
    The fused kernel must leave the cache and q exactly as the two reference
    steps do, so the attention output equals the oracle's within the fp16
    bound.
    """
    case = make_case("c3", seed=3, device="cpu")
    T, Hq, Hkv, D = case.query.shape[0], 14, 2, 64
    g = torch.Generator().manual_seed(8)
    q = torch.randn(T, Hq, D, generator=g).half()
    k = torch.randn(T, Hkv, D, generator=g).half()
    v = torch.randn(T, Hkv, D, generator=g).half()
    md = case.md
    pos = []
    for sl, ql in zip(md.seq_lens_cpu, md.query_lens_cpu):
        pos += list(range(sl - ql, sl))
    rot = RotaryEmbedding(D, 32768)
    cos, sin = rope_cos_sin_ref(rot.cos_cached, rot.sin_cached, torch.tensor(pos), torch.float16)
    eq, ek, ev = rope_reshape_and_cache_ref(q, k, v, cos, sin, case.k_cache, case.v_cache, md.slot_mapping)
    want = paged_attention_ref(eq, ek, ev, md, 1.0 / math.sqrt(D))

    cache = PagedKVCache(case.k_cache.shape[0], case.k_cache.shape[1], 1, Hkv, D, torch.float16, DEV)
    cache.k_cache[0].copy_(case.k_cache)
    cache.v_cache[0].copy_(case.v_cache)
    gmd = md_to(md, DEV)
    rot.to(DEV)
    gcos, gsin = rot.cos_sin(torch.tensor(pos, device=DEV), torch.float16)
    gq = rope_reshape_and_cache(q.to(DEV), k.to(DEV), v.to(DEV), gcos, gsin,
                                cache.k_cache[0], cache.v_cache[0], gmd.slot_mapping)
    out = paged_attention_hip(gq, cache.k_cache[0], cache.v_cache[0], gmd, 1.0 / math.sqrt(D))
    torch.cuda.synchronize()
    _assert_bits(gq, eq, "q")
    _assert_bits(cache.k_cache[0], ek, "k_cache")
    err = (out.float().cpu() - want).abs().max().item()
    assert err <= 2e-3, f"max abs err {err:.3e}"


def test_unfused_reference_path_equals_fused():
    """Two HIP-side steps (oracle rotation, then the HIP cache write) == the fused launch."""
    q, k, v, cos, sin, kc, vc, slots = _case(64, 14, 2, 64, 6, 16, torch.float16, seed=9)
    qa, ka = rope_apply_ref(q, k, cos, sin)
    gk1, gv1 = kc.to(DEV), vc.to(DEV)
    reshape_and_cache(ka.to(DEV), v.to(DEV), gk1, gv1, slots.to(DEV))
    gk2, gv2 = kc.to(DEV), vc.to(DEV)
    gq = rope_reshape_and_cache(q.to(DEV), k.to(DEV), v.to(DEV), cos.to(DEV), sin.to(DEV), gk2, gv2,
                                slots.to(DEV))
    torch.cuda.synchronize()
    _assert_bits(gq, qa, "q")
    _assert_bits(gk2, gk1, "k_cache")
    _assert_bits(gv2, gv1, "v_cache")
