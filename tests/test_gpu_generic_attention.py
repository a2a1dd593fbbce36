"""The generic kernel: float32, head sizes other than 64/128, block sizes that are
not powers of two and wide query groups, on an MI355X.

The reference's own paged-attention tests run float32 at head size 8 with block
sizes 4, 8 and 16 (tests/test_paged_attention.py:97-134): those cases are
repeated here through the HIP path against the float64 textbook reference at
the reference's tolerance (2e-5).  Float16/bfloat16 cases at other head sizes
are held to the MFMA kernels' tolerances against the float32 oracle.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from nanoserve_amd import paged_attention_hip
from oracle.paged_attention import dense_reference, paged_attention_ref
from tests._helpers import build_paged, make_md, md_to

pytestmark = pytest.mark.gpu

DEV = "cuda"
TOL = {torch.float32: 2e-5, torch.float16: 2e-3, torch.bfloat16: 1e-2}


def _run(q, kc, vc, md, scale):
    out = paged_attention_hip(q.to(DEV), kc.to(DEV), vc.to(DEV), md_to(md, DEV), scale)
    torch.cuda.synchronize()
    assert out.dtype == q.dtype and out.shape == q.shape
    return out.float().cpu()


def _case(seqs, query_lens, Hq, Hkv, D, bs, dtype, seed=7, fill=0.0, index_dtype=torch.int32):
    nb = sum(-(-s // bs) for s in seqs) + 6
    kc, vc, tables, truth = build_paged(seqs, nb, bs, Hkv, D, dtype=dtype, fill=fill)
    md = make_md(seqs, query_lens, tables, bs, index_dtype=index_dtype)
    q = torch.randn(sum(query_lens), Hq, D, generator=torch.Generator().manual_seed(seed)).to(dtype)
    return q, kc, vc, md, truth


@pytest.mark.parametrize("block_size", [4, 8, 16])
@pytest.mark.parametrize("seqs", [[7], [16], [5, 13, 1], [1, 1, 1, 1]])
def test_reference_prefill_case_float32_head_size_8(block_size, seqs):
    print(f"generic prefill fp32 D=8 bs={block_size} seqs={seqs}", flush=True)
    q, kc, vc, md, truth = _case(seqs, seqs, 4, 2, 8, block_size, torch.float32)
    got = _run(q, kc, vc, md, 1.0 / math.sqrt(8))
    off = 0
    for i, sl in enumerate(seqs):
        K, V = truth[i]
        ref = dense_reference(q[off:off + sl], K, V, 0, 2)
        np.testing.assert_allclose(got[off:off + sl].numpy(), ref, atol=2e-5, rtol=2e-5)
        off += sl


@pytest.mark.parametrize("block_size", [4, 16])
@pytest.mark.parametrize("seqs", [[1, 9, 33], [16, 16], [64, 3, 17, 40]])
def test_reference_decode_case_float32_head_size_8(block_size, seqs):
    print(f"generic decode fp32 D=8 bs={block_size} seqs={seqs}", flush=True)
    q, kc, vc, md, truth = _case(seqs, [1] * len(seqs), 6, 2, 8, block_size, torch.float32, seed=11)
    assert md.is_decode_only
    got = _run(q, kc, vc, md, 1.0 / math.sqrt(8))
    for i, sl in enumerate(seqs):
        K, V = truth[i]
        ref = dense_reference(q[i:i + 1], K, V, sl - 1, 3)
        np.testing.assert_allclose(got[i:i + 1].numpy(), ref, atol=2e-5, rtol=2e-5)


def test_float32_decode_ignores_stale_kv_in_padded_slots():
    """The reference's stale-slot case (tests/test_paged_attention.py:137-160) in float32:
    slots past a sequence's length hold 1e3 and must not change its row."""
    seqs = [3, 29, 16]
    q, kc, vc, md, truth = _case(seqs, [1, 1, 1], 4, 2, 16, 8, torch.float32, fill=1e3)
    got = _run(q, kc, vc, md, 0.25)
    for i, sl in enumerate(seqs):
        ref = dense_reference(q[i:i + 1], truth[i][0], truth[i][1], sl - 1, 2, 0.25)
        np.testing.assert_allclose(got[i:i + 1].numpy(), ref, atol=2e-5, rtol=2e-5)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("Hq,Hkv,D,bs", [(14, 2, 64, 16), (4, 2, 32, 16), (8, 2, 96, 16), (4, 1, 256, 16),
                                         (14, 2, 64, 12), (40, 2, 64, 16), (6, 3, 80, 5)])
def test_mixed_batch_against_the_oracle(dtype, Hq, Hkv, D, bs):
    """Decode rows, a whole prompt and a chunk behind cached context in one call."""
    if dtype != torch.float32 and D in (64, 128) and bs & (bs - 1) == 0 and Hq // Hkv <= 16:
        pytest.skip("the MFMA kernels take this shape (tests/test_gpu_attention.py)")
    print(f"generic mixed {dtype} Hq={Hq} Hkv={Hkv} D={D} bs={bs}", flush=True)
    seqs, qls = [1, 70, 37, 130, 9], [1, 1, 37, 40, 9]
    q, kc, vc, md, _ = _case(seqs, qls, Hq, Hkv, D, bs, dtype)
    scale = 1.0 / math.sqrt(D)
    got = _run(q, kc, vc, md, scale)
    ref = paged_attention_ref(q, kc, vc, md, scale)
    err = (got - ref.float()).abs().max().item()
    assert err <= TOL[dtype] * (1.0 if dtype != torch.float32 else max(1.0, ref.abs().max().item())), err


@pytest.mark.parametrize("index_dtype", [torch.int32, torch.int64])
def test_decode_only_float32_long_contexts(index_dtype):
    seqs = [1000, 1, 333, 64]
    q, kc, vc, md, _ = _case(seqs, [1] * 4, 14, 2, 64, 16, torch.float32, index_dtype=index_dtype)
    got = _run(q, kc, vc, md, 0.125)
    ref = paged_attention_ref(q, kc, vc, md, 0.125)
    assert (got - ref).abs().max().item() <= 2e-5


def test_empty_context_is_zero_and_a_bad_block_poisons_only_its_row():
    seqs = [0, 20, 20]
    kc, vc, tables, _ = build_paged([1, 20, 20], 12, 4, 2, 8, dtype=torch.float32)
    md = make_md(seqs, [1, 1, 1], tables, 4)
    md.block_tables[2, 1] = 10_000  # beyond the cache: never dereferenced
    q = torch.randn(3, 4, 8)
    got = _run(q, kc, vc, md, 0.3)
    assert torch.count_nonzero(got[0]) == 0
    assert torch.isnan(got[2]).all()
    ok = make_md(seqs, [1, 1, 1], tables, 4)
    ref = paged_attention_ref(q, kc, vc, ok, 0.3)
    assert (got[1] - ref[1]).abs().max().item() <= 2e-5


def test_chunked_prefill_equals_whole_prefill_float32():
    """A prompt prefilled in two chunks gives the rows of the whole prefill (the second
    chunk sees the first chunk's keys through the cache)."""
    seqs = [50]
    q, kc, vc, md, _ = _case(seqs, seqs, 4, 2, 24, 6, torch.float32)
    whole = _run(q, kc, vc, md, 0.2)
    md1 = make_md([30], [30], [md.block_tables[0].tolist()], 6)
    md2 = make_md([50], [20], [md.block_tables[0].tolist()], 6)
    first = _run(q[:30], kc, vc, md1, 0.2)
    second = _run(q[30:], kc, vc, md2, 0.2)
    assert (torch.cat([first, second]) - whole).abs().max().item() <= 1e-6
