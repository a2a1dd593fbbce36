"""HIP paged attention against the CPU oracle (runs on an MI355X).

Tolerances are the ones the build is held to: max-abs error <= 2e-3 for fp16
and <= 1e-2 for bf16 outputs against the fp32-accumulated oracle, which is the
reference's gather+SDPA restated on the CPU.  Cases mirror the reference's
tests (tests/test_paged_attention.py:97-229) at the kernels' head sizes, plus
the benchmark configurations and the edge cases of the boundary (int32/int64
indices, stale slots, empty contexts, invalid block ids, ragged batches).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from nanoserve_amd import paged_attention_hip
from nanoserve_amd.attention import _attention, _workspaces, prepare_decode_plan
from nanoserve_amd.capture import graph_capture
from nanoserve_amd.workloads import make_case, metadata_for
from oracle.paged_attention import dense_reference, paged_attention_ref
from tests._helpers import build_paged, make_md, md_to

pytestmark = pytest.mark.gpu

TOL = {torch.float16: 2e-3, torch.bfloat16: 1e-2}
DEV = "cuda"


def _run(q, kc, vc, md, scale):
    out = paged_attention_hip(q.to(DEV), kc.to(DEV), vc.to(DEV), md_to(md, DEV), scale)
    torch.cuda.synchronize()
    return out.float().cpu()


def _assert_close(got, ref, dtype, what=""):
    err = (got.float() - ref.float()).abs().max().item()
    assert err <= TOL[dtype], f"{what} max abs err {err:.3e} > {TOL[dtype]:.0e}"
    return err


def _case(seqs, query_lens, Hq, Hkv, D, bs, dtype, num_blocks=None, q_seed=7, index_dtype=torch.int32):
    nb = num_blocks or sum(-(-s // bs) for s in seqs) + 8
    kc, vc, tables, truth = build_paged(seqs, nb, bs, Hkv, D, dtype=dtype)
    md = make_md(seqs, query_lens, tables, bs, index_dtype=index_dtype)
    q = torch.randn(sum(query_lens), Hq, D, generator=torch.Generator().manual_seed(q_seed)).to(dtype)
    return q, kc, vc, md, tables, truth


# ---- the reference's GPU test, at its own shapes --------------------------------
@pytest.mark.parametrize("block_size", [16, 32])
@pytest.mark.parametrize("seqs", [[1, 9, 33], [128, 7], [64] * 8])
def test_decode_matches_oracle_reference_shapes(block_size, seqs):
    q, kc, vc, md, _, _ = _case(seqs, [1] * len(seqs), 6, 2, 64, block_size, torch.float16, num_blocks=512)
    scale = 1.0 / math.sqrt(64)
    _assert_close(_run(q, kc, vc, md, scale), paged_attention_ref(q, kc, vc, md, scale), torch.float16)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("group", [1, 2, 7, 8, 16])
def test_decode_head_shapes(dtype, D, group):
    Hkv = 2
    seqs = [1, 15, 16, 17, 255, 256, 257, 700, 1500]
    q, kc, vc, md, _, truth = _case(seqs, [1] * len(seqs), group * Hkv, Hkv, D, 16, dtype, q_seed=group)
    scale = 1.0 / math.sqrt(D)
    got = _run(q, kc, vc, md, scale)
    _assert_close(got, paged_attention_ref(q, kc, vc, md, scale), dtype)
    for i, sl in enumerate(seqs[:3]):
        ref = dense_reference(q[i:i + 1].float(), truth[i][0].float(), truth[i][1].float(), sl - 1, group, scale)
        assert np.abs(got[i:i + 1].numpy() - ref).max() <= TOL[dtype]


@pytest.mark.parametrize("block_size", [8, 16, 32, 64])
def test_decode_block_sizes(block_size):
    seqs = [3, 40, 333, 1024, 2049]
    q, kc, vc, md, _, _ = _case(seqs, [1] * len(seqs), 14, 2, 64, block_size, torch.float16)
    scale = 0.125
    _assert_close(_run(q, kc, vc, md, scale), paged_attention_ref(q, kc, vc, md, scale), torch.float16)


def test_decode_int32_and_int64_indices_agree():
    seqs = [5, 300, 4000, 77]
    q, kc, vc, md32, tables, _ = _case(seqs, [1] * 4, 14, 2, 64, 16, torch.float16, index_dtype=torch.int32)
    md64 = make_md(seqs, [1] * 4, tables, 16, index_dtype=torch.int64)
    a = _run(q, kc, vc, md32, 0.125)
    b = _run(q, kc, vc, md64, 0.125)
    assert torch.equal(a, b)
    _assert_close(a, paged_attention_ref(q, kc, vc, md32, 0.125), torch.float16)


def test_decode_ignores_stale_kv_in_padded_slots():
    Hq, Hkv, D, bs = 14, 2, 64, 16
    seqs = [3, 40, 1000]
    kc, vc, tables, truth = build_paged(seqs, 128, bs, Hkv, D, dtype=torch.float16, fill=1e3)
    kf, vf = kc.view(-1, Hkv, D), vc.view(-1, Hkv, D)
    for i, sl in enumerate(seqs):  # poison the owned blocks' unused tail too
        for p in range(sl, len(tables[i]) * bs):
            kf[tables[i][p // bs] * bs + p % bs] = 1e3
            vf[tables[i][p // bs] * bs + p % bs] = 1e3
    md = make_md(seqs, [1] * 3, tables, bs)
    q = torch.randn(3, Hq, D, generator=torch.Generator().manual_seed(3)).half()
    got = _run(q, kc, vc, md, 0.125)
    for i, sl in enumerate(seqs):
        ref = dense_reference(q[i:i + 1].float(), truth[i][0].float(), truth[i][1].float(), sl - 1, 7, 0.125)
        assert np.abs(got[i:i + 1].numpy() - ref).max() <= 2e-3


def test_decode_empty_context_is_zero():
    seqs = [0, 20]
    kc, vc, tables, _ = build_paged([1, 20], 8, 16, 2, 64, dtype=torch.float16)
    md = make_md(seqs, [1, 1], tables, 16)
    q = torch.randn(2, 14, 64).half()
    got = _run(q, kc, vc, md, 0.125)
    assert torch.count_nonzero(got[0]) == 0
    _assert_close(got, paged_attention_ref(q, kc, vc, md, 0.125), torch.float16)


def test_decode_invalid_block_id_poisons_only_its_sequence():
    seqs = [40, 40]
    kc, vc, tables, _ = build_paged(seqs, 16, 16, 2, 64, dtype=torch.float16)
    md = make_md(seqs, [1, 1], tables, 16)
    md.block_tables[0, 1] = 10_000  # beyond the cache: must never be dereferenced
    q = torch.randn(2, 14, 64).half()
    got = _run(q, kc, vc, md, 0.125)
    assert torch.isnan(got[0]).all()
    md_ok = make_md(seqs, [1, 1], tables, 16)
    _assert_close(got[1:], paged_attention_ref(q, kc, vc, md_ok, 0.125)[1:], torch.float16)


def test_decode_table_permutation_invariance():
    seqs = [100, 900, 17]
    ka, va, ta, _ = build_paged(seqs, 80, 16, 2, 64, dtype=torch.float16, shuffle=True, seed=5)
    kb, vb, tb, _ = build_paged(seqs, 80, 16, 2, 64, dtype=torch.float16, shuffle=False, seed=5)
    q = torch.randn(3, 14, 64).half()
    a = _run(q, ka, va, make_md(seqs, [1] * 3, ta, 16), 0.125)
    b = _run(q, kb, vb, make_md(seqs, [1] * 3, tb, 16), 0.125)
    _assert_close(a, b, torch.float16)


def test_decode_wider_table_and_larger_max_seq_len():
    """Wider tables / larger max_seq_len change the split plan, not the result."""
    seqs = [5000, 700, 33]
    q, kc, vc, md, tables, _ = _case(seqs, [1] * 3, 14, 2, 64, 16, torch.float16, num_blocks=600)
    a = _run(q, kc, vc, md, 0.125)
    wide = make_md(seqs, [1] * 3, [t + [0] * 100 for t in tables], 16)
    wide.max_seq_len = 40000
    wide.block_tables = torch.cat([wide.block_tables, torch.zeros(3, 3000, dtype=torch.int32)], dim=1)
    b = _run(q, kc, vc, wide, 0.125)
    _assert_close(a, b, torch.float16)
    _assert_close(a, paged_attention_ref(q, kc, vc, md, 0.125), torch.float16)


def test_decode_prepared_plan_and_per_call_plan_agree_bitwise():
    """The decode plan is built on the device from seq_lens: by the step's first
    call and stored on md, explicitly before it (prepare_decode_plan), or by the
    library inside a call that shares none; with or without the host copies of
    the lengths the same plan, arithmetic and merge order give identical bits."""
    seqs = [5, 300, 4000, 77, 1, 2048, 0]
    q, kc, vc, md, tables, _ = _case(seqs, [1] * len(seqs), 14, 2, 64, 16, torch.float16)
    md_nolist = make_md(seqs, [1] * len(seqs), tables, 16, with_cpu_lists=False)
    a = _run(q, kc, vc, md, 0.125)
    b = _run(q, kc, vc, md_nolist, 0.125)
    mdd = md_to(md, DEV)
    prepare_decode_plan(mdd, kc.to(DEV))
    assert mdd.decode_plan is not None
    c = paged_attention_hip(q.to(DEV), kc.to(DEV), vc.to(DEV), mdd, 0.125).float().cpu()
    own = md_to(md, DEV)
    d = _attention(q.to(DEV), kc.to(DEV), vc.to(DEV), own, 0.125, share_plan=False).float().cpu()
    assert own.decode_plan is None  # the library planned inside the call
    assert torch.equal(a, b) and torch.equal(a, c) and torch.equal(a, d)
    _assert_close(a, paged_attention_ref(q, kc, vc, md, 0.125), torch.float16)


def test_first_call_of_a_step_builds_the_plan_the_others_reuse():
    """The unchanged reference call pattern (qwen2.py:59-65: one md, one call
    per layer, no per-step hook): the first call stores the plan on md, later
    calls reuse that same buffer, and a new md (the next step) gets its own."""
    seqs = [700, 33, 1900, 260]
    q, kc, vc, md, tables, _ = _case(seqs, [1] * 4, 14, 2, 64, 16, torch.float16)
    mdd = md_to(md, DEV)
    assert mdd.decode_plan is None
    first = paged_attention_hip(q.to(DEV), kc.to(DEV), vc.to(DEV), mdd, 0.125)
    plan = mdd.decode_plan
    assert plan is not None
    again = paged_attention_hip(q.to(DEV), kc.to(DEV), vc.to(DEV), mdd, 0.125)
    assert mdd.decode_plan is plan
    nxt = md_to(md, DEV)
    paged_attention_hip(q.to(DEV), kc.to(DEV), vc.to(DEV), nxt, 0.125)
    assert nxt.decode_plan is not None and nxt.decode_plan is not plan
    torch.cuda.synchronize()
    assert torch.equal(first, again)
    _assert_close(first.float().cpu(), paged_attention_ref(q, kc, vc, md, 0.125), torch.float16)


def test_decode_plan_is_shared_by_the_layers_of_a_step():
    """One plan, several layers (each its own caches and queries): every call
    equals the same call planning for itself, and a plan built for other sizes
    is not used."""
    seqs = [700, 33, 1900, 260]
    q, kc, vc, md, tables, _ = _case(seqs, [1] * 4, 14, 2, 64, 16, torch.float16)
    mdd = md_to(md, DEV)
    prepare_decode_plan(mdd, kc.to(DEV))
    for layer in range(3):
        g = torch.Generator().manual_seed(40 + layer)
        ql = torch.randn(q.shape, generator=g).half().to(DEV)
        kl = torch.randn(kc.shape, generator=g).half().to(DEV)
        vl = torch.randn(vc.shape, generator=g).half().to(DEV)
        shared = paged_attention_hip(ql, kl, vl, mdd, 0.125)
        own = _attention(ql, kl, vl, md_to(md, DEV), 0.125, share_plan=False)
        torch.cuda.synchronize()
        assert torch.equal(shared, own), f"layer {layer}"
    # A plan for another head size does not apply to this call: it plans for itself.
    other = md_to(md, DEV)
    prepare_decode_plan(other, torch.empty(1, 16, 2, 128, device=DEV, dtype=torch.float16))
    got = _run(q, kc, vc, other, 0.125)
    _assert_close(got, paged_attention_ref(q, kc, vc, md, 0.125), torch.float16)


def test_decode_many_items_per_pair_and_rounds():
    """100 x ~2000 tokens: several rounds of items, each pair cut into several
    items merged in-launch; the waves pipeline several steps per item."""
    seqs = [2000 + 7 * i for i in range(100)]
    q, kc, vc, md, tables, _ = _case(seqs, [1] * len(seqs), 14, 2, 64, 16, torch.float16, q_seed=3)
    got = _run(q, kc, vc, md, 0.125)
    _assert_close(got, paged_attention_ref(q, kc, vc, md, 0.125), torch.float16)


def test_decode_more_pairs_than_items_per_round():
    """More (sequence, kv head) pairs than a round of items: one item per pair,
    the workgroups loop over them."""
    seqs = [37 + (7 * i) % 500 for i in range(400)]  # 800 pairs
    q, kc, vc, md, _, _ = _case(seqs, [1] * len(seqs), 14, 2, 64, 16, torch.float16, q_seed=4)
    _assert_close(_run(q, kc, vc, md, 0.125), paged_attention_ref(q, kc, vc, md, 0.125), torch.float16)


def test_decode_follows_the_device_lengths_whatever_the_host_copy_says():
    """Decode rows are planned from the device lengths: a host copy that
    disagrees (shorter or longer) changes nothing."""
    seqs = [300, 1000, 50]
    q, kc, vc, md, tables, _ = _case(seqs, [1] * 3, 14, 2, 64, 16, torch.float16)
    ref = paged_attention_ref(q, kc, vc, md, 0.125)
    shorter = make_md(seqs, [1] * 3, tables, 16)
    shorter.seq_lens_cpu = [300, 600, 50]
    _assert_close(_run(q, kc, vc, shorter, 0.125), ref, torch.float16)
    longer = make_md([300, 1500, 50], [1] * 3, [t + [0] * 40 for t in tables], 16)
    longer.seq_lens = md.seq_lens
    _assert_close(_run(q, kc, vc, longer, 0.125), ref, torch.float16)
    _assert_close(_run(q, kc, vc, md, 0.125), ref, torch.float16)


# ---- benchmark configurations ---------------------------------------------------------
# Seeds 0-3: the four steps the benchmark cycles through, so every timed input is checked.
@pytest.mark.parametrize("seed", [0, 1, 2, 3])
@pytest.mark.parametrize("config", ["c1", "c2"])
def test_config_decode_matches_oracle(config, seed):
    case = make_case(config, seed=seed)
    got = _run(case.query, case.k_cache, case.v_cache, case.md, case.scale)
    ref = paged_attention_ref(case.query, case.k_cache, case.v_cache, case.md, case.scale)
    _assert_close(got, ref, case.query.dtype, f"{config} seed {seed}")


@pytest.mark.parametrize("block_size", [16, 32])
def test_c4_subset_matches_oracle(block_size):
    """C4's head shape and length law, 8 sequences, full oracle check."""
    from nanoserve_amd.workloads import sample_lengths
    lens = sample_lengths("c4", 3)[0][:8]
    case = make_case("c4", seed=3, block_size=block_size, seq_lens=lens)
    got = _run(case.query, case.k_cache, case.v_cache, case.md, case.scale)
    ref = paged_attention_ref(case.query, case.k_cache, case.v_cache, case.md, case.scale, per_seq_decode=True)
    _assert_close(got, ref, torch.bfloat16, f"c4 bs{block_size}")


@pytest.mark.parametrize("block_size", [16, 32])
def test_c4_full_batch_sampled_rows(block_size):
    """Full C4 batch on the GPU; 8 sampled sequences checked against the oracle."""
    case = make_case("c4", seed=0, block_size=block_size, device=DEV, gen_device=DEV)
    out = paged_attention_hip(case.query, case.k_cache, case.v_cache, case.md, case.scale).float().cpu()
    rows = np.random.default_rng(block_size).choice(case.md.num_seqs, 8, replace=False).tolist()
    rows = sorted(set(rows) | {int(np.argmax(case.seq_lens))})
    bs = block_size
    for i in rows:
        L, t = case.seq_lens[i], case.tables[i]
        slots = torch.tensor([t[p // bs] * bs + p % bs for p in range(L)], device=DEV)
        K = case.k_cache.view(-1, 4, 128).index_select(0, slots).float().cpu()
        V = case.v_cache.view(-1, 4, 128).index_select(0, slots).float().cpu()
        ref = dense_reference(case.query[i:i + 1].float().cpu(), K, V, L - 1, 7, case.scale)
        err = np.abs(out[i:i + 1].numpy() - ref).max()
        assert err <= 1e-2, f"row {i} (L={L}) err {err}"


# ---- prefill / chunked / mixed ---------------------------------------------------------
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("block_size", [8, 16])
@pytest.mark.parametrize("seqs", [[7], [16], [5, 13, 1], [130, 3, 64]])
def test_prefill_matches_oracle(dtype, block_size, seqs):
    q, kc, vc, md, _, truth = _case(seqs, seqs, 14, 2, 64, block_size, dtype)
    got = _run(q, kc, vc, md, 0.125)
    _assert_close(got, paged_attention_ref(q, kc, vc, md, 0.125), dtype)
    off = 0
    for i, sl in enumerate(seqs):
        ref = dense_reference(q[off:off + sl].float(), truth[i][0].float(), truth[i][1].float(), 0, 7, 0.125)
        assert np.abs(got[off:off + sl].numpy() - ref).max() <= TOL[dtype]
        off += sl


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("group", [1, 7, 16])
def test_prefill_head_shapes(D, group):
    seqs, qls = [300, 40, 129], [300, 17, 64]
    q, kc, vc, md, _, _ = _case(seqs, qls, group * 2, 2, D, 16, torch.float16, q_seed=group)
    scale = 1.0 / math.sqrt(D)
    _assert_close(_run(q, kc, vc, md, scale), paged_attention_ref(q, kc, vc, md, scale), torch.float16)


@pytest.mark.parametrize("seqs,qls", [([9000, 300], [5, 40]), ([4200, 70], [150, 70])])
def test_prefill_block_size_one_crosses_table_windows(seqs, qls):
    """Block size 1 makes one table entry per key, so a workgroup's keys span
    several 4096-entry table windows (the second case puts a window edge
    inside the causal band of the chunk)."""
    q, kc, vc, md, _, _ = _case(seqs, qls, 14, 2, 64, 1, torch.float16)
    _assert_close(_run(q, kc, vc, md, 0.125), paged_attention_ref(q, kc, vc, md, 0.125), torch.float16)


@pytest.mark.parametrize("D,dtype", [(64, torch.float16), (128, torch.bfloat16)])
def test_prefill_long_context_splits_match_unsplit(D, dtype):
    """With host offsets the long key ranges of a chunked prefill are split
    across workgroups and merged in-launch; without them every column block
    walks its whole range.  Both match the oracle."""
    seqs, qls = [4000, 900, 35], [300, 900, 1]
    q, kc, vc, md, tables, _ = _case(seqs, qls, 14, 2, D, 16, dtype)
    md_plain = make_md(seqs, qls, tables, 16, with_cpu_lists=False)
    ref = paged_attention_ref(q, kc, vc, md, 0.125)
    _assert_close(_run(q, kc, vc, md, 0.125), ref, dtype, "planned")
    _assert_close(_run(q, kc, vc, md_plain, 0.125), ref, dtype, "unplanned")


def test_prefill_host_offsets_that_disagree_poison_only_their_sequence():
    seqs, qls = [3000, 64], [200, 64]
    q, kc, vc, md, _, _ = _case(seqs, qls, 14, 2, 64, 16, torch.float16)
    ref = paged_attention_ref(q, kc, vc, md, 0.125)
    md.query_lens_cpu = [100, 64]
    md.query_start_loc_cpu = [0, 100, 164]  # sequence 0's host query length is wrong
    got = _run(q, kc, vc, md, 0.125)
    assert torch.isnan(got[:200]).any()
    _assert_close(got[200:], ref[200:], torch.float16)


def test_prefill_invalid_block_id_poisons_only_its_sequence():
    seqs = [300, 64]
    kc, vc, tables, _ = build_paged(seqs, 32, 16, 2, 64, dtype=torch.float16)
    md = make_md(seqs, seqs, tables, 16)
    md.block_tables[0, 0] = 10_000  # every row of sequence 0 needs block 0
    q = torch.randn(sum(seqs), 14, 64).half()
    got = _run(q, kc, vc, md, 0.125)
    assert torch.isnan(got[:300]).all()
    md_ok = make_md(seqs, seqs, tables, 16)
    _assert_close(got[300:], paged_attention_ref(q, kc, vc, md_ok, 0.125)[300:], torch.float16)


def test_chunked_prefill_matches_whole_prefill():
    sl = 200
    q, kc, vc, md, tables, _ = _case([sl], [sl], 14, 2, 64, 16, torch.float16)
    whole = _run(q, kc, vc, md, 0.125)
    pieces = [_run(q[a:b], kc, vc, make_md([b], [b - a], tables, 16), 0.125)
              for a, b in ((0, 70), (70, 130), (130, 199), (199, 200))]
    _assert_close(torch.cat(pieces), whole, torch.float16)


def test_mixed_batch_of_prefill_and_decode():
    seqs, qls = [12, 300, 5, 2000, 64], [12, 1, 5, 1, 20]
    q, kc, vc, md, _, _ = _case(seqs, qls, 14, 2, 64, 16, torch.float16, q_seed=17)
    assert not md.is_decode_only
    _assert_close(_run(q, kc, vc, md, 0.125), paged_attention_ref(q, kc, vc, md, 0.125), torch.float16)


def test_mixed_batch_with_empty_query_rows():
    seqs, qls = [12, 30, 9, 50], [12, 0, 1, 0]
    q, kc, vc, md, _, _ = _case(seqs, qls, 14, 2, 64, 16, torch.float16)
    got = _run(q, kc, vc, md, 0.125)
    _assert_close(got, paged_attention_ref(q, kc, vc, md, 0.125), torch.float16)


@pytest.mark.parametrize("seed", [0, 1, 2, 3])
def test_c3_mixed_matches_oracle(seed):
    case = make_case("c3", seed=seed)
    assert case.md.num_tokens == 2076
    got = _run(case.query, case.k_cache, case.v_cache, case.md, case.scale)
    ref = paged_attention_ref(case.query, case.k_cache, case.v_cache, case.md, case.scale)
    _assert_close(got, ref, torch.float16, f"c3 seed {seed}")


def test_engine_int64_metadata_layout():
    """Metadata as the runner stages it: int64 views into one buffer, zero-padded rows."""
    from nanoserve_amd.metadata import ScheduledSeq, build_metadata
    seqs, qls = [100, 37, 512], [1, 37, 12]
    kc, vc, tables, _ = build_paged(seqs, 64, 16, 2, 64, dtype=torch.float16)
    batch = [ScheduledSeq(t, L - q, L, i) for i, (t, L, q) in enumerate(zip(tables, seqs, qls))]
    _, md = build_metadata(batch, 16, DEV)
    assert md.block_tables.dtype == torch.int64
    q = torch.randn(sum(qls), 14, 64).half()
    got = paged_attention_hip(q.to(DEV), kc.to(DEV), vc.to(DEV), md, 0.125).float().cpu()
    ref = paged_attention_ref(q, kc, vc, make_md(seqs, qls, tables, 16), 0.125)
    _assert_close(got, ref, torch.float16)


def test_repeated_calls_reuse_workspace():
    """Split-K counters are left at zero: back-to-back calls give identical results."""
    case = make_case("c2", seed=4, device=DEV, gen_device=DEV)
    outs = [paged_attention_hip(case.query, case.k_cache, case.v_cache, case.md, case.scale).clone()
            for _ in range(5)]
    torch.cuda.synchronize()
    for o in outs[1:]:
        assert torch.equal(o, outs[0])


@pytest.mark.parametrize("config", ["c2", "c3"])
def test_graph_replays_match_eager(config):
    """Capture calls in a HIP graph; every replay matches the eager result.

    Eager calls run between replays, so the split-K counters a replay leaves
    behind are exercised by the eager path and the other way round.  The mixed
    c3 batch forks its decode rows onto the shim's aux stream, so its capture
    records the fork and the join.
    """
    case = make_case(config, seed=5, device=DEV, gen_device=DEV)
    eager = paged_attention_hip(case.query, case.k_cache, case.v_cache, case.md, case.scale).clone()
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):  # warm the workspace of this stream before capture
        paged_attention_hip(case.query, case.k_cache, case.v_cache, case.md, case.scale)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with graph_capture(graph, stream=s):
        out = paged_attention_hip(case.query, case.k_cache, case.v_cache, case.md, case.scale)
    with torch.inference_mode():
        for _ in range(4):
            out.fill_(0)
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, eager)
            again = paged_attention_hip(case.query, case.k_cache, case.v_cache, case.md, case.scale)
            torch.cuda.synchronize()
            assert torch.equal(again, eager)


def test_workspace_reused_across_shapes():
    """One workspace (per stream) serves calls of different shapes back to
    back: partials of one call never land on another call's counters."""
    cases = [
        ([37 + (13 * i) % 900 for i in range(60)], None),   # decode, many split pairs
        ([4000, 900, 35], [300, 900, 1]),                   # prefill splits + decode rows
        ([5, 17], None),                                    # tiny decode
        ([2500, 64], [64, 64]),                             # prefill splits again
    ]
    for _ in range(2):
        for seqs, qls in cases:
            qls = qls or [1] * len(seqs)
            q, kc, vc, md, _, _ = _case(seqs, qls, 14, 2, 64, 16, torch.float16)
            _assert_close(_run(q, kc, vc, md, 0.125), paged_attention_ref(q, kc, vc, md, 0.125),
                          torch.float16, f"{len(seqs)} seqs")


def test_rejects_unsupported_shapes():
    """Head sizes past 256 and non-float dtypes are refused; float32, head size 96 and 32
    query heads per KV head run the generic kernel (tests/test_gpu_generic_attention.py)."""
    md = metadata_for([5], [1], [[0]], 16, DEV)
    kc = torch.zeros(4, 16, 1, 320, device=DEV, dtype=torch.float16)
    with pytest.raises(RuntimeError):
        paged_attention_hip(torch.zeros(1, 2, 320, device=DEV, dtype=torch.float16), kc, kc, md, 0.1)
    kc = torch.zeros(4, 16, 1, 64, device=DEV, dtype=torch.float64)
    with pytest.raises(TypeError):
        paged_attention_hip(torch.zeros(1, 2, 64, device=DEV, dtype=torch.float64), kc, kc, md, 0.1)
    kc = torch.zeros(4, 16, 1, 64, device=DEV, dtype=torch.float16)
    with pytest.raises(TypeError):
        paged_attention_hip(torch.zeros(1, 2, 64, device=DEV), kc, kc, md, 0.1)  # dtypes differ
    for D, Hq, dtype in ((96, 2, torch.float16), (64, 32, torch.float16), (64, 2, torch.float32)):
        kc = torch.zeros(4, 16, 1, D, device=DEV, dtype=dtype)
        out = paged_attention_hip(torch.zeros(1, Hq, D, device=DEV, dtype=dtype), kc, kc, md, 0.1)
        torch.cuda.synchronize()
        assert out.shape == (1, Hq, D) and torch.count_nonzero(out) == 0  # zero values average to zero


def test_workspace_counters_and_prefill_slots_are_left_zero():
    """The arrival counters (the first 4 MiB) and the prefill split-K slots
    (the 36 MiB after the 8 MiB head) go back to zero after decode calls with
    merged splits and after a mixed call whose prefill rows split, so a
    workspace reused by calls of other shapes starts every protocol clean;
    only the decode slots after them keep partials."""
    cases = [([4000, 900, 35, 2000, 1], None), ([4000, 900, 35], [300, 900, 1]), ([5000, 64], [64, 64])]
    head, prefill = 8 << 20, 36 << 20
    for seqs, qls in cases:
        qls = qls or [1] * len(seqs)
        q, kc, vc, md, _, _ = _case(seqs, qls, 14, 2, 64, 16, torch.float16)
        _assert_close(_run(q, kc, vc, md, 0.125), paged_attention_ref(q, kc, vc, md, 0.125), torch.float16)
        stream = torch.cuda.current_stream().cuda_stream
        ws = _workspaces[(torch.cuda.current_device(), stream)]
        torch.cuda.synchronize()
        assert ws.numel() >= head + prefill
        assert not ws[:4 << 20].any(), "arrival counters must be back at zero"
        assert not ws[head:head + prefill].any(), f"{len(seqs)} seqs: prefill split slots not cleared"
