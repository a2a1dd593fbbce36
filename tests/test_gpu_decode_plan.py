"""The device-side decode plan (ns_paged_decode_plan), read back and checked.

The plan is the decode kernel's whole schedule, so it is checked on its own,
against properties that do not restate how it is computed:
  * the items of each decode row's (sequence, kv head) pair partition its
    context [0, L) into contiguous, 16-aligned, non-empty ranges (one empty
    item for an empty context), stored next to each other in split order;
  * sequences that are not decode rows (more than one query row in a mixed
    batch) get no items, and each item's query row is the sequence's row;
  * item sizes never exceed the plan's tokens per item, which is a multiple of
    16 no smaller than the minimum, and the item count stays within the
    buffer's capacity and the round target (or one item per pair, or, when
    even the longest items leave more, the plan takes that longest length);
  * a plan of more items than the device has CUs lists its pairs longest
    sequence first (the items run in several rounds); a plan that runs in one
    round keeps the batch's order.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from nanoserve_amd.attention import prepare_decode_plan
from nanoserve_amd.workloads import metadata_for

pytestmark = pytest.mark.gpu
DEV = "cuda"


ITEM_WORDS = 40  # s, qtok, t0, t1, first, nsplit, kvh, split, then 32 first-step block ids


def _read_plan(buf: torch.Tensor, with_blocks=False):
    words = buf.cpu().view(torch.int32).numpy().view(np.uint32)
    n_items, num_seqs, hkv, item_tokens, item_cap = (int(x) for x in words[:5])
    rows = words[16:16 + ITEM_WORDS * n_items].reshape(n_items, ITEM_WORDS)
    items = rows[:, :8].astype(np.int64)
    if with_blocks:
        return n_items, num_seqs, hkv, item_tokens, item_cap, items, rows[:, 8:].view(np.int32).astype(np.int64)
    return n_items, num_seqs, hkv, item_tokens, item_cap, items


def _plan_for(seq_lens, query_lens, hkv=2, d=64, bs=16, index_dtype=torch.int64, with_blocks=False):
    rng = np.random.default_rng(len(seq_lens))
    pool = rng.permutation(sum(-(-max(L, 1) // bs) for L in seq_lens)).tolist()
    tables, at = [], 0
    for L in seq_lens:
        n = -(-max(L, 1) // bs)
        tables.append(pool[at:at + n])
        at += n
    md = metadata_for(seq_lens, query_lens, tables, bs, DEV, index_dtype=index_dtype)
    cache = torch.empty(1, bs, hkv, d, device=DEV, dtype=torch.float16)
    prepare_decode_plan(md, cache)
    torch.cuda.synchronize()
    return md, tables, _read_plan(md.decode_plan.buffer, with_blocks)


def _check(seq_lens, query_lens, hkv=2, d=64, bs=16, index_dtype=torch.int64):
    md, tables, (n, S, H, T, cap, items, blocks) = _plan_for(seq_lens, query_lens, hkv, d, bs, index_dtype, True)
    assert (S, H) == (len(seq_lens), hkv)
    assert T % 16 == 0 and T >= (128 if d == 64 else 64) and n <= cap
    qsl = np.concatenate([[0], np.cumsum(query_lens)])
    decode_rows = [s for s, q in enumerate(query_lens) if q == 1]
    pairs = len(decode_rows) * hkv
    # At most the round target (CUs x rounds, rounds <= 16) or one item per pair,
    # unless even the longest items (kMaxItemTokens = 4096, or the longest
    # context below that) leave more: the plan then takes that length.
    if n > max(256 * 16, pairs):
        assert T == min(4096, -(-max(seq_lens) // 16) * 16), (n, T)
    seen = {}
    for idx, (s, qtok, t0, t1, first, nsplit, kvh, split) in enumerate(items):
        assert s in decode_rows and 0 <= kvh < hkv
        assert qtok == (s if md.is_decode_only else qsl[s])
        assert first + split == idx and split < nsplit
        assert t1 - t0 <= T and t0 % 16 == 0
        seen.setdefault((s, kvh), []).append((split, nsplit, t0, t1, first))
    assert sorted(seen) == [(s, h) for s in decode_rows for h in range(hkv)]
    for (s, h), its in seen.items():
        its.sort()
        L = seq_lens[s]
        nsplit = its[0][1]
        assert [i[0] for i in its] == list(range(nsplit)) and all(i[1] == nsplit for i in its)
        assert len({i[4] for i in its}) == 1
        if L == 0:
            assert its == [(0, 1, 0, 0, its[0][4])]
            continue
        assert its[0][2] == 0 and its[-1][3] == L
        for a, b in zip(its, its[1:]):
            assert a[3] == b[2], f"pair {(s, h)}: ranges not contiguous"
        assert all(i[3] > i[2] for i in its), f"pair {(s, h)}: empty item"
    # Block ids of every wave's first steps (4 waves; 4 tiles of 16 tokens per
    # step at D 64 and 2 at D 128, so 2 and 4 steps fill the 32 entries).
    if bs >= 16:
        nt = 4 if d == 64 else 2
        steps = 32 // (4 * nt)
        for it, blk in zip(items, blocks):
            s, t0, t1 = int(it[0]), int(it[2]), int(it[3])
            per_wave = -(-(-(-(t1 - t0) // 16)) // 4) * 16
            for w in range(4):
                end = min(t1, t0 + (w + 1) * per_wave)
                for st in range(steps):
                    for j in range(nt):
                        t = t0 + w * per_wave + 16 * (st * nt + j)
                        want = tables[s][t // bs] if t < end else 0
                        assert blk[(w * steps + st) * nt + j] == want, (s, t0, w, st, j)
    # Longest sequence first when the items run in rounds; batch order otherwise.
    order = [int(items[i][0]) for i in range(n) if items[i][7] == 0 and items[i][6] == 0]
    if n > torch.cuda.get_device_properties(0).multi_processor_count:
        lens = [seq_lens[s] for s in order]
        assert lens == sorted(lens, reverse=True)
    else:
        assert order == sorted(order)
    return T, n


@pytest.mark.parametrize("index_dtype", [torch.int32, torch.int64])
def test_plan_of_config_like_decode_batches(index_dtype):
    rng = np.random.default_rng(0)
    c2 = np.clip(rng.lognormal(np.log(1024), 0.8, 32).astype(int), 16, 8192).tolist()
    T, n = _check(c2, [1] * 32, index_dtype=index_dtype)
    assert n <= 256, "a c2-sized batch is one round of items"
    c1 = rng.integers(64, 513, 8).tolist()
    _check(c1, [1] * 8, index_dtype=index_dtype)
    c4 = np.clip(rng.lognormal(np.log(4096), 1.0, 64).astype(int), 128, 32768).tolist()
    _check(c4, [1] * 64, hkv=4, d=128, index_dtype=index_dtype)


def test_one_round_plans_keep_long_items_while_half_the_cus_get_one():
    """A one-round D=64 plan takes 512-token items when the batch still has at
    least half as many items as CUs at that length (fewer split-K merges) or
    when every context fits one such item (no merge at all), and keeps shorter
    items otherwise (the parallelism is needed)."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    rng = np.random.default_rng(0)
    c2 = np.clip(rng.lognormal(np.log(1024), 0.8, 32).astype(int), 16, 8192).tolist()
    at512 = 2 * sum(max(1, -(-L // 512)) for L in c2)
    T, n = _check(c2, [1] * 32)
    if 2 * at512 >= min(cus, 256):
        assert T == 512 and n == at512
    single = [400] * 32  # every context fits one 512-token item
    T, n = _check(single, [1] * 32)
    assert T == 512 and n == 64
    mixed = [400] * 31 + [900]  # 66 items at 512 tokens and one pair split: short items
    T, n = _check(mixed, [1] * 32)
    assert T < 512 and n > 66


def test_plan_edge_cases():
    _check([0, 0, 5], [1, 1, 1])                       # empty contexts
    _check([1], [1])                                   # a single token
    _check([16, 17, 31, 32, 33], [1] * 5, bs=8)        # tile boundaries
    _check([37 + (7 * i) % 500 for i in range(400)], [1] * 400)  # more pairs than a round
    _check([5000] * 3 + [20] * 200, [1] * 203)        # long pairs beside many short ones


def test_plan_of_a_mixed_batch_lists_only_decode_rows():
    seqs = [700, 1200, 64, 900, 2048]
    qls = [1, 300, 1, 64, 1]
    _check(seqs, qls)
    _check([100, 200], [100, 200])  # no decode row at all: no items


@pytest.mark.parametrize("num_seqs,max_len", [(64, 16384), (256, 16384), (512, 16384), (1024, 32768)])
def test_plan_grid_slices_of_every_size(num_seqs, max_len):
    # The plan kernel's grid writes the fewest whole passes of 8 items per
    # workgroup that keep it within 256 workgroups: these batches' capacities
    # (640, 2560, 5120, 18432 items) give slices of 8, 16, 24 and 32 items, the
    # last on a grid of 576 workgroups.  Every slice must write its items whole.
    rng = np.random.default_rng(num_seqs)
    seqs = rng.integers(1, max_len, num_seqs, endpoint=True).tolist()
    seqs[0] = max_len
    _check(seqs, [1] * num_seqs)


def test_plan_with_more_sequences_than_the_ranked_window():
    rng = np.random.default_rng(3)
    seqs = rng.integers(1, 300, 5000).tolist()
    md, _, (n, S, H, T, cap, items) = _plan_for(seqs, [1] * len(seqs))
    # Beyond 4096 sequences the batch keeps its order; coverage still holds.
    covered = {}
    for s, _, t0, t1, _, _, kvh, _ in items:
        covered[(int(s), int(kvh))] = covered.get((int(s), int(kvh)), 0) + int(t1 - t0)
    assert all(covered[(s, h)] == seqs[s] for s in range(len(seqs)) for h in range(2))
