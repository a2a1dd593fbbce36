"""ns_paged_attention_noalloc against ns_paged_attention, through the C ABI (MI355X).

The no-alloc entry point runs the same kernels on a library-held scratch array
instead of a caller workspace, so its outputs must equal the workspace entry
point's bit for bit.  Two calls in a row on the same scratch, the second with
a smaller batch, check that a call leaves the scratch ready for the next (the
split-K counters back at zero) whatever the shape; a mixed batch covers the
prefill split state; a shape whose workspace exceeds the 128 MiB scratch is
refused with NS_ERR_WORKSPACE.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from nanoserve_amd import _lib
from nanoserve_amd.workloads import make_case

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _args(case, out):
    md = case.md
    q, kc, vc = case.query, case.k_cache, case.v_cache
    T, Hq, D = q.shape
    NB, BS, Hkv, _ = kc.shape
    bt, sl = md.block_tables, md.seq_lens
    qsl = None if md.is_decode_only else md.query_start_loc
    lens = (ctypes.c_int64 * md.num_seqs)(*md.seq_lens_cpu)
    qslh = None if md.is_decode_only else (ctypes.c_int64 * (md.num_seqs + 1))(*md.query_start_loc_cpu)
    return [out.data_ptr(), q.data_ptr(), kc.data_ptr(), vc.data_ptr(),
            bt.data_ptr(), bt.stride(0), bt.shape[1], int(bt.dtype == torch.int64),
            sl.data_ptr(), int(sl.dtype == torch.int64),
            None if qsl is None else qsl.data_ptr(), int(qsl is not None and qsl.dtype == torch.int64),
            lens, 1, qslh, 1,
            md.num_seqs, md.num_tokens, md.max_query_len, md.max_seq_len, int(md.is_decode_only),
            Hq, Hkv, D, BS, NB, case.scale, _lib.DTYPE_CODES[q.dtype], None, 0]


def _with_workspace(case):
    lib = _lib.load()
    md = case.md
    T, Hq, D = case.query.shape
    _, BS, Hkv, _ = case.k_cache.shape
    n = lib.ns_paged_attention_workspace_size(md.num_seqs, Hq, Hkv, D, BS, md.max_seq_len, md.max_query_len,
                                              md.num_tokens, int(md.is_decode_only))
    ws = torch.zeros(n, dtype=torch.uint8, device=DEV)
    out = torch.empty_like(case.query)
    stream = torch.cuda.current_stream().cuda_stream
    rc = lib.ns_paged_attention(*_args(case, out), ws.data_ptr(), ws.numel(), stream, None, None, None)
    _lib.check(rc, "ns_paged_attention")
    return out


def _no_alloc(case):
    lib = _lib.load()
    out = torch.empty_like(case.query)
    stream = torch.cuda.current_stream().cuda_stream
    rc = lib.ns_paged_attention_noalloc(*_args(case, out), stream, None, None, None)
    _lib.check(rc, "ns_paged_attention_noalloc")
    return out


@pytest.mark.parametrize("first,second", [("c2", "c1"), ("c3", "c1")])
def test_no_alloc_matches_the_workspace_entry_on_consecutive_calls(first, second):
    for seed, config in enumerate((first, second)):
        print(f"no-alloc {config} seed {seed}", flush=True)
        case = make_case(config, seed=seed, device=DEV, gen_device=DEV)
        got = _no_alloc(case)
        want = _with_workspace(case)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"{config}: no-alloc output differs from the workspace entry point"
        assert torch.isfinite(got.float()).all()


def test_no_alloc_is_repeatable_and_refuses_oversized_shapes():
    case = make_case("c2", seed=7, device=DEV, gen_device=DEV)
    a = _no_alloc(case)
    b = _no_alloc(case)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    lib = _lib.load()
    # 256 sequences of up to 64K tokens, 16 query heads per kv head at head_dim
    # 128: the plan fits the workspace's plan region, the decode split-K
    # slots do not fit the scratch.
    big = lib.ns_paged_attention_workspace_size(256, 64, 4, 128, 16, 65536, 1, 256, 1)
    assert big > 128 << 20
    out = torch.empty(16, device=DEV)
    rc = lib.ns_paged_attention_noalloc(out.data_ptr(), out.data_ptr(), out.data_ptr(), out.data_ptr(),
                                        out.data_ptr(), 4096, 4096, 0, out.data_ptr(), 0, None, 0, None, 0,
                                        None, 0, 256, 256, 1, 65536, 1, 64, 4, 128, 16, 1 << 20,
                                        0.1, _lib.NS_DTYPE_BF16, None, 0, torch.cuda.current_stream().cuda_stream,
                                        None, None, None)
    assert rc == _lib.NS_ERR_WORKSPACE
