"""HIP greedy selection (ns_argmax_rows) against torch.argmax's rules (MI355X).

torch.argmax(dim=-1) -- what the reference's greedy sampler calls
(nanoserve/sampler.py:24-27) -- returns the first index among equal maxima
and the first NaN when a row holds one.  Checked on the CPU copy with
numpy's argmax (also first-maximum) and explicit NaN/tie cases.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from nanoserve_amd.sampling import argmax_rows

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _want(x: torch.Tensor) -> list[int]:
    a = x.float().cpu().numpy()
    out = []
    for r in a:
        nan = np.flatnonzero(np.isnan(r))
        out.append(int(nan[0]) if nan.size else int(np.argmax(r)))
    return out


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("M,N", [(1, 151936), (32, 151936), (7, 1000), (3, 13), (64, 512)])
def test_matches_first_maximum(dtype, M, N):
    g = torch.Generator().manual_seed(M * N)
    x = (torch.randn(M, N, generator=g) * 4).to(dtype)
    got = argmax_rows(x.to(DEV))
    torch.cuda.synchronize()
    assert got.dtype == torch.int64 and got.tolist() == _want(x)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_ties_pick_the_first_index_and_nan_wins(dtype):
    N = 151936
    x = torch.zeros(5, N, dtype=dtype)
    x[0, 100] = x[0, 90000] = x[0, 151935] = 3.0           # tie across threads and vector lanes
    x[1, :] = -1.0                                          # all equal: index 0
    x[2, 777] = float("nan")
    x[2, 10] = float("inf")
    x[2, 77777] = float("nan")                              # first NaN wins over inf
    x[3, 151935] = 1.0                                      # maximum in the last element
    x[4, :] = float("-inf")
    x[4, 5] = -1e30 if dtype == torch.bfloat16 else -60000.0
    got = argmax_rows(x.to(DEV))
    torch.cuda.synchronize()
    assert got.tolist() == [100, 0, 777, 151935, 5]
    assert got.tolist() == torch.argmax(x.to(DEV), dim=-1).tolist()


def test_signed_zeros_are_equal():
    x = torch.full((2, 9000), -1.0)
    x[0, 3], x[0, 7] = -0.0, 0.0          # equal maxima: the first wins
    x[1, 8191], x[1, 8192] = 0.0, -0.0    # across a slice boundary
    got = argmax_rows(x.half().to(DEV))
    torch.cuda.synchronize()
    assert got.tolist() == [3, 8191]


def test_strided_rows_and_unaligned_width():
    g = torch.Generator().manual_seed(3)
    wide = torch.randn(6, 1030, generator=g).half().to(DEV)
    x = wide[:, :1001]            # row stride 1030 elements (2060 bytes: not a multiple of 16)
    got = argmax_rows(x)
    torch.cuda.synchronize()
    assert got.tolist() == _want(x)
