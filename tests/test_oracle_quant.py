"""Pins the INT4 oracle (oracle/quant.py) and the product's quantiser.

The checks are the reference's own quant tests (reference
tests/test_quant.py:46-94) restated against the oracle, plus closed forms that
do not share its code: weights on the quantisation grid round-trip exactly, a
per-element loop decodes the packed bytes, and the float64 linear equals
integer arithmetic on integer inputs.  The product's setup-time quantiser
(nanoserve_amd/quant.py) must produce the oracle's bytes exactly.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from nanoserve_amd.quant import quantize_int4_groupwise
from oracle.quant import dequantize_int4_ref, int4_linear_ref, quantize_int4_ref


def _w(out_f, in_f, seed=0):
    return np.random.default_rng(seed).standard_normal((out_f, in_f)).astype(np.float32)


def test_packing_halves_the_bytes():
    packed, s, z = quantize_int4_ref(_w(32, 256), 128)
    assert packed.dtype == np.uint8 and packed.shape == (32, 128)
    assert s.shape == (32, 2) and s.dtype == np.float32 and z.shape == (32, 2) and z.dtype == np.uint8


def test_nibbles_unpack_in_the_right_order():
    w = _w(4, 128, 1)
    packed, s, z = quantize_int4_ref(w, 128)
    q = np.clip(np.round(w / s[:, :1]) + z[:, :1], 0, 15).astype(np.uint8)
    assert np.array_equal(packed & 0x0F, q[:, 0::2])
    assert np.array_equal(packed >> 4, q[:, 1::2])


def test_roundtrip_error_is_bounded_by_the_group_step():
    w = _w(16, 256, 2)
    packed, s, z = quantize_int4_ref(w, 128)
    deq = dequantize_int4_ref(packed, s, z, 128)
    assert (np.abs(deq - w) <= np.repeat(s, 128, axis=1) * 0.51 + 1e-6).all()


def test_grouping_beats_per_tensor_on_outliers():
    w = _w(8, 256, 3) * 0.01
    w[:, 0] = 50.0
    fine = dequantize_int4_ref(*quantize_int4_ref(w, 128), 128)
    coarse = dequantize_int4_ref(*quantize_int4_ref(w, 256), 256)
    assert np.abs(fine[:, 1:] - w[:, 1:]).mean() < np.abs(coarse[:, 1:] - w[:, 1:]).mean()


def test_bad_group_size_is_rejected():
    with pytest.raises(ValueError):
        quantize_int4_ref(_w(4, 100), 128)
    with pytest.raises(ValueError):
        quantize_int4_groupwise(torch.randn(4, 100), 128)


def test_grid_weights_roundtrip_exactly():
    """w = (q - z) * s with every group spanning codes 0..15 is reproduced bit for bit."""
    rng = np.random.default_rng(4)
    N, K, gs = 6, 256, 128
    q = rng.integers(0, 16, (N, K))
    q[:, 0], q[:, 1], q[:, 128], q[:, 129] = 0, 15, 0, 15
    z = rng.integers(0, 16, (N, K // gs))
    s = 2.0 ** rng.integers(-8, 0, (N, K // gs))
    w = ((q - np.repeat(z, gs, axis=1)) * np.repeat(s, gs, axis=1)).astype(np.float32)
    packed, s2, z2 = quantize_int4_ref(w, gs)
    assert np.array_equal(s2, s.astype(np.float32)) and np.array_equal(z2, z)
    assert np.array_equal(dequantize_int4_ref(packed, s2, z2, gs), w)


def test_dequantizer_matches_a_per_element_loop():
    packed, s, z = quantize_int4_ref(_w(3, 256, 5), 128)
    deq = dequantize_int4_ref(packed, s, z, 128)
    for n in range(3):
        for k in range(256):
            b = int(packed[n, k // 2])
            code = (b & 15) if k % 2 == 0 else (b >> 4)
            want = np.float32(np.float32(code - int(z[n, k // 128])) * s[n, k // 128])
            assert deq[n, k] == want


def test_dequantizer_rounds_to_the_model_dtype():
    packed, s, z = quantize_int4_ref(_w(8, 256, 6), 128)
    f32 = dequantize_int4_ref(packed, s, z, 128)
    assert np.array_equal(dequantize_int4_ref(packed, s, z, 128, "float16"), f32.astype(np.float16).astype(np.float32))
    want = torch.from_numpy(f32).to(torch.bfloat16).float().numpy()
    assert np.array_equal(dequantize_int4_ref(packed, s, z, 128, "bfloat16"), want)


def test_linear_matches_integer_arithmetic():
    rng = np.random.default_rng(7)
    x = rng.integers(-8, 9, (5, 64))
    w = rng.integers(-8, 9, (12, 64))
    b = rng.integers(-100, 101, 12)
    y = int4_linear_ref(x.astype(np.float32), w.astype(np.float32), b.astype(np.float32))
    assert np.array_equal(y, (x @ w.T + b).astype(np.float64))


@pytest.mark.parametrize("shape,gs", [((64, 256), 128), ((1152, 896), 128), ((40, 512), 64)])
def test_product_quantizer_equals_oracle(shape, gs):
    w = _w(*shape, seed=8) * 0.05
    w[0, :gs] = 0.0                     # a constant group: scale clamps to 1e-8
    packed, s, z = quantize_int4_groupwise(torch.from_numpy(w), gs)
    rp, rs, rz = quantize_int4_ref(w, gs)
    assert np.array_equal(packed.numpy(), rp)
    assert np.array_equal(s.numpy(), rs)
    assert np.array_equal(z.numpy(), rz)


@pytest.mark.parametrize("heads,D", [(18, 64), (8, 128), (1, 16)])
def test_rope_pair_row_order(heads, D):
    """The stored order of a rope-paired q|k|v weight: a permutation of each head's
    rows in which row r and row r + 8 of every 16-row tile are a rotate_half pair
    (dims d and d + D/2), lane groups g and g ^ 2 of the MFMA result; the
    product's order (nanoserve_amd.quant.rope_pair_order) is the oracle's."""
    from oracle.qwen2 import _rope_pair_order_ref
    from nanoserve_amd.quant import rope_pair_order

    order = _rope_pair_order_ref(heads, D)
    assert sorted(order) == list(range(heads * D))
    for t in range(0, heads * D, 16):
        tile = order[t:t + 16]
        head = tile[0] // D
        assert all(o // D == head for o in tile)
        for r in range(8):
            assert tile[r + 8] - tile[r] == D // 2 and tile[r] % D < D // 2
    assert rope_pair_order(heads, D).tolist() == order


# quantize_model: the reference's model-level checks (tests/test_quant.py:120-166)
# on the CPU; the conversion is setup-time tensor code and runs no kernel.

def test_quantize_model_reports_real_compression():
    from nanoserve_amd.quant import Int4Linear, quantize_model

    m = torch.nn.Sequential(torch.nn.Linear(256, 256, bias=False), torch.nn.SiLU(),
                            torch.nn.Linear(256, 256, bias=False))
    report = quantize_model(m, 128, skip=())
    assert report["mode"] == "int4" and report["group_size"] == 128
    assert report["layers_quantized"] == 2
    assert isinstance(m[0], Int4Linear) and isinstance(m[2], Int4Linear)
    # 2 x 256 x 256 fp32 = 512 KiB before; after, per layer 256 x 128 code bytes
    # + 256 x 2 scales (4 B) + 256 x 2 zero points (1 B) = 35,328 B.
    assert report["weight_mib_before"] * 2**20 == 2 * 256 * 256 * 4
    assert report["weight_mib_after"] * 2**20 == 2 * (256 * 128 + 256 * 2 * 4 + 256 * 2)
    assert report["compression"] == pytest.approx(524288 / 70656)
    assert report["freed_mib"] == pytest.approx(report["weight_mib_before"] - report["weight_mib_after"])


def test_quantize_model_honours_skip_and_shape():
    from nanoserve_amd.quant import Int4Linear, quantize_model

    m = torch.nn.Sequential()
    m.add_module("keep_me", torch.nn.Linear(128, 128, bias=False))
    m.add_module("other", torch.nn.Linear(128, 128, bias=True))
    inner = torch.nn.Sequential()
    inner.add_module("deep", torch.nn.Linear(128, 64))
    m.add_module("keep_me_too", inner)                  # a skipped subtree stays whole
    m.add_module("ragged_in", torch.nn.Linear(100, 128))  # not a whole number of groups
    m.add_module("ragged_out", torch.nn.Linear(128, 40))  # not a whole number of 16-row tiles
    report = quantize_model(m, 128, skip=("keep_me",))
    assert report["layers_quantized"] == 1
    assert isinstance(m.other, Int4Linear) and m.other.bias is not None
    for name in ("keep_me", "ragged_in", "ragged_out"):
        assert type(getattr(m, name)) is torch.nn.Linear
    assert type(m.keep_me_too.deep) is torch.nn.Linear


def test_quantize_model_counts_tied_weights_once():
    from nanoserve_amd.quant import quantize_model

    a = torch.nn.Linear(64, 64, bias=False)
    b = torch.nn.Linear(64, 64, bias=False)
    b.weight = a.weight
    m = torch.nn.Sequential(a, b)
    report = quantize_model(m, 64, skip=("0", "1"))
    assert report["layers_quantized"] == 0
    assert report["weight_mib_before"] * 2**20 == 64 * 64 * 4 == report["weight_mib_after"] * 2**20


def test_quantized_modules_hold_the_quantiser_bytes():
    from nanoserve_amd.quant import quantize_model

    torch.manual_seed(3)
    m = torch.nn.Sequential(torch.nn.Linear(256, 128))
    w = m[0].weight.detach().numpy().copy()
    bias = m[0].bias.detach().clone()
    quantize_model(m, 128, skip=())
    rp, rs, rz = quantize_int4_ref(w, 128)
    assert np.array_equal(m[0].qweight.numpy(), rp)
    assert np.array_equal(m[0].scales.numpy(), rs)
    assert np.array_equal(m[0].zeros.numpy(), rz)
    assert torch.equal(m[0].bias.data, bias)
