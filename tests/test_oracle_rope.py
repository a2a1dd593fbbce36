"""Pins the rotary oracle (oracle/rope.py) before the HIP path is checked against it.

rope_apply_ref restates the reference's tensor arithmetic (reference
nanoserve/layers.py:81-90).  It is checked bit for bit against a numpy
restatement with an explicit rounding after every op (numpy's own float16
arithmetic, an integer bfloat16 rounding), against closed forms
(cos=1/sin=0 is the identity, cos=0/sin=1 is rotate_half) and, in float64,
against the textbook definition of RoPE: pair (x[i], x[i+D/2]) is the complex
number x[i] + j*x[i+D/2] multiplied by exp(j * pos * base**(-2i/D)).  That
last check fixes the sign of rotate_half, which half pairs with which
frequency, and the table; a rotation in the wrong direction or with the
halves swapped fails it.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle.paged_attention import reshape_and_cache_ref
from oracle.rope import (rope_apply_bits, rope_apply_ref, rope_cos_sin_ref, rope_reshape_and_cache_ref,
                         rope_table_ref, rotate_half_ref)

DTYPES = {torch.float16: "float16", torch.bfloat16: "bfloat16", torch.float32: "float32"}


def _values(shape, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=g) * torch.exp(torch.randn(*shape, generator=g) * 3)
    flat = x.view(-1)
    flat[:8] = torch.tensor([0.0, -0.0, 65504.0, -60000.0, 2 ** -24, 3 * 2 ** -25, 1 + 2 ** -11, 1e-30])
    return x.to(dtype)


def _same(a: torch.Tensor, b: np.ndarray):
    a = a.float().numpy()
    nan = np.isnan(a)
    assert np.array_equal(nan, np.isnan(b))
    assert np.array_equal(a[~nan].view(np.uint32), b[~nan].astype(np.float32).view(np.uint32))


@pytest.mark.parametrize("dtype", list(DTYPES))
def test_apply_matches_numpy_per_op_rounding(dtype):
    T, H, D = 37, 5, 64
    q = _values((T, H, D), dtype, 1)
    cos_t, sin_t = rope_table_ref(D, 5000)
    pos = torch.randint(0, 5000, (T,), generator=torch.Generator().manual_seed(2))
    cos, sin = rope_cos_sin_ref(cos_t, sin_t, pos, dtype)
    qr, _ = rope_apply_ref(q, q[:, :1], cos, sin)
    want = rope_apply_bits(q.float().numpy(), cos.float().numpy(), sin.float().numpy(), DTYPES[dtype])
    _same(qr, want)


@pytest.mark.parametrize("dtype", list(DTYPES))
def test_apply_with_arbitrary_tables_matches_numpy(dtype):
    """cos/sin need not be a rotation: any values round the same way."""
    T, H, D = 11, 3, 128
    q = _values((T, H, D), dtype, 3)
    cos = _values((T, 1, D), dtype, 4)
    sin = _values((T, 1, D), dtype, 5)
    qr, _ = rope_apply_ref(q, q, cos, sin)
    want = rope_apply_bits(q.float().numpy(), cos.float().numpy(), sin.float().numpy(), DTYPES[dtype])
    _same(qr, want)


@pytest.mark.parametrize("dtype", list(DTYPES))
def test_closed_forms_identity_and_rotate_half(dtype):
    T, H, D = 9, 4, 64
    q = _values((T, H, D), dtype, 6)
    one, zero = torch.ones(T, 1, D, dtype=dtype), torch.zeros(T, 1, D, dtype=dtype)
    same, _ = rope_apply_ref(q, q, one, zero)
    assert torch.equal(same, q)
    rot, _ = rope_apply_ref(q, q, zero, one)
    assert torch.equal(rot, torch.cat((-q[..., D // 2:], q[..., :D // 2]), dim=-1))


def test_rotate_half_matches_index_loop():
    x = torch.arange(2 * 3 * 8, dtype=torch.float32).view(2, 3, 8)
    y = rotate_half_ref(x)
    for i in range(8):
        want = -x[..., i + 4] if i < 4 else x[..., i - 4]
        assert torch.equal(y[..., i], want)


@pytest.mark.parametrize("D,base", [(64, 10000.0), (128, 1000000.0)])
def test_float64_rotation_is_complex_multiplication(D, base):
    """RoPE as x[i] + j x[i+D/2] times exp(j pos theta_i), theta_i = base**(-2i/D)."""
    T, H = 23, 3
    g = torch.Generator().manual_seed(7)
    q = torch.randn(T, H, D, generator=g, dtype=torch.float64)
    pos = torch.randint(0, 32768, (T,), generator=g).to(torch.float64)
    h = D // 2
    theta = torch.tensor([base ** (-2.0 * i / D) for i in range(h)], dtype=torch.float64)
    ang = torch.cat((torch.outer(pos, theta),) * 2, dim=-1).unsqueeze(1)
    qr, _ = rope_apply_ref(q, q, ang.cos(), ang.sin())
    z = torch.complex(q[..., :h], q[..., h:]) * torch.polar(torch.ones_like(ang[..., :h]), ang[..., :h])
    np.testing.assert_allclose(qr[..., :h].numpy(), z.real.numpy(), rtol=0, atol=1e-12)
    np.testing.assert_allclose(qr[..., h:].numpy(), z.imag.numpy(), rtol=0, atol=1e-12)
    # Norm of every pair is preserved, and rotations compose.
    n0 = q[..., :h] ** 2 + q[..., h:] ** 2
    n1 = qr[..., :h] ** 2 + qr[..., h:] ** 2
    np.testing.assert_allclose(n1.numpy(), n0.numpy(), rtol=1e-12)
    q2, _ = rope_apply_ref(qr, qr, ang.cos(), ang.sin())
    q2d, _ = rope_apply_ref(q, q, (2 * ang).cos(), (2 * ang).sin())
    np.testing.assert_allclose(q2.numpy(), q2d.numpy(), rtol=0, atol=1e-10)


@pytest.mark.parametrize("D,base", [(64, 10000.0), (128, 1000000.0)])
def test_table_matches_float64_closed_form(D, base):
    P = 4096
    cos, sin = rope_table_ref(D, P, base)
    assert cos.shape == (P, D) and cos.dtype == torch.float32
    assert torch.equal(cos[:, :D // 2], cos[:, D // 2:]) and torch.equal(sin[:, :D // 2], sin[:, D // 2:])
    assert torch.equal(cos[0], torch.ones(D)) and torch.equal(sin[0], torch.zeros(D))
    for p in (1, 7, 100, 1023, 4095):
        for i in range(D // 2):
            ang = p * base ** (-2.0 * i / D)
            tol = 2.5e-7 * p + 1e-6  # float32 inv_freq and product rounding, scaled by the angle
            assert abs(float(cos[p, i]) - math.cos(ang)) <= tol
            assert abs(float(sin[p, i]) - math.sin(ang)) <= tol


def test_cos_sin_lookup_shape_and_cast():
    cos_t, sin_t = rope_table_ref(64, 100)
    pos = torch.tensor([5, 0, 99, 5])
    cos, sin = rope_cos_sin_ref(cos_t, sin_t, pos, torch.float16)
    assert cos.shape == (4, 1, 64) and cos.dtype == torch.float16
    assert torch.equal(cos[0], cos[3]) and torch.equal(cos[1, 0], torch.ones(64, dtype=torch.float16))
    assert torch.equal(sin[2, 0], sin_t[99].half())


def test_fused_ref_is_apply_then_write():
    T, Hq, Hkv, D, NB, BS = 10, 14, 2, 64, 4, 16
    dt = torch.float16
    q, k, v = _values((T, Hq, D), dt, 8), _values((T, Hkv, D), dt, 9), _values((T, Hkv, D), dt, 10)
    cos_t, sin_t = rope_table_ref(D, 64)
    cos, sin = rope_cos_sin_ref(cos_t, sin_t, torch.arange(T) * 3, dt)
    kc = torch.zeros(NB, BS, Hkv, D, dtype=dt)
    vc = torch.zeros_like(kc)
    slots = torch.tensor([3, -1, 17, 40, 63, 0, 64, 5, 22, 9])
    qr, gk, gv = rope_reshape_and_cache_ref(q, k, v, cos, sin, kc, vc, slots)
    qa, ka = rope_apply_ref(q, k, cos, sin)
    assert torch.equal(qr, qa)
    keep = (slots >= 0) & (slots < NB * BS)
    ek, ev = reshape_and_cache_ref(ka[keep], v[keep], kc, vc, slots[keep])
    assert torch.equal(gk, ek) and torch.equal(gv, ev)
    assert torch.equal(gk.view(-1, Hkv, D)[17], ka[2]) and torch.equal(gv.view(-1, Hkv, D)[63], v[4])
    assert int((gk.view(-1, Hkv, D).abs().sum(dim=(1, 2)) > 0).sum()) <= 8
