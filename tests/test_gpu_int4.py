"""HIP INT4 dequant-GEMM (ns_int4_linear) against the oracle (MI355X).

The weights the MFMA sees must be the reference's dequantised weights bit for
bit (checked through an identity input, whose products are exact), and the
output must equal x · W^T + bias rounded once to the model dtype: within one
rounding of the float64 result (|err| <= 2^-10 |ref| for fp16, 2^-7 |ref| for
bf16, plus an absolute 1e-5 · max|ref| for fp32 accumulation order).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from nanoserve_amd.quant import Int4Linear, int4_linear, quantize_int4_groupwise, quantize_model
from oracle.quant import dequantize_int4_ref, int4_linear_ref

pytestmark = pytest.mark.gpu
DEV = "cuda"
RTOL = {torch.float16: 2.0 ** -10, torch.bfloat16: 2.0 ** -7}
NAME = {torch.float16: "float16", torch.bfloat16: "bfloat16"}

# Qwen2.5-0.5B projections (in -> out): q, k/v, o, gate/up, down, and fused q|k|v, gate|up.
# Arrival-counter region at the head of every split-K workspace (256 tiles x u32).
SPLITK_COUNTER_BYTES = 1024

QWEN = [(896, 896), (896, 128), (896, 4864), (4864, 896), (896, 1152), (896, 9728)]


def _weights(N, K, gs, seed, scale=0.05):
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(N, K, generator=g) * scale
    return quantize_int4_groupwise(w, gs)


def _check(got: torch.Tensor, ref: np.ndarray, dtype, what=""):
    got = got.float().cpu().numpy().astype(np.float64)
    tol = RTOL[dtype] * np.abs(ref) + 1e-5 * max(1.0, np.abs(ref).max())
    bad = np.abs(got - ref) > tol
    assert not bad.any(), (f"{what}: {bad.sum()} of {bad.size} outside one rounding; "
                           f"max err {np.abs(got - ref).max():.3e}")


def _run(M, N, K, dtype, gs=128, bias=True, seed=0, x_scale=1.0, method="auto"):
    packed, s, z = _weights(N, K, gs, seed)
    g = torch.Generator().manual_seed(seed + 1)
    x = (torch.randn(M, K, generator=g) * x_scale).to(dtype)
    b = (torch.randn(N, generator=g) * 0.1).to(dtype) if bias else None
    got = int4_linear(x.to(DEV), packed.to(DEV), s.to(DEV), z.to(DEV), None if b is None else b.to(DEV), gs,
                      method=method)
    torch.cuda.synchronize()
    w = dequantize_int4_ref(packed.numpy(), s.numpy(), z.numpy(), gs, NAME[dtype])
    ref = int4_linear_ref(x.float().numpy(), w, None if b is None else b.float().numpy())
    _check(got, ref, dtype, f"M={M} N={N} K={K} {dtype}")
    return got, x, (packed, s, z), b


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("K,N", QWEN, ids=[f"{k}x{n}" for k, n in QWEN])
@pytest.mark.parametrize("M", [1, 32])
def test_decode_shapes(dtype, K, N, M):
    print(f"int4 M={M} N={N} K={K} {dtype}", flush=True)
    _run(M, N, K, dtype, seed=M + N)


@pytest.mark.parametrize("M", [7, 17, 33, 64, 100, 2076])
def test_row_counts_across_tiles(M):
    _run(M, 1152, 896, torch.float16, seed=M)


@pytest.mark.parametrize("gs", [32, 64, 256])
def test_group_sizes(gs):
    _run(20, 256, 512, torch.float16, gs=gs, seed=gs)


def test_without_bias():
    _run(9, 128, 896, torch.bfloat16, bias=False)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_identity_input_reproduces_dequantised_weights_bit_exactly(dtype):
    """x = I: y[m][n] = W[n][m] (one exact product per output), so y^T is the dequantised weight."""
    K, N, gs = 128, 64, 128
    packed, s, z = _weights(N, K, gs, 3, scale=1.0)
    eye = torch.eye(K, dtype=dtype, device=DEV)
    y = int4_linear(eye, packed.to(DEV), s.to(DEV), z.to(DEV), None, gs)
    torch.cuda.synchronize()
    want = dequantize_int4_ref(packed.numpy(), s.numpy(), z.numpy(), gs, NAME[dtype])
    assert np.array_equal(y.float().cpu().numpy().T, want)


def test_strided_rows_and_leading_dims():
    """x as a column slice of a wider activation, with a [B, T, K] leading shape."""
    K, N = 896, 1152
    packed, s, z = _weights(N, K, 128, 5)
    g = torch.Generator().manual_seed(6)
    wide = torch.randn(2, 11, K + 64, generator=g).half()
    x = wide[..., 64:]
    got = int4_linear(x.to(DEV), packed.to(DEV), s.to(DEV), z.to(DEV), None, 128)
    torch.cuda.synchronize()
    assert got.shape == (2, 11, N)
    w = dequantize_int4_ref(packed.numpy(), s.numpy(), z.numpy(), 128, "float16")
    ref = int4_linear_ref(x.reshape(-1, K).float().numpy(), w, None)
    _check(got.reshape(-1, N), ref, torch.float16, "strided")


def test_matches_reference_quantlinear_path():
    """The reference's forward (dequantise to fp16, then F.linear) within one fp16 rounding of each other."""
    lin = torch.nn.Linear(896, 4864, bias=True).half().to(DEV)
    q = Int4Linear.from_linear(lin, 128)
    x = torch.randn(32, 896, device=DEV).half()
    got = q(x)
    w = torch.from_numpy(dequantize_int4_ref(q.qweight.cpu().numpy(), q.scales.cpu().numpy(),
                                             q.zeros.cpu().numpy(), 128, "float16")).half().to(DEV)
    want = F.linear(x.float(), w.float(), q.bias.float())
    torch.cuda.synchronize()
    err = (got.float() - want).abs()
    assert (err <= 2.0 ** -10 * want.abs() + 1e-4).all(), f"max err {err.max().item():.3e}"


def test_quantize_model_replaces_linears_and_stays_close():
    torch.manual_seed(0)
    m = torch.nn.Sequential(torch.nn.Linear(256, 256, bias=False), torch.nn.SiLU(),
                            torch.nn.Linear(256, 256, bias=False)).half().to(DEV)
    x = torch.randn(4, 256, device=DEV).half()
    ref = m(x).float()
    report = quantize_model(m, 128, skip=())
    assert report["layers_quantized"] == 2 and report["compression"] > 3.4
    got = m(x).float()
    torch.cuda.synchronize()
    cos = F.cosine_similarity(got.flatten(), ref.flatten(), dim=0).item()
    assert cos > 0.98, f"int4 output cosine similarity {cos:.4f}"


def _round(a: np.ndarray, dtype) -> np.ndarray:
    return torch.from_numpy(np.asarray(a, np.float32)).to(dtype).double().numpy()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("K,N,M", [(896, 896, 32), (4864, 896, 32), (4864, 896, 5), (896, 1152, 100),
                                   (896, 896, 300), (4864, 896, 1030)])
def test_residual_epilogue(dtype, K, N, M):
    """out = round(round(x W^T + b) + residual), also in place on the residual
    (M of 300 and 1030: the tiled GEMM's epilogue)."""
    packed, s, z = _weights(N, K, 128, 11)
    g = torch.Generator().manual_seed(12)
    x = torch.randn(M, K, generator=g).to(dtype)
    b = (torch.randn(N, generator=g) * 0.1).to(dtype)
    res = torch.randn(M, N, generator=g).to(dtype)
    w = dequantize_int4_ref(packed.numpy(), s.numpy(), z.numpy(), 128, NAME[dtype])
    y = int4_linear_ref(x.float().numpy(), w, b.float().numpy())
    want = _round(y, dtype) + res.double().numpy()
    gres = res.to(DEV)
    got = int4_linear(x.to(DEV), packed.to(DEV), s.to(DEV), z.to(DEV), b.to(DEV), 128, residual=gres)
    inplace = gres.clone()
    int4_linear(x.to(DEV), packed.to(DEV), s.to(DEV), z.to(DEV), b.to(DEV), 128, residual=inplace, out=inplace)
    torch.cuda.synchronize()
    # The first rounding may differ by one unit where fp32 sums of different order round apart.
    tol = 2 * RTOL[dtype] * (np.abs(y) + np.abs(res.double().numpy())) + 1e-5
    for t in (got, inplace):
        err = np.abs(t.double().cpu().numpy() - want)
        assert (err <= tol).all(), f"max err {err.max():.3e}"


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("M", [1, 32, 70, 300, 1100])
def test_silu_mul_epilogue_on_interleaved_gate_up(dtype, M):
    """Interleaved (gate, up) rows -> round(round(silu(round(g))) * round(u)), [M, N/2]
    (M = 300: the tiled GEMM's epilogue on 64 x 64 tiles; 1100: on 128 x 128 tiles,
    the last one partly past M)."""
    from nanoserve_amd.quant import Int4Linear

    K, I = 896, 4864
    g = torch.Generator().manual_seed(13)
    gate = torch.nn.Linear(K, I, bias=False).to(dtype)
    up = torch.nn.Linear(K, I, bias=False).to(dtype)
    with torch.no_grad():
        gate.weight.copy_(torch.randn(I, K, generator=g) * 0.05)
        up.weight.copy_(torch.randn(I, K, generator=g) * 0.05)
    qg, qu = Int4Linear.from_linear(gate, 128).to(DEV), Int4Linear.from_linear(up, 128).to(DEV)
    fused = Int4Linear.gate_up_pairs(qg, qu)
    x = torch.randn(M, K, generator=g).to(dtype)
    got = fused(x.to(DEV))
    torch.cuda.synchronize()
    assert got.shape == (M, I)

    def proj(q):
        w = dequantize_int4_ref(q.qweight.cpu().numpy(), q.scales.cpu().numpy(), q.zeros.cpu().numpy(), 128,
                                NAME[dtype])
        return int4_linear_ref(x.float().numpy(), w, None)

    gv, uv = _round(proj(qg), dtype), _round(proj(qu), dtype)
    act = _round(gv / (1.0 + np.exp(-gv)), dtype)
    want = _round(act * uv, dtype)
    err = np.abs(got.double().cpu().numpy() - want)
    # Gate and up may each round one unit apart (fp32 sums in another order);
    # silu and the product carry that through plus their own rounding.
    tol = 4 * RTOL[dtype] * np.abs(want) + 4 * RTOL[dtype] * np.abs(act * uv).max() * 1e-2 + 1e-4
    assert (err <= tol).all(), f"max err {err.max():.3e}"
    # The unfused composition through separate launches agrees within the same bound.
    sep = torch.nn.functional.silu(qg(x.to(DEV))) * qu(x.to(DEV))
    torch.cuda.synchronize()
    assert (np.abs(sep.double().cpu().numpy() - want) <= tol).all()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("K,M", [(896, 1), (896, 32), (896, 100), (256, 7), (1024, 40)])
def test_rmsnorm_prologue(dtype, K, M):
    """int4_linear(x, norm_weight=w) == linear(round((x * rsqrt(mean(x^2) + eps)) * w))."""
    N = 1152
    packed, s, z = _weights(N, K, 128, 21)
    g = torch.Generator().manual_seed(22)
    x = (torch.randn(M, K, generator=g) * 3).to(dtype)
    w = (1 + 0.1 * torch.randn(K, generator=g)).to(dtype)
    b = (torch.randn(N, generator=g) * 0.1).to(dtype)
    got = int4_linear(x.to(DEV), packed.to(DEV), s.to(DEV), z.to(DEV), b.to(DEV), 128,
                      norm_weight=w.to(DEV), norm_eps=1e-6)
    torch.cuda.synchronize()
    xf = x.double().numpy()
    rstd = 1.0 / np.sqrt((xf ** 2).mean(axis=1, keepdims=True) + 1e-6)
    xn = _round(xf * rstd * w.double().numpy(), dtype)
    wq = dequantize_int4_ref(packed.numpy(), s.numpy(), z.numpy(), 128, NAME[dtype])
    ref = int4_linear_ref(xn, wq, b.float().numpy())
    # The normalised operands may round one unit apart (rsqrt and sum order),
    # which moves the result by at most that unit times |w| summed over K.
    tol = 2 * RTOL[dtype] * np.abs(xn) @ np.abs(wq).T + RTOL[dtype] * np.abs(ref) + 1e-4
    err = np.abs(got.double().cpu().numpy() - ref)
    assert (err <= tol).all(), f"max err {err.max():.3e}"
    # Same result as normalising with torch first.
    sep = int4_linear(torch.nn.functional.rms_norm(x.to(DEV), (K,), w.to(DEV), 1e-6), packed.to(DEV),
                      s.to(DEV), z.to(DEV), b.to(DEV), 128)
    torch.cuda.synchronize()
    assert (np.abs(sep.double().cpu().numpy() - ref) <= tol).all()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("M", [1, 16, 32, 64, 100])
def test_rmsnorm_with_gate_up_silu_mul(dtype, M):
    """Qwen2's MLP input: silu(gate(rms_norm(x))) * up(rms_norm(x)) in one launch, at
    gate|up's width (4864 pairs), where 16-64 tokens take two feature tiles per
    workgroup and 100 tokens a 64-token tile."""
    K, I = 896, 4864
    g = torch.Generator().manual_seed(31)
    gate = torch.nn.Linear(K, I, bias=False).to(dtype)
    up = torch.nn.Linear(K, I, bias=False).to(dtype)
    with torch.no_grad():
        gate.weight.copy_(torch.randn(I, K, generator=g) * 0.05)
        up.weight.copy_(torch.randn(I, K, generator=g) * 0.05)
    qg, qu = Int4Linear.from_linear(gate, 128).to(DEV), Int4Linear.from_linear(up, 128).to(DEV)
    fused = Int4Linear.gate_up_pairs(qg, qu)
    assert fused.fuses_norm
    x = (torch.randn(M, K, generator=g) * 3).to(dtype)
    w = (1 + 0.1 * torch.randn(K, generator=g)).to(dtype)
    got = int4_linear(x.to(DEV), fused.qweight, fused.scales, fused.zeros, None, 128, silu_mul=True,
                      norm_weight=w.to(DEV), norm_eps=1e-6)
    torch.cuda.synchronize()
    assert got.shape == (M, I)

    xf = x.double().numpy()
    rstd = 1.0 / np.sqrt((xf ** 2).mean(axis=1, keepdims=True) + 1e-6)
    xn = _round(xf * rstd * w.double().numpy(), dtype)

    def proj(q):
        wq = dequantize_int4_ref(q.qweight.cpu().numpy(), q.scales.cpu().numpy(), q.zeros.cpu().numpy(), 128,
                                 NAME[dtype])
        ref = int4_linear_ref(xn, wq, None)
        # The normalised operands may round one unit apart, which moves a
        # projection by at most that unit times |w| summed over K.
        return ref, 2 * RTOL[dtype] * np.abs(xn) @ np.abs(wq).T + RTOL[dtype] * np.abs(ref) + 1e-4

    (gr, tg), (ur, tu) = proj(qg), proj(qu)
    gv, uv = _round(gr, dtype), _round(ur, dtype)
    act = _round(gv / (1.0 + np.exp(-gv)), dtype)
    want = _round(act * uv, dtype)
    # silu' is at most 1.1; the product carries both operands' bounds, then rounds.
    tol = 1.1 * tg * np.abs(uv) + np.abs(act) * tu + tg * tu + 4 * RTOL[dtype] * np.abs(want) + 1e-4
    err = np.abs(got.double().cpu().numpy() - want)
    assert (err <= tol).all(), f"max err {err.max():.3e}"
    # Normalising with torch first agrees within the same bound.
    sep = int4_linear(F.rms_norm(x.to(DEV), (K,), w.to(DEV), 1e-6), fused.qweight, fused.scales, fused.zeros,
                      None, 128, silu_mul=True)
    torch.cuda.synchronize()
    assert (np.abs(sep.double().cpu().numpy() - want) <= tol).all()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("N,K,gs", [(1152, 896, 128), (896, 4864, 128), (64, 256, 32)])
def test_dequantize_is_bit_exact(dtype, N, K, gs):
    from nanoserve_amd.quant import int4_dequantize

    packed, s, z = _weights(N, K, gs, 31, scale=0.7)
    got = int4_dequantize(packed.to(DEV), s.to(DEV), z.to(DEV), gs, dtype)
    torch.cuda.synchronize()
    want = dequantize_int4_ref(packed.numpy(), s.numpy(), z.numpy(), gs, NAME[dtype])
    assert np.array_equal(got.float().cpu().numpy(), want)


@pytest.mark.parametrize("M", [129, 700, 2048])
def test_large_row_counts_take_the_tiled_gemm_within_one_rounding(M):
    """Every tile shape of the GEMM: 64 x 64 (all but the cases below), 128 tokens
    x 64 features (K = 4864 at 2048 tokens), 128 x 128 (N = 4096 at 2048 tokens).
    method="fused" keeps the long-K layer on the tiled GEMM, which "auto" leaves
    above 1024 tokens."""
    _run(M, 1152, 896, torch.float16, seed=M, method="fused")
    _run(M, 896, 4864, torch.bfloat16, seed=M + 1, method="fused")
    _run(M, 4096, 512, torch.bfloat16, seed=M + 2, method="fused")


@pytest.mark.parametrize("M,K,dequant", [(1024, 4864, False), (1025, 4864, True), (2048, 4864, True),
                                         (2048, 896, False), (1100, 2048, True), (1100, 1920, False)])
def test_auto_takes_the_faster_path_per_shape(M, K, dequant):
    """Eagerly "auto" is the tiled GEMM (bit-identical to method="fused"); recorded into a
    graph it takes the dequantise + library GEMM steps exactly when K >= LONG_K and
    M > LONG_K_TILED_MAX_ROWS (bit-identical to method="dequant"), and every replay stays
    bit-identical with eager work between replays."""
    from nanoserve_amd.capture import graph_capture

    N = 896
    got, x, (packed, s, z), b = _run(M, N, K, torch.float16, seed=M + K)
    xd, pd, sd, zd, bd = x.to(DEV), packed.to(DEV), s.to(DEV), z.to(DEV), b.to(DEV)
    fused = int4_linear(xd, pd, sd, zd, bd, 128, method="fused")
    torch.cuda.synchronize()
    assert torch.equal(got.to(DEV), fused)
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        want = int4_linear(xd, pd, sd, zd, bd, 128, method="dequant" if dequant else "fused")  # takes the scratch
    stream.synchronize()
    g = torch.cuda.CUDAGraph()
    with graph_capture(g, stream=stream):
        out = int4_linear(xd, pd, sd, zd, bd, 128)
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want)
        fused.add_(0)  # eager work between replays


@pytest.mark.parametrize("gs", [32, 64, 256])
@pytest.mark.parametrize("M,N", [(130, 2048), (513, 1152)])
def test_tiled_gemm_group_sizes_and_partial_tiles(gs, M, N):
    """Token tiles past M (rows repeat the last one and are never stored), feature
    tiles past N (N = 1152 is nine 128-row tiles; 2048 sixteen), and group sizes
    below (32: the fused kernel, as a 64-wide K step of the GEMM would span two
    groups) and above the 64-wide K step."""
    _run(M, N, 768, torch.float16, gs=gs, seed=M + gs)
    _run(M, N, 512, torch.bfloat16, gs=gs, bias=False, seed=M + gs + 1)


@pytest.mark.parametrize("method", ["fused", "dequant"])
def test_both_methods_agree_on_every_epilogue(method):
    K, I = 896, 1024
    g = torch.Generator().manual_seed(41)
    pk, s, z = _weights(2 * I, K, 128, 42)
    pk, s, z = pk.to(DEV), s.to(DEV), z.to(DEV)
    x = torch.randn(200, K, generator=g).half().to(DEV)
    w = (1 + 0.1 * torch.randn(K, generator=g)).half().to(DEV)
    res = torch.randn(200, 2 * I, generator=g).half().to(DEV)
    outs = {}
    for m in ("fused", "dequant"):
        outs[m] = (int4_linear(x, pk, s, z, None, 128, method=m, silu_mul=True),
                   int4_linear(x, pk, s, z, None, 128, method=m, residual=res),
                   int4_linear(x, pk, s, z, None, 128, method=m, norm_weight=w))
    torch.cuda.synchronize()
    for a, b in zip(outs["fused"], outs["dequant"]):
        err = (a.float() - b.float()).abs()
        assert (err <= 4 * 2.0 ** -10 * b.float().abs() + 1e-3).all(), f"max err {err.max().item():.3e}"


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("K", [896, 928, 256])
def test_a_row_does_not_depend_on_the_rest_of_the_batch(dtype, K):
    """Row m's output is bit-identical whether it is launched alone or among 64 rows.

    8 rows run one 16-feature tile per workgroup; 16 or more rows over a wide
    N run two tiles that share each x load (a different grid), so this pins
    the two-tile path bit for bit against the one-tile path on every epilogue
    and on the 32-wide tail steps (K = 928).
    """
    N = 2048
    packed, s, z = (t.to(DEV) for t in _weights(N, K, 32 if K == 928 else 128, 51))
    gs = 32 if K == 928 else 128
    g = torch.Generator().manual_seed(52)
    x = torch.randn(64, K, generator=g).to(dtype).to(DEV)
    b = (torch.randn(N, generator=g) * 0.1).to(dtype).to(DEV)
    res = torch.randn(64, N, generator=g).to(dtype).to(DEV)
    w = (1 + 0.1 * torch.randn(K, generator=g)).to(dtype).to(DEV)
    cases = {"bias": {}, "residual": {"residual": None}, "silu_mul": {"silu_mul": True}}
    if K % 128 == 0:
        cases["rmsnorm"] = {"norm_weight": w}
    for name, kw in cases.items():
        def call(m):
            args = dict(kw)
            if "residual" in args:
                args["residual"] = res[:m].contiguous()
            return int4_linear(x[:m].contiguous(), packed, s, z, b, gs, **args)
        few, many = call(8), call(64)
        torch.cuda.synchronize()
        assert torch.equal(few, many[:8]), f"{name}: rows differ between the 8-row and 64-row launches"
        # The 64-row launch also stands on its own against the oracle (bias case).
        if name == "bias":
            wq = dequantize_int4_ref(packed.cpu().numpy(), s.cpu().numpy(), z.cpu().numpy(), gs, NAME[dtype])
            _check(many, int4_linear_ref(x.float().cpu().numpy(), wq, b.float().cpu().numpy()), dtype,
                   f"M=64 N={N} K={K}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("M", [1, 7, 32, 64, 100, 200])
@pytest.mark.parametrize("heads", [(14, 2, 64), (4, 2, 128)], ids=["qwen0.5b", "d128"])
@pytest.mark.parametrize("with_norm", [True, False], ids=["norm", "no_norm"])
def test_rope_cache_epilogue_matches_projection_then_rotary(dtype, M, heads, with_norm):
    """ns_int4_linear_rope_cache == q|k|v projection, then ns_rope_reshape_and_cache, bit for bit.

    Checks q', the rotated keys and the values in both caches, with padding
    slots (-1) that must stay untouched, int32 and int64 slot mappings, and
    the >128-token fallback through the dequantised weight."""
    from nanoserve_amd.model import RMSNorm
    from nanoserve_amd.quant import Int4Linear, int4_qkv_rope_cache
    from nanoserve_amd.rotary import RotaryEmbedding, rope_reshape_and_cache

    Hq, Hkv, D = heads
    K = 896 if D == 64 else 512
    N = (Hq + 2 * Hkv) * D
    g = torch.Generator().manual_seed(61 + M)
    lin = torch.nn.Linear(K, N, bias=True).to(dtype)
    with torch.no_grad():
        lin.weight.copy_(torch.randn(N, K, generator=g) * 0.05)
        lin.bias.copy_(torch.randn(N, generator=g) * 0.1)
    plain = Int4Linear.from_linear(lin, 128).to(DEV)
    paired = Int4Linear.rope_pairs(plain, Hq, Hkv, D)
    norm = None
    if with_norm:
        norm = RMSNorm(K, eps=1e-6).to(dtype).to(DEV)
        with torch.no_grad():
            norm.weight.copy_((1 + 0.1 * torch.randn(K, generator=g)).to(dtype))
    x = (torch.randn(M, K, generator=g) * 2).to(dtype).to(DEV)
    rot = RotaryEmbedding(D, 4096, base=1e6, device=DEV)
    pos = torch.randint(0, 4096, (M,), generator=g).to(DEV)
    cos, sin = rot.cos_sin(pos, dtype)
    nb, bs = 64, 16
    slots = torch.randperm(nb * bs, generator=g)[:M]
    slots[::5] = -1
    kc0 = torch.randn(nb, bs, Hkv, D, generator=g).to(dtype).to(DEV)
    vc0 = torch.randn(nb, bs, Hkv, D, generator=g).to(dtype).to(DEV)
    for slot_dtype in (torch.int32, torch.int64):
        sm = slots.to(slot_dtype).to(DEV)
        y = plain(x, norm=norm)
        q, k, v = y[:, :Hq * D].view(M, Hq, D), y[:, Hq * D:(Hq + Hkv) * D].view(M, Hkv, D), y[:, (Hq + Hkv) * D:].view(M, Hkv, D)
        kc_a, vc_a = kc0.clone(), vc0.clone()
        q_a = rope_reshape_and_cache(q, k, v, cos, sin, kc_a, vc_a, sm)
        kc_b, vc_b = kc0.clone(), vc0.clone()
        q_b = int4_qkv_rope_cache(x, paired, cos, sin, kc_b, vc_b, sm, norm=norm)
        torch.cuda.synchronize()
        assert torch.equal(q_a, q_b), f"q' differs: {(q_a.float() - q_b.float()).abs().max().item():.3e}"
        assert torch.equal(kc_a, kc_b), "key cache differs"
        assert torch.equal(vc_a, vc_b), "value cache differs"
        # The module still returns rows in q|k|v order.
        assert torch.equal(paired(x, norm=norm), y)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("M", [1, 16, 33, 64, 100, 200, 700, 2048])
def test_splitk_down_projection(dtype, M):
    """ns_int4_linear_splitk on down_proj's shape (N 896, K 4864; 4 splits per
    16-token tile up to 16 tokens, 2 up to 32, none at 33-64; beyond 64 tokens the
    tiles are 64 tokens wide and split twice again; above 128 tokens the tiled GEMM
    splits its 64 x 64 tiles 4 times up to 896 tokens and 3 times up to 1152, and
    from 1793 tokens its 128 x 64 tiles twice): within one rounding of the oracle on
    the residual epilogue, identical on a repeated call (the arrival counters are back
    at zero), identical rows for a batch and its first row alone when both split the
    same way, and within one rounding of the unsplit kernel."""
    from nanoserve_amd.quant import splitk_workspace_bytes

    N, K = 896, 4864
    packed, s, z = (t.to(DEV) for t in _weights(N, K, 128, 71))
    g = torch.Generator().manual_seed(72)
    x = torch.randn(M, K, generator=g).to(dtype)
    b = (torch.randn(N, generator=g) * 0.1).to(dtype)
    res = torch.randn(M, N, generator=g).to(dtype)
    ws = torch.zeros(splitk_workspace_bytes(N, K), dtype=torch.uint8, device=DEV)
    assert ws.numel() > 0
    xd, bd, rd = x.to(DEV), b.to(DEV), res.to(DEV)
    first = int4_linear(xd, packed, s, z, bd, 128, residual=rd, workspace=ws)
    again = int4_linear(xd, packed, s, z, bd, 128, residual=rd, workspace=ws)
    plain = int4_linear(xd, packed, s, z, bd, 128, residual=rd)
    head = int4_linear(xd[:1].contiguous(), packed, s, z, bd, 128, residual=rd[:1].contiguous(), workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(first, again)
    if M <= 16:  # same split count as the one-row launch: the batch does not change a row's sums
        assert torch.equal(head, first[:1])
    assert not ws[:SPLITK_COUNTER_BYTES].any(), "arrival counters must be left at zero"
    w = dequantize_int4_ref(packed.cpu().numpy(), s.cpu().numpy(), z.cpu().numpy(), 128, NAME[dtype])
    y = int4_linear_ref(x.float().numpy(), w, b.float().numpy())
    want = _round(y, dtype) + res.double().numpy()
    tol = 2 * RTOL[dtype] * (np.abs(y) + np.abs(res.double().numpy())) + 1e-5
    for t in (first, plain):
        err = np.abs(t.double().cpu().numpy() - want)
        assert (err <= tol).all(), f"max err {err.max():.3e}"


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_splitk_workspace_reused_across_token_counts(dtype):
    """One split-K workspace serves down_proj calls whose token counts change from
    call to call, as a layer's decode steps do (M = 1, 32, 100, 1, 17, 8): each call
    equals, bit for bit, the same call on a fresh zeroed workspace, and the whole
    arrival-counter region is back at zero after every call.  A small-M call's
    partial sums must never land where a larger-M call keeps its counters (the
    300-token call splits every tile of the tiled GEMM, the 4700-token call the
    tiles of its last dispatch round, the 1500-token call none; the rest split
    in the fused kernel)."""
    from nanoserve_amd.quant import splitk_workspace_bytes

    N, K = 896, 4864
    packed, s, z = (t.to(DEV) for t in _weights(N, K, 128, 81))
    nbytes = splitk_workspace_bytes(N, K)
    shared = torch.zeros(nbytes, dtype=torch.uint8, device=DEV)
    g = torch.Generator().manual_seed(82)
    b = (torch.randn(N, generator=g) * 0.1).to(dtype).to(DEV)
    for M in (1, 32, 300, 100, 1, 1500, 4700, 17, 8, 32):
        print(f"splitk reuse M={M} {dtype}", flush=True)
        x = torch.randn(M, K, generator=g).to(dtype).to(DEV)
        res = torch.randn(M, N, generator=g).to(dtype).to(DEV)
        got = int4_linear(x, packed, s, z, b, 128, residual=res, workspace=shared)
        fresh_ws = torch.zeros(nbytes, dtype=torch.uint8, device=DEV)
        want = int4_linear(x, packed, s, z, b, 128, residual=res, workspace=fresh_ws)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"M={M}: reused workspace differs from a fresh one"
        assert not shared[:SPLITK_COUNTER_BYTES].any(), f"M={M}: counters left non-zero"
        assert not fresh_ws[:SPLITK_COUNTER_BYTES].any()


# (N, K, M, epilogue): tiled-GEMM calls on long-K layers whose tiles take more
# than one dispatch round with a part-filled last one, which the library splits
# over K while the earlier rounds' tiles run whole.  down_proj at 4700 tokens:
# 518 128 x 64 tiles on 512 slots, the last 6 (the partial token tile among
# them) split 4 ways; at 10000 tokens: 553 128 x 128 tiles, the last 41 split 4
# ways (residual epilogue); a 1152 x 2048 layer at 3700 tokens: 522 128 x 64
# tiles, the last 10 split 4 ways (bias); a 9728 x 2048 gate|up at 800
# tokens: 532 128 x 128 tiles, the last 20 split 4 ways (SiLU-mul).
TAIL_SPLITS = [(896, 4864, 4700, "residual"), (896, 4864, 10000, "residual"), (1152, 2048, 3700, "bias"),
               (9728, 2048, 800, "silu")]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("N,K,M,epi", TAIL_SPLITS, ids=[f"{n}x{k}-M{m}-{e}" for n, k, m, e in TAIL_SPLITS])
def test_tiled_gemm_splits_the_last_rounds_tiles(dtype, N, K, M, epi):
    """Within one rounding of the oracle (and of the unsplit call, which takes no
    workspace), identical on a repeated call on the same workspace, and the
    arrival counters back at zero."""
    from nanoserve_amd.quant import splitk_workspace_bytes
    from nanoserve_amd import _lib

    lib = _lib.load()
    assert lib.ns_int4_linear_splitk_workspace_size(M, N, K) > SPLITK_COUNTER_BYTES, "the call must split"
    print(f"tail split N={N} K={K} M={M} {epi} {dtype}", flush=True)
    packed, s, z = (t.to(DEV) for t in _weights(N, K, 128, N + M))
    g = torch.Generator().manual_seed(M)
    x = torch.randn(M, K, generator=g).to(dtype)
    b = (torch.randn(N, generator=g) * 0.1).to(dtype) if epi == "bias" else None
    res = torch.randn(M, N, generator=g).to(dtype) if epi == "residual" else None
    ws = torch.zeros(splitk_workspace_bytes(N, K), dtype=torch.uint8, device=DEV)
    kw = dict(residual=None if res is None else res.to(DEV), silu_mul=epi == "silu")
    bd = None if b is None else b.to(DEV)
    xd = x.to(DEV)
    first = int4_linear(xd, packed, s, z, bd, 128, workspace=ws, **kw)
    again = int4_linear(xd, packed, s, z, bd, 128, workspace=ws, **kw)
    plain = int4_linear(xd, packed, s, z, bd, 128, **kw)
    torch.cuda.synchronize()
    assert torch.equal(first, again)
    assert not ws[:SPLITK_COUNTER_BYTES].any(), "arrival counters must be left at zero"
    w = dequantize_int4_ref(packed.cpu().numpy(), s.cpu().numpy(), z.cpu().numpy(), 128, NAME[dtype])
    y = int4_linear_ref(x.float().numpy(), w, None if b is None else b.float().numpy())
    if epi == "silu":
        gv, uv = _round(y[:, 0::2], dtype), _round(y[:, 1::2], dtype)
        act = _round(gv / (1.0 + np.exp(-gv)), dtype)
        want = _round(act * uv, dtype)
        tol = 4 * RTOL[dtype] * np.abs(want) + 4 * RTOL[dtype] * np.abs(act * uv).max() * 1e-2 + 1e-4
    elif epi == "residual":
        want = _round(y, dtype) + res.double().numpy()
        tol = 2 * RTOL[dtype] * (np.abs(y) + np.abs(res.double().numpy())) + 1e-5
    else:
        want = y
        tol = RTOL[dtype] * np.abs(y) + 1e-5 * max(1.0, np.abs(y).max())
    for t, what in ((first, "split"), (plain, "unsplit")):
        err = np.abs(t.double().cpu().numpy() - want)
        assert (err <= tol).all(), f"{what}: max err {err.max():.3e}"
