"""The C-ABI library: it loads, exports every declared symbol, and rejects bad
arguments on the host before touching the GPU (runs without a GPU)."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from nanoserve_amd import _lib

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "nanoserve_paged.h"


def _declared_functions() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ns_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_entry_points():
    names = _declared_functions()
    for n in ("ns_reshape_and_cache", "ns_paged_attention", "ns_paged_attention_workspace_size",
              "ns_rope_reshape_and_cache", "ns_int4_linear", "ns_int4_dequantize", "ns_argmax_rows",
              "ns_error_string", "ns_version"):
        assert n in names


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(_lib.LIB_PATH))
    for name in _declared_functions():
        assert hasattr(lib, name), f"{name} declared in {HEADER.name} but not exported"
    assert set(_declared_functions()) == set(_lib.SIGNATURES)


def test_the_benchmark_probe_lives_outside_the_product_library():
    from nanoserve_amd import _build

    assert not hasattr(ctypes.CDLL(str(_lib.LIB_PATH)), "ns_stream_read")
    if not _build.FLOORS_LIB_PATH.exists():
        pytest.skip("the benchmark's probe library is not built")
    assert hasattr(ctypes.CDLL(str(_build.FLOORS_LIB_PATH)), "ns_stream_read")


def test_status_strings_and_version():
    lib = _lib.load()
    assert lib.ns_version() >= 100
    for code in (0, -1, -2, -3, -4):
        assert lib.ns_error_string(code)
    assert lib.ns_error_string(-99) == b"unknown status"


def _attn_args(**over):
    a = dict(out=16, query=16, k_cache=16, v_cache=16, bt=16, bt_stride=4, bt_width=4, bt64=0,
             sl=16, sl64=0, qsl=16, qsl64=0, slh=None, slh64=0, qslh=None, qslh64=0, S=2, T=2, maxq=1, maxs=64, decode_only=1,
             Hq=14, Hkv=2, D=64, bs=16, nb=32, scale=0.125, dtype=_lib.NS_DTYPE_F16, plan=None, plan_bytes=0,
             ws=16, ws_bytes=1 << 30, stream=None, aux=None, fork=None, join=None)
    a.update(over)
    return list(a.values())


@pytest.mark.parametrize("over,code", [
    (dict(out=None), _lib.NS_ERR_INVALID_ARG),
    (dict(bt=None), _lib.NS_ERR_INVALID_ARG),
    (dict(decode_only=0, qsl=None), _lib.NS_ERR_INVALID_ARG),
    (dict(T=3), _lib.NS_ERR_INVALID_ARG),                 # decode-only needs T == S
    (dict(Hq=15), _lib.NS_ERR_INVALID_ARG),               # Hq not a multiple of Hkv
    (dict(D=320), _lib.NS_ERR_UNSUPPORTED),               # beyond the generic kernel's 256
    (dict(D=0), _lib.NS_ERR_INVALID_ARG),
    (dict(bs=0), _lib.NS_ERR_INVALID_ARG),
    (dict(dtype=7), _lib.NS_ERR_UNSUPPORTED),              # no such dtype code
    (dict(dtype=_lib.NS_DTYPE_F32, out=18), _lib.NS_ERR_INVALID_ARG),  # float32 rows misaligned
    (dict(D=96, query=17), _lib.NS_ERR_INVALID_ARG),       # generic path: fp16 element misaligned
    (dict(ws=None), _lib.NS_ERR_WORKSPACE),
    (dict(ws_bytes=8), _lib.NS_ERR_WORKSPACE),
    (dict(bt_stride=2), _lib.NS_ERR_INVALID_ARG),         # stride below width
    (dict(out=18), _lib.NS_ERR_INVALID_ARG),              # misaligned output
    (dict(scale=float("nan")), _lib.NS_ERR_INVALID_ARG),
    (dict(aux=16), _lib.NS_ERR_INVALID_ARG),              # aux stream without its events
    (dict(aux=16, fork=16), _lib.NS_ERR_INVALID_ARG),
    (dict(aux=16, fork=16, join=16, stream=16), _lib.NS_ERR_INVALID_ARG),  # aux == stream
    (dict(plan=16, plan_bytes=64), _lib.NS_ERR_INVALID_ARG),  # plan buffer smaller than the plan
    (dict(plan=24, plan_bytes=1 << 20), _lib.NS_ERR_INVALID_ARG),  # misaligned plan
])
def test_paged_attention_rejects_bad_arguments(over, code):
    lib = _lib.load()
    assert lib.ns_paged_attention(*_attn_args(**over)) == code


def test_empty_batch_is_a_no_op():
    lib = _lib.load()
    assert lib.ns_paged_attention(*_attn_args(S=0, T=0, out=None)) == _lib.NS_OK


def test_generic_shapes_need_only_a_token_workspace():
    """float32, head sizes other than 64/128, non-power-of-two blocks and wide groups run the
    generic kernel, which reads no workspace; head sizes past 256 are refused."""
    lib = _lib.load()
    for Hq, Hkv, D, bs in ((14, 2, 96, 16), (14, 2, 64, 24), (64, 2, 64, 16), (4, 2, 8, 4)):
        assert lib.ns_paged_attention_workspace_size(8, Hq, Hkv, D, bs, 512, 1, 8, 1) == 256
    assert lib.ns_paged_attention_workspace_size(8, 14, 2, 320, 16, 512, 1, 8, 1) == 0


def test_workspace_size_is_monotone_in_context():
    lib = _lib.load()
    sizes = [lib.ns_paged_attention_workspace_size(32, 14, 2, 64, 16, L, 1, 32, 1)
             for L in (16, 256, 1024, 8192, 65536)]
    assert all(s > 0 for s in sizes)
    assert sizes == sorted(sizes)
    assert lib.ns_paged_attention_workspace_size(32, 14, 2, 0, 16, 100, 1, 32, 1) == 0


def _rc_args(**over):
    a = dict(key=16, value=16, kst=128, ksh=64, vst=128, vsh=64, kc=16, vc=16, slots=16, s64=1,
             T=4, Hkv=2, D=64, bs=16, nb=8, src=_lib.NS_DTYPE_F16, dst=_lib.NS_DTYPE_F16, stream=None)
    a.update(over)
    return list(a.values())


@pytest.mark.parametrize("over,code", [
    (dict(key=None), _lib.NS_ERR_INVALID_ARG),
    (dict(slots=None), _lib.NS_ERR_INVALID_ARG),
    (dict(Hkv=0), _lib.NS_ERR_INVALID_ARG),
    (dict(src=7), _lib.NS_ERR_UNSUPPORTED),
    (dict(D=60), _lib.NS_ERR_UNSUPPORTED),                # rows not a whole number of 16-byte chunks
    (dict(kc=18), _lib.NS_ERR_INVALID_ARG),
])
def test_reshape_and_cache_rejects_bad_arguments(over, code):
    lib = _lib.load()
    assert lib.ns_reshape_and_cache(*_rc_args(**over)) == code


def test_reshape_and_cache_zero_tokens_is_a_no_op():
    lib = _lib.load()
    assert lib.ns_reshape_and_cache(*_rc_args(T=0, key=None)) == _lib.NS_OK


def _rope_args(**over):
    a = dict(qo=16, q=16, qst=14 * 64, qsh=64, k=16, kst=128, ksh=64, v=16, vst=128, vsh=64,
             cos=16, sin=16, cst=64, kc=16, vc=16, slots=16, s64=1,
             T=4, Hq=14, Hkv=2, D=64, bs=16, nb=8, dt=_lib.NS_DTYPE_F16, cdt=_lib.NS_DTYPE_F16, stream=None)
    a.update(over)
    return list(a.values())


@pytest.mark.parametrize("over,code", [
    (dict(q=None), _lib.NS_ERR_INVALID_ARG),
    (dict(cos=None), _lib.NS_ERR_INVALID_ARG),
    (dict(slots=None), _lib.NS_ERR_INVALID_ARG),
    (dict(Hq=0), _lib.NS_ERR_INVALID_ARG),
    (dict(nb=0), _lib.NS_ERR_INVALID_ARG),
    (dict(dt=7), _lib.NS_ERR_UNSUPPORTED),
    (dict(cdt=7), _lib.NS_ERR_UNSUPPORTED),
    (dict(D=72), _lib.NS_ERR_UNSUPPORTED),               # half a row not a whole number of 16-byte chunks
    (dict(D=68, dt=_lib.NS_DTYPE_F32, qst=14 * 68, qsh=68, kst=136, ksh=68, vst=136, vsh=68, cst=68),
     _lib.NS_ERR_UNSUPPORTED),                           # f32: 4 per chunk, 34 per half
    (dict(qsh=60), _lib.NS_ERR_INVALID_ARG),             # stride not a whole number of chunks
    (dict(cst=4), _lib.NS_ERR_INVALID_ARG),
    (dict(k=18), _lib.NS_ERR_INVALID_ARG),               # misaligned row base
    (dict(sin=24), _lib.NS_ERR_INVALID_ARG),
])
def test_rope_reshape_and_cache_rejects_bad_arguments(over, code):
    lib = _lib.load()
    assert lib.ns_rope_reshape_and_cache(*_rope_args(**over)) == code


def test_rope_reshape_and_cache_zero_tokens_is_a_no_op():
    lib = _lib.load()
    assert lib.ns_rope_reshape_and_cache(*_rope_args(T=0, q=None, k=None)) == _lib.NS_OK


def _i4_args(**over):
    a = dict(out=16, x=16, xs=256, qw=16, sc=16, zp=16, bias=None, res=None, epi=_lib.NS_EPILOGUE_NONE,
             nw=None, eps=1e-6, M=4, N=64, K=256, gs=128, dt=_lib.NS_DTYPE_F16, stream=None)
    a.update(over)
    return list(a.values())


@pytest.mark.parametrize("over,code", [
    (dict(x=None), _lib.NS_ERR_INVALID_ARG),
    (dict(qw=None), _lib.NS_ERR_INVALID_ARG),
    (dict(N=0), _lib.NS_ERR_INVALID_ARG),
    (dict(dt=_lib.NS_DTYPE_F32), _lib.NS_ERR_UNSUPPORTED),
    (dict(N=72), _lib.NS_ERR_UNSUPPORTED),                # features not a whole number of 16-row tiles
    (dict(K=240, xs=240), _lib.NS_ERR_UNSUPPORTED),       # K not a multiple of the group size
    (dict(gs=48), _lib.NS_ERR_UNSUPPORTED),
    (dict(xs=250), _lib.NS_ERR_INVALID_ARG),              # row stride not 16-byte aligned
    (dict(xs=128), _lib.NS_ERR_INVALID_ARG),              # row stride shorter than a row
    (dict(x=24), _lib.NS_ERR_INVALID_ARG),
    (dict(out=20), _lib.NS_ERR_INVALID_ARG),
    (dict(qw=24), _lib.NS_ERR_INVALID_ARG),               # codes are read as 16-byte vectors
    (dict(epi=3), _lib.NS_ERR_UNSUPPORTED),
    (dict(epi=_lib.NS_EPILOGUE_RESIDUAL), _lib.NS_ERR_INVALID_ARG),  # residual epilogue without residual
    (dict(nw=16, K=2048, xs=2048), _lib.NS_ERR_UNSUPPORTED),          # RMSNorm prologue: K at most 1024
    (dict(nw=16, K=96, xs=96, gs=32), _lib.NS_ERR_UNSUPPORTED),       # RMSNorm prologue: whole 128-chunks
    (dict(nw=24), _lib.NS_ERR_INVALID_ARG),                          # misaligned norm weight
])
def test_int4_linear_rejects_bad_arguments(over, code):
    lib = _lib.load()
    assert lib.ns_int4_linear(*_i4_args(**over)) == code


def test_int4_linear_splitk_checks_its_workspace():
    """down_proj's shape splits (a workspace is required and sized by the query);
    a shape that does not split needs none.  Rejected before any launch."""
    lib = _lib.load()
    M, N, K = 16, 896, 4864
    need = lib.ns_int4_linear_splitk_workspace_size(M, N, K)
    assert need > 0 and lib.ns_int4_linear_splitk_workspace_size(16, 64, 256) == 0
    assert lib.ns_int4_linear_splitk_workspace_size(-1, N, K) == 0
    base = _i4_args(M=M, N=N, K=K, xs=K)[:-1]
    for ws, nbytes in ((None, need), (256, need - 1), (128, need)):  # missing, too small, misaligned
        assert lib.ns_int4_linear_splitk(*base, ws, nbytes, None) == _lib.NS_ERR_INVALID_ARG
    assert lib.ns_int4_linear_splitk(*_i4_args(M=M, N=N, K=K, xs=K, x=None)[:-1], 256, need, None) == \
        _lib.NS_ERR_INVALID_ARG


@pytest.mark.parametrize("N,K", [(896, 4864), (896, 896), (1152, 896), (9728, 896), (4096, 8192)])
def test_splitk_workspace_bytes_cover_every_token_count(N, K):
    """The module-level workspace (sized once per layer by a scan of token counts)
    is at least what the library asks for at every M: densely through the
    register kernel's range and the tiled GEMM's first rounds, then at strided and
    odd token counts far past the scan's end (the GEMM's last-round splits
    recur at any size).  The GEMM splits down_proj (K 4864) at prefill sizes,
    including the part-filled last round of 4700 and 10000 tokens, and never a
    K-896 layer (14 steps: under 8 a split); the splits only ever fill idle
    slots of one round, so the partials never exceed 512 workgroups' 128 x 128
    fp32 tiles."""
    from nanoserve_amd.quant import splitk_workspace_bytes

    lib = _lib.load()
    have = splitk_workspace_bytes(N, K)
    rows = list(range(1, 6000)) + list(range(6007, 400_000, 997)) + [131_071, 131_073, 262_145, 1_000_003]
    sizes = [lib.ns_int4_linear_splitk_workspace_size(m, N, K) for m in rows]
    assert max(sizes) <= have
    assert have <= 1024 + 512 * 128 * 128 * 4
    if (N, K) == (896, 4864):
        for m in (1024, 2048, 4700, 10000):
            assert lib.ns_int4_linear_splitk_workspace_size(m, N, K) > 0
    if K == 896:
        assert max(sizes[128:]) == 0


def test_int4_linear_rope_cache_rejects_bad_arguments():
    lib = _lib.load()

    def call(**over):
        a = dict(q=16, x=16, xs=896, qw=16, sc=16, zp=16, bias=None, nw=None, eps=1e-6, cos=16, sin=16, css=64,
                 kc=16, vc=16, slots=16, s64=1, M=4, K=896, gs=128, hq=14, hkv=2, d=64, bs=16, nb=8,
                 dt=_lib.NS_DTYPE_F16, stream=None)
        a.update(over)
        return lib.ns_int4_linear_rope_cache(*a.values())

    assert call(M=0, x=None) == _lib.NS_OK
    assert call(dt=_lib.NS_DTYPE_F32) == _lib.NS_ERR_UNSUPPORTED
    assert call(d=40) == _lib.NS_ERR_UNSUPPORTED           # head_dim not a multiple of 16
    assert call(K=2048, xs=2048) == _lib.NS_ERR_UNSUPPORTED  # more than 8 chunks
    assert call(kc=None) == _lib.NS_ERR_INVALID_ARG
    assert call(cos=20) == _lib.NS_ERR_INVALID_ARG         # cos/sin rows read as 8-byte vectors
    assert call(css=62) == _lib.NS_ERR_INVALID_ARG
    assert call(hkv=0) == _lib.NS_ERR_INVALID_ARG


def test_int4_linear_zero_rows_is_a_no_op():
    lib = _lib.load()
    assert lib.ns_int4_linear(*_i4_args(M=0, x=None)) == _lib.NS_OK


@pytest.mark.parametrize("args,code", [
    ((16, 16, 104, 4, 100, 7, 16, 1 << 20, None), _lib.NS_ERR_UNSUPPORTED),
    ((None, 16, 104, 4, 100, _lib.NS_DTYPE_F16, 16, 1 << 20, None), _lib.NS_ERR_INVALID_ARG),
    ((16, 16, 99, 4, 100, _lib.NS_DTYPE_F16, 16, 1 << 20, None), _lib.NS_ERR_INVALID_ARG),   # stride < row
    ((16, 16, 100, 4, 100, _lib.NS_DTYPE_F16, 16, 1 << 20, None), _lib.NS_ERR_INVALID_ARG),  # 200-byte rows
    ((16, 24, 104, 4, 100, _lib.NS_DTYPE_F16, 16, 1 << 20, None), _lib.NS_ERR_INVALID_ARG),  # misaligned base
    ((16, 16, 104, 4, 100, _lib.NS_DTYPE_F16, None, 0, None), _lib.NS_ERR_WORKSPACE),
    ((16, 16, 104, 4, 100, _lib.NS_DTYPE_F16, 16, 8, None), _lib.NS_ERR_WORKSPACE),          # 4 rows need 32 B
    ((16, 16, 104, 0, 100, _lib.NS_DTYPE_F16, None, 0, None), _lib.NS_OK),                   # no rows: no launch
])
def test_argmax_rows_rejects_bad_arguments(args, code):
    assert _lib.load().ns_argmax_rows(*args) == code


def test_argmax_workspace_size():
    lib = _lib.load()
    assert lib.ns_argmax_rows_workspace_size(32, 151936) == 32 * 38 * 8
    assert lib.ns_argmax_rows_workspace_size(1, 4096) == 8
    assert lib.ns_argmax_rows_workspace_size(0, 10) == 0


@pytest.mark.parametrize("args,code", [
    ((None, 16, 16, 16, 64, 256, 128, _lib.NS_DTYPE_F16, None), _lib.NS_ERR_INVALID_ARG),
    ((16, 16, 16, 16, 64, 256, 128, _lib.NS_DTYPE_F32, None), _lib.NS_ERR_UNSUPPORTED),
    ((16, 16, 16, 16, 64, 260, 130, _lib.NS_DTYPE_F16, None), _lib.NS_ERR_UNSUPPORTED),
    ((24, 16, 16, 16, 64, 256, 128, _lib.NS_DTYPE_F16, None), _lib.NS_ERR_INVALID_ARG),
    ((16, 16, 16, 16, 0, 256, 128, _lib.NS_DTYPE_F16, None), _lib.NS_ERR_INVALID_ARG),
])
def test_int4_dequantize_rejects_bad_arguments(args, code):
    assert _lib.load().ns_int4_dequantize(*args) == code


@pytest.mark.parametrize("Hq,Hkv,D,bs", [(14, 2, 64, 16), (28, 4, 128, 32), (14, 2, 96, 16), (4, 2, 8, 4),
                                         (14, 2, 64, 12), (64, 2, 64, 16), (6, 3, 256, 1)])
def test_the_shim_and_the_library_pick_the_same_kernel_family(Hq, Hkv, D, bs):
    """attention.py skips the decode plan and the aux stream for the shapes the library
    runs on its generic kernel; both must draw the line in the same place (the
    library's workspace size is the token 256 bytes exactly for those shapes)."""
    import torch

    from nanoserve_amd.attention import takes_generic_kernel

    lib = _lib.load()
    generic_py = takes_generic_kernel(torch.float16, D, bs, Hq // Hkv)
    assert takes_generic_kernel(torch.float32, D, bs, Hq // Hkv)
    ws = lib.ns_paged_attention_workspace_size(8, Hq, Hkv, D, bs, 512, 1, 8, 1)
    assert (ws == 256) == generic_py, (Hq, Hkv, D, bs, ws)
