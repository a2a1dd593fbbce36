"""ctypes binding of the C ABI declared in include/nanoserve_paged.h.

Loading order matters: torch ships its own libamdhip64.so.7, and the library
must bind to that same runtime so torch's streams and allocations are valid
inside it.  Importing torch first makes the dynamic linker resolve the
library's libamdhip64.so.7 dependency to the copy torch already loaded.

There is no fallback.  If the library is missing or does not export the
expected symbols, `load()` raises.
"""

from __future__ import annotations

import ctypes
import threading
from ctypes import c_float, c_int, c_int64, c_size_t, c_void_p, c_char_p

import torch  # noqa: F401  (binds libamdhip64 before the library is loaded)

from ._build import LIB_PATH

NS_OK = 0
NS_ERR_INVALID_ARG = -1
NS_ERR_UNSUPPORTED = -2
NS_ERR_WORKSPACE = -3
NS_ERR_HIP = -4

NS_DTYPE_F32 = 0
NS_DTYPE_F16 = 1
NS_DTYPE_BF16 = 2

NS_EPILOGUE_NONE = 0
NS_EPILOGUE_RESIDUAL = 1
NS_EPILOGUE_SILU_MUL = 2

DTYPE_CODES = {
    torch.float32: NS_DTYPE_F32,
    torch.float16: NS_DTYPE_F16,
    torch.bfloat16: NS_DTYPE_BF16,
}

# Exported symbol -> (restype, argtypes).  Kept in the order of the header.
SIGNATURES = {
    "ns_error_string": (c_char_p, [c_int]),
    "ns_version": (c_int, []),
    "ns_reshape_and_cache": (c_int, [
        c_void_p, c_void_p,                      # key, value
        c_int64, c_int64, c_int64, c_int64,      # key/value token and head strides
        c_void_p, c_void_p,                      # k_cache, v_cache
        c_void_p, c_int,                         # slot_mapping, is_int64
        c_int64, c_int, c_int, c_int, c_int64,   # T, Hkv, D, block_size, num_blocks
        c_int, c_int, c_void_p,                  # src dtype, cache dtype, stream
    ]),
    "ns_rope_reshape_and_cache": (c_int, [
        c_void_p, c_void_p, c_int64, c_int64,    # q_out, query, query token / head strides
        c_void_p, c_int64, c_int64,              # key, token / head strides
        c_void_p, c_int64, c_int64,              # value, token / head strides
        c_void_p, c_void_p, c_int64,             # cos, sin, token stride
        c_void_p, c_void_p,                      # k_cache, v_cache
        c_void_p, c_int,                         # slot_mapping, is_int64
        c_int64, c_int, c_int, c_int,            # T, Hq, Hkv, D
        c_int, c_int64,                          # block_size, num_blocks
        c_int, c_int, c_void_p,                  # model dtype, cache dtype, stream
    ]),
    "ns_int4_linear": (c_int, [
        c_void_p, c_void_p, c_int64,             # out, x, x row stride
        c_void_p, c_void_p, c_void_p, c_void_p,  # qweight, scales, zeros, bias (or None)
        c_void_p, c_int,                         # residual (or None), epilogue
        c_void_p, c_float,                       # RMSNorm weight (or None), eps
        c_int64, c_int, c_int, c_int,            # M, N, K, group_size
        c_int, c_void_p,                         # dtype, stream
    ]),
    "ns_int4_linear_splitk_workspace_size": (c_size_t, [c_int64, c_int, c_int]),  # M, N, K
    "ns_int4_linear_splitk": (c_int, [
        c_void_p, c_void_p, c_int64,             # out, x, x row stride
        c_void_p, c_void_p, c_void_p, c_void_p,  # qweight, scales, zeros, bias (or None)
        c_void_p, c_int,                         # residual (or None), epilogue
        c_void_p, c_float,                       # RMSNorm weight (or None), eps
        c_int64, c_int, c_int, c_int,            # M, N, K, group_size
        c_int,                                   # dtype
        c_void_p, c_size_t, c_void_p,            # workspace, bytes, stream
    ]),
    "ns_int4_linear_rope_cache": (c_int, [
        c_void_p, c_void_p, c_int64,             # q_out, x, x row stride
        c_void_p, c_void_p, c_void_p, c_void_p,  # qweight, scales, zeros, bias (or None)
        c_void_p, c_float,                       # RMSNorm weight (or None), eps
        c_void_p, c_void_p, c_int64,             # cos, sin, token stride
        c_void_p, c_void_p,                      # k_cache, v_cache
        c_void_p, c_int,                         # slot_mapping, is_int64
        c_int64, c_int, c_int,                   # M, K, group_size
        c_int, c_int, c_int,                     # Hq, Hkv, D
        c_int, c_int64,                          # block_size, num_blocks
        c_int, c_void_p,                         # dtype, stream
    ]),
    "ns_int4_dequantize": (c_int, [
        c_void_p, c_void_p, c_void_p, c_void_p,  # out [N, K], qweight, scales, zeros
        c_int, c_int, c_int, c_int, c_void_p,    # N, K, group_size, dtype, stream
    ]),
    "ns_argmax_rows_workspace_size": (c_size_t, [c_int64, c_int64]),  # M, N
    "ns_argmax_rows": (c_int, [
        c_void_p, c_void_p, c_int64,             # out (int64), x, x row stride
        c_int64, c_int64, c_int,                 # M, N, dtype
        c_void_p, c_size_t, c_void_p,            # workspace, bytes, stream
    ]),
    "ns_paged_attention_workspace_size": (c_size_t, [
        c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int64, c_int,
    ]),
    "ns_paged_decode_plan_size": (c_size_t, [c_int, c_int, c_int, c_int, c_int]),  # S, Hkv, D, bs, max_seq_len
    "ns_paged_decode_plan": (c_int, [
        c_void_p, c_size_t,                      # plan, bytes
        c_void_p, c_int64, c_int64, c_int,       # block_tables, row stride, width, is_int64
        c_void_p, c_int, c_void_p, c_int,        # seq_lens, is_int64, query_start_loc (or None), is_int64
        c_int, c_int, c_int, c_int, c_int,       # S, decode_only, Hkv, D, block_size
        c_int, c_void_p,                         # max_seq_len, stream
    ]),
    "ns_paged_attention": (c_int, [
        c_void_p, c_void_p,                      # out, query
        c_void_p, c_void_p,                      # k_cache, v_cache
        c_void_p, c_int64, c_int64, c_int,       # block_tables, row stride, width, is_int64
        c_void_p, c_int,                         # seq_lens, is_int64
        c_void_p, c_int,                         # query_start_loc, is_int64
        c_void_p, c_int,                         # seq_lens_host (host memory, optional), is_int64
        c_void_p, c_int,                         # query_start_loc_host (host memory, optional), is_int64
        c_int, c_int64, c_int, c_int, c_int,     # S, T, max_query_len, max_seq_len, decode_only
        c_int, c_int, c_int, c_int, c_int64,     # Hq, Hkv, D, block_size, num_blocks
        c_float, c_int,                          # scale, dtype
        c_void_p, c_size_t,                      # decode plan (or None), bytes
        c_void_p, c_size_t, c_void_p,            # workspace, bytes, stream
        c_void_p, c_void_p, c_void_p,            # aux stream, fork event, join event (all or none)
    ]),
    "ns_paged_attention_noalloc": (c_int, [
        c_void_p, c_void_p,                      # out, query
        c_void_p, c_void_p,                      # k_cache, v_cache
        c_void_p, c_int64, c_int64, c_int,       # block_tables, row stride, width, is_int64
        c_void_p, c_int,                         # seq_lens, is_int64
        c_void_p, c_int,                         # query_start_loc, is_int64
        c_void_p, c_int,                         # seq_lens_host (host memory, optional), is_int64
        c_void_p, c_int,                         # query_start_loc_host (host memory, optional), is_int64
        c_int, c_int64, c_int, c_int, c_int,     # S, T, max_query_len, max_seq_len, decode_only
        c_int, c_int, c_int, c_int, c_int64,     # Hq, Hkv, D, block_size, num_blocks
        c_float, c_int,                          # scale, dtype
        c_void_p, c_size_t, c_void_p,            # decode plan (or None), bytes, stream
        c_void_p, c_void_p, c_void_p,            # aux stream, fork event, join event (all or none)
    ]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None
_capture_info = None


def load() -> ctypes.CDLL:
    """Load the library once; raise if it is absent or incomplete."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m nanoserve_amd._build` "
                "(the paged-attention path has no non-HIP fallback)"
            )
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)  # AttributeError if the export is missing
            fn.restype = res
            fn.argtypes = args
        _lib = lib
        return lib


def check(rc: int, what: str) -> None:
    if rc != NS_OK:
        msg = load().ns_error_string(rc).decode()
        raise RuntimeError(f"{what} failed: {msg} (status {rc})")


def stream_capture_id(stream: int) -> int:
    """The id of the graph capture under way on `stream` (a hipStream_t as an
    int), or 0 when the stream is not capturing.

    Read with the HIP runtime's hipStreamGetCaptureInfo from the copy torch
    loaded (the library's own dependency resolves to it, see the top)."""
    global _capture_info
    if _capture_info is None:
        fn = ctypes.CDLL("libamdhip64.so.7").hipStreamGetCaptureInfo
        fn.restype = c_int
        fn.argtypes = [c_void_p, ctypes.POINTER(c_int), ctypes.POINTER(ctypes.c_ulonglong)]
        _capture_info = fn
    status, cid = c_int(0), ctypes.c_ulonglong(0)
    rc = _capture_info(c_void_p(stream), ctypes.byref(status), ctypes.byref(cid))
    if rc != 0:
        raise RuntimeError(f"hipStreamGetCaptureInfo failed with HIP error {rc}")
    return int(cid.value) if status.value == 1 else 0  # 1: hipStreamCaptureStatusActive
