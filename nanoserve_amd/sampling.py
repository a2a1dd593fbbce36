"""Greedy token selection on the GPU (ns_argmax_rows).

The reference's sampler takes logits.argmax(dim=-1) for greedy requests
(nanoserve/sampler.py:24-27); `argmax_rows` is the same selection -- first
index among equal maxima, first NaN if any -- in one HIP launch per batch.
"""

from __future__ import annotations

import torch

from . import _lib

# One slice-key workspace per (device, stream), grown on demand; graph capture
# records its pointer, so it is allocated by the warm-up call before capture.
_workspaces: dict[tuple[int, int], torch.Tensor] = {}
# Buffers a larger one replaced: a graph captured with one of them keeps its
# address (and torch recycles stream handles), so they are never freed.
_retired: list[torch.Tensor] = []


def _workspace(device: torch.device, stream: int, nbytes: int) -> torch.Tensor:
    key = (device.index if device.index is not None else torch.cuda.current_device(), stream)
    ws = _workspaces.get(key)
    if ws is None or ws.numel() < nbytes:
        if torch.cuda.is_current_stream_capturing():
            # A graph captured earlier with the old buffer would keep its freed
            # address; callers warm up every shape before capturing.
            raise RuntimeError(
                f"argmax_rows needs a {nbytes}-byte workspace on stream {stream:#x} during graph "
                f"capture, but has {0 if ws is None else ws.numel()} bytes: run the largest shape "
                "once on this stream before capturing")
        if ws is not None:
            _retired.append(ws)
        ws = torch.empty(max(nbytes, 1 << 16), dtype=torch.uint8, device=device)
        _workspaces[key] = ws
    return ws


@torch.inference_mode()
def argmax_rows(logits: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """[M, N] logits (f32/f16/bf16, unit element stride) -> [M] int64 indices."""
    if logits.dim() != 2:
        raise ValueError(f"logits must be [M, N], got {tuple(logits.shape)}")
    if not logits.is_cuda:
        raise ValueError("argmax_rows needs a GPU tensor (the HIP path has no CPU fallback)")
    if logits.dtype not in _lib.DTYPE_CODES:
        raise TypeError(f"unsupported dtype {logits.dtype}")
    x = logits
    esz = x.element_size()
    if x.stride(1) != 1 or (x.stride(0) * esz) % 16 != 0 or x.data_ptr() % 16 != 0:
        x = x.contiguous()
        if (x.shape[1] * esz) % 16 != 0:
            pad = -x.shape[1] % (16 // esz)
            x = torch.nn.functional.pad(x, (0, pad), value=float("-inf"))[:, :logits.shape[1]]
    M, N = logits.shape
    if out is None:
        out = torch.empty(M, dtype=torch.int64, device=x.device)
    lib = _lib.load()
    stream = torch.cuda.current_stream(x.device).cuda_stream
    ws = _workspace(x.device, stream, lib.ns_argmax_rows_workspace_size(M, N))
    rc = lib.ns_argmax_rows(out.data_ptr(), x.data_ptr(), x.stride(0), M, N, _lib.DTYPE_CODES[x.dtype],
                            ws.data_ptr(), ws.numel(), stream)
    _lib.check(rc, "ns_argmax_rows")
    return out
