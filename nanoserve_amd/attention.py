"""Paged attention on MI355X: the attn_fn drop-in over the HIP kernels.

`paged_attention_hip(query, k_cache, v_cache, md, scale)` keeps the signature
and the semantics of the reference's unified op (nanoserve/attention.py:99-151,
decode fast path 154-190, Triton wrapper triton_attention.py:117-161): prefill,
decode, chunked prefill and mixed batches are one call; query row j of a
sequence with context length L and query length ql attends to keys
[0, L - ql + j]; the kv head of query head h is h // (Hq // Hkv).

Everything runs on the GPU through libnanoserve_paged.so: the decode rows of a
batch are one kernel launch over a work plan built on the device, with
split-K partials merged inside the launch; any other batch adds one launch of
the variable-length MFMA kernel.  Those kernels take float16/bfloat16 at head
sizes 64 and 128; float32, other head sizes (up to 256), block sizes that are
not powers of two and more than 16 query heads per KV head run the library's
generic one-wave-per-row kernel instead.  There is no torch or Triton
fallback; a missing library or an unsupported shape raises.

The plan belongs to the step, like the metadata: the reference builds one
AttentionMetadata per step and hands the same object to every layer
(model_runner.py:85-147, qwen2.py:105-113), so the first call that sees an
`md` builds its plan (one small launch) and stores it on the `md`; the other
layers' calls find it there.  A caller that rewrites an md's device tensors in
place for a new step must clear `md.decode_plan` (or call
`prepare_decode_plan` again); the engine builds a new md per step, and a
captured graph rebuilds the plan in every replay.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from . import _lib


@dataclass
class AttentionMetadata:
    """Per-step addressing shared by all layers (reference attention.py:31-54).

    Index tensors may be int32 or int64 and must live on the query's device.
    The engine stages all of them as int64 slices of one buffer
    (reference model_runner.py:128-137); the reference tests use int32.
    """

    slot_mapping: torch.Tensor      # [num_tokens] cache slot of each new token
    query_start_loc: torch.Tensor   # [num_seqs + 1] prefix sums of query_lens
    seq_lens: torch.Tensor          # [num_seqs] context length including this step
    block_tables: torch.Tensor      # [num_seqs, max_blocks] physical block ids
    max_query_len: int
    max_seq_len: int
    num_seqs: int
    num_tokens: int
    is_decode_only: bool            # every query_len == 1

    query_lens_cpu: list[int] = None          # type: ignore[assignment]
    seq_lens_cpu: list[int] = None            # type: ignore[assignment]
    query_start_loc_cpu: list[int] = None     # type: ignore[assignment]
    # The step's device-side decode plan (prepare_decode_plan), built by the
    # step's first attention call (or explicitly before it) and read by every
    # layer's call.
    decode_plan: "DecodePlan | None" = None


@dataclass(frozen=True)
class DecodePlan:
    """A device buffer holding ns_paged_decode_plan's output, the call sizes it
    is valid for, and the graph capture that built it (0: none).  A plan built
    inside a capture is written by that graph's replays only."""

    buffer: torch.Tensor
    key: tuple
    capture: int = 0


_INDEX_DTYPES = (torch.int32, torch.int64)

# Split-K workspaces, one per (device, stream).  The library requires the
# buffer to be zero once and leaves its counters at zero after every call, so
# a cached buffer is reused without clearing.  Calls on different streams may
# overlap in time and therefore get different buffers.
_workspaces: dict[tuple[int, int], torch.Tensor] = {}
# Buffers a larger one replaced.  A graph captured while one of them was
# current still holds its address, so they stay allocated for the process
# (torch hands out recycled stream handles, so a key can also be reused by a
# later, unrelated stream).  Growth is geometric: they add up to less than
# the current buffer.
_retired: list[torch.Tensor] = []
# Plans built inside a graph capture and later replaced on their md (the md
# was used again eagerly or in another capture): the graph still writes and
# reads the buffer on every replay, so it is never freed.
_captured_plans: list["DecodePlan"] = []

# Per (device, stream): the second stream and fork/join events a mixed batch
# overlaps its decode launch on.  The shim owns them; the library only uses
# what it is handed.
_aux: dict[tuple[int, int], tuple[torch.cuda.Stream, torch.cuda.Event, torch.cuda.Event]] = {}


def _device_index(device: torch.device) -> int:
    return device.index if device.index is not None else torch.cuda.current_device()


def _workspace(device: torch.device, stream: int, nbytes: int) -> torch.Tensor:
    key = (_device_index(device), stream)
    ws = _workspaces.get(key)
    if ws is None or ws.numel() < nbytes:
        if torch.cuda.is_current_stream_capturing():
            # A graph captured with the old buffer would keep its freed
            # address, and the new buffer's zero fill would be recorded into
            # this graph.  Callers warm up every shape before capturing.
            raise RuntimeError(
                f"paged attention needs a {nbytes}-byte workspace on stream {stream:#x} during graph "
                f"capture, but has {0 if ws is None else ws.numel()} bytes: run the largest shape "
                "once on this stream before capturing")
        # Grow geometrically so a slowly growing max_seq_len reallocates rarely.
        size = max(nbytes, 2 * ws.numel() if ws is not None else 0, 1 << 20)
        if ws is not None:
            _retired.append(ws)
        ws = torch.zeros(size, dtype=torch.uint8, device=device)
        _workspaces[key] = ws
    return ws


def _aux_stream(device: torch.device, stream: int):
    """(aux stream, fork event, join event) handles for overlapping a mixed batch."""
    key = (_device_index(device), stream)
    aux = _aux.get(key)
    if aux is None:
        if torch.cuda.is_current_stream_capturing():
            return None, None, None  # created on first use outside capture; run in order meanwhile
        side = torch.cuda.Stream(device)  # default priority
        fork, join = torch.cuda.Event(), torch.cuda.Event()
        fork.record(side)  # creates the HIP events (torch creates them lazily)
        join.record(side)
        side.synchronize()
        aux = _aux[key] = (side, fork, join)
    side, fork, join = aux
    return side.cuda_stream, fork.cuda_event, join.cuda_event


def _index(t: torch.Tensor, name: str, device: torch.device) -> torch.Tensor:
    if t.device != device:
        raise ValueError(f"{name} is on {t.device}, expected {device}")
    if t.dtype not in _INDEX_DTYPES:
        t = t.to(torch.int64)
    return t


def _plan_key(md: AttentionMetadata, num_kv_heads: int, head_dim: int, block_size: int,
              device: torch.device) -> tuple:
    """What a plan depends on besides the device lengths it reads: the call sizes,
    the metadata tensors it was built from and, when the metadata carries them,
    the host copies of the lengths and query offsets."""
    lens = None if md.seq_lens_cpu is None else tuple(md.seq_lens_cpu[:md.num_seqs])
    qsl = None if md.is_decode_only or md.query_start_loc_cpu is None else tuple(md.query_start_loc_cpu)
    return (md.num_seqs, num_kv_heads, head_dim, block_size, md.max_seq_len, int(md.block_tables.shape[1]),
            bool(md.is_decode_only), md.seq_lens.data_ptr(),
            None if md.query_start_loc is None else md.query_start_loc.data_ptr(), _device_index(device),
            lens, qsl)


@torch.inference_mode()
def prepare_decode_plan(md: AttentionMetadata, cache: torch.Tensor) -> None:
    """Build md's decode plan on the device (one launch on the current stream)
    for attention calls over caches shaped like `cache` ([NB, BS, Hkv, D]).

    The reference builds a step's metadata once and hands it to every layer
    (model_runner.py:85-147, qwen2.py:105-113); the plan belongs to that step
    in the same way: it is read from the device lengths, so a captured graph
    that calls this rebuilds it from the replayed step's lengths.  Calls whose
    sizes differ from the plan's build their own instead.
    """
    if md.num_seqs == 0 or md.num_tokens == 0:
        return
    lib = _lib.load()
    _, block_size, num_kv_heads, head_dim = cache.shape
    if takes_generic_kernel(cache.dtype, head_dim, block_size, 1):
        return  # the generic kernel reads no plan
    device = cache.device
    bt = _index(md.block_tables, "block_tables", device)
    sl = _index(md.seq_lens, "seq_lens", device).contiguous()
    decode_only = bool(md.is_decode_only)
    qsl_ptr, qsl64 = None, 0
    if not decode_only:
        qsl = _index(md.query_start_loc, "query_start_loc", device).contiguous()
        qsl_ptr, qsl64 = qsl.data_ptr(), int(qsl.dtype == torch.int64)
    nbytes = int(lib.ns_paged_decode_plan_size(md.num_seqs, num_kv_heads, head_dim, block_size, md.max_seq_len))
    if nbytes == 0:
        raise RuntimeError(f"unsupported decode plan shape: Hkv={num_kv_heads} D={head_dim} block_size={block_size}")
    buf = torch.empty(nbytes, dtype=torch.uint8, device=device)
    if bt.stride(1) != 1:
        raise ValueError("block_tables rows must be contiguous")
    rc = lib.ns_paged_decode_plan(buf.data_ptr(), nbytes, bt.data_ptr(), bt.stride(0), bt.shape[1],
                                  int(bt.dtype == torch.int64), sl.data_ptr(), int(sl.dtype == torch.int64),
                                  qsl_ptr, qsl64, md.num_seqs, int(decode_only), num_kv_heads, head_dim,
                                  block_size, md.max_seq_len, torch.cuda.current_stream(device).cuda_stream)
    _lib.check(rc, "ns_paged_decode_plan")
    stream = torch.cuda.current_stream(device).cuda_stream
    capture = _lib.stream_capture_id(stream) if torch.cuda.is_current_stream_capturing() else 0
    old = md.decode_plan
    if old is not None and old.capture not in (0, capture):
        _captured_plans.append(old)
    md.decode_plan = DecodePlan(buf, _plan_key(md, num_kv_heads, head_dim, block_size, device), capture)


def takes_generic_kernel(dtype: torch.dtype, head_dim: int, block_size: int, group: int) -> bool:
    """Whether the library runs this shape on its generic kernel (float32, head sizes
    other than 64/128, block sizes that are not powers of two, more than 16 query heads
    per KV head), which takes no decode plan and no second stream.  The library draws
    the same line (generic_attention_takes in csrc/generic_attention.h)."""
    return (dtype == torch.float32 or head_dim not in (64, 128)
            or block_size & (block_size - 1) != 0 or group > 16)


def workspace_bytes(md: AttentionMetadata, num_heads: int, num_kv_heads: int,
                    head_dim: int, block_size: int) -> int:
    """Device workspace ns_paged_attention needs for this metadata."""
    return int(_lib.load().ns_paged_attention_workspace_size(
        md.num_seqs, num_heads, num_kv_heads, head_dim, block_size,
        md.max_seq_len, md.max_query_len, md.num_tokens, int(bool(md.is_decode_only))))


@torch.inference_mode()
def paged_attention_hip(
    query: torch.Tensor,        # [num_tokens, num_heads, head_dim]
    k_cache: torch.Tensor,      # [num_blocks, block_size, num_kv_heads, head_dim]
    v_cache: torch.Tensor,
    md: AttentionMetadata,
    scale: float,
) -> torch.Tensor:
    """Unified paged attention on the GPU.  Returns [num_tokens, num_heads, head_dim].

    The reference's attn_fn contract (attention.py:99-151).  The decode plan
    is shared by the calls of one md: built by the first, reused by the rest."""
    return _attention(query, k_cache, v_cache, md, scale, share_plan=True)


def _attention(query, k_cache, v_cache, md: AttentionMetadata, scale: float, share_plan: bool) -> torch.Tensor:
    """paged_attention_hip's body.  share_plan=False leaves md.decode_plan
    unused and untouched: the library then plans the decode rows inside the
    call (in its workspace)."""
    lib = _lib.load()
    if query.dim() != 3 or k_cache.dim() != 4 or v_cache.shape != k_cache.shape:
        raise ValueError(
            f"expected query [T,Hq,D] and caches [NB,BS,Hkv,D], got "
            f"{tuple(query.shape)}, {tuple(k_cache.shape)}, {tuple(v_cache.shape)}")
    num_tokens, num_heads, head_dim = query.shape
    num_blocks, block_size, num_kv_heads, cache_dim = k_cache.shape
    if cache_dim != head_dim:
        raise ValueError(f"head_dim mismatch: query {head_dim}, cache {cache_dim}")
    if not query.is_cuda:
        raise ValueError("paged_attention_hip needs GPU tensors (the HIP path has no CPU fallback)")
    device = query.device
    if k_cache.device != device or v_cache.device != device:
        raise ValueError("query and caches must be on the same device")
    if query.dtype != k_cache.dtype or v_cache.dtype != k_cache.dtype:
        raise TypeError(f"query/cache dtypes differ: {query.dtype}, {k_cache.dtype}, {v_cache.dtype}")
    if query.dtype not in _lib.DTYPE_CODES:
        raise TypeError(f"paged_attention_hip supports float32/float16/bfloat16, got {query.dtype}")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("caches must be contiguous [num_blocks, block_size, num_kv_heads, head_dim]")
    if md.num_tokens != num_tokens:
        raise ValueError(f"metadata has {md.num_tokens} tokens, query has {num_tokens}")

    q = query.contiguous()
    out = torch.empty_like(q)
    if num_tokens == 0 or md.num_seqs == 0:
        return out.view(query.shape)

    bt = _index(md.block_tables, "block_tables", device)
    if bt.dim() != 2 or bt.shape[0] < md.num_seqs:
        raise ValueError(f"block_tables must be [num_seqs, max_blocks], got {tuple(bt.shape)}")
    if bt.stride(1) != 1:
        bt = bt.contiguous()
    max_blk = (md.max_seq_len + block_size - 1) // block_size
    if bt.shape[1] < max_blk:
        raise ValueError(
            f"block_tables has {bt.shape[1]} columns but max_seq_len={md.max_seq_len} needs {max_blk}")
    sl = _index(md.seq_lens, "seq_lens", device).contiguous()
    decode_only = bool(md.is_decode_only)
    if decode_only:
        qsl_ptr, qsl64 = None, 0
        if num_tokens != md.num_seqs:
            raise ValueError("is_decode_only needs one query token per sequence")
    else:
        qsl = _index(md.query_start_loc, "query_start_loc", device).contiguous()
        qsl_ptr, qsl64 = qsl.data_ptr(), int(qsl.dtype == torch.int64)

    # The host copies of the lengths and query offsets let the library size
    # its grids exactly: one decode workgroup per split (longest sequences
    # first), and prefill key ranges split across the CUs.
    lens_host = None
    if md.seq_lens_cpu is not None:
        if len(md.seq_lens_cpu) < md.num_seqs:
            raise ValueError("seq_lens_cpu is shorter than num_seqs")
        lens_host = (ctypes.c_int64 * md.num_seqs)(*md.seq_lens_cpu[:md.num_seqs])
    qsl_host = None
    if not decode_only and md.query_start_loc_cpu is not None:
        if len(md.query_start_loc_cpu) < md.num_seqs + 1:
            raise ValueError("query_start_loc_cpu is shorter than num_seqs + 1")
        qsl_host = (ctypes.c_int64 * (md.num_seqs + 1))(*md.query_start_loc_cpu[:md.num_seqs + 1])

    stream = torch.cuda.current_stream(device).cuda_stream
    nbytes = lib.ns_paged_attention_workspace_size(
        md.num_seqs, num_heads, num_kv_heads, head_dim, block_size,
        md.max_seq_len, md.max_query_len, num_tokens, int(decode_only))
    if nbytes == 0:
        raise RuntimeError(
            f"unsupported attention shape: Hq={num_heads} Hkv={num_kv_heads} D={head_dim} "
            f"block_size={block_size}")
    ws = _workspace(device, stream, nbytes)
    generic = takes_generic_kernel(q.dtype, head_dim, block_size, num_heads // num_kv_heads)
    aux = (None, None, None) if decode_only or generic else _aux_stream(device, stream)
    plan = None
    # A batch whose host offsets show no one-row sequence has no decode rows:
    # the library launches no decode kernel and needs no plan.
    has_decode_rows = decode_only or qsl_host is None or lens_host is None or any(
        b - a == 1 for a, b in zip(md.query_start_loc_cpu[:md.num_seqs], md.query_start_loc_cpu[1:md.num_seqs + 1]))
    if share_plan and has_decode_rows and not generic:
        # Reuse md's plan only in the context that built it: eagerly, or inside
        # the same graph capture (whose replays rebuild it).  Anywhere else
        # this call builds the step's plan anew; a replaced plan that a
        # captured graph owns stays allocated for that graph.
        capture = _lib.stream_capture_id(stream) if torch.cuda.is_current_stream_capturing() else 0
        plan = md.decode_plan
        if plan is None or plan.capture != capture or \
                plan.key != _plan_key(md, num_kv_heads, head_dim, block_size, device):
            prepare_decode_plan(md, k_cache)  # this step's first call here (or md changed shape)
            plan = md.decode_plan

    rc = lib.ns_paged_attention(
        out.data_ptr(), q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
        bt.data_ptr(), bt.stride(0), bt.shape[1], int(bt.dtype == torch.int64),
        sl.data_ptr(), int(sl.dtype == torch.int64),
        qsl_ptr, qsl64,
        lens_host, 1,
        qsl_host, 1,
        md.num_seqs, num_tokens, md.max_query_len, md.max_seq_len, int(decode_only),
        num_heads, num_kv_heads, head_dim, block_size, num_blocks,
        float(scale), _lib.DTYPE_CODES[q.dtype],
        None if plan is None else plan.buffer.data_ptr(), 0 if plan is None else plan.buffer.numel(),
        ws.data_ptr(), ws.numel(), stream, *aux)
    _lib.check(rc, "ns_paged_attention")
    return out.view(query.shape)


# The per-step hook a forward calls once before its layers (Qwen2Model.forward).
paged_attention_hip.prepare = prepare_decode_plan


def get_attention_backend(name: str = "auto"):
    """Resolve a backend name to (callable, name) with attn_fn's signature.

    Mirrors reference attention.py:193-206, with one backend: "auto" and "hip"
    return the HIP path and raise if its library cannot be loaded.  The
    reference's "torch" (gather+SDPA) and "triton" backends are not product
    paths here and are rejected rather than silently substituted.
    """
    if name in ("auto", "hip"):
        _lib.load()
        return paged_attention_hip, "hip"
    if name in ("torch", "triton"):
        raise ValueError(
            f"attention backend {name!r} is not provided: nanoserve_amd runs paged attention "
            "only through its HIP kernels")
    raise ValueError(f"unknown attention backend {name!r}")
