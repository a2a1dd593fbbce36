"""A minimal continuous-batching engine around the HIP path.

Enough of the reference engine (nanoserve/engine.py, model_runner.py,
metrics.py) to run the end-to-end serving benchmark with the kernels inside
the model: requests join and leave the batch every step, prefill and decode
share one token budget, long prompts are prefilled in chunks, and when
blocks run out sequences are evicted and later recomputed (the scheduling
rules live in `scheduling.py`).  Sampling is greedy (the benchmark's
setting).  A step's metadata is built in scheduler order with int64 indices
in one host-to-device copy (model_runner.py:52-147); a sequence yields a
token only in the step that computes its last uncomputed token.
"""

from __future__ import annotations

import time
from dataclasses import dataclass

import numpy as np
import torch

from .attention import AttentionMetadata, get_attention_backend
from .block_manager import BlockSpaceManager
from .capture import no_cycle_collection
from .kv_cache import PagedKVCache
from .sampling import argmax_rows
from .scheduling import RequestMetrics, SamplingParams, Scheduler, SchedulerConfig, Sequence, SeqState

__all__ = ["DecodeGraphs", "LLMEngine", "ModelRunner", "RequestMetrics", "SamplingParams", "Scheduler",
           "SchedulerConfig", "Sequence", "SeqState", "summarize"]


class ModelRunner:
    """Scheduler decision -> metadata -> forward -> greedy tokens.

    With `use_graphs`, decode-only steps replay a HIP graph of the whole
    forward (embedding to greedy token) captured once per batch-size bucket;
    other steps run eagerly.  See `DecodeGraphs`.
    """

    def __init__(self, model, kv_cache: PagedKVCache, block_manager: BlockSpaceManager, device,
                 backend: str = "auto", use_graphs: bool = False, max_model_len: int = 4096,
                 graph_batch_sizes: tuple[int, ...] = (1, 2, 4, 8, 16, 24, 32, 48, 64)) -> None:
        self.model = model
        self.kv_cache = kv_cache
        self.block_manager = block_manager
        self.device = torch.device(device)
        self.block_size = kv_cache.block_size
        self.attn_fn, self.backend_name = get_attention_backend(backend)
        self._host: torch.Tensor | None = None
        self._dev: torch.Tensor | None = None
        self.graphs = DecodeGraphs(self, graph_batch_sizes, max_model_len) if use_graphs else None

    def _stage(self, chunks: list[list[int]]) -> list[torch.Tensor]:
        """All integer vectors in one pinned host buffer and one copy (model_runner.py:52-83)."""
        sizes = [len(c) for c in chunks]
        total = sum(sizes)
        if self._host is None or self._host.numel() < total:
            n = max(2 * total, 8192)
            self._host = torch.empty(n, dtype=torch.int64, pin_memory=self.device.type == "cuda")
            self._dev = torch.empty(n, dtype=torch.int64, device=self.device)
        flat = np.fromiter((v for c in chunks for v in c), dtype=np.int64, count=total)
        self._host[:total].copy_(torch.from_numpy(flat))
        self._dev[:total].copy_(self._host[:total])  # blocking: the buffer is reused next step
        views, off = [], 0
        for n in sizes:
            views.append(self._dev[off:off + n])
            off += n
        return views

    def build_inputs(self, scheduled):
        """(input_ids, positions, md, sample_indices or None, sample_seqs) for one step."""
        input_ids, positions, slots, seq_lens, query_lens = [], [], [], [], []
        qsl = [0]
        sample_indices, sample_seqs = [], []
        for seq, q in scheduled:
            start, end = seq.num_computed_tokens, seq.num_computed_tokens + q
            input_ids.extend(seq.token_slice(start, end))
            positions.extend(range(start, end))
            slots.extend(self.block_manager.slot_mapping(seq, start, end))
            qsl.append(qsl[-1] + q)
            seq_lens.append(end)
            query_lens.append(q)
            if end == seq.num_tokens:
                sample_indices.append(qsl[-1] - 1)
                sample_seqs.append(seq)
        max_seq_len = max(seq_lens)
        max_blocks = -(-max_seq_len // self.block_size)
        bt: list[int] = []
        for seq, _ in scheduled:
            row = seq.block_table[:max_blocks]
            bt.extend(row)
            bt.extend([0] * (max_blocks - len(row)))
        ids_t, pos_t, slot_t, qsl_t, sl_t, bt_t, samp_t = self._stage(
            [input_ids, positions, slots, qsl, seq_lens, bt, sample_indices])
        md = AttentionMetadata(
            slot_mapping=slot_t, query_start_loc=qsl_t, seq_lens=sl_t,
            block_tables=bt_t.view(len(scheduled), max_blocks),
            max_query_len=max(query_lens), max_seq_len=max_seq_len,
            num_seqs=len(scheduled), num_tokens=len(input_ids),
            is_decode_only=all(q == 1 for q in query_lens),
            query_lens_cpu=query_lens, seq_lens_cpu=seq_lens, query_start_loc_cpu=qsl)
        return ids_t, pos_t, md, (samp_t if sample_indices else None), sample_seqs

    @torch.inference_mode()
    def execute(self, scheduled) -> list[tuple[Sequence, int]]:
        if self.graphs is not None and self.graphs.covers(scheduled):
            return self.graphs.execute(scheduled)
        ids, pos, md, sample_idx, sample_seqs = self.build_inputs(scheduled)
        hidden = self.model(ids, pos, self.kv_cache, md, self.attn_fn)
        for seq, q in scheduled:
            seq.mark_computed(q)
        if sample_idx is None:
            return []
        logits = self.model.compute_logits(hidden, sample_idx)
        tokens = argmax_rows(logits).tolist()  # greedy; the step's one device-to-host sync
        return list(zip(sample_seqs, tokens))


class DecodeGraphs:
    """HIP graphs of the decode step, one per batch-size bucket.

    A decode step is ~12 launches per layer plus the logits; replaying a
    captured graph removes the per-launch host cost, which dominates at
    Qwen2.5-0.5B size.  Each graph reads its inputs from one static int64
    device buffer (token ids, positions, slots, lengths, block tables) that
    is refilled by a single host-to-device copy before the replay, and leaves
    the greedy tokens in a static output.  Batches are padded to the bucket
    with slot -1 (the cache write skips it) and length 1.

    The forward builds the step's decode plan on the device from the replayed
    lengths (attn_fn.prepare, once per step), so attention inside the graph is
    scheduled from the step's actual lengths.  Graphs are also keyed by a
    context bucket (powers of two up to max_model_len), which sets the width
    of the graph's block table and so the bytes the fill copies.

    `launch` and `tokens` split a step so that the engine can plan and launch
    the next step before reading this one's tokens back: the next step's input
    ids are then gathered on the device from this step's greedy output.  Two
    pinned staging buffers alternate, so filling step N+1 never overwrites the
    buffer step N's copy may still be reading.

    Lifetimes.  The object keeps the runner's model, cache and attention
    function but not the runner itself, so an engine and its graphs form no
    reference cycle and are freed as soon as the engine is dropped, not by a
    later cycle collection (which could otherwise run inside another graph's
    capture; see `capture.no_cycle_collection`).  Each graph is kept with the
    metadata it was captured with, so the step's decode-plan buffer -- a
    tensor of the graph's private pool that every replay rewrites and reads
    -- stays allocated for the graph's lifetime and is never handed to a
    later capture.
    """

    def __init__(self, runner: "ModelRunner", sizes: tuple[int, ...], max_model_len: int) -> None:
        self.model = runner.model
        self.kv_cache = runner.kv_cache
        self.attn_fn = runner.attn_fn
        self.block_size = runner.block_size
        self.device = runner.device
        self.sizes = sorted(sizes)
        self.max_model_len = max_model_len
        self.width = -(-max_model_len // runner.block_size)
        self.ctx_sizes = sorted({max_model_len >> k for k in range(4) if (max_model_len >> k) >= 256}
                                | {max_model_len})
        n = max(self.sizes)
        self._per = 5 * n + n * self.width  # ids, pos, slots, lens, gather rows, tables
        pin = runner.device.type == "cuda"
        self._host = [torch.zeros(self._per, dtype=torch.int64, pin_memory=pin) for _ in range(2)]
        self._host_np = [h.numpy() for h in self._host]
        self._tok = [torch.zeros(n, dtype=torch.int64, pin_memory=pin) for _ in range(2)]
        self._next = 0  # staging buffer of the next launch
        self._dev = torch.zeros(self._per, dtype=torch.int64, device=runner.device)
        # What each table row of a staging buffer holds: (table width, and per
        # row the block_table list written there and how many of its entries).
        # Tables only grow in place (BlockSpaceManager.allocate extends the
        # list; free installs a new one), so a row holding the same list keeps
        # valid entries and a decode step writes only blocks added since.
        # Holding the lists keeps their ids from reuse.
        self._rows: list[tuple[int, list[tuple[list, int]]]] = [(0, []), (0, [])]
        self._graphs: dict[tuple[int, int], CapturedStep] = {}
        self.last_logits: torch.Tensor | None = None  # graph-owned logits of the latest replay
        self._pool = None
        self._stream = torch.cuda.Stream(runner.device) if runner.device.type == "cuda" else None

    def covers(self, scheduled) -> bool:
        return (len(scheduled) <= self.sizes[-1] and all(q == 1 for _, q in scheduled)
                and all(s.num_tokens <= self.max_model_len for s, _ in scheduled))

    def _table_width(self, ctx: int) -> int:
        return -(-ctx // self.block_size)

    def _views(self, b: int, ctx: int):
        n, w = max(self.sizes), self._table_width(ctx)
        d = self._dev
        return (d[0:b], d[n:n + b], d[2 * n:2 * n + b], d[3 * n:3 * n + b],
                d[5 * n:5 * n + b * w].view(b, w))

    def _metadata(self, b: int, ctx: int) -> tuple[torch.Tensor, torch.Tensor, AttentionMetadata]:
        ids, pos, slots, lens, tables = self._views(b, ctx)
        md = AttentionMetadata(
            slot_mapping=slots, query_start_loc=None, seq_lens=lens, block_tables=tables,
            max_query_len=1, max_seq_len=ctx, num_seqs=b, num_tokens=b,
            is_decode_only=True, query_lens_cpu=None, seq_lens_cpu=None, query_start_loc_cpu=None)
        return ids, pos, md

    def _fill(self, scheduled, b: int, ctx: int, gather: list[int] | None) -> int:
        """Write the step's inputs for rows [0, b) into the next staging buffer
        and copy them to the device; returns the staging buffer used.

        Only what the graph reads is written: each row's token, position,
        slot and length, and its block-table entries up to its length
        (entries past a row's length are never read, so stale ones stay);
        padding rows get slot -1 (no cache write), length 1 and block 0.
        With `gather`, row i's token is not known on the host yet and is row
        gather[i] of the previous launch's greedy output."""
        n, bs, w = max(self.sizes), self.block_size, self._table_width(ctx)
        slot_i = self._next
        self._next ^= 1
        h = self._host_np[slot_i]
        ids, pos, slots, lens, rows_src = h[0:n], h[n:2 * n], h[2 * n:3 * n], h[3 * n:4 * n], h[4 * n:5 * n]
        tab = h[5 * n:5 * n + b * w].reshape(b, w)
        k = len(scheduled)
        ids[k:b] = 0
        pos[k:b] = 0
        slots[k:b] = -1
        lens[k:b] = 1
        tab[k:b, 0] = 0
        width, prev = self._rows[slot_i]
        prev = prev if width == w else []
        rows = []
        tok, at, slot = [], [], []
        for i, (seq, _) in enumerate(scheduled):
            p = seq.num_computed_tokens
            plen = len(seq.prompt_token_ids)
            bt = seq.block_table
            tok.append(seq.output_token_ids[p - plen] if p >= plen else seq.prompt_token_ids[p])
            at.append(p)
            slot.append(bt[p // bs] * bs + p % bs)
            nb = p // bs + 1
            have = prev[i][1] if i < len(prev) and prev[i][0] is bt else 0
            if nb > have:
                tab[i, have:nb] = bt[have:nb]
            rows.append((bt, max(nb, have)))
        self._rows[slot_i] = (w, rows)
        ids[:k] = tok if gather is None else 0
        pos[:k] = at
        slots[:k] = slot
        lens[:k] = at
        lens[:k] += 1
        if gather is not None:
            rows_src[:k] = gather
        end = 5 * n + b * w
        # Asynchronous: this staging buffer is written again two launches
        # later, after the engine has read back the tokens of the launch in
        # between, which comes after this copy on the stream.
        self._dev[:end].copy_(self._host[slot_i][:end], non_blocking=True)
        return slot_i

    def _capture(self, b: int, ctx: int):
        ids, pos, md = self._metadata(b, ctx)
        model, kv_cache, attn_fn = self.model, self.kv_cache, self.attn_fn

        def forward():
            hidden = model(ids, pos, kv_cache, md, attn_fn)
            logits = model.compute_logits(hidden)
            return argmax_rows(logits), logits

        s = self._stream
        s.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(s):  # warm-up: workspaces and allocator state for this stream
            forward()
            forward()
        s.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, pool=self._pool, stream=s):
            out, logits = forward()
        if self._pool is None:
            self._pool = g.pool()
        self._graphs[(b, ctx)] = CapturedStep(g, out, logits, md)

    def capture_all(self) -> None:
        """Capture every bucket up front, largest first (the pool then fits the rest).

        The cycle collector is held off for the whole sequence (pending
        garbage is collected first), so no destructor of unrelated objects
        runs inside a capture."""
        self._dev.zero_()
        self._dev[3 * max(self.sizes):4 * max(self.sizes)] = 1
        self._dev[2 * max(self.sizes):3 * max(self.sizes)] = -1
        with no_cycle_collection():
            for ctx in sorted(self.ctx_sizes, reverse=True):
                for b in sorted(self.sizes, reverse=True):
                    if (b, ctx) not in self._graphs:
                        self._capture(b, ctx)

    @torch.inference_mode()
    def launch(self, scheduled, after: "GraphLaunch | None" = None) -> "GraphLaunch":
        """Replay the step's graph; with `after`, every row's token comes from
        that earlier launch's greedy output (gathered on the device)."""
        b = next(x for x in self.sizes if x >= len(scheduled))
        longest = max(seq.num_computed_tokens + 1 for seq, _ in scheduled)
        ctx = next(c for c in self.ctx_sizes if c >= longest)
        if (b, ctx) not in self._graphs:
            self.capture_all()
        step = self._graphs[(b, ctx)]
        g, out, logits = step.graph, step.out, step.logits
        gather = None
        if after is not None:
            where = {seq.seq_id: i for i, (seq, _) in enumerate(after.scheduled)}
            gather = [where[seq.seq_id] for seq, _ in scheduled]
        slot_i = self._fill(scheduled, b, ctx, gather)
        k = len(scheduled)
        if after is not None:
            n = max(self.sizes)
            torch.index_select(after.out, 0, self._dev[4 * n:4 * n + k], out=self._dev[0:k])
        g.replay()
        self.last_logits = logits[:k]
        # The tokens leave the graph's output before a later replay of the
        # same graph can overwrite it.
        tok = self._tok[slot_i]
        tok[:k].copy_(out[:k], non_blocking=True)
        done = torch.cuda.Event()
        done.record()
        return GraphLaunch(list(scheduled), out, tok, done)

    def tokens(self, launch: "GraphLaunch") -> list[int]:
        launch.done.synchronize()
        return launch.tokens_host[:len(launch.scheduled)].tolist()

    def execute(self, scheduled) -> list[tuple[Sequence, int]]:
        launch = self.launch(scheduled)
        tokens = self.tokens(launch)
        for seq, q in scheduled:
            seq.mark_computed(q)
        return [(seq, tok) for (seq, _), tok in zip(scheduled, tokens)]


@dataclass
class CapturedStep:
    """One captured decode step: the graph, its static outputs, and the
    metadata (with the decode-plan buffer) its kernels were captured with."""

    graph: torch.cuda.CUDAGraph
    out: torch.Tensor        # greedy token per row
    logits: torch.Tensor     # [bucket, vocab]
    md: AttentionMetadata    # keeps md.decode_plan's buffer allocated


@dataclass
class GraphLaunch:
    """A replayed decode step whose tokens may not have been read back yet."""

    scheduled: list
    out: torch.Tensor          # the graph's greedy output (device)
    tokens_host: torch.Tensor  # pinned copy of it, valid once `done` has completed
    done: torch.cuda.Event


class LLMEngine:
    """add_request / step / run_all over a model, a paged cache and the scheduler."""

    def __init__(self, model, num_blocks: int, block_size: int = 16, device="cuda",
                 scheduler_config: SchedulerConfig | None = None, eos_token_id: int | None = None,
                 max_model_len: int = 4096, use_graphs: bool = False, pipeline_decode: bool = True) -> None:
        self.model = model.eval().requires_grad_(False)
        self.device = torch.device(device)
        dtype = model.model.embed_tokens.weight.dtype
        self.kv_cache = PagedKVCache(num_blocks, block_size, model.num_layers, model.num_kv_heads,
                                     model.head_dim, dtype, device)
        self.block_manager = BlockSpaceManager(block_size, num_blocks, watermark=0.0)
        self.scheduler = Scheduler(scheduler_config or SchedulerConfig(), self.block_manager)
        self.runner = ModelRunner(model, self.kv_cache, self.block_manager, device,
                                  use_graphs=use_graphs, max_model_len=max_model_len)
        self.eos_token_id = eos_token_id
        self.max_model_len = max_model_len
        self._next_id = 0
        self.finished: list[Sequence] = []
        # A graph-replayed decode step whose tokens have not been read back.
        self._inflight: GraphLaunch | None = None
        self.pipeline_decode = pipeline_decode

    def add_request(self, prompt_token_ids: list[int], sampling: SamplingParams | None = None) -> int:
        sampling = sampling or SamplingParams()
        if len(prompt_token_ids) + sampling.max_new_tokens > self.max_model_len:
            raise ValueError("request exceeds max_model_len")
        seq = Sequence(self._next_id, list(prompt_token_ids), sampling)
        self._next_id += 1
        self.scheduler.add(seq)
        return seq.seq_id

    @property
    def has_unfinished_requests(self) -> bool:
        return self.scheduler.has_work or self._inflight is not None

    def _pipelines(self, scheduled) -> bool:
        """A decode step can be launched before the previous step's tokens are
        read back when it replays a graph and no sequence in it can stop on a
        token value: stops then depend on lengths alone, so the schedule does
        not depend on the tokens."""
        g = self.runner.graphs
        return (self.pipeline_decode and g is not None and g.covers(scheduled)
                and (self.eos_token_id is None or all(s.sampling.ignore_eos for s, _ in scheduled)))

    def _record(self, seq: Sequence, now: float) -> None:
        m = seq.metrics
        if m.first_token == 0.0:
            m.first_token = now
        m.output_tokens = len(seq.output_token_ids)
        m.end = now

    def _run(self, scheduled) -> list[Sequence]:
        results = self.runner.execute(scheduled)
        now = time.perf_counter()
        for seq, tok in results:
            seq.output_token_ids.append(tok)
            self._record(seq, now)
            seq.check_done(self.eos_token_id)
        done = self.scheduler.free_finished()
        self.finished.extend(done)
        return done

    def step(self) -> list[Sequence]:
        """One scheduling step.  Decode steps that replay a graph are pipelined:
        step N is launched, its sequences are advanced with placeholder tokens
        (stops by length only), step N+1 is scheduled and launched with its
        input ids gathered on the device from step N's output, and only then
        are step N's tokens read back into the placeholders.  Token values and
        order are those of the unpipelined engine."""
        pending, self._inflight = self._inflight, None
        done: list[Sequence] = []
        held: list[int] = []
        if pending is not None:
            for seq, _ in pending.scheduled:
                seq.mark_computed(1)
                seq.output_token_ids.append(-1)  # placeholder until the tokens are read back
                held.append(len(seq.output_token_ids) - 1)
                seq.check_done(None)
            done = self.scheduler.free_finished()
            self.finished.extend(done)
        sched = self.scheduler.schedule()
        nxt = None
        if sched and self._pipelines(sched.scheduled):
            if pending is None:
                nxt = self.runner.graphs.launch(sched.scheduled)
            elif {s.seq_id for s, _ in sched.scheduled} <= {s.seq_id for s, _ in pending.scheduled}:
                nxt = self.runner.graphs.launch(sched.scheduled, after=pending)
        if pending is not None:
            tokens = self.runner.graphs.tokens(pending)
            now = time.perf_counter()
            for (seq, _), at, tok in zip(pending.scheduled, held, tokens):
                seq.output_token_ids[at] = tok
                self._record(seq, now)
        if nxt is not None:
            self._inflight = nxt
        elif sched:
            done += self._run(sched.scheduled)
        return done

    def run_all(self) -> list[Sequence]:
        out: list[Sequence] = []
        while self.has_unfinished_requests:
            out.extend(self.step())
        return sorted(out, key=lambda s: s.seq_id)


def summarize(records: list[RequestMetrics], wall_time: float) -> dict:
    """Throughput over wall time and TTFT/TPOT/E2E percentiles (reference metrics.py:45-78)."""
    def pct(v, q):
        return float(np.percentile(v, q)) if len(v) else 0.0

    ttft = [r.ttft * 1e3 for r in records]
    tpot = [r.tpot * 1e3 for r in records if r.output_tokens > 1]
    e2e = [r.e2e * 1e3 for r in records]
    out_tok = sum(r.output_tokens for r in records)
    in_tok = sum(r.prompt_tokens for r in records)
    res = {
        "num_requests": len(records),
        "wall_time_s": wall_time,
        "prompt_tokens": in_tok,
        "output_tokens": out_tok,
        "output_tok_per_s": out_tok / wall_time if wall_time else 0.0,
        "total_tok_per_s": (in_tok + out_tok) / wall_time if wall_time else 0.0,
    }
    for name, v in (("ttft", ttft), ("tpot", tpot), ("e2e", e2e)):
        res[f"{name}_mean_ms"] = float(np.mean(v)) if v else 0.0
        for q in (50, 90, 99):
            res[f"{name}_p{q}_ms"] = pct(v, q)
    return res
