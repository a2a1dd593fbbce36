"""Request state and the continuous-batching scheduler of the engine harness.

Config 5 is a workload of the reference engine, so which sequences run
together in a step, when a prompt is cut into chunks and who loses its cache
blocks under memory pressure follow the reference's rules
(nanoserve/scheduler.py:91-262, sequence.py:29-145):

1. A step has a token budget (`max_num_batched_tokens`).  Running sequences
   are served first, in admission order, each granted
   min(tokens still without KV, budget left).  Without chunked prefill a
   prompt is granted whole or not at all in this step.
2. A grant needs cache blocks up to its last token.  While the cache cannot
   provide them, the most recently admitted running sequence that holds no
   grant in this step is evicted: its blocks are freed, its KV will be
   recomputed, and it goes to the head of the queue.  When nobody is left to
   evict, a request larger than the whole cache is an error and otherwise
   the requester itself is evicted.
3. Queued requests are then admitted in arrival order while budget, the
   sequence cap and blocks outside the watermark allow; admission stops at a
   request evicted in the same step.

A sequence produces a token only in the step that computes its last token
without KV; evicted sequences keep their generated tokens and recompute them
as part of their next prefill.
"""

from __future__ import annotations

import enum
import time
from collections import deque
from dataclasses import dataclass, field

from .block_manager import BlockSpaceManager


@dataclass
class SamplingParams:
    max_new_tokens: int = 16
    ignore_eos: bool = False


PREEMPTION_MODES = ("recompute", "none")


@dataclass
class SchedulerConfig:
    """Step budget, sequence cap, prompt chunking and what happens when the
    cache runs out of blocks (reference config.py:68-83).

    preemption_mode "recompute" evicts as rule 2 of the module docstring says;
    "none" evicts nobody, so a grant the cache cannot hold stops the engine
    with a RuntimeError (the reference's ablation, scheduler.py:213-243).
    """

    max_num_batched_tokens: int = 2048
    max_num_seqs: int = 64
    enable_chunked_prefill: bool = True
    preemption_mode: str = "recompute"

    def __post_init__(self) -> None:
        if self.preemption_mode not in PREEMPTION_MODES:
            raise ValueError(f"preemption_mode must be one of {PREEMPTION_MODES}, got {self.preemption_mode!r}")


class SeqState(enum.Enum):
    QUEUED = "queued"
    RUNNING = "running"
    EVICTED = "evicted"          # blocks taken back; queued for recompute
    DONE_LENGTH = "done_length"  # reached max_new_tokens
    DONE_EOS = "done_eos"        # produced the end-of-sequence token

    @property
    def done(self) -> bool:
        return self is SeqState.DONE_LENGTH or self is SeqState.DONE_EOS


@dataclass
class RequestMetrics:
    """Timestamps of one request (perf_counter seconds) and its derived
    latencies, as the reference reports them (metrics.py:10-38)."""

    request_id: int
    prompt_tokens: int
    arrival: float
    start: float = 0.0
    first_token: float = 0.0
    end: float = 0.0
    output_tokens: int = 0

    @property
    def ttft(self) -> float:
        return self.first_token - self.arrival

    @property
    def e2e(self) -> float:
        return self.end - self.arrival

    @property
    def tpot(self) -> float:
        """Mean seconds per output token after the first."""
        return 0.0 if self.output_tokens <= 1 else (self.end - self.first_token) / (self.output_tokens - 1)


class Sequence:
    """Tokens, cache blocks and progress of one request.

    `num_computed_tokens` counts the leading tokens (prompt, then outputs)
    whose K/V are in the cache; the rest are fed to the model in later steps.
    Identity, not value, tells two sequences apart (the scheduler looks them
    up in its lists).
    """

    __slots__ = ("seq_id", "prompt_token_ids", "output_token_ids", "sampling", "state", "block_table",
                 "num_computed_tokens", "num_evictions", "metrics")

    def __init__(self, seq_id: int, prompt_token_ids: list[int], sampling: SamplingParams,
                 arrival: float | None = None) -> None:
        self.seq_id = seq_id
        self.prompt_token_ids = prompt_token_ids
        self.output_token_ids: list[int] = []
        self.sampling = sampling
        self.state = SeqState.QUEUED
        self.block_table: list[int] = []
        self.num_computed_tokens = 0
        self.num_evictions = 0
        t = time.perf_counter() if arrival is None else arrival
        self.metrics = RequestMetrics(seq_id, len(prompt_token_ids), t)

    def __repr__(self) -> str:
        return (f"Sequence({self.seq_id}, {self.state.value}, prompt={len(self.prompt_token_ids)}, "
                f"out={len(self.output_token_ids)}, computed={self.num_computed_tokens})")

    @property
    def prompt_len(self) -> int:
        return len(self.prompt_token_ids)

    @property
    def num_tokens(self) -> int:
        return len(self.prompt_token_ids) + len(self.output_token_ids)

    @property
    def pending_tokens(self) -> int:
        """Tokens whose K/V are not in the cache yet."""
        return self.num_tokens - self.num_computed_tokens

    @property
    def in_prompt(self) -> bool:
        """Whether some prompt token still lacks K/V (the sequence prefills)."""
        return self.num_computed_tokens < len(self.prompt_token_ids)

    def token_slice(self, start: int, end: int) -> list[int]:
        """Token ids at positions [start, end) of prompt + outputs."""
        n = len(self.prompt_token_ids)
        head = self.prompt_token_ids[start:min(end, n)] if start < n else []
        tail = self.output_token_ids[max(start - n, 0):end - n] if end > n else []
        return head + tail

    def mark_computed(self, n: int) -> None:
        if self.num_computed_tokens + n > self.num_tokens:
            raise ValueError(f"sequence {self.seq_id}: {n} more computed tokens exceed its "
                             f"{self.num_tokens} tokens ({self.num_computed_tokens} computed)")
        self.num_computed_tokens += n

    def check_done(self, eos_token_id: int | None) -> bool:
        """Mark the sequence done after its latest token if a stop condition holds."""
        if len(self.output_token_ids) >= self.sampling.max_new_tokens:
            self.state = SeqState.DONE_LENGTH
        elif (eos_token_id is not None and not self.sampling.ignore_eos and self.output_token_ids
              and self.output_token_ids[-1] == eos_token_id):
            self.state = SeqState.DONE_EOS
        return self.state.done


@dataclass
class SchedulerOutput:
    """One step's grants, in the order the runner lays the batch out."""

    scheduled: list[tuple[Sequence, int]] = field(default_factory=list)
    preempted: list[Sequence] = field(default_factory=list)  # evicted during this step
    num_prefill_seqs: int = 0
    num_decode_seqs: int = 0
    num_batched_tokens: int = 0

    def __bool__(self) -> bool:
        return bool(self.scheduled)


class Scheduler:
    """Grants each step's token budget to running and queued sequences (rules in the module docstring)."""

    def __init__(self, cfg: SchedulerConfig, block_manager: BlockSpaceManager) -> None:
        self.cfg = cfg
        self.blocks = block_manager
        self.waiting: deque[Sequence] = deque()
        self.running: list[Sequence] = []
        self.num_preemptions = 0

    def add(self, seq: Sequence) -> None:
        seq.state = SeqState.QUEUED
        self.waiting.append(seq)

    @property
    def has_work(self) -> bool:
        return bool(self.waiting) or bool(self.running)

    def schedule(self) -> SchedulerOutput:
        step = SchedulerOutput()
        left = self._serve_running(step, self.cfg.max_num_batched_tokens)
        self._admit_queued(step, left)
        # Classified now: the runner advances num_computed_tokens afterwards.
        for seq, n in step.scheduled:
            step.num_batched_tokens += n
            if seq.in_prompt:
                step.num_prefill_seqs += 1
            else:
                step.num_decode_seqs += 1
        return step

    def free_finished(self) -> list[Sequence]:
        """Drop finished sequences from the running set and return their blocks."""
        finished = [s for s in self.running if s.state.done]
        if finished:
            self.running = [s for s in self.running if not s.state.done]
            for s in finished:
                self.blocks.free(s)
        return finished

    # -- internals ---------------------------------------------------------
    def _grant_size(self, seq: Sequence, left: int) -> int:
        """Tokens `seq` may take from `left`; 0 when an unchunked prompt does not fit."""
        if self.cfg.enable_chunked_prefill or not seq.in_prompt:
            return min(seq.pending_tokens, left)
        whole = seq.pending_tokens
        if whole > self.cfg.max_num_batched_tokens:
            raise ValueError(f"request {seq.seq_id}: a {whole}-token prompt can never fit "
                             f"max_num_batched_tokens={self.cfg.max_num_batched_tokens} unchunked; "
                             "enable chunked prefill")
        return whole if whole <= left else 0

    def _serve_running(self, step: SchedulerOutput, left: int) -> int:
        admitted_order = list(self.running)
        granted: set[int] = set()
        for seq in admitted_order:
            if seq.state is not SeqState.RUNNING or left <= 0:
                continue  # evicted earlier in this step, or no budget left (stays running)
            n = self._grant_size(seq, left)
            if n and self._reserve_blocks(seq, seq.num_computed_tokens + n, admitted_order, granted, step):
                step.scheduled.append((seq, n))
                granted.add(seq.seq_id)
                left -= n
        self.running = [s for s in admitted_order if s.state is SeqState.RUNNING]
        return left

    def _reserve_blocks(self, seq: Sequence, upto: int, admitted_order: list[Sequence], granted: set[int],
                        step: SchedulerOutput) -> bool:
        """Blocks for positions [0, upto) of `seq`, evicting newer sequences as needed."""
        evicting = self.cfg.preemption_mode == "recompute"
        while not self.blocks.allocate(seq, upto):
            victim = None
            for cand in reversed(admitted_order) if evicting else ():
                if cand is not seq and cand.state is SeqState.RUNNING and cand.seq_id not in granted:
                    victim = cand
                    break
            if victim is None:
                usable = self.blocks.num_total_blocks - self.blocks.watermark_blocks
                needed = self.blocks.blocks_for(upto)
                if needed > usable:
                    raise ValueError(f"request {seq.seq_id} cannot fit the KV cache: {upto} tokens need "
                                     f"{needed} blocks of {self.blocks.block_size}, {usable} are usable")
                if not evicting:
                    raise RuntimeError(
                        f"KV cache exhausted with preemption_mode='none': sequence {seq.seq_id} needs blocks "
                        f"up to token {upto}, and the {len(self.running)} running sequences hold all "
                        f"{self.blocks.num_total_blocks} blocks")
                self._evict(seq, step)
                return False
            self._evict(victim, step)
        return True

    def _admit_queued(self, step: SchedulerOutput, left: int) -> None:
        evicted_now = {s.seq_id for s in step.preempted}
        while self.waiting and left > 0 and len(self.running) < self.cfg.max_num_seqs:
            seq = self.waiting[0]
            if seq.seq_id in evicted_now:
                break  # re-admitting it would take back the blocks just freed
            n = self._grant_size(seq, left)
            upto = seq.num_computed_tokens + n
            if n == 0 or not self.blocks.can_allocate(seq, upto) or not self.blocks.allocate(seq, upto):
                break
            self.waiting.popleft()
            seq.state = SeqState.RUNNING
            if not seq.metrics.start:
                seq.metrics.start = time.perf_counter()
            self.running.append(seq)
            step.scheduled.append((seq, n))
            left -= n

    def _evict(self, seq: Sequence, step: SchedulerOutput) -> None:
        """Recompute-style eviction: free the blocks, forget the KV, requeue first."""
        self.blocks.free(seq)
        seq.num_computed_tokens = 0
        seq.state = SeqState.EVICTED
        seq.num_evictions += 1
        self.num_preemptions += 1
        step.preempted.append(seq)
        self.waiting.appendleft(seq)
