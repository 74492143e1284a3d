"""Iteration-level (continuous batching) scheduler, host side.

Counterpart of the reference's Scheduler (src/tinybatch/scheduler.py:71-154):
every running sequence decodes one token per step; waiting requests are
admitted first come first served while the step's token budget, the running
cap and the pool allow (scheduler.py:112-130); a decode that cannot get a
slot preempts the youngest running sequence, whose blocks are freed and which
restarts from its prompt (scheduler.py:92-110,141-154). With
``preemption="swap"`` the preempted sequence keeps its tokens instead: the
blocks holding its written positions are listed for a swap-out to host
memory (the engine runs it before the step's forward, so blocks reused in the
same step are read first), and it resumes, before any new admission, in fresh
blocks filled by a swap-in.

One deliberate difference: the decode slot is reserved for the position the
step writes. The engine writes the last sampled token at position
context_len - 1 (reference engine.py:116-117), while the reference reserves
room for index len(all_token_ids) (scheduler.py:97 with
block_manager.py:133-134), one position later. For a prompt whose length is a
multiple of the block size that leaves the first decode without a block for
its position (the reference raises IndexError in kv_cache.py:35). Here the
slot is reserved for all_token_ids()[:-1], i.e. index context_len - 1.
"""
from __future__ import annotations

import itertools
import time
from dataclasses import dataclass, field
from enum import Enum

from .block_manager import BlockManager, OutOfBlocks
from .config import EngineConfig

_ids = itertools.count()


class Status(Enum):
    WAITING = "waiting"
    RUNNING = "running"
    SWAPPED = "swapped"
    FINISHED = "finished"


@dataclass
class Request:
    prompt_token_ids: list[int]
    max_new_tokens: int
    temperature: float = 0.0
    top_p: float = 1.0
    req_id: int = field(default_factory=lambda: next(_ids))
    arrival_time: float = field(default_factory=time.perf_counter)
    status: Status = Status.WAITING
    output_token_ids: list[int] = field(default_factory=list)
    block_table: list[int] = field(default_factory=list)
    num_cached_tokens: int = 0
    first_token_time: float | None = None
    finish_time: float | None = None
    preemptions: int = 0
    swap_blocks: int = 0                    # blocks held in host memory while swapped
    swap_staging: object = field(default=None, repr=False)   # the host copy (set by the engine)

    def all_token_ids(self) -> list[int]:
        return self.prompt_token_ids + self.output_token_ids

    def context_len(self) -> int:
        return len(self.prompt_token_ids) + len(self.output_token_ids)

    def last_token_id(self) -> int:
        return self.output_token_ids[-1] if self.output_token_ids else self.prompt_token_ids[-1]


@dataclass
class ScheduledBatch:
    prefill: list[Request]
    decode: list[Request]
    swap_out: list[tuple[Request, list[int]]] = field(default_factory=list)   # (request, pool blocks to save)
    swap_in: list[tuple[Request, list[int]]] = field(default_factory=list)    # (request, pool blocks to fill)

    def is_empty(self) -> bool:
        return not self.prefill and not self.decode


class Scheduler:
    def __init__(self, config: EngineConfig, block_manager: BlockManager):
        self.cfg = config
        self.bm = block_manager
        self.waiting: list[Request] = []
        self.running: list[Request] = []
        self.swapped: list[Request] = []
        if config.preemption not in ("recompute", "swap"):
            raise ValueError(f"unknown preemption mode {config.preemption!r}")
        self._swap_out: list[tuple[Request, list[int]]] = []

    def add(self, req: Request) -> None:
        self.waiting.append(req)

    def has_work(self) -> bool:
        return bool(self.waiting or self.running or self.swapped)

    def _reserve_decode_slot(self, req: Request) -> None:
        # room for the position this step writes: context_len - 1
        self.bm.append_slot(req.block_table, req.all_token_ids()[:-1])

    def schedule(self) -> ScheduledBatch:
        budget = self.cfg.max_batch_tokens
        self._swap_out = []
        decode: list[Request] = []
        for req in list(self.running):
            if req.status is not Status.RUNNING:
                continue                                  # preempted earlier in this pass
            try:
                self._reserve_decode_slot(req)
            except OutOfBlocks:
                if self._preempt_youngest() is req:
                    continue
                try:
                    self._reserve_decode_slot(req)
                except OutOfBlocks:
                    self._preempt(req)
                    continue
            decode.append(req)
            budget -= 1
        decode = [r for r in decode if r.status is Status.RUNNING]

        swap_in: list[tuple[Request, list[int]]] = []
        while self.swapped and not self._swap_out and budget > 0 and len(self.running) < self.cfg.max_running:
            req = self.swapped[0]
            need = req.swap_blocks + (1 if (req.context_len() - 1) % self.bm.block_size == 0 else 0)
            if need > self.bm.num_free():
                break
            self.swapped.pop(0)
            req.block_table = self.bm.allocate_private(req.swap_blocks, req.all_token_ids()[:-1])
            self._reserve_decode_slot(req)
            req.status = Status.RUNNING
            self.running.append(req)
            swap_in.append((req, req.block_table[:req.swap_blocks]))
            decode.append(req)
            budget -= 1
        if self.swapped:
            # swapped sequences resume first: no new admission while any waits
            return ScheduledBatch(prefill=[], decode=decode, swap_out=self._swap_out, swap_in=swap_in)

        prefill: list[Request] = []
        while self.waiting and len(self.running) < self.cfg.max_running:
            req = self.waiting[0]
            n = len(req.prompt_token_ids)                 # upper bound before prefix hits
            if n > budget or self.bm.blocks_needed(n) > self.bm.num_free():
                break
            self.waiting.pop(0)
            req.block_table, req.num_cached_tokens = self.bm.allocate_prompt(req.prompt_token_ids)
            if req.num_cached_tokens >= n:                # the last prompt token's logits are needed
                req.num_cached_tokens = n - 1
            req.status = Status.RUNNING
            self.running.append(req)
            prefill.append(req)
            budget -= n - req.num_cached_tokens
        return ScheduledBatch(prefill=prefill, decode=decode, swap_out=self._swap_out, swap_in=swap_in)

    def finish(self, req: Request) -> None:
        req.status = Status.FINISHED
        req.finish_time = time.perf_counter()
        self.running.remove(req)
        self.bm.free_table(req.block_table)
        req.block_table = []

    def _preempt(self, req: Request) -> None:
        req.preemptions += 1
        self.running.remove(req)
        if self.cfg.preemption == "swap" and req.output_token_ids:
            # keep the tokens: positions 0 .. context_len - 2 are written, the last
            # sampled token is written by the step that resumes it
            written = req.context_len() - 1
            req.swap_blocks = self.bm.blocks_needed(written)
            self._swap_out.append((req, list(req.block_table[:req.swap_blocks])))
            self.bm.free_table(req.block_table)
            req.block_table = []
            req.status = Status.SWAPPED
            self.swapped.insert(0, req)
            return
        req.status = Status.WAITING
        self.bm.free_table(req.block_table)
        req.block_table = []
        req.output_token_ids = []                         # recompute from the prompt
        req.num_cached_tokens = 0
        self.waiting.insert(0, req)

    def _preempt_youngest(self) -> Request:
        victim = self.running[-1]
        self._preempt(victim)
        return victim
