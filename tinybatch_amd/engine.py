"""The engine: schedule -> one flat-batch forward -> sample (token ids in and out).

Counterpart of LLMEngine (reference src/tinybatch/engine.py:32-171) without a
tokenizer: requests carry token ids, outputs are token ids. One ``step`` runs
one iteration of continuous batching: prefills of newly admitted requests
(their uncached prompt tokens) followed by one decode token for every running
sequence, in that order in the flat batch (engine.py:99-120), then greedy
(or temperature / top-p) sampling of each sequence's next token
(engine.py:145-159).

MI355X-side choices: the step's metadata is built once and shared by all
layers (the cache object memoises it on the positions tensor); greedy rows
are sampled by one batched argmax and one device-to-host copy instead of one
``int()`` synchronisation per sequence; greedy decode-only steps replay a
captured HIP graph of the whole forward (DecodeGraphs) instead of issuing
its launches one by one.

Pipelined decode (EngineConfig.pipeline_decode): while the batch is steady -
nothing waiting or swapped, every running request greedy, a free block for
each - a graph step is queued before the previous one's tokens are on the
host. Its rows read their input tokens from the previous step's ids on the
device; on the host each request gets a placeholder token (PENDING) that the
previous step's ids replace once collected, one step later, so the scheduler
sees the right context lengths throughout. A request that reaches its token
budget finishes at launch (its last token is on the way; blocks freed now are
only reused by later steps, which the stream orders behind this one). A stop
token seen at collection ends its request there and drops the placeholder of
the step already queued for it (that step computed one row more than a
synchronous run would have; rows do not interact). Anything else drains the
pipeline first and runs the synchronous step.
"""
from __future__ import annotations

import time
from dataclasses import dataclass, field

import torch

from . import ops
from .block_manager import BlockManager
from .config import EngineConfig
from .decode_graphs import DecodeGraphs, MergeErrors
from .kv_cache import PagedKVCache
from .model import ModelConfig, Qwen2Paged
from .scheduler import Request, Scheduler, Status

PENDING = -1    # placeholder of a token still on the device


@dataclass
class StepOutput:
    req_id: int
    token_id: int
    finished: bool
    request: Request = field(repr=False)


class LLMEngine:
    def __init__(self, config: EngineConfig | None = None, model_config: ModelConfig | None = None,
                 model: Qwen2Paged | None = None):
        self.cfg = config or EngineConfig()
        self.device = torch.device(self.cfg.device)
        self.dtype = getattr(torch, self.cfg.dtype)
        self.model = model or Qwen2Paged(model_config or ModelConfig.qwen2_0_5b(), self.device, self.dtype,
                                         seed=self.cfg.seed)
        mc = self.model.cfg
        self.kv_cache = PagedKVCache(mc.n_layers, self.cfg.num_blocks, self.cfg.block_size, mc.n_kv_heads,
                                     mc.head_dim, self.device, self.dtype)
        self.block_manager = BlockManager(self.cfg.num_blocks, self.cfg.block_size, self.cfg.enable_prefix_caching)
        self.scheduler = Scheduler(self.cfg, self.block_manager)
        self.eos_ids = set(self.cfg.stop_token_ids)
        self.steps = 0
        self.last_step_prefills = 0
        self.graph_steps = 0
        self.pipelined_steps = 0
        self.merge_failures = 0         # eager steps recomputed after an in-launch merge error
        self.graphs = (DecodeGraphs(self.model, self.kv_cache, self.cfg.max_running, self.cfg.max_model_len)
                       if self.cfg.decode_graphs else None)
        self.swap_outs = 0
        self.swap_ins = 0
        self._swap_reads: list[torch.Tensor] = []   # host copies read by the last step's swap-ins
        self._inflight: dict | None = None           # the queued graph step whose tokens are not collected

    # ---- API -----------------------------------------------------------------
    def add_request(self, prompt_token_ids: list[int], *, max_new_tokens: int | None = None,
                    temperature: float | None = None, top_p: float | None = None) -> Request:
        ids = list(prompt_token_ids)[: self.cfg.max_model_len - 1]
        if not ids:
            raise ValueError("empty prompt")
        req = Request(prompt_token_ids=ids,
                      max_new_tokens=self.cfg.max_new_tokens if max_new_tokens is None else max_new_tokens,
                      temperature=self.cfg.temperature if temperature is None else temperature,
                      top_p=self.cfg.top_p if top_p is None else top_p)
        self.scheduler.add(req)
        return req

    def generate(self, prompts: list[list[int]], **kw) -> list[list[int]]:
        reqs = [self.add_request(p, **kw) for p in prompts]
        while self.has_work():
            self.step()
        return [r.output_token_ids for r in reqs]

    # ---- one iteration ---------------------------------------------------------
    @staticmethod
    def build_step(prefill: list[Request], decode: list[Request]):
        """Flat-batch inputs of a step (engine.py:99-120)."""
        token_ids: list[int] = []
        positions: list[int] = []
        seq_slices: list[tuple[int, int]] = []
        block_tables: list[list[int]] = []
        context_lens: list[int] = []
        for req in prefill:
            start = len(token_ids)
            token_ids.extend(req.prompt_token_ids[req.num_cached_tokens:])
            positions.extend(range(req.num_cached_tokens, len(req.prompt_token_ids)))
            seq_slices.append((start, len(token_ids)))
            block_tables.append(req.block_table)
            context_lens.append(len(req.prompt_token_ids))
        for req in decode:
            start = len(token_ids)
            token_ids.append(req.last_token_id())
            positions.append(req.context_len() - 1)
            seq_slices.append((start, len(token_ids)))
            block_tables.append(req.block_table)
            context_lens.append(req.context_len())
        return token_ids, positions, seq_slices, block_tables, context_lens

    def _swap(self, batch) -> None:
        """Run the step's swaps on the compute stream, ahead of its forward: swap-outs
        read blocks that this step may hand to others, swap-ins fill the blocks the
        resumed sequences decode from (K3 gather / scatter to pinned host memory)."""
        self._swap_reads = []          # the previous step ended with a synchronising copy
        for req, blocks in batch.swap_out:
            staging = torch.empty((self.model.cfg.n_layers, len(blocks)) + tuple(self.kv_cache.pools[0].shape[1:]),
                                  dtype=self.dtype, pin_memory=True)
            self.kv_cache.swap_out(blocks, list(staging))
            req.swap_staging = staging
            self.swap_outs += 1
        for req, blocks in batch.swap_in:
            self.kv_cache.swap_in(list(req.swap_staging), blocks)
            self._swap_reads.append(req.swap_staging)
            req.swap_staging = None
            self.swap_ins += 1

    def has_work(self) -> bool:
        return self.scheduler.has_work() or self._inflight is not None

    def step(self) -> list[StepOutput]:
        """One iteration. Pipelined decode steps return the outputs of the step
        queued before them (tokens arrive one call late); other steps first
        collect a queued step and return its outputs ahead of their own."""
        if self._can_pipeline():
            return self._step_pipelined()
        outs = self._collect(self._inflight) if self._inflight is not None else []
        return outs + self._step_sync()

    def _can_pipeline(self) -> bool:
        sch = self.scheduler
        return (self.cfg.pipeline_decode and self.graphs is not None and not sch.waiting and not sch.swapped
                and bool(sch.running) and self.graphs.bucket(len(sch.running)) is not None
                and self.block_manager.num_free() >= len(sch.running)      # no preemption this step
                and all(r.temperature <= 0.0 for r in sch.running))

    def _step_pipelined(self) -> list[StepOutput]:
        batch = self.scheduler.schedule()
        if batch.prefill or batch.swap_out or batch.swap_in or len(batch.decode) != len(self.scheduler.running):
            raise RuntimeError("a steady decode batch was expected")
        ordered = batch.decode
        prev = self._inflight
        row_of = prev["row_of"] if prev is not None else {}
        src = [row_of.get(r.req_id, -1) for r in ordered]
        tokens = [0 if s >= 0 else r.last_token_id() for r, s in zip(ordered, src)]
        ctx = [r.context_len() for r in ordered]
        handle = self.graphs.launch(tokens, [c - 1 for c in ctx], [r.block_table for r in ordered], ctx,
                                    src_rows=src)
        if handle is None:
            # two rows on one slot (the graph's fused append cannot serve it): collect the
            # queued step, whose tokens these rows take as input, then run the rows unfused
            outs = self._collect(prev) if prev is not None else []
            return outs + self._run([], [r for r in ordered if r.status is Status.RUNNING], graphs=False)
        self.graph_steps += 1
        self.pipelined_steps += 1
        self.last_step_prefills = 0
        idx = []
        for r in ordered:
            r.output_token_ids.append(PENDING)
            idx.append(len(r.output_token_ids) - 1)
            if len(r.output_token_ids) >= r.max_new_tokens or r.context_len() >= self.cfg.max_model_len:
                self.scheduler.finish(r)
        self._inflight = {"reqs": ordered, "handle": handle, "idx": idx,
                          "row_of": {r.req_id: i for i, r in enumerate(ordered)},
                          "tokens": tokens, "src": src, "ctx": ctx}
        return self._collect(prev) if prev is not None else []

    def _collect(self, rec: dict) -> list[StepOutput]:
        """A queued step's tokens into its requests' placeholders."""
        if "ids" in rec:                      # computed again after a merge error
            ids = rec["ids"]
        else:
            try:
                ids = self.graphs.collect(rec["handle"])
            except MergeErrors:
                ids = self._recompute_queued(rec)
        if self._inflight is rec:
            self._inflight = None
        now = time.perf_counter()
        outputs = []
        for r, i, t in zip(rec["reqs"], rec["idx"], ids):
            if i >= len(r.output_token_ids):
                continue                      # dropped: the request stopped at an earlier step
            r.output_token_ids[i] = t
            if r.first_token_time is None:
                r.first_token_time = now
            finished = r.status is Status.FINISHED and i == len(r.output_token_ids) - 1
            if t in self.eos_ids:
                del r.output_token_ids[i + 1:]   # the step queued after this one computed past the stop
                # a request whose budget ends with the queued step was finished at that launch
                if r.status is not Status.FINISHED:
                    self.scheduler.finish(r)
                finished = True
            outputs.append(StepOutput(r.req_id, t, finished, r))
        self.steps += 1
        return outputs

    def _recompute_queued(self, rec: dict) -> list[int]:
        """A captured step whose in-launch merges reported errors (the graphs now run
        the work items and in-launch merges are off): that step again, eagerly, and the
        step queued after it from its ids, whose ids are kept for its own collect and
        written where the next launch reads its source rows. Running a step again
        appends its rows to the same slots; a step with a request that finished at its
        launch (its blocks are freed) cannot be run again, which raises."""
        self.merge_failures += 1
        self.kv_cache.clear_metadata()
        nxt = self._inflight if self._inflight is not None and self._inflight is not rec else None
        steps = [rec] + ([nxt] if nxt is not None else [])
        if any(not r.block_table for st in steps for r in st["reqs"]):
            raise RuntimeError("a captured decode step reported in-launch merge errors after some of its "
                               "requests finished (their blocks are freed): its tokens cannot be computed again")

        def again(st, prev_ids):
            toks = []
            for i, (r, s) in enumerate(zip(st["reqs"], st["src"])):
                if s < 0:
                    toks.append(st["tokens"][i])
                elif prev_ids is not None:
                    toks.append(prev_ids[s])
                else:                         # the previous step's token, collected before this one
                    toks.append(r.output_token_ids[st["idx"][i] - 1])
            n, ctx = len(toks), st["ctx"]
            return self._forward_eager(st["reqs"], toks, [c - 1 for c in ctx], [(i, i + 1) for i in range(n)],
                                       [r.block_table for r in st["reqs"]], ctx)

        ids = again(rec, None)
        if nxt is not None:
            nxt["ids"] = again(nxt, ids)
            self.graphs.ids[:len(nxt["ids"])].copy_(torch.tensor(nxt["ids"], dtype=torch.int64))
        return ids

    def _step_sync(self) -> list[StepOutput]:
        batch = self.scheduler.schedule()
        self._swap(batch)
        if batch.is_empty():
            return []
        return self._run(batch.prefill, batch.decode)

    def _run(self, prefill: list[Request], decode: list[Request], graphs: bool = True) -> list[StepOutput]:
        """Forward and sample the scheduled rows: a graph replay for greedy
        decode-only steps the graphs accept, the eager forward otherwise."""
        ordered = prefill + decode
        self.last_step_prefills = len(prefill)
        if not ordered:
            return []
        token_ids, positions, seq_slices, block_tables, context_lens = self.build_step(prefill, decode)
        if (graphs and self.graphs is not None and not prefill and all(r.temperature <= 0.0 for r in ordered)
                and self.graphs.bucket(len(ordered)) is not None):
            try:
                next_ids = self.graphs.run(token_ids, positions, block_tables, context_lens)
            except MergeErrors:               # the step again, eagerly (in-launch merges are off now)
                self.merge_failures += 1
                self.kv_cache.clear_metadata()
                next_ids = None
            if next_ids is not None:
                self.graph_steps += 1
                return self._finish_step(ordered, next_ids)
        next_ids = self._forward_eager(ordered, token_ids, positions, seq_slices, block_tables, context_lens)
        return self._finish_step(ordered, next_ids)

    def _forward_eager(self, ordered, token_ids, positions, seq_slices, block_tables, context_lens) -> list[int]:
        """Launch by launch: per layer the separate append (its last writer wins on
        a shared slot) then attention, as the reference's forward orders them.

        The step's attention may merge split rows inside its launches (the decode
        kernel, the merged launch), which assume a workgroup placement on the XCDs. The
        device's error count rides on the step's one synchronising copy (the sampled
        ids); if a merge reported an error the step's outputs are unusable, so merges
        are switched off for the rest of the process and the step runs again through
        the work items (re-appending the same rows to the same slots)."""
        tok = torch.tensor(token_ids, dtype=torch.int64).pin_memory().to(self.device, non_blocking=True)
        pos = torch.tensor(positions, dtype=torch.int64).pin_memory().to(self.device, non_blocking=True)
        hq = self.model.cfg.n_heads
        guard = ops.decode_device(self.device) if self.device.type == "cuda" else None
        for attempt in range(2):
            # the step's metadata, built from the host lists (no device round trip) and shared by every layer
            self.kv_cache.step_metadata(pos, seq_slices, block_tables, context_lens,
                                        self.kv_cache.rows_per_item(hq), host_positions=positions, num_heads=hq)
            logits = self.model.forward(tok, pos, seq_slices, block_tables, context_lens, self.kv_cache)
            errs = guard.errors_async() if guard is not None else None
            ids = self._sample(logits, ordered)          # synchronises: errs holds the count
            if errs is None or int(errs[0]) == 0:
                return ids
            if attempt == 1:
                break
            self.merge_failures += 1
            guard.disable_merges()
            self.kv_cache.clear_metadata()
        raise RuntimeError("attention kept reporting merge errors with in-launch merges switched off")

    def _finish_step(self, ordered: list[Request], next_ids: list[int]) -> list[StepOutput]:
        now = time.perf_counter()
        outputs = []
        for req, t in zip(ordered, next_ids):
            if req.first_token_time is None:
                req.first_token_time = now
            req.output_token_ids.append(t)
            finished = (t in self.eos_ids or len(req.output_token_ids) >= req.max_new_tokens
                        or req.context_len() >= self.cfg.max_model_len)
            if finished:
                self.scheduler.finish(req)
            outputs.append(StepOutput(req.req_id, t, finished, req))
        self.steps += 1
        return outputs

    def _sample(self, logits: torch.Tensor, reqs: list[Request]) -> list[int]:
        greedy = logits.argmax(dim=-1).cpu().tolist()        # one copy for the whole batch
        out = []
        for i, req in enumerate(reqs):
            if req.temperature <= 0.0:
                out.append(int(greedy[i]))
                continue
            probs = torch.softmax(logits[i] / req.temperature, dim=-1)
            if req.top_p < 1.0:
                sorted_p, idx = probs.sort(descending=True)
                keep = sorted_p.cumsum(0) - sorted_p < req.top_p
                probs = torch.zeros_like(probs).scatter(0, idx[keep], sorted_p[keep])
                probs = probs / probs.sum()
            out.append(int(torch.multinomial(probs, 1)))
        return out

    def stats(self) -> dict:
        bm = self.block_manager
        return {"kv_pool_mb": round(self.kv_cache.memory_bytes() / 2**20, 1), "free_blocks": bm.num_free(),
                "prefix_hit_rate": round(bm.hit_rate(), 3), "running": len(self.scheduler.running),
                "waiting": len(self.scheduler.waiting), "swapped": len(self.scheduler.swapped), "steps": self.steps,
                "graph_steps": self.graph_steps, "pipelined_steps": self.pipelined_steps, "swap_outs": self.swap_outs, "swap_ins": self.swap_ins}
