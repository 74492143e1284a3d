"""HIP-graph replays of decode-only engine steps.

A decode step of B running sequences is the same chain of ~240 launches every
time (24 layers of norm, projections, RoPE, fused append + paged attention,
MLP); only the metadata changes. Each batch-size bucket (B padded up) gets one
graph, captured once, whose launches read fixed device buffers:

* tokens, positions and source rows [Bmax] (row i's input token is the
  previous step's id of row src[i] where src[i] >= 0, else tokens[i]);
* the step metadata at fixed capacities — slot mapping, block tables
  [Bmax, ceil(max_model_len / BS)], work items for every partition a row can
  have, partition offsets, split rows — plus the device counts the attention
  kernels read at run time (tb_paged_attention's device_counts), so a launch
  sized for the capacities only runs this step's work items;
* the output token ids (argmax inside the graph; for 16-bit batches of up
  to 32 rows the LM head and the argmax are one fused kernel that never
  writes the logits).

Attention in the captured step is one launch per layer. A 16-bit model on a
device whose workgroups land on its XCDs round robin (ops.DecodeDevice) runs
tb_paged_attention_merged: the partitions of a split row run on one XCD and
the last one to finish merges them, with no combine launch. Its grid is the
bucket's slot capacity (the bound of the slot map's longest-first packing:
num_xcds * (ceil(items * kv heads / num_xcds) + partitions per row)); the
step's slot map (tb_build_xcd_slot_map over its work items, padded with -1,
whose workgroups exit at once) rides in the staging buffer. The device's
merge error count is copied back with every step's token ids: a nonzero count
makes ``collect`` raise MergeErrors after switching the graphs to the work
items and their combine launch (recaptured on next use) and in-launch merges
off on the device. Otherwise (fp32, no split rows, another placement) the
work-item kernel reads the device counts, and a combine launch merges split rows.

Per step the host packs the tokens, positions and metadata straight into one
pinned staging buffer (pack_decode_step: the arrays build_step_metadata would
give, built for decode rows only), copies it with one host-to-device copy, and
replays. ``launch`` returns without waiting: the step's token ids come back
through a pinned buffer and an event (``collect``), and a row may take its
input token from the previous step's ids still on the device (its source row),
so the host can queue step N+1 while step N runs. Two staging and two id
buffers alternate; a step's buffers are reused two launches later, so each
launch is collected before the launch after next. Padded rows get no work
items and slot -1: they read nothing and write nothing, and their outputs are
ignored.
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from . import layer_ops, ops
from .kv_cache import PagedKVCache
from .metadata import MERGED_MAX_PARTS, StepMetadata, decode_staging_offsets, pack_decode_step
from .model import Qwen2Paged

DEFAULT_BUCKETS = (1, 2, 4, 8, 16, 24, 32, 48, 64, 96, 128, 192, 256)


class MergeErrors(RuntimeError):
    """A captured step's in-launch merges reported errors: its token ids, and those of
    any step launched from them, cannot be used. The graphs have switched to the work
    items and their combine launch; the steps must be computed again."""


class DecodeGraphs:
    def __init__(self, model: Qwen2Paged, kv_cache: PagedKVCache, max_batch: int, max_model_len: int,
                 buckets=DEFAULT_BUCKETS):
        self.model, self.cache = model, kv_cache
        self.dev = kv_cache.device
        c = model.cfg
        self.BS = kv_cache.block_size
        self.P = kv_cache.partition_tokens
        self.max_nb = -(-max_model_len // self.BS)
        self.max_parts = -(-max_model_len // self.P)
        self.buckets = sorted({b for b in buckets if b < max_batch} | {max_batch})
        B = self.buckets[-1]
        self.wcap = B * self.max_parts
        # one staging buffer, one copy per step: the int32 metadata (decode_staging_offsets)
        # followed by int64 tokens [B], positions [B] and source rows [B] (-1: the token
        # comes from the host; r >= 0: row r of the previous step's ids)
        self.offs = decode_staging_offsets(B, self.max_nb, self.max_parts)
        n = int(self.offs[-1])
        # the merged launch (see the module docstring): its slot map follows the int64 tail
        d = ops.decode_device(self.dev)
        self.num_xcds = d.num_xcds
        self.merged = (d.merge_in_kernel and d.num_xcds > 1 and model.dtype in (torch.float16, torch.bfloat16)
                       and c.n_heads // c.n_kv_heads <= 16 and 1 < self.max_parts <= MERGED_MAX_PARTS)
        self.slots = self._slot_capacity(B) if self.merged else 0
        nbytes = 4 * n + 24 * B + 4 * self.slots
        self.dev_buf = torch.zeros(nbytes, dtype=torch.uint8, device=self.dev)
        self.host_bufs = [torch.zeros(nbytes, dtype=torch.uint8).pin_memory() for _ in range(2)]
        self.dev_i32 = self.dev_buf[:4 * n].view(torch.int32)
        self.host_nps = [h[:4 * n].view(torch.int32).numpy() for h in self.host_bufs]
        self.host_tps = [h[4 * n:4 * n + 24 * B].view(torch.int64).view(3, B).numpy() for h in self.host_bufs]
        tail = self.dev_buf[4 * n:4 * n + 24 * B].view(torch.int64).view(3, B)
        self.tok, self.pos, self.src = tail[0], tail[1], tail[2]
        self.dev_slots = self.dev_buf[4 * n + 24 * B:].view(torch.int32)
        self.host_slots = [h[4 * n + 24 * B:].view(torch.int32).numpy() for h in self.host_bufs]
        self.host_errs = [torch.zeros(1, dtype=torch.int32).pin_memory() for _ in range(2)]
        self.ids = torch.zeros(B, dtype=torch.int64, device=self.dev)
        self.host_ids = [torch.zeros(B, dtype=torch.int64).pin_memory() for _ in range(2)]
        self.turn = 0       # which staging / id buffer the next launch uses
        self.last_use = [None, None]   # the event of the launch that last used each buffer
        ws_bytes = ops._lib.lib().tb_paged_attention_workspace_bytes(self.wcap, c.n_heads, c.head_dim)
        self.ws = torch.empty(max(int(ws_bytes), 16), dtype=torch.uint8, device=self.dev)
        # the LM head with greedy sampling fused (streamed batches): its candidate slots
        self.head_fused = (model.fused_mlp and model._streamed(torch.empty(B, 0, dtype=model.dtype))
                           and c.vocab_size % 16 == 0 and c.d_model % 32 == 0)
        head_bytes = ops._lib.lib().tb_linear_argmax_workspace_bytes(B, c.vocab_size) if self.head_fused else 0
        self.head_ws = torch.empty(max(int(head_bytes), 16), dtype=torch.uint8, device=self.dev)
        self.graphs: dict[int, torch.cuda.CUDAGraph] = {}
        self.pool = None    # graph memory pool shared by the buckets

    def _slot_capacity(self, Bp: int) -> int:
        """Slots of the merged launch for a bucket: the longest-first packing's bound."""
        X, hkv = self.num_xcds, self.model.cfg.n_kv_heads
        return X * (-(-Bp * self.max_parts * hkv // X) + self.max_parts)

    # ---- metadata at capacity ---------------------------------------------------
    def _view(self, i: int, n: int) -> torch.Tensor:
        return self.dev_i32.narrow(0, int(self.offs[i]), n)

    def _meta(self, Bp: int) -> StepMetadata:
        e = np.zeros(0, np.int32)
        m = StepMetadata(num_tokens=Bp, num_seqs=Bp, block_size=self.BS, partition_tokens=self.P,
                         max_blocks_per_seq=self.max_nb, num_work_items=Bp * self.max_parts,
                         total_partitions=Bp * self.max_parts, max_parts_per_row=self.max_parts,
                         decode_only=True, rows_per_item=1, num_prefill_tiles=0,
                         num_split_rows=Bp if self.max_parts > 1 else 0,   # rows of one partition never split
                         slot_mapping_np=e, block_tables_np=e, work_np=e, row_part_off_np=e, row_ctx_np=e,
                         prefill_tiles_np=e, split_rows_np=e)
        m.slot_mapping = self._view(0, Bp)
        m.block_tables = self._view(1, Bp * self.max_nb).view(Bp, self.max_nb)
        m.work = self._view(2, Bp * self.max_parts * 4).view(-1, 4)
        m.row_part_off = self._view(3, Bp + 1)
        m.split_rows = self._view(4, Bp * 4).view(Bp, 4)
        m.prefill_tiles = m.split_rows            # never read: no tiles in a decode step
        m.device_counts = self._view(5, 4)
        if self.merged:
            m.slot_map = self.dev_slots[:self._slot_capacity(Bp)]
        return m

    # ---- the captured step -------------------------------------------------------
    @torch.inference_mode()
    def _forward(self, Bp: int, meta: StepMetadata) -> None:
        m, c = self.model, self.model.cfg

        rope = m.rope if m.fused_rope else None

        def attention(i, q, k, v):   # fused append + attention (a decode step), RoPE in the kernel
            return ops.paged_attention(q, self.cache.pools[i], meta, num_heads=c.n_heads, k_new=k, v_new=v,
                                       workspace=self.ws, rope=rope)

        src = self.src[:Bp]
        tok = torch.where(src >= 0, self.ids.index_select(0, src.clamp(min=0)), self.tok[:Bp])
        x = m.run_layers(tok, self.pos[:Bp], attention, fused_rope=m.fused_rope)
        if self.head_fused:
            layer_ops.linear_argmax(x, m.lm_head, out=self.ids[:Bp], workspace=self.head_ws)
        else:
            self.ids[:Bp].copy_(F.linear(x, m.lm_head).argmax(dim=-1))

    def bucket(self, B: int) -> int | None:
        for b in self.buckets:
            if b >= B:
                return b
        return None

    def _capture(self, Bp: int) -> torch.cuda.CUDAGraph:
        meta = self._meta(Bp)
        torch.cuda.synchronize(self.dev)                            # no step in flight reads the buffers
        self.dev_i32[int(self.offs[5]):int(self.offs[5]) + 4].zero_()   # no work: warm-up launches exit at once
        if self.merged:
            meta.slot_map.fill_(-1)                                 # no slot runs an item in the warm-up
        self.src.zero_()                                            # in-range source rows for the warm-up
        ids = self.ids.clone()          # the last step's tokens, which the next launch may read
        stream = torch.cuda.Stream(device=self.dev)
        stream.wait_stream(torch.cuda.current_stream(self.dev))
        with torch.cuda.stream(stream):
            self._forward(Bp, meta)                                 # eager warm-up outside the graph
        torch.cuda.synchronize(self.dev)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream, pool=self.pool):
            self._forward(Bp, meta)
        self.ids.copy_(ids)             # the warm-up overwrote them
        torch.cuda.synchronize(self.dev)
        if self.pool is None:
            self.pool = g.pool()
        return g

    def capture_all(self) -> None:
        """Capture every bucket now (otherwise each is captured on first use)."""
        for b in self.buckets:
            if b not in self.graphs:
                self.graphs[b] = self._capture(b)

    def launch(self, tokens: list[int], positions: list[int], block_tables: list[list[int]],
               context_lens: list[int], src_rows: list[int] | None = None):
        """Queue one decode step (one row per sequence) without waiting for it. Row i's
        input token is tokens[i], or, where src_rows[i] >= 0, the id the previous launch
        produced for its row src_rows[i]. Returns the handle ``collect`` takes, or None
        when two rows' newest positions map to one pool slot (nothing is queued: such a
        step needs the separate append, whose last writer wins, before attention)."""
        B = len(tokens)
        Bp = self.bucket(B)
        if Bp is None:
            raise ValueError(f"batch {B} exceeds the largest bucket {self.buckets[-1]}")
        if max(context_lens) > self.max_nb * self.BS:
            raise ValueError("context longer than max_model_len")
        g = self.graphs.get(Bp)
        if g is None:
            g = self.graphs[Bp] = self._capture(Bp)
        k = self.turn
        self.turn ^= 1
        if self.last_use[k] is not None:
            self.last_use[k].synchronize()   # its copies are done before the buffers are rewritten
        h, tp = self.host_nps[k], self.host_tps[k]
        if not pack_decode_step(h, self.offs, Bp, self.max_nb, context_lens, block_tables,
                                block_size=self.BS, num_blocks=self.cache.num_blocks, partition_tokens=self.P):
            # Two rows write one slot. The reference appends the whole batch first, the
            # last row in batch order winning, and then both rows attend to the winner's
            # K/V; the fused append of the captured step would have each row store and
            # read its own. Nothing is queued: the caller runs this step unfused.
            self.turn ^= 1
            return None
        if self.merged:
            import ctypes

            from . import _lib
            W = int(h[self.offs[5]])
            work = h[self.offs[2]:self.offs[2] + 4 * W]
            vp = lambda a: a.ctypes.data_as(ctypes.c_void_p)
            _lib.check(_lib.lib().tb_build_xcd_slot_map(vp(work), W, self.model.cfg.n_kv_heads, self.num_xcds,
                                                        vp(self.host_slots[k]), self._slot_capacity(Bp)),
                       "tb_build_xcd_slot_map")
        tp[0, :B] = tokens
        tp[1, :B] = positions
        tp[2, :B] = -1 if src_rows is None else src_rows
        tp[0:2, B:Bp] = 0
        tp[2, B:Bp] = -1
        self.dev_buf.copy_(self.host_bufs[k], non_blocking=True)
        g.replay()
        self.host_ids[k][:Bp].copy_(self.ids[:Bp], non_blocking=True)
        if self.merged:
            self.host_errs[k].copy_(ops.decode_device(self.dev).violations, non_blocking=True)
        ev = torch.cuda.Event()
        ev.record()
        self.last_use[k] = ev
        return (B, k, ev)

    def collect(self, handle) -> list[int]:
        """The token ids of a launched step (waits for that step only). Call it
        before the launch after next, which reuses the step's id buffer."""
        B, k, ev = handle
        ev.synchronize()
        if self.merged and int(self.host_errs[k][0]) != 0:
            torch.cuda.synchronize(self.dev)         # nothing in flight uses the graphs or the counters
            ops.decode_device(self.dev).disable_merges()
            self.merged = False
            self.graphs.clear()                      # recaptured with the work items on next use
            raise MergeErrors("a captured decode step's in-launch merges reported errors")
        return self.host_ids[k][:B].tolist()

    def run(self, tokens: list[int], positions: list[int], block_tables: list[list[int]],
            context_lens: list[int]) -> list[int]:
        """Greedy next token of each decode row (one row per sequence), or None for a
        step with two rows on one slot (see ``launch``)."""
        handle = self.launch(tokens, positions, block_tables, context_lens)
        return None if handle is None else self.collect(handle)
