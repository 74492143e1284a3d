"""Drop-in PagedKVCache backed by the HIP kernels.

Same constructor, attributes and methods as the reference's
``tinybatch.kv_cache.PagedKVCache`` (src/tinybatch/kv_cache.py:13-45):

* ``pools[layer]`` is a ``[num_blocks, 2, n_kv_heads, block_size, head_dim]``
  tensor (K = index 0, V = index 1 of axis 1), zero-initialised. The layers are
  views into one allocation so that K3 can copy a block in every layer with
  one launch.
* ``write(layer, k, v, positions, seq_slices, block_tables)`` appends through
  K1 instead of a per-sequence ``index_put`` loop.
* ``gather(layer, table, context_len)`` returns contiguous ``[ctx, kvh, hd]``
  K and V, as the reference does.

Added for the fused data path (no reference counterpart):

* ``attention(layer, q, positions, seq_slices, block_tables, context_lens)``
  is the whole per-sequence attention region of Qwen2Paged.forward
  (model.py:130-147) as one K2 launch; returns ``attn_out [T, Hq*D]``.
* ``copy_blocks(src, dst)`` (K3, every layer) and ``swap_out``/``swap_in``.

The per-step metadata (slot mapping, padded int32 block tables, attention work
list) is built once and reused by every layer of the step; it is rebuilt when
the step's arguments change.
"""
from __future__ import annotations

import numpy as np
import torch

from . import _lib, ops
from .metadata import StepMetadata, build_step_metadata


class PagedKVCache:
    def __init__(self, n_layers: int, num_blocks: int, block_size: int, n_kv_heads: int, head_dim: int,
                 device: torch.device, dtype: torch.dtype, partition_tokens: int | None = None):
        device = torch.device(device)
        if device.type != "cuda":
            raise RuntimeError("tinybatch_amd.PagedKVCache needs a GPU device (no CPU fallback)")
        self.block_size = block_size
        self.num_blocks = num_blocks
        self.n_kv_heads = n_kv_heads
        self.head_dim = head_dim
        self.dtype = dtype
        self.device = device
        self.partition_tokens = partition_tokens or ops.partition_tokens(dtype, head_dim)
        self.storage = torch.zeros(n_layers, num_blocks, 2, n_kv_heads, block_size, head_dim,
                                   device=device, dtype=dtype)
        self.pools = [self.storage[i] for i in range(n_layers)]
        self._meta_cache: list[dict] = []

    def memory_bytes(self) -> int:
        return sum(p.numel() * p.element_size() for p in self.pools)

    # ---- per-step metadata -------------------------------------------------
    def step_metadata(self, positions, seq_slices, block_tables, context_lens=None,
                      rows_per_item: int = 1, host_positions=None, num_heads: int | None = None) -> StepMetadata:
        """Build (or reuse) the step's device metadata.

        Every layer of a forward pass passes the same argument objects, so the
        metadata is built once per step: an entry is reused when the positions
        object is the same one (held by the cache, so its identity cannot be
        recycled) with an unchanged in-place version, and the slices, tables
        and context lengths compare equal. write() (no context lengths) may
        reuse an entry built for attention(). ``host_positions`` (the same
        positions as a host list) spares the device-to-host copy of a device
        ``positions`` tensor; the entry is still keyed on ``positions``. With
        ``num_heads`` (query heads), a decode-only step that the streaming decode
        kernel serves faster (ops.decode_kernel_preferred) also gets its plan, and
        attention() / decode_step() with this metadata then run that kernel; a
        prefill-only step goes to tb_paged_prefill, and a step of whole prefills
        beside a run of decode rows to tb_paged_prefill and the decode kernel, each
        on its own rows (ops.attach_split_parts), when the decode rows gain by it.
        """
        pos_key = (positions, positions._version) if isinstance(positions, torch.Tensor) else list(positions)
        for e in self._meta_cache:
            # write() (no context lengths) takes any entry of the step; attention() only one
            # built for its row grouping and query heads (the heads decide the kernel routing)
            if (_same_positions(e["pos"], pos_key) and e["slices"] == [tuple(x) for x in seq_slices]
                    and e["tables"] == block_tables
                    and (context_lens is None or (e["ctx"] == context_lens and e["rows"] == rows_per_item
                                                  and e["heads"] == num_heads))):
                return e["meta"]
        # 16-bit pools serve long runs of new rows (prefills) with the tile kernel; a
        # step of prefills only (every sequence >= 16 new rows, its context within
        # the kernel's limit) goes to tb_paged_prefill instead: a step that also has
        # decode rows keeps them in the one launch with the tiles
        tile = self.pools[0].dtype in (torch.float16, torch.bfloat16)
        route = None
        if num_heads is not None and context_lens is not None and self.device.type == "cuda" and tile:
            r = ops.prefill_route(self.dtype, num_heads, self.n_kv_heads, self.head_dim, self.device)
            qlens = [e - b for b, e in seq_slices]
            if r is not None and any(qlens) and all(
                    n == 0 or (n >= 16 and c <= r.max_context) for n, c in zip(qlens, context_lens)):
                route = r
        meta = build_step_metadata(positions if host_positions is None else host_positions,
                                   seq_slices, block_tables, context_lens,
                                   block_size=self.block_size, num_blocks=self.num_blocks,
                                   partition_tokens=self.partition_tokens, rows_per_item=rows_per_item,
                                   tile_prefill=tile, prefill_route=route)
        if num_heads is not None and context_lens is not None and self.device.type == "cuda" and tile \
                and route is None:
            # whole prefills beside a run of decode rows: tb_paged_prefill and the
            # streaming decode kernel on their own rows, when the decode rows gain
            ops.attach_split_parts(meta, positions if host_positions is None else host_positions, seq_slices,
                                   block_tables, context_lens, num_heads=num_heads, num_kv_heads=self.n_kv_heads,
                                   head_dim=self.head_dim, dtype=self.dtype, device=self.device,
                                   rows=rows_per_item)
        if (num_heads is not None and context_lens is not None and self.device.type == "cuda"
                and ops.decode_kernel_preferred(meta, num_kv_heads=self.n_kv_heads, head_dim=self.head_dim,
                                                dtype=self.dtype)):
            ops.attach_decode_plan(meta, num_heads=num_heads, num_kv_heads=self.n_kv_heads,
                                   head_dim=self.head_dim, dtype=self.dtype, device=self.device)
        meta.to(self.device)
        entry = {"pos": pos_key, "slices": [tuple(x) for x in seq_slices],
                 "tables": [list(t) for t in block_tables],
                 "ctx": None if context_lens is None else list(context_lens), "rows": rows_per_item,
                 "heads": num_heads, "meta": meta}
        self._meta_cache = [entry] + self._meta_cache[:1]
        return meta

    def check(self) -> None:
        """Raise RuntimeError when an in-launch merge of this device reported an error
        since the last check (a unit's partials on two XCDs: the placement the decode
        kernel and the merged launch assume did not hold), so attention outputs since
        then cannot be trusted. Synchronises the device; a caller checks at a point it
        synchronises anyway (the engine does it with each eager step's token copy and
        recomputes the step, ops.DecodeDevice.disable_merges)."""
        if self.device.type != "cuda":
            return
        n = ops.decode_device(self.device).errors()
        if n:
            raise RuntimeError(f"{n} in-launch merge errors on {self.device}: attention outputs since the last "
                               "check are unusable (ops.DecodeDevice.disable_merges, then recompute)")

    def clear_metadata(self) -> None:
        """Forget the cached step metadata (its kernel routing), e.g. after disable_merges."""
        self._meta_cache = []

    # ---- reference API -----------------------------------------------------
    def write(self, layer: int, k: torch.Tensor, v: torch.Tensor, positions: torch.Tensor,
              seq_slices: list[tuple[int, int]], block_tables: list[list[int]],
              rope: ops.Rope | None = None) -> None:
        """Scatter each new token's K/V into its sequence's blocks (reference kv_cache.py:25-38).
        With ``rope``, k is the projection before rotation and is rotated at ``positions``
        (a device int64 tensor) on its way to the pool."""
        meta = self._lookup_or_build(positions, seq_slices, block_tables, None, k.shape[0])
        ops.kv_append(self.pools[layer], k, v, meta.slot_mapping, rope=rope, positions=positions)

    def gather(self, layer: int, table: list[int], context_len: int) -> tuple[torch.Tensor, torch.Tensor]:
        """Contiguous K, V [context_len, n_kv_heads, head_dim] (reference kv_cache.py:40-45)."""
        nb_needed = (context_len + self.block_size - 1) // self.block_size
        if nb_needed > len(table):
            # the reference slices a shorter gather silently; out-of-table reads are refused here
            raise IndexError(f"context_len {context_len} needs {nb_needed} blocks, table has {len(table)}")
        for b in table[:nb_needed]:
            if not 0 <= b < self.num_blocks:
                raise IndexError(f"block id {b} outside the pool of {self.num_blocks} blocks")
        t = torch.tensor(list(table[:max(nb_needed, 1)]), dtype=torch.int32).to(self.device)
        return ops.kv_gather(self.pools[layer], t, context_len)

    # ---- fused data path ---------------------------------------------------
    def rows_per_item(self, num_heads: int) -> int:
        """Query rows per attention work item for this cache's dtype and geometry."""
        return ops.rows_per_item(self.dtype, num_heads, self.n_kv_heads)

    def attention(self, layer: int, q: torch.Tensor, positions, seq_slices, block_tables, context_lens,
                  *, num_heads: int | None = None, scale: float | None = None,
                  out: torch.Tensor | None = None, rope: ops.Rope | None = None) -> torch.Tensor:
        """attn_out [T, Hq*D] for the whole flat batch (reference model.py:130-147). With
        ``rope``, q is the projection before rotation (rotated inside the kernels)."""
        hq = num_heads if num_heads is not None else q.shape[1]
        rows = self.rows_per_item(hq)
        meta = self._lookup_or_build(positions, seq_slices, block_tables, context_lens, q.shape[0], rows, hq)
        return ops.paged_attention(q, self.pools[layer], meta, num_heads=hq, scale=scale, out=out, rope=rope)

    def append_attention(self, layer: int, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, positions,
                         seq_slices, block_tables, context_lens, *, num_heads: int | None = None,
                         scale: float | None = None, out: torch.Tensor | None = None,
                         rope: ops.Rope | None = None) -> torch.Tensor:
        """write() then attention() (model.py:128-147) with the append folded into the
        attention kernels where the step's kernels can do both: decode-only steps, steps
        of whole prefills (tb_paged_prefill) and mixed steps split into those two sides,
        when no slot is written by two rows of the step; otherwise the two calls. With
        ``rope`` q and k are the projections before rotation."""
        hq = num_heads if num_heads is not None else q.shape[1]
        rows = self.rows_per_item(hq)
        meta = self._lookup_or_build(positions, seq_slices, block_tables, context_lens, q.shape[0], rows, hq)
        if self._fusable(meta):
            return ops.paged_attention(q, self.pools[layer], meta, num_heads=hq, scale=scale, out=out, rope=rope,
                                       k_new=k, v_new=v)
        self.write(layer, k, v, positions, seq_slices, block_tables, rope=rope)
        return ops.paged_attention(q, self.pools[layer], meta, num_heads=hq, scale=scale, out=out, rope=rope)

    @staticmethod
    def _fusable(meta: StepMetadata) -> bool:
        sm = meta.slot_mapping_np
        if sm.size and np.any((sm < 0) & (meta.row_ctx_np > 0)):
            return False                                  # a superseded writer: the separate append
        if meta.parts is not None or meta.decode_only:
            return True
        return bool(meta.num_prefill_work and not meta.num_work_items and not meta.num_prefill_tiles)

    def decode_step(self, layer: int, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, meta: StepMetadata,
                    *, num_heads: int | None = None, scale: float | None = None,
                    out: torch.Tensor | None = None) -> torch.Tensor:
        """Append + attention of a decode-only step in one launch (fused K1+K2)."""
        hq = num_heads if num_heads is not None else q.shape[1]
        return ops.paged_attention(q, self.pools[layer], meta, num_heads=hq, scale=scale, out=out,
                                   k_new=k, v_new=v)

    def copy_blocks(self, src, dst) -> None:
        """pool_l[dst[i]] <- pool_l[src[i]] in every layer (K3, one launch)."""
        ops.block_copy(self.pools, src, dst)

    def swap_out(self, blocks, staging: list[torch.Tensor]) -> None:
        """staging[l][i] <- pools[l][blocks[i]] for every layer."""
        for pool, st in zip(self.pools, staging):
            ops.block_gather(pool, blocks, st)

    def swap_in(self, staging: list[torch.Tensor], blocks) -> None:
        for pool, st in zip(self.pools, staging):
            ops.block_scatter(st, pool, blocks)

    def _lookup_or_build(self, positions, seq_slices, block_tables, context_lens, num_tokens,
                         rows_per_item: int = 1, num_heads: int | None = None) -> StepMetadata:
        meta = self.step_metadata(positions, seq_slices, block_tables, context_lens, rows_per_item,
                                  num_heads=num_heads)
        if meta.num_tokens != num_tokens:
            raise ValueError(f"{num_tokens} tokens given, positions describe {meta.num_tokens}")
        return meta


def _same_positions(a, b) -> bool:
    if isinstance(a, tuple) and isinstance(b, tuple):
        return a[0] is b[0] and a[1] == b[1]
    if isinstance(a, list) and isinstance(b, list):
        return a == b
    return False
