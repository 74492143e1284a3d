"""Once-per-step device metadata for the paged kernels.

The reference converts each sequence's block table to a device tensor inside
every layer (src/tinybatch/kv_cache.py:35,43) and builds a boolean mask per
sequence per layer (src/tinybatch/model.py:142-145). Here the host lists that
LLMEngine.step produces (src/tinybatch/engine.py:99-126: positions,
seq_slices, block_tables, context_lens) are turned into int32 arrays once per
step and uploaded in a single host-to-device copy:

* ``slot_mapping[T]``  - pool slot of every token's new K/V
  (table[pos // BS] * BS + pos % BS, kv_cache.py:35-36); -1 for tokens outside
  every slice and for all but the last writer of a duplicated slot, so the
  parallel append equals the reference's sequential "last in batch order wins".
* ``block_tables[B, max_nb]`` - tables padded with 0 (padding is never read).
* ``work[W, 4]`` - (row, seq, partition | (rows-1) << 24, row_ctx) for the
  attention kernel: rows row .. row+rows-1 of one sequence (rows = 1 unless
  ``rows_per_item`` > 1 groups consecutive prefill rows, never across a change
  of partition count), where row_ctx = ctx - q_len + i + 1 is the number of
  positions query row i may see (the mask rule j <= ctx - q_len + i of
  model.py:139-145) and the group's later rows see one more position each.
* ``row_part_off[T + 1]`` - running count of partitions per row.
* ``split_rows[S, 4]`` - (row, first partial slot, partial count, 0) of every
  row whose work spans more than one partition (their partials are merged by
  the combine pass; the record saves it the lookups in row_part_off).
* ``prefill_tiles[N, 4]`` - (row0, seq, rows | partition << 8, pos0) when
  ``tile_prefill``: sequences with many new rows (full prefills and long
  prefill tails) are cut into tiles of up to TILE_ROWS consecutive rows (row0
  at position pos0), one item per tile and TILE_PARTITION-position partition
  its last row reaches; the prefill kernel serves them and their rows get no
  work items. A tile row counts ceil(row_ctx / TILE_PARTITION) partitions in
  row_part_off (a split tile row leaves partials like any split row). Items
  are ordered by the positions they cover, most first.

Errors mirror the reference: a table too short for a position raises
IndexError (kv_cache.py:35), a block id outside the pool raises IndexError
(pool indexing, kv_cache.py:37,43).
"""
from __future__ import annotations

import itertools
from dataclasses import dataclass

from typing import NamedTuple

import numpy as np
import torch


@dataclass
class StepMetadata:
    num_tokens: int
    num_seqs: int
    block_size: int
    partition_tokens: int
    max_blocks_per_seq: int
    num_work_items: int
    total_partitions: int
    max_parts_per_row: int
    decode_only: bool            # every sequence has exactly one query row
    rows_per_item: int
    num_prefill_tiles: int
    num_split_rows: int
    # host copies
    slot_mapping_np: np.ndarray
    block_tables_np: np.ndarray
    work_np: np.ndarray
    row_part_off_np: np.ndarray
    row_ctx_np: np.ndarray       # [T] visible positions per row (0 for rows outside slices)
    prefill_tiles_np: np.ndarray  # [N, 4]
    split_rows_np: np.ndarray     # [S, 4]
    # device views (int32, one backing buffer)
    device_buffer: torch.Tensor | None = None
    slot_mapping: torch.Tensor | None = None
    block_tables: torch.Tensor | None = None
    work: torch.Tensor | None = None
    row_part_off: torch.Tensor | None = None
    prefill_tiles: torch.Tensor | None = None
    split_rows: torch.Tensor | None = None
    # set for capacity-sized (graph) metadata: {work items, split rows, tiles} on the device
    device_counts: torch.Tensor | None = None
    # decode plan (tb_paged_decode): set by attach_decode_plan for decode-only steps
    rows_are_seqs: bool = False  # decode-only with row b = sequence b (the decode kernel's layout)
    decode_plan_np: np.ndarray | None = None
    decode_workgroups: int = 0
    decode_waves: int = 0
    decode_stride: int = 0
    decode_pieces: int = 0
    decode_unit_cost: int = 0
    decode_units: int = 0
    decode_plan: torch.Tensor | None = None
    # the same plan built on the device by meta.to (attach_decode_plan(on_device=True)):
    # the count words and the segment descriptors (tb_build_decode_segments)
    decode_counts_np: np.ndarray | None = None
    decode_segments_np: np.ndarray | None = None
    decode_kv_heads: int = 0
    decode_head_dim: int = 0
    num_blocks: int = 0          # blocks of the pool the step's tables index
    # slot map of the work-item kernel with split rows merged inside the launch
    # (tb_paged_attention_merged): set by attach_xcd_slot_map
    slot_map_np: np.ndarray | None = None
    slot_map: torch.Tensor | None = None
    # whole prefill sequences served by tb_paged_prefill (build_step_metadata's
    # prefill_route): its work list and the most tiles one entry holds
    prefill_work_np: np.ndarray | None = None
    num_prefill_work: int = 0
    prefill_max_tiles: int = 0
    prefill_work: torch.Tensor | None = None
    # a mixed step served as sub-steps (split_step_parts): (first row, end row, the
    # sub-step's metadata with rows counted from the first row); the arrays above
    # still describe the whole step (its slot mapping serves the append)
    parts: list | None = None

    def to(self, device: torch.device) -> "StepMetadata":
        """Upload every array with one host-to-device copy (views into one buffer);
        the parts' arrays get copies of their own."""
        for _, _, m in self.parts or ():
            m.to(device)
        parts = [self.slot_mapping_np, self.block_tables_np.reshape(-1), self.work_np.reshape(-1),
                 self.row_part_off_np, self.prefill_tiles_np.reshape(-1), self.split_rows_np.reshape(-1)]
        extra = [x for x in (self.decode_plan_np, self.slot_map_np, self.prefill_work_np, self.decode_counts_np,
                             self.decode_segments_np) if x is not None]
        parts += extra
        sizes = [pad4(p.size) for p in parts]
        host = np.zeros(sum(sizes), dtype=np.int32)
        offs = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int64)
        for p, o in zip(parts, offs):
            host[o:o + p.size] = p.reshape(-1)
        src = torch.from_numpy(host)
        if device.type == "cuda":
            src = src.pin_memory()
        buf = src.to(device, non_blocking=True)
        self.device_buffer = buf
        self.slot_mapping = buf.narrow(0, int(offs[0]), parts[0].size)
        self.block_tables = buf.narrow(0, int(offs[1]), parts[1].size).view(-1, self.max_blocks_per_seq)
        self.work = buf.narrow(0, int(offs[2]), parts[2].size).view(-1, 4)
        self.row_part_off = buf.narrow(0, int(offs[3]), parts[3].size)
        self.prefill_tiles = buf.narrow(0, int(offs[4]), parts[4].size).view(-1, 4)
        self.split_rows = buf.narrow(0, int(offs[5]), parts[5].size).view(-1, 4)
        k = 6
        if self.decode_plan_np is not None:
            self.decode_plan = buf.narrow(0, int(offs[k]), parts[k].size)
            k += 1
        if self.slot_map_np is not None:
            self.slot_map = buf.narrow(0, int(offs[k]), parts[k].size)
            k += 1
        if self.prefill_work_np is not None:
            self.prefill_work = buf.narrow(0, int(offs[k]), parts[k].size)
            k += 1
        if self.decode_segments_np is not None:
            counts = buf.narrow(0, int(offs[k]), parts[k].size)
            segs = buf.narrow(0, int(offs[k + 1]), parts[k + 1].size)
            self.decode_plan = _expand_decode_plan(self, counts, segs, device)
        return self


def split_step_parts(positions, seq_slices, block_tables, context_lens, *, block_size: int, num_blocks: int,
                     partition_tokens: int, rows_per_item: int, prefill_route: "PrefillRoute") -> list | None:
    """A mixed step whose sequences are whole prefills that ``prefill_route`` serves
    (>= 16 new rows, context within its limit) on one side and decode rows (one
    new row each) on the other, each side a contiguous run of rows: the two
    sub-steps as [(row0, row1, metadata), ...] in row order, rows counted from
    row0 (so q[row0:row1] and out[row0:row1] are the sub-step's rows). The
    prefill side's metadata carries only its tb_paged_prefill work list. None
    for any other step shape."""
    B = len(seq_slices)
    if B < 2 or context_lens is None or prefill_route is None:
        return None
    pos = _host_positions(positions)
    qlens = [int(e) - int(b) for b, e in seq_slices]
    is_pre = [n >= 16 and int(c) <= prefill_route.max_context for n, c in zip(qlens, context_lens)]
    is_dec = [n == 1 for n in qlens]
    if not all(p or d for p, d in zip(is_pre, is_dec)):
        return None
    # one change of kind in sequence order, and rows contiguous in that order
    kinds = [0 if d else 1 for d in is_dec]
    cut = next((i for i in range(1, B) if kinds[i] != kinds[i - 1]), None)
    if cut is None or any(kinds[i] != kinds[cut] for i in range(cut, B)):
        return None
    if any(int(seq_slices[i][0]) != int(seq_slices[i - 1][1]) for i in range(1, B)):
        return None
    parts = []
    for lo, hi in ((0, cut), (cut, B)):
        r0, r1 = int(seq_slices[lo][0]), int(seq_slices[hi - 1][1])
        sl = [(int(b) - r0, int(e) - r0) for b, e in seq_slices[lo:hi]]
        pre = kinds[lo] == 1
        m = build_step_metadata(pos[r0:r1], sl, block_tables[lo:hi], list(context_lens[lo:hi]),
                                block_size=block_size, num_blocks=num_blocks, partition_tokens=partition_tokens,
                                rows_per_item=rows_per_item, tile_prefill=pre,
                                prefill_route=prefill_route if pre else None)
        if pre and (m.num_work_items or m.num_prefill_tiles):
            return None
        parts.append((r0, r1, m))
    return parts


# The prefill kernel's tile shape (TB_PREFILL_TILE_ROWS / TB_PREFILL_TILE_PARTITION
# in include/tinybatch_amd.h): query rows per tile, positions per tile partition.
TILE_ROWS = 64
TILE_PARTITION = 1024
# partitions of one row the merged launch counts (8-bit per-XCD arrival fields,
# TB_MERGED_MAX_PARTS)
MERGED_MAX_PARTS = 255


class PrefillRoute(NamedTuple):
    """Where whole prefill sequences go to tb_paged_prefill: the step's kv heads and
    head dim, and the longest context that kernel serves (ops.prefill_route)."""
    num_kv_heads: int
    head_dim: int
    max_context: int
    num_xcds: int = 1


def build_prefill_work(first_rows, seqs, pos0s, new_rows, *, num_kv_heads: int, head_dim: int,
                       num_xcds: int = 1) -> tuple[np.ndarray, int]:
    """tb_build_prefill_work: one entry (first row, sequence, pos0, new rows | pair <<
    16 | kv head << 24) per (sequence, kv head, pair of 16-row blocks), the entries of
    one (sequence, kv head) on one XCD, and the most 16-position tiles one entry holds."""
    import ctypes

    from . import _lib

    cols = [np.ascontiguousarray(np.asarray(x, dtype=np.int32).reshape(-1)) for x in (first_rows, seqs, pos0s, new_rows)]
    n = cols[0].size
    lib = _lib.lib()
    ptrs = [c.ctypes.data_as(ctypes.c_void_p) for c in cols]
    count = lib.tb_prefill_work_count(ptrs[3], n, num_kv_heads)
    if count < 0:
        raise ValueError("bad prefill sequences (new rows must be >= 1)")
    work = np.zeros((max(count, 1), 4), dtype=np.int32)
    tiles = ctypes.c_int32()
    st = lib.tb_build_prefill_work(*ptrs, n, num_kv_heads, head_dim, num_xcds, work.ctypes.data_as(ctypes.c_void_p),
                                   count, ctypes.byref(tiles))
    _lib.check(st, "tb_build_prefill_work")
    return work[:count], int(tiles.value)


def tiles_sequence(q_len: int, ctx: int, min_rows: int = 16, max_ctx: int = 4096) -> bool:
    """Whether a sequence's rows go to prefill tiles: many new rows, and a context
    short enough (or a tail long enough) that one workgroup's serial walk over it
    is not the critical path. Short tails of long contexts stay with the split
    row groups, which spread the context over partitions."""
    return q_len >= min_rows and (ctx <= max_ctx or ctx <= 16 * q_len)


def pad4(n: int) -> int:
    return (n + 3) // 4 * 4


def _host_positions(positions) -> np.ndarray:
    if isinstance(positions, torch.Tensor):
        return positions.detach().to("cpu", torch.int64).numpy().reshape(-1)
    return np.asarray(positions, dtype=np.int64).reshape(-1)


def build_step_metadata(positions, seq_slices, block_tables, context_lens, *, block_size: int,
                        num_blocks: int, partition_tokens: int, num_tokens: int | None = None,
                        validate_attention: bool = True, rows_per_item: int = 1,
                        tile_prefill: bool = False, prefill_route: PrefillRoute | None = None) -> StepMetadata:
    """Build the per-step arrays (host side). See the module docstring. With
    ``prefill_route``, sequences of >= 16 new rows whose context is at most its
    max_context go to tb_paged_prefill whole (prefill_work_np); their rows get no
    work items, tiles or partition slots."""
    if block_size <= 0 or block_size & (block_size - 1):
        raise ValueError(f"block_size must be a power of two, got {block_size}")
    pos = _host_positions(positions)
    T = int(pos.size if num_tokens is None else num_tokens)
    if pos.size != T:
        raise ValueError(f"positions has {pos.size} entries, expected {T}")
    B = len(seq_slices)
    if len(block_tables) != B:
        raise ValueError("seq_slices and block_tables differ in length")
    if context_lens is not None and len(context_lens) != B:
        raise ValueError("seq_slices and context_lens differ in length")

    starts = np.fromiter((s for s, _ in seq_slices), dtype=np.int64, count=B)
    ends = np.fromiter((e for _, e in seq_slices), dtype=np.int64, count=B)
    qlens = ends - starts
    if B and (np.any(starts < 0) or np.any(ends > T) or np.any(qlens < 0)):
        raise ValueError("seq_slices out of range of the flat batch")
    tab_lens = np.fromiter((len(t) for t in block_tables), dtype=np.int64, count=B)
    max_nb = max(1, int(tab_lens.max()) if B else 1)
    tables = np.zeros((max(B, 1), max_nb), dtype=np.int64)
    for b, t in enumerate(block_tables):
        if len(t):
            tables[b, :len(t)] = t
    if B:
        used = np.arange(max_nb)[None, :] < tab_lens[:, None]
        bad = used & ((tables[:B] < 0) | (tables[:B] >= num_blocks))
        if bad.any():
            b, i = np.argwhere(bad)[0]
            raise IndexError(f"block id {tables[b, i]} of sequence {b} is outside the pool of {num_blocks} blocks")

    # ---- rows (query tokens that belong to a slice) ----
    tot = int(qlens.sum()) if B else 0
    row_seq = np.repeat(np.arange(B, dtype=np.int64), qlens)
    seq_row_base = np.concatenate([[0], np.cumsum(qlens)[:-1]]) if B else np.zeros(0, np.int64)
    row_i = np.arange(tot, dtype=np.int64) - np.repeat(seq_row_base, qlens)
    row_ids = np.repeat(starts, qlens) + row_i

    # ---- slot mapping (kv_cache.py:34-38) ----
    slots = np.full(T, -1, dtype=np.int64)
    if tot:
        p = pos[row_ids]
        if np.any(p < 0):
            raise ValueError("negative position")
        bidx = p // block_size
        over = bidx >= tab_lens[row_seq]
        if over.any():
            r = int(np.argmax(over))
            raise IndexError(f"position {int(p[r])} of sequence {int(row_seq[r])} needs block index "
                             f"{int(bidx[r])} but its table has {int(tab_lens[row_seq[r]])} blocks")
        s = tables[row_seq, bidx] * block_size + p % block_size
        slots[row_ids] = s
        # last writer wins: keep only the final occurrence of each slot
        rev = s[::-1]
        _, first_in_rev = np.unique(rev, return_index=True)
        keep = np.zeros(tot, dtype=bool)
        keep[tot - 1 - first_in_rev] = True
        slots[row_ids[~keep]] = -1

    # ---- attention work items ----
    P = int(partition_tokens)
    row_ctx_by_row = np.zeros(T, dtype=np.int64)
    tiles: list[tuple[int, int, int, int, int]] = []
    stream_seqs: list[tuple[int, int, int, int]] = []
    tiled = np.zeros(T, dtype=bool)
    nparts_by_row = np.zeros(T, dtype=np.int64)
    if tot and context_lens is not None:
        ctx = np.asarray(context_lens, dtype=np.int64)
        if np.any(ctx < qlens):
            b = int(np.argmax(ctx < qlens))
            raise ValueError(f"context_len {int(ctx[b])} of sequence {b} is shorter than its {int(qlens[b])} new tokens")
        if validate_attention:
            need = (ctx + block_size - 1) // block_size
            short = (need > tab_lens) & (qlens > 0)
            if short.any():
                b = int(np.argmax(short))
                raise IndexError(f"context_len {int(ctx[b])} of sequence {b} needs {int(need[b])} blocks "
                                 f"but its table has {int(tab_lens[b])}")
        row_ctx = np.repeat(ctx - qlens, qlens) + row_i + 1
        row_ctx_by_row[row_ids] = row_ctx
        nparts_by_row[row_ids] = (row_ctx + P - 1) // P
        if prefill_route is not None:
            for b in range(B):
                n, c = int(qlens[b]), int(ctx[b])
                if n >= 16 and c <= prefill_route.max_context:
                    s0 = int(starts[b])
                    tiled[s0:s0 + n] = True               # served by tb_paged_prefill
                    nparts_by_row[s0:s0 + n] = 0
                    stream_seqs.append((s0, b, c - n, n))
        if tile_prefill:
            for b in range(B):
                n, c = int(qlens[b]), int(ctx[b])
                if n and not tiled[int(starts[b])] and tiles_sequence(n, c):
                    s0 = int(starts[b])
                    tiled[s0:s0 + n] = True               # served by tiles, not work items
                    rc = row_ctx_by_row[s0:s0 + n]
                    nparts_by_row[s0:s0 + n] = (rc + TILE_PARTITION - 1) // TILE_PARTITION
                    for r in range(0, n, TILE_ROWS):
                        rows = min(TILE_ROWS, n - r)
                        pos0 = c - n + r
                        end = pos0 + rows                 # positions the tile's last row sees
                        for part in range((end + TILE_PARTITION - 1) // TILE_PARTITION):
                            tiles.append((s0 + r, b, rows | (part << 8), pos0,
                                          min(TILE_PARTITION, end - part * TILE_PARTITION)))
    row_part_off = np.zeros(T + 1, dtype=np.int64)
    np.cumsum(nparts_by_row, out=row_part_off[1:])
    if not 1 <= rows_per_item <= 16:
        raise ValueError("rows_per_item must be in [1, 16]")
    total_parts = int(row_part_off[-1])
    # groups of consecutive rows of one sequence with equal partition counts
    grp_row, grp_len = row_ids, np.ones(tot, dtype=np.int64)
    if rows_per_item > 1 and tot:
        starts_l, lens_l = [], []
        for b in range(B):
            s0, e0 = int(starts[b]), int(ends[b])
            i = s0
            while i < e0:
                j = min(e0, i + rows_per_item)
                k = i + 1
                while k < j and nparts_by_row[k] == nparts_by_row[i]:
                    k += 1
                starts_l.append(i)
                lens_l.append(k - i)
                i = k
        grp_row = np.asarray(starts_l, dtype=np.int64)
        grp_len = np.asarray(lens_l, dtype=np.int64)
    grp_parts = nparts_by_row[grp_row] if tot else np.zeros(0, np.int64)
    keep = (grp_parts > 0) & ~tiled[grp_row] if tot else grp_parts > 0
    grp_row, grp_len, grp_parts = grp_row[keep], grp_len[keep], grp_parts[keep]
    W = int(grp_parts.sum())
    work = np.zeros((W, 4), dtype=np.int64)
    if W:
        rep_rows = np.repeat(grp_row, grp_parts)
        seq_of_row = np.zeros(T, dtype=np.int64)
        seq_of_row[row_ids] = row_seq
        item_off = np.concatenate([[0], np.cumsum(grp_parts)[:-1]])
        part = np.arange(W) - np.repeat(item_off, grp_parts)
        work[:, 0] = rep_rows
        work[:, 1] = seq_of_row[rep_rows]
        work[:, 2] = part | ((np.repeat(grp_len, grp_parts) - 1) << 24)
        work[:, 3] = row_ctx_by_row[rep_rows]
        # Shortest partitions first (stable): on the 64-row decode step
        # (U[512, 4096] contexts) 20.4-20.5 us per call against 20.7-20.8 in
        # row order; nothing depends on the order (slots come from
        # row_part_off and the partition index).
        length = np.minimum(P, work[:, 3] - P * part)
        work = work[np.argsort(length, kind="stable")]
    if max(T, W, max_nb, total_parts) >= 2**24 - 1:
        raise ValueError("step too large for int32 metadata")
    tiles.sort(key=lambda t: -t[4])                   # most positions first (stable)
    tiles_np = np.asarray([t[:4] for t in tiles], dtype=np.int64).reshape(-1, 4)
    split_ids = np.nonzero(nparts_by_row > 1)[0]
    split_rows = np.zeros((split_ids.size, 4), dtype=np.int64)
    split_rows[:, 0] = split_ids
    split_rows[:, 1] = row_part_off[split_ids]
    split_rows[:, 2] = nparts_by_row[split_ids]
    prefill_work, prefill_tiles_max = None, 0
    if stream_seqs:
        cols = np.asarray(stream_seqs, dtype=np.int64).T
        prefill_work, prefill_tiles_max = build_prefill_work(
            cols[0], cols[1], cols[2], cols[3], num_kv_heads=prefill_route.num_kv_heads,
            head_dim=prefill_route.head_dim, num_xcds=prefill_route.num_xcds)

    return StepMetadata(
        num_tokens=T, num_seqs=B, block_size=block_size, partition_tokens=P,
        max_blocks_per_seq=max_nb, num_work_items=W, total_partitions=total_parts,
        max_parts_per_row=int(nparts_by_row.max()) if T else 0,
        decode_only=bool(B) and bool(np.all(qlens == 1)),
        rows_are_seqs=bool(B) and T == B and bool(np.all(starts == np.arange(B))) and bool(np.all(qlens == 1)),
        rows_per_item=int(rows_per_item),
        num_prefill_tiles=int(tiles_np.shape[0]),
        num_split_rows=int(split_ids.size),
        slot_mapping_np=slots.astype(np.int32),
        block_tables_np=tables[:max(B, 1)].astype(np.int32),
        work_np=work.astype(np.int32),
        row_part_off_np=row_part_off.astype(np.int32),
        row_ctx_np=row_ctx_by_row.astype(np.int32),
        prefill_tiles_np=tiles_np.astype(np.int32),
        split_rows_np=split_rows.astype(np.int32),
        num_blocks=int(num_blocks),
        prefill_work_np=prefill_work,
        num_prefill_work=0 if prefill_work is None else int(prefill_work.shape[0]),
        prefill_max_tiles=prefill_tiles_max,
    )


# ---- decode-only steps, packed for a captured graph ----------------------------
# Staging layout of a decode graph (int32, each part 16-byte aligned): slot [B] |
# block tables [B, max_nb] | work items [B * max_parts, 4] | row_part_off [B + 1] |
# split-row records [B, 4] | counts (work items, split rows, tiles, 0).
def decode_staging_offsets(max_batch: int, max_nb: int, max_parts: int) -> np.ndarray:
    sizes = [pad4(n) for n in (max_batch, max_batch * max_nb, max_batch * max_parts * 4, max_batch + 1,
                               max_batch * 4, 4)]
    return np.concatenate([[0], np.cumsum(sizes)]).astype(np.int64)


def pack_step(h: np.ndarray, offs: np.ndarray, Bp: int, max_nb: int, meta: StepMetadata) -> None:
    """A decode step's metadata (from build_step_metadata) into staging buffer h,
    padded to Bp rows: padded rows get slot -1 and no work."""
    o = offs
    B = meta.num_tokens
    h[o[0]:o[0] + Bp] = -1
    h[o[0]:o[0] + B] = meta.slot_mapping_np
    tab = h[o[1]:o[1] + Bp * max_nb].reshape(Bp, max_nb)
    nb = min(meta.block_tables_np.shape[1], max_nb)   # entries past the context are never read
    tab[:B, :nb] = meta.block_tables_np[:B, :nb]
    W = meta.num_work_items
    h[o[2]:o[2] + W * 4] = meta.work_np.reshape(-1)
    h[o[3]:o[3] + B + 1] = meta.row_part_off_np
    h[o[3] + B + 1:o[3] + Bp + 1] = meta.row_part_off_np[-1]
    S = meta.num_split_rows
    h[o[4]:o[4] + 4 * S] = meta.split_rows_np.reshape(-1)
    h[o[5]:o[5] + 4] = (W, S, 0, 0)


def pack_decode_step(h: np.ndarray, offs: np.ndarray, Bp: int, max_nb: int, context_lens, block_tables, *,
                     block_size: int, num_blocks: int, partition_tokens: int) -> bool:
    """Pack a decode-only step (row b = sequence b, one new token at position
    context_lens[b] - 1) straight into staging buffer h: the arrays that
    build_step_metadata + pack_step write, for a fraction of the host time (the
    engine's per-step cost). Returns False, writing nothing that matters, when
    two rows map to one slot (then the general builder's last-writer rule
    applies); raises as the general builder does on block ids outside the pool
    or tables shorter than their contexts."""
    B = len(context_lens)
    BS, P, o = int(block_size), int(partition_tokens), offs
    ctx = np.fromiter(context_lens, np.int64, B)
    lens = np.fromiter(map(len, block_tables), np.int64, B)
    if B == 0 or ctx.min() < 1:
        raise ValueError("a decode row needs a context of at least one position")
    need = (ctx + BS - 1) // BS
    short = need > lens
    if short.any():
        b = int(short.argmax())
        raise IndexError(f"context_len {int(ctx[b])} of sequence {b} needs {int(need[b])} blocks "
                         f"but its table has {int(lens[b])}")
    if int(need.max()) > max_nb:
        raise ValueError("context longer than the staging tables")
    flat = np.fromiter(itertools.chain.from_iterable(block_tables), np.int64, int(lens.sum()))
    if flat.min() < 0 or flat.max() >= num_blocks:
        i = int(((flat < 0) | (flat >= num_blocks)).argmax())
        b = int(np.searchsorted(np.cumsum(lens), i, side="right"))
        raise IndexError(f"block id {int(flat[i])} of sequence {b} is outside the pool of {num_blocks} blocks")
    # table entries the kernels read: the first need[b] of each row
    first = np.cumsum(lens) - lens
    tot = int(need.sum())
    row = np.repeat(np.arange(B, dtype=np.int64), need)
    col = np.arange(tot, dtype=np.int64) - np.repeat(np.cumsum(need) - need, need)
    tab = h[o[1]:o[1] + Bp * max_nb].reshape(Bp, max_nb)
    tab[row, col] = flat[np.repeat(first, need) + col]
    last = ctx - 1
    slots = flat[first + last // BS] * BS + last % BS
    if len(set(slots.tolist())) != B:
        return False
    h[o[0]:o[0] + Bp] = -1
    h[o[0]:o[0] + B] = slots
    # work items, shortest partition first (stable), as build_step_metadata orders them
    nparts = (ctx + P - 1) // P
    W = int(nparts.sum())
    wrow = np.repeat(np.arange(B, dtype=np.int64), nparts)
    part = np.arange(W, dtype=np.int64) - np.repeat(np.cumsum(nparts) - nparts, nparts)
    wctx = ctx[wrow]
    order = np.argsort(np.minimum(P, wctx - P * part), kind="stable")
    work = h[o[2]:o[2] + W * 4].reshape(W, 4)
    work[:, 0] = wrow[order]
    work[:, 1] = wrow[order]
    work[:, 2] = part[order]
    work[:, 3] = wctx[order]
    rpo = h[o[3]:o[3] + Bp + 1]
    rpo[0] = 0
    np.cumsum(nparts, out=rpo[1:B + 1])
    rpo[B + 1:] = W
    split = np.nonzero(nparts > 1)[0]
    S = int(split.size)
    rec = h[o[4]:o[4] + 4 * S].reshape(S, 4)
    rec[:, 0] = split
    rec[:, 1] = rpo[split]
    rec[:, 2] = nparts[split]
    rec[:, 3] = 0
    h[o[5]:o[5] + 4] = (W, S, 0, 0)
    return True


# ---- decode plans (tb_paged_decode) ---------------------------------------------
def decode_defaults(head_dim: int):
    """(waves per workgroup, per-unit cost) the decode kernel uses for this head dim by
    default, or None when it does not serve the head dim."""
    import ctypes

    from . import _lib

    w, uc = ctypes.c_int32(), ctypes.c_int32()
    st = _lib.lib().tb_decode_defaults(head_dim, ctypes.byref(w), ctypes.byref(uc))
    return (w.value, uc.value) if st == 0 else None


def decode_unit_cost(context_lens, *, num_kv_heads: int, head_dim: int, workgroups: int, num_xcds: int,
                     waves: int) -> int:
    """tb_decode_unit_cost: the per-unit cost a step's decode plan is built with by
    default (the head dim's default cost, or 2 lower when that gives the busiest worker
    >= 5% fewer entries)."""
    import ctypes

    from . import _lib

    ctx = np.ascontiguousarray(np.asarray(context_lens, dtype=np.int32).reshape(-1))
    uc = ctypes.c_int32()
    st = _lib.lib().tb_decode_unit_cost(ctx.ctypes.data_as(ctypes.c_void_p), int(ctx.size), num_kv_heads,
                                        head_dim, workgroups, waves, num_xcds, ctypes.byref(uc))
    if st == _lib.TB_ERR_UNSUPPORTED and decode_defaults(head_dim) is not None:
        return decode_defaults(head_dim)[1]   # no plan serves the step: the builder says so
    _lib.check(st, "tb_decode_unit_cost")
    return uc.value


def build_decode_plan(context_lens, block_tables, *, block_size: int, num_blocks: int, num_kv_heads: int,
                      head_dim: int, workgroups: int, num_xcds: int, waves: int | None = None,
                      unit_cost: int | None = None) -> tuple[np.ndarray, int, int, int] | None:
    """tb_build_decode_plan for a decode step (row b = sequence b with context_lens[b]
    positions, block_tables[b] its blocks): (int32 plan, waves, stride, partial slots),
    or None when the kernel does not serve the step (head dim, or a unit cut over more
    than 255 workers)."""
    import ctypes

    from . import _lib

    dflt = decode_defaults(head_dim)
    if dflt is None:
        return None
    waves = dflt[0] if waves is None else int(waves)
    L = _lib.lib()
    if not L.tb_decode_variant_supported(head_dim, waves):
        raise ValueError(f"the decode kernel has no {waves}-wave variant for head_dim {head_dim}")
    ctx = np.ascontiguousarray(np.asarray(context_lens, dtype=np.int32).reshape(-1))
    B = int(ctx.size)
    if B == 0 or np.any(ctx <= 0):
        raise ValueError("a decode plan needs >= 1 sequence, each with >= 1 position")
    if unit_cost is None:
        unit_cost = decode_unit_cost(ctx, num_kv_heads=num_kv_heads, head_dim=head_dim, workgroups=workgroups,
                                     num_xcds=num_xcds, waves=waves)
    unit_cost = int(unit_cost)
    tables = np.ascontiguousarray(np.asarray(block_tables, dtype=np.int32).reshape(B, -1))
    vp = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    me, pieces = ctypes.c_int32(), ctypes.c_int32()
    st = L.tb_decode_plan_shape(vp(ctx), B, num_kv_heads, head_dim, workgroups, waves, num_xcds, unit_cost,
                                ctypes.byref(me), ctypes.byref(pieces))
    if st == _lib.TB_ERR_UNSUPPORTED:
        return None
    _lib.check(st, "tb_decode_plan_shape")
    stride = max(2, (me.value + 1) // 2 * 2)
    words = int(L.tb_decode_plan_words(workgroups * waves, stride))
    plan = np.zeros(words, dtype=np.int32)
    st = L.tb_build_decode_plan(vp(ctx), B, num_kv_heads, head_dim, vp(tables), tables.shape[1], block_size,
                                num_blocks, workgroups, waves, num_xcds, unit_cost, stride, vp(plan), words)
    if st == _lib.TB_ERR_UNSUPPORTED:
        return None
    if st == _lib.TB_ERR_INDEX:
        raise IndexError("a block table is too short for its context, or holds a block outside the pool")
    _lib.check(st, "tb_build_decode_plan")
    return plan, waves, stride, pieces.value


def build_decode_segments(context_lens, block_tables, *, block_size: int, num_kv_heads: int, head_dim: int,
                          workgroups: int, num_xcds: int, waves: int | None = None, unit_cost: int | None = None):
    """tb_build_decode_segments: the host half of a decode plan built on the device
    (count words [workers padded to 4], descriptors int32 [n, 8], waves, stride, partial
    slots), or None when the kernel does not serve the step."""
    import ctypes

    from . import _lib

    dflt = decode_defaults(head_dim)
    if dflt is None:
        return None
    waves = dflt[0] if waves is None else int(waves)
    L = _lib.lib()
    if not L.tb_decode_variant_supported(head_dim, waves):
        raise ValueError(f"the decode kernel has no {waves}-wave variant for head_dim {head_dim}")
    ctx = np.ascontiguousarray(np.asarray(context_lens, dtype=np.int32).reshape(-1))
    B = int(ctx.size)
    if B == 0 or np.any(ctx <= 0):
        raise ValueError("a decode plan needs >= 1 sequence, each with >= 1 position")
    if unit_cost is None:
        unit_cost = decode_unit_cost(ctx, num_kv_heads=num_kv_heads, head_dim=head_dim, workgroups=workgroups,
                                     num_xcds=num_xcds, waves=waves)
    unit_cost = int(unit_cost)
    tables = np.ascontiguousarray(np.asarray(block_tables, dtype=np.int32).reshape(B, -1))
    workers = workgroups * waves
    counts = np.zeros((workers + 3) // 4 * 4, dtype=np.int32)
    cap = B * num_kv_heads + workers
    segs = np.zeros((cap, 8), dtype=np.int32)
    vp = lambda a: a.ctypes.data_as(ctypes.c_void_p)   # noqa: E731
    ns, me, pieces = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int32()
    st = L.tb_build_decode_segments(vp(ctx), B, num_kv_heads, head_dim, vp(tables), tables.shape[1], block_size,
                                    workgroups, waves, num_xcds, unit_cost, vp(counts), vp(segs), cap,
                                    ctypes.byref(ns), ctypes.byref(me), ctypes.byref(pieces))
    if st == _lib.TB_ERR_UNSUPPORTED:
        return None
    if st == _lib.TB_ERR_INDEX:
        raise IndexError("a block table is too short for its context")
    _lib.check(st, "tb_build_decode_segments")
    stride = max(2, (me.value + 1) // 2 * 2)
    return counts, segs[:ns.value].copy(), waves, stride, pieces.value


def _expand_decode_plan(meta: StepMetadata, counts: torch.Tensor, segs: torch.Tensor,
                        device: torch.device) -> torch.Tensor:
    """The decode plan on the device: the count words, then the tile entries written by
    tb_expand_decode_plan from the descriptors and the uploaded block tables, on the
    device's current stream."""
    from . import _lib, ops

    workers = meta.decode_workgroups * meta.decode_waves
    words = int(_lib.lib().tb_decode_plan_words(workers, meta.decode_stride))
    plan = torch.empty(words, dtype=torch.int32, device=device)
    plan[:counts.numel()].copy_(counts)
    hkv, d = meta.decode_kv_heads, meta.decode_head_dim
    _lib.check(_lib.lib().tb_expand_decode_plan(
        segs.data_ptr(), int(meta.decode_segments_np.shape[0]), meta.block_tables.data_ptr(),
        meta.max_blocks_per_seq, meta.block_size, meta.num_blocks, hkv, d, workers, meta.decode_stride,
        plan.data_ptr(), ops.decode_device(device).violations.data_ptr(), _lib.stream_handle(device)),
        "tb_expand_decode_plan")
    return plan


def attach_decode_plan(meta: StepMetadata, *, num_heads: int, num_kv_heads: int, head_dim: int,
                       dtype: torch.dtype, workgroups: int, num_xcds: int, waves: int | None = None,
                       unit_cost: int | None = None, on_device: bool = False) -> bool:
    """Give a decode-only step (row b = sequence b) the plan of the decode kernel, to be
    uploaded with the rest of its metadata by ``meta.to``. Returns whether it applies:
    16-bit rows, head_dim 64 / 128, at most 8 query heads per kv head, at most 16 kv
    heads, blocks of >= 16 positions. With ``on_device`` the host only assigns the
    tiles (tb_build_decode_segments) and ``meta.to`` writes the plan's entries on the
    device (tb_expand_decode_plan); the plan is the same."""
    if (not meta.rows_are_seqs or dtype not in (torch.float16, torch.bfloat16) or meta.block_size < 16
            or meta.device_buffer is not None or meta.num_blocks <= 0 or num_heads % num_kv_heads
            or num_heads // num_kv_heads > 8 or num_kv_heads > 16):
        return False
    B = meta.num_seqs
    dflt = decode_defaults(head_dim)
    if dflt is None:
        return False
    if unit_cost is None:
        unit_cost = decode_unit_cost(meta.row_ctx_np[:B], num_kv_heads=num_kv_heads, head_dim=head_dim,
                                     workgroups=workgroups, num_xcds=num_xcds,
                                     waves=dflt[0] if waves is None else int(waves))
    meta.decode_unit_cost = int(unit_cost)
    if on_device:
        got = build_decode_segments(meta.row_ctx_np[:B], meta.block_tables_np[:B], block_size=meta.block_size,
                                    num_kv_heads=num_kv_heads, head_dim=head_dim, workgroups=workgroups,
                                    num_xcds=num_xcds, waves=waves, unit_cost=unit_cost)
        if got is None:
            return False
        counts, segs, w, stride, pieces = got
        meta.decode_counts_np, meta.decode_segments_np = counts, segs
        meta.decode_workgroups, meta.decode_waves, meta.decode_stride = workgroups, w, stride
        meta.decode_units = B * num_kv_heads
        meta.decode_pieces = pieces
        meta.decode_kv_heads, meta.decode_head_dim = num_kv_heads, head_dim
        return True
    got = build_decode_plan(meta.row_ctx_np[:B], meta.block_tables_np[:B], block_size=meta.block_size,
                            num_blocks=meta.num_blocks, num_kv_heads=num_kv_heads, head_dim=head_dim,
                            workgroups=workgroups, num_xcds=num_xcds, waves=waves, unit_cost=unit_cost)
    if got is None:
        return False
    plan, w, stride, pieces = got
    meta.decode_plan_np = plan
    meta.decode_workgroups = workgroups
    meta.decode_waves = w
    meta.decode_stride = stride
    meta.decode_units = B * num_kv_heads
    meta.decode_pieces = pieces
    return True


def build_xcd_slot_map(work, num_work_items: int, num_kv_heads: int, num_xcds: int) -> np.ndarray:
    """tb_build_xcd_slot_map: the grid of tb_paged_attention_merged for these work items
    (int32 [num_work_items, 4]): every row group's items of one kv head on one XCD."""
    import ctypes

    from . import _lib

    w = np.ascontiguousarray(np.asarray(work, dtype=np.int32).reshape(-1, 4)[:num_work_items])
    L = _lib.lib()
    vp = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    n = int(L.tb_xcd_slot_map_slots(vp(w), num_work_items, num_kv_heads, num_xcds))
    if n < 0:
        _lib.check(n, "tb_xcd_slot_map_slots")
    out = np.full(max(n, 1), -1, dtype=np.int32)
    _lib.check(L.tb_build_xcd_slot_map(vp(w), num_work_items, num_kv_heads, num_xcds, vp(out), n),
               "tb_build_xcd_slot_map")
    return out[:n]


def attach_xcd_slot_map(meta: StepMetadata, *, num_heads: int, num_kv_heads: int, dtype: torch.dtype,
                        num_xcds: int) -> bool:
    """Give a step of work items with split rows the slot map of the merged launch, to be
    uploaded by ``meta.to``. Applies to 16-bit steps without prefill tiles, with at most
    16 query heads per kv head and no capacity counts; returns whether it does."""
    if (dtype not in (torch.float16, torch.bfloat16) or meta.num_prefill_tiles > 0 or meta.num_split_rows == 0
            or num_heads // num_kv_heads > 16 or meta.device_buffer is not None or meta.num_work_items == 0):
        return False
    if meta.max_parts_per_row > MERGED_MAX_PARTS:
        # the merged launch counts a row's partitions in 8-bit fields; the combine
        # kernel serves such steps
        return False
    meta.slot_map_np = build_xcd_slot_map(meta.work_np, meta.num_work_items, num_kv_heads, num_xcds)
    return meta.slot_map_np.size > 0
