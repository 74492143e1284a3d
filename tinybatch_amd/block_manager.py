"""Block tables, reference counts and the prefix cache (host side).

Counterpart of the reference's BlockManager (src/tinybatch/block_manager.py:43-175):
the same contract, because the tables it produces are what the paged kernels
read (slot(pos) = table[pos // block_size] * block_size + pos % block_size).

* Free ids are handed out last-in first-out, starting from the highest id
  (block_manager.py:50,70), so fresh tables are descending runs.
* A full block is addressed by the hash of every token from the start of the
  sequence through the block's end (block_manager.py:38-40); a prompt reuses
  the longest run of cached full blocks (block_manager.py:92-107). The partial
  tail block is never cached (block_manager.py:109-114).
* A block filled by decoding is published when the next block is reserved
  (block_manager.py:127-156).
* Cached blocks whose count drops to zero stay cached and are evicted least
  recently freed first (block_manager.py:68-79,160-170).
* ``OutOfBlocks`` when nothing is left; a double free trips an assertion
  (block_manager.py:25-26,164).

``compact`` has no reference counterpart: it moves live blocks into the lowest
ids (a compaction round) and returns the (src, dst) pairs for the block-copy
kernel, remapping every table it is given and the prefix-cache index.
"""
from __future__ import annotations

from collections import OrderedDict
from dataclasses import dataclass, field


class OutOfBlocks(Exception):
    """No free or evictable block is left."""


@dataclass
class Block:
    block_id: int
    ref_count: int = 0
    prefix_hash: int | None = None          # set once the block is full and cached
    token_ids: list[int] = field(default_factory=list)


def hash_prefix(token_ids) -> int:
    """Content key of a whole prefix (sequence start .. end of a block)."""
    return hash(tuple(token_ids))


class BlockManager:
    def __init__(self, num_blocks: int, block_size: int, enable_prefix_caching: bool = True):
        if num_blocks <= 0 or block_size <= 0:
            raise ValueError("num_blocks and block_size must be positive")
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.enable_prefix_caching = enable_prefix_caching
        self.blocks = [Block(i) for i in range(num_blocks)]
        self.free_ids: list[int] = list(range(num_blocks))     # popped from the end
        self.cache: dict[int, int] = {}                          # prefix hash -> block id
        self.evictable: OrderedDict[int, None] = OrderedDict()   # cached, unreferenced; oldest first
        self.prefix_hits = 0
        self.prefix_queries = 0

    # ---- accounting --------------------------------------------------------
    def num_free(self) -> int:
        return len(self.free_ids) + len(self.evictable)

    def blocks_needed(self, num_tokens: int) -> int:
        return -(-num_tokens // self.block_size)

    def hit_rate(self) -> float:
        return self.prefix_hits / self.prefix_queries if self.prefix_queries else 0.0

    # ---- allocation ----------------------------------------------------------
    def _fresh(self) -> Block:
        if self.free_ids:
            return self.blocks[self.free_ids.pop()]
        if self.evictable:
            bid, _ = self.evictable.popitem(last=False)         # least recently freed
            blk = self.blocks[bid]
            if blk.prefix_hash is not None:
                self.cache.pop(blk.prefix_hash, None)
            blk.prefix_hash = None
            blk.token_ids = []
            return blk
        raise OutOfBlocks(f"all {self.num_blocks} KV blocks are in use")

    def allocate_prompt(self, token_ids: list[int]) -> tuple[list[int], int]:
        """Table for a prompt and how many leading tokens the prefix cache serves."""
        bs = self.block_size
        table: list[int] = []
        cached = 0
        n_full = len(token_ids) // bs
        still_matching = self.enable_prefix_caching
        for b in range(n_full):
            self.prefix_queries += 1
            key = hash_prefix(token_ids[:(b + 1) * bs])
            hit = self.cache.get(key) if still_matching else None
            if hit is None:
                still_matching = False                          # later blocks cannot match
                blk = self._fresh()
                blk.ref_count = 1
                blk.token_ids = list(token_ids[b * bs:(b + 1) * bs])
                if self.enable_prefix_caching:
                    blk.prefix_hash = key
                    self.cache[key] = blk.block_id
                table.append(blk.block_id)
            else:
                self.blocks[hit].ref_count += 1
                self.evictable.pop(hit, None)
                table.append(hit)
                cached += bs
                self.prefix_hits += 1
        if len(token_ids) % bs:
            blk = self._fresh()
            blk.ref_count = 1
            blk.token_ids = list(token_ids[n_full * bs:])
            table.append(blk.block_id)
        return table, cached

    def allocate_private(self, num_blocks: int, token_ids: list[int]) -> list[int]:
        """A table of fresh, uncached blocks for ``token_ids`` (a sequence coming back
        from host memory: its contents are copied in, not looked up in the prefix cache)."""
        if num_blocks > self.num_free():
            raise OutOfBlocks(f"{num_blocks} blocks requested, {self.num_free()} free")
        bs = self.block_size
        table = []
        for b in range(num_blocks):
            blk = self._fresh()
            blk.ref_count = 1
            blk.token_ids = list(token_ids[b * bs:(b + 1) * bs])
            table.append(blk.block_id)
        return table

    def append_slot(self, table: list[int], seq_token_ids: list[int]) -> bool:
        """Make room for the token at index len(seq_token_ids) (call it before
        that token joins the sequence). Returns True when a block was added."""
        bs = self.block_size
        pos = len(seq_token_ids)
        if pos % bs == 0:
            blk = self._fresh()
            blk.ref_count = 1
            blk.token_ids = []
            table.append(blk.block_id)
            if self.enable_prefix_caching and len(table) >= 2:
                self._publish(table, len(table) - 2, seq_token_ids)
            return True
        self.blocks[table[-1]].token_ids = list(seq_token_ids[(len(table) - 1) * bs:pos])
        return False

    def _publish(self, table: list[int], idx: int, seq_token_ids: list[int]) -> None:
        blk = self.blocks[table[idx]]
        if blk.prefix_hash is not None or blk.ref_count != 1:
            return                      # already cached, or shared (its first owner published it)
        key = hash_prefix(seq_token_ids[:(idx + 1) * self.block_size])
        if key in self.cache:
            return                      # the same content is cached under another id
        blk.prefix_hash = key
        blk.token_ids = list(seq_token_ids[idx * self.block_size:(idx + 1) * self.block_size])
        self.cache[key] = blk.block_id

    # ---- release -------------------------------------------------------------
    def free_table(self, table: list[int]) -> None:
        for bid in table:
            blk = self.blocks[bid]
            blk.ref_count -= 1
            assert blk.ref_count >= 0, "double free"
            if blk.ref_count == 0:
                if blk.prefix_hash is not None:
                    self.evictable[bid] = None
                else:
                    blk.token_ids = []
                    self.free_ids.append(bid)

    # ---- compaction (no reference counterpart) ------------------------------
    def compact(self, tables: list[list[int]]) -> tuple[list[int], list[int]]:
        """Move every referenced or cached block into the lowest ids.

        Rewrites ``tables`` in place and the prefix-cache index, and returns
        (src, dst) block-id lists for one copy round (dst ids are free before
        the copy, so no id is both a source and a destination). Afterwards the
        free ids are exactly the top of the pool.
        """
        live = sorted(b.block_id for b in self.blocks if b.ref_count > 0 or b.prefix_hash is not None)
        target = set(range(len(live)))
        movers = [b for b in live if b not in target]
        holes = sorted(target.difference(live))
        mapping = dict(zip(movers, holes))
        for src, dst in mapping.items():
            a, b = self.blocks[src], self.blocks[dst]
            b.ref_count, b.prefix_hash, b.token_ids = a.ref_count, a.prefix_hash, a.token_ids
            a.ref_count, a.prefix_hash, a.token_ids = 0, None, []
            if b.prefix_hash is not None:
                self.cache[b.prefix_hash] = dst
        for t in tables:
            t[:] = [mapping.get(x, x) for x in t]
        self.evictable = OrderedDict((mapping.get(x, x), None) for x in self.evictable)
        self.free_ids = list(range(self.num_blocks - 1, len(live) - 1, -1))
        return list(mapping.keys()), list(mapping.values())
