"""Paged KV-cache block accounting: the slot / block-table contract the kernels read.

Call surface of engine/block_manager.py (mohsinmubarak/iitj-llm-coopt): BlockManager(num_blocks,
block_size), ensure (:86-93), truncate (:95-103), free (:105-110), blocks_for (:48-49),
can_fit (:54-55), num_free / usage (:40-46), slot_mapping (:216-220), block_table_tensor
(:222-229), OutOfBlocks (:22-23), and the elastic pool's add_blocks / migrate_out_of /
withdraw_free / take_free_excluding (:159-213).  Token p of a sequence lives in slot
table[p // block_size] * block_size + p % block_size.  Prefix caching (hashes, reference counts,
the evictable LRU) is a control-plane feature outside this path: every block here belongs to
one table, and evictable blocks do not exist.

`free_order` lets a caller fix the order in which blocks are handed out (e.g. a seeded
permutation, so that block tables are scattered over the pool as in a long-running server).
"""
from collections import deque

import numpy as np
import torch

__all__ = ["BlockManager", "OutOfBlocks"]


class OutOfBlocks(Exception):
    """The pool cannot hold the requested tokens."""


class BlockManager:
    def __init__(self, num_blocks: int, block_size: int = 16, free_order=None):
        if num_blocks <= 0 or block_size <= 0:
            raise ValueError("num_blocks and block_size must be positive")
        self.num_blocks, self.block_size = int(num_blocks), int(block_size)
        order = range(self.num_blocks) if free_order is None else [int(b) for b in free_order]
        if sorted(order) != list(range(self.num_blocks)):
            raise ValueError("free_order must be a permutation of range(num_blocks)")
        self._free = deque(order)
        self.tables: dict[int, list[int]] = {}

    # ---- capacity ------------------------------------------------------------------------
    @property
    def num_free(self) -> int:
        return len(self._free)

    @property
    def free_blocks(self):
        return self._free

    @property
    def usage(self) -> float:
        return 1.0 - self.num_free / self.num_blocks

    def blocks_for(self, num_tokens: int) -> int:
        return (int(num_tokens) + self.block_size - 1) // self.block_size

    def extra_blocks_needed(self, seq_id: int, total_tokens: int) -> int:
        have = len(self.tables.get(seq_id, ()))
        return max(0, self.blocks_for(total_tokens) - have)

    def can_fit(self, seq_id: int, total_tokens: int) -> bool:
        return self.extra_blocks_needed(seq_id, total_tokens) <= self.num_free

    # ---- allocation ------------------------------------------------------------------------
    def ensure(self, seq_id: int, total_tokens: int) -> None:
        """Grows seq_id's table to hold total_tokens tokens (all or nothing)."""
        need = self.extra_blocks_needed(seq_id, total_tokens)
        if need > self.num_free:
            raise OutOfBlocks(f"cannot grow sequence {seq_id} by {need} blocks: only {self.num_free} are free")
        table = self.tables.setdefault(seq_id, [])
        table.extend(self._free.popleft() for _ in range(need))

    def truncate(self, seq_id: int, total_tokens: int) -> None:
        """Returns trailing blocks beyond total_tokens (speculative rollback), last first."""
        table = self.tables.get(seq_id)
        if not table:
            return
        keep = self.blocks_for(total_tokens)
        while len(table) > keep:
            self._free.append(table.pop())

    def free(self, seq_id: int) -> int:
        table = self.tables.pop(seq_id, [])
        self._free.extend(table)
        return len(table)

    # ---- pool growth, shrinkage and migration (the elastic buffer's park / unpark) ----------
    def add_blocks(self, ids) -> None:
        """Grows the pool with blocks whose memory was just handed over (engine/block_manager.py
        :159-163); they join the end of the free list in the given order."""
        ids = [int(b) for b in ids]
        self._free.extend(ids)
        self.num_blocks += len(ids)

    def take_free_excluding(self, excluded) -> int:
        """Takes the first free block not in `excluded` (engine/block_manager.py:202-213)."""
        for i, b in enumerate(self._free):
            if b not in excluded:
                del self._free[i]
                return b
        raise OutOfBlocks("every free block lies inside the excluded id range")

    def migrate_out_of(self, ids, copy_fn) -> int:
        """Moves every in-use block in `ids` to a free block outside `ids`, in ascending id
        order, calling copy_fn(src, dst) for each and rewriting every table that holds it; the
        source joins the end of the free list (engine/block_manager.py:165-187).  Returns the
        number moved, or -1 (nothing changed) when too few free blocks lie outside `ids`.
        Sources are all in `ids` and destinations all outside, so the copies may run in any
        order, e.g. batched into one kv_blocks.copy_blocks launch."""
        ids = set(int(b) for b in ids)
        used = sorted({b for t in self.tables.values() for b in t if b in ids})
        if sum(1 for b in self._free if b not in ids) < len(used):
            return -1
        where = {}
        for sid, t in self.tables.items():
            for i, b in enumerate(t):
                if b in ids:
                    where.setdefault(b, []).append((sid, i))
        for src in used:
            dst = self.take_free_excluding(ids)
            copy_fn(src, dst)
            for sid, i in where[src]:
                self.tables[sid][i] = dst
            self._free.append(src)
        return len(used)

    def withdraw_free(self, ids) -> None:
        """Shrinks the pool by the blocks `ids`, which must all be free
        (engine/block_manager.py:189-199); raises OutOfBlocks otherwise, changing nothing."""
        ids = set(int(b) for b in ids)
        remaining = deque(b for b in self._free if b not in ids)
        if len(self._free) - len(remaining) != len(ids):
            raise OutOfBlocks("withdraw_free: not every requested block is free")
        self._free = remaining
        self.num_blocks -= len(ids)

    # ---- tensors for the kernels -------------------------------------------------------------
    def slot_mapping(self, seq_id: int, start: int, end: int) -> torch.Tensor:
        """Cache slots of positions [start, end) of seq_id, int64 CPU tensor."""
        table = np.asarray(self.tables[seq_id], dtype=np.int64)
        pos = np.arange(start, end, dtype=np.int64)
        blk = pos // self.block_size
        if len(pos) and blk[-1] >= len(table):
            raise IndexError(f"position {end - 1} of seq {seq_id} has no block (call ensure)")
        return torch.from_numpy(table[blk] * self.block_size + pos % self.block_size)

    def block_table_tensor(self, seq_ids, width=None) -> torch.Tensor:
        """[B, width] int32 block tables; rows past a table's end are 0 (never read: the
        kernels stop at seq_lens)."""
        w = max((len(self.tables[s]) for s in seq_ids), default=0) if width is None else width
        out = np.zeros((len(seq_ids), w), dtype=np.int32)
        for i, s in enumerate(seq_ids):
            t = self.tables[s]
            if len(t) > w:
                raise ValueError(f"seq {s} has {len(t)} blocks > width {w}")
            out[i, :len(t)] = t
        return torch.from_numpy(out)
