"""Which fixed-size blocks of the KV pool each sequence owns (CPU bookkeeping).

Same contract as the reference's BlockManager (engine/block_manager.py:19-137), because block-table indexing
must be bit-exact with it:
  - a token's slot is table[p // B] * B + p % B;
  - free blocks form a LIFO stack that initially hands out block 0, then 1, ...; a freed sequence's blocks go
    back in reverse table order, so the next allocation receives them in their old table order, and long-lived
    pools end up with scattered, non-monotonic tables;
  - per-block reference counts (0 or 1 without sharing), free listeners, OutOfBlocks leaves state unchanged.
"""

from __future__ import annotations

from typing import Callable

import numpy as np


class OutOfBlocks(RuntimeError):
    """A request needed more free blocks than the pool had; the manager is left as it was before the call."""


class BlockManager:
    def __init__(self, num_blocks: int, block_size: int = 16):
        """A pool of num_blocks blocks of block_size tokens, all free."""
        if num_blocks < 1 or block_size < 1:
            raise ValueError(f"a pool needs num_blocks >= 1 and block_size >= 1, got {num_blocks} and {block_size}")
        self.num_blocks, self.block_size = num_blocks, block_size
        # The top of the stack is the end of the list: block 0 is handed out first.
        self._free: list[int] = list(reversed(range(num_blocks)))
        self._ref = [0] * num_blocks
        self._tables: dict[int, list[int]] = {}
        self._lengths: dict[int, int] = {}
        # int32 mirror of every table (capacity doubles as it grows), so per-forward metadata is built with array
        # copies instead of Python list work: _arrays[seq][:len(table)] == table.
        self._arrays: dict[int, np.ndarray] = {}
        self._free_listeners: list[Callable[[list[int]], None]] = []
        self._table_listeners: list[Callable[[int, int], None]] = []

    # ---- queries -------------------------------------------------------------------------------------------------

    def blocks_for(self, n_tokens: int) -> int:
        """ceil(n_tokens / block_size)."""
        return (n_tokens + self.block_size - 1) // self.block_size

    def num_free_blocks(self) -> int:
        """Blocks owned by no sequence."""
        return len(self._free)

    def can_allocate(self, n_tokens: int, watermark_blocks: int = 0) -> bool:
        """Whether a new sequence of n_tokens fits while keeping watermark_blocks free."""
        return self.blocks_for(n_tokens) + watermark_blocks <= len(self._free)

    def new_blocks_needed(self, seq_id: int, n: int = 1) -> int:
        """Blocks that appending n tokens to seq_id takes from the free stack."""
        return self.blocks_for(self._lengths[seq_id] + n) - len(self._tables[seq_id])

    def can_append(self, seq_id: int, n: int = 1) -> bool:
        """Whether n more tokens fit for seq_id."""
        return self.new_blocks_needed(seq_id, n) <= len(self._free)

    def ref_count(self, block: int) -> int:
        """Sequences holding `block`."""
        return self._ref[block]

    def block_table(self, seq_id: int) -> list[int]:
        """The sequence's blocks in token order (a copy)."""
        return self._tables[seq_id][:]

    def seq_len(self, seq_id: int) -> int:
        """Tokens the sequence holds."""
        return self._lengths[seq_id]

    def seq_ids(self) -> list[int]:
        """Live sequences."""
        return list(self._tables)

    def table_array(self, seq_id: int) -> np.ndarray:
        """The sequence's blocks in token order as a read-only int32 array view (valid until its next change)."""
        v = self._arrays[seq_id][:len(self._tables[seq_id])]
        v.flags.writeable = False
        return v

    def _mirror_extend(self, seq_id: int, blocks: list[int]) -> None:
        arr = self._arrays.get(seq_id)
        n = len(self._tables[seq_id])  # table length after the extension
        if arr is None or arr.shape[0] < n:
            grown = np.empty(max(16, 2 * n), dtype=np.int32)
            if arr is not None:
                grown[:n - len(blocks)] = arr[:n - len(blocks)]
            arr = self._arrays[seq_id] = grown
        arr[n - len(blocks):n] = blocks
        for fn in self._table_listeners:
            fn(seq_id, n - len(blocks))

    def slots(self, seq_id: int, start: int, end: int) -> list[int]:
        """Slots of positions [start, end) of the sequence."""
        n = self._lengths[seq_id]
        if not (0 <= start <= end <= n):
            raise ValueError(f"sequence {seq_id} holds {n} tokens; slots of positions {start}..{end - 1} asked for")
        table, B = self._tables[seq_id], self.block_size
        return [table[p // B] * B + p % B for p in range(start, end)]

    # ---- mutations -----------------------------------------------------------------------------------------------

    def add_free_listener(self, fn: Callable[[list[int]], None]) -> None:
        """Call fn(blocks) with the blocks each free() returns to the stack."""
        self._free_listeners.append(fn)

    def add_table_listener(self, fn: Callable[[int, int], None]) -> None:
        """Call fn(seq_id, first) when a sequence's table is created (first = 0) or gains blocks from index first
        on, and fn(seq_id, -1) when the sequence is freed (no counterpart in the reference: device-side copies
        of the tables follow these changes)."""
        self._table_listeners.append(fn)

    def remove_table_listener(self, fn: Callable[[int, int], None]) -> None:
        """Stop calling fn (added by add_table_listener)."""
        self._table_listeners.remove(fn)

    def _pop_blocks(self, count: int) -> list[int]:
        taken = self._free[len(self._free) - count:][::-1]  # top of the stack first
        del self._free[len(self._free) - count:]
        for b in taken:
            if self._ref[b]:
                raise AssertionError(f"block {b} came off the free stack while {self._ref[b]} sequence(s) hold it")
            self._ref[b] = 1
        return taken

    def allocate(self, seq_id: int, n_tokens: int) -> list[int]:
        """Create seq_id holding n_tokens (>= 0) and return their slots."""
        if seq_id in self._tables:
            raise ValueError(f"sequence {seq_id} is already live")
        if n_tokens < 0:
            raise ValueError(f"a sequence cannot hold {n_tokens} tokens")
        need = self.blocks_for(n_tokens)
        if need > len(self._free):
            raise OutOfBlocks(f"a new sequence of {n_tokens} tokens takes {need} blocks; the pool has "
                              f"{len(self._free)} free")
        self._tables[seq_id] = self._pop_blocks(need)
        self._lengths[seq_id] = n_tokens
        self._mirror_extend(seq_id, self._tables[seq_id])
        return self.slots(seq_id, 0, n_tokens)

    def append_slots(self, seq_id: int, n: int = 1) -> list[int]:
        """Extend seq_id by n tokens and return their slots."""
        need = self.new_blocks_needed(seq_id, n)
        if need > len(self._free):
            raise OutOfBlocks(f"{n} more tokens for sequence {seq_id} take {need} blocks; the pool has "
                              f"{len(self._free)} free")
        new = self._pop_blocks(need)
        self._tables[seq_id].extend(new)
        if new:
            self._mirror_extend(seq_id, new)
        start = self._lengths[seq_id]
        self._lengths[seq_id] = start + n
        return self.slots(seq_id, start, start + n)

    def append_slot(self, seq_id: int) -> int:
        """Extend seq_id by one token and return its slot."""
        return self.append_slots(seq_id, 1)[0]

    def free(self, seq_id: int) -> None:
        """Release seq_id; a block returns to the stack when its reference count reaches 0."""
        table = self._tables.pop(seq_id)
        del self._lengths[seq_id]
        self._arrays.pop(seq_id, None)
        released = []
        for b in table[::-1]:  # last block first, so the stack hands the blocks out again in table order
            self._ref[b] -= 1
            if self._ref[b] < 0:
                raise AssertionError(f"block {b} released more often than it was taken")
            if self._ref[b] == 0:
                self._free.append(b)
                released.append(b)
        for fn in self._free_listeners:
            fn(released)
        for fn in self._table_listeners:
            fn(seq_id, -1)

    # ---- checking ------------------------------------------------------------------------------------------------

    def check_invariants(self) -> None:
        """Raise AssertionError unless the bookkeeping is consistent: each block is on the free stack exactly when
        no table holds it, reference counts equal the number of holding tables, every table has the blocks its
        length needs, and the int32 mirrors match the tables."""
        def fail(msg: str) -> None:
            raise AssertionError(msg)

        free = set(self._free)
        if len(free) != len(self._free):
            fail("the free stack holds some block more than once")
        owners = np.zeros(self.num_blocks, dtype=np.int64)
        for seq_id, table in self._tables.items():
            if len(table) != self.blocks_for(self._lengths[seq_id]):
                fail(f"sequence {seq_id} holds {len(table)} blocks for {self._lengths[seq_id]} tokens")
            if self._arrays[seq_id][:len(table)].tolist() != table:
                fail(f"the int32 mirror of sequence {seq_id} is out of date")
            np.add.at(owners, np.asarray(table, dtype=np.int64), 1)
        for b in range(self.num_blocks):
            n = int(owners[b])
            if n != self._ref[b]:
                fail(f"block {b} has reference count {self._ref[b]} but {n} holding tables")
            if (b in free) == (n > 0):
                fail(f"block {b} is {'both free and held' if n else 'neither free nor held'}")
