"""Block tables kept on the device, and per-forward metadata derived there in one launch.

The reference rebuilds every forward's packed metadata on the host from Python lists and ships it in 8 + S
host-to-device copies (engine/paged_cache.py:55-90); at batch 512 that is tens of milliseconds per step. Here each
live sequence owns one row of a persistent device table that follows the block manager's changes (a decode step
uploads only the blocks sequences gained since the last step, one copy and one scatter), and
`sipa_paged_metadata` derives positions, slots, the packed -1 padded tables, context lengths and last-token rows
from the forward's (row, start, query start) triples, uploaded in one copy. The result is a PagedMetadata with the
same contents as build_metadata's, so the caches' begin / write / attend run on it unchanged.
"""

from __future__ import annotations

import ctypes
from collections.abc import Sequence

import numpy as np
import torch

from . import _hip
from .block_manager import BlockManager
from .paged_cache import PagedMetadata, PerSequence


class _LazyList(Sequence):
    """A list made by `make()` on first access (the host-side slot list, which only INT8 format B reads)."""

    def __init__(self, n: int, make):
        self._n, self._make, self._list = n, make, None

    def _get(self) -> list:
        if self._list is None:
            self._list = self._make()
        return self._list

    def __len__(self) -> int:
        return self._n

    def __getitem__(self, i):
        return self._get()[i]

    def __eq__(self, other) -> bool:
        return self._get() == list(other)

    def __repr__(self) -> str:
        return repr(self._get())


class DeviceBlockTables:
    """Device copies of the block tables of `manager`'s live sequences (one row each, up to max_seqs sequences of
    up to max_blocks blocks), kept current through the manager's table listener."""

    def __init__(self, manager: BlockManager, device: str | torch.device, max_seqs: int, max_blocks: int):
        if max_seqs < 1 or max_blocks < 1:
            raise ValueError("max_seqs and max_blocks must be positive")
        self.manager, self.device = manager, torch.device(device)
        self.max_seqs, self.max_blocks = max_seqs, max_blocks
        self.table = torch.full((max_seqs, max_blocks), -1, dtype=torch.int32, device=self.device)
        self._row_of: dict[int, int] = {}
        self._free_rows = list(reversed(range(max_seqs)))
        self._dirty: dict[int, int] = {}  # sequence -> first table column changed since the last sync
        manager.add_table_listener(self._on_change)
        for seq in manager.seq_ids():
            self._on_change(seq, 0)

    def close(self) -> None:
        """Stop following the block manager."""
        self.manager.remove_table_listener(self._on_change)

    def row(self, seq_id: int) -> int:
        """The table row of a live sequence."""
        return self._row_of[seq_id]

    def _on_change(self, seq_id: int, first: int) -> None:
        if first < 0:  # freed: its row returns to the pool (its stale entries are never read: rows are rebuilt)
            row = self._row_of.pop(seq_id, None)
            self._dirty.pop(seq_id, None)
            if row is not None:
                self._free_rows.append(row)
            return
        if seq_id not in self._row_of:
            if not self._free_rows:
                raise RuntimeError(f"more than {self.max_seqs} live sequences for the device block tables")
            self._row_of[seq_id] = self._free_rows.pop()
            first = 0
        self._dirty[seq_id] = min(self._dirty.get(seq_id, first), first)

    def sync(self) -> None:
        """Copy every table entry changed since the last sync to the device: one upload, one scatter."""
        if not self._dirty:
            return
        flat, vals = [], []
        W = self.max_blocks
        for seq, first in self._dirty.items():
            arr = self.manager.table_array(seq)[:W]  # a longer sequence keeps its first W blocks (build refuses it)
            if arr.shape[0] > first:
                row = self._row_of[seq]
                flat.append(np.arange(row * W + first, row * W + arr.shape[0], dtype=np.int64))
                vals.append(arr[first:].astype(np.int64))
        self._dirty.clear()
        if not flat:
            return
        both = torch.from_numpy(np.stack([np.concatenate(flat), np.concatenate(vals)])).to(self.device)
        self.table.view(-1)[both[0]] = both[1].to(torch.int32)

    def build(self, batch: list[tuple[int, int, int]]) -> PagedMetadata:
        """Metadata for a forward over batch = [(seq_id, start, n), ...], with build_metadata's contents and
        errors (reference engine/paged_cache.py:55-90), derived on the device."""
        S = len(batch)
        if S == 0:
            raise ValueError("a forward needs at least one sequence")
        m, B = self.manager, self.manager.block_size
        seqs = [b[0] for b in batch]
        starts = np.fromiter((b[1] for b in batch), dtype=np.int64, count=S)
        counts = np.fromiter((b[2] for b in batch), dtype=np.int64, count=S)
        held = np.fromiter((m.seq_len(s) for s in seqs), dtype=np.int64, count=S)
        ctx = starts + counts
        bad = np.flatnonzero((counts < 1) | (held < ctx) | (starts < 0))
        if bad.size:
            i = int(bad[0])
            if counts[i] < 1:
                raise ValueError(f"sequence {seqs[i]}: a forward needs at least one new token")
            if held[i] < ctx[i]:
                raise ValueError(f"sequence {seqs[i]} holds {held[i]} tokens, forward needs {ctx[i]}")
            raise ValueError(f"sequence {seqs[i]}: negative start {starts[i]}")
        if int(ctx.max()) > self.max_blocks * B:
            i = int(np.argmax(ctx))
            raise ValueError(f"sequence {seqs[i]}: context {ctx[i]} exceeds the device tables' "
                             f"{self.max_blocks * B} tokens")
        self.sync()
        rows = np.fromiter((self._row_of[s] for s in seqs), dtype=np.int64, count=S)
        qs = np.zeros(S + 1, dtype=np.int64)
        np.cumsum(counts, out=qs[1:])
        T = int(qs[-1])
        width = int(-(-ctx.max() // B))
        info = torch.from_numpy(np.concatenate([rows, starts, qs]).astype(np.int32)).to(self.device)
        d64 = torch.empty(4 * T + S, dtype=torch.int64, device=self.device)
        d32 = torch.empty(S * width + S, dtype=torch.int32, device=self.device)
        p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
        _hip.check(_hip.lib().sipa_paged_metadata(
            p(self.table), self.table.stride(0), self.max_seqs, self.max_blocks, p(info), S, T, B, width,
            p(d64), p(d64[T:]), p(d64[2 * T:]), p(d64[3 * T:]), p(d64[4 * T:]), p(d32), p(d32[S * width:]),
            _hip.stream_of(d64)), "paged metadata")
        tables = [m.table_array(s) for s in seqs]  # views, valid for this forward
        nbs = (-(-ctx // B)).tolist()

        def slot_list() -> list[int]:
            out: list[int] = []
            for t, st, n in zip(tables, starts.tolist(), counts.tolist()):
                pos = np.arange(st, st + n, dtype=np.int64)
                out.extend((t[pos // B].astype(np.int64) * B + pos % B).tolist())
            return out

        return PagedMetadata(
            num_tokens=T,
            query_starts=qs.tolist(),
            context_lens=ctx.tolist(),
            positions=d64[:T],
            slots_cpu=_LazyList(T, slot_list),
            slot_mapping=d64[T:2 * T],
            slot_blocks=d64[2 * T:3 * T],
            slot_offsets=d64[3 * T:4 * T],
            block_ids=PerSequence(S, lambda i: torch.from_numpy(tables[i][:nbs[i]].astype(np.int64)).to(self.device)),
            block_ids_cpu=PerSequence(S, lambda i: tables[i][:nbs[i]].tolist()),
            block_tables=d32[:S * width].view(S, width),
            context_lens_t=d32[S * width:],
            last_token_indices=d64[4 * T:],
        )
