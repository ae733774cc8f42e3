"""Decode steps replayed from HIP graphs: the whole forward of a batch of one-token rows (embedding, every layer's
GEMMs, the HIP store and paged-decode launches, the LM head) captured once per batch-size bucket and replayed with
one host-to-device copy of the step's metadata.

The reference launches every kernel of a decode step from Python (about 800 launches per step for Qwen2.5-0.5B,
reference README.md:144,172 and docs/implementation-plan.md:126), so small-batch steps are bound by launch
overhead. Capture needs every launch to be shape-static and every pointer fixed: the metadata lives in persistent
device buffers (one int64 and one int32 buffer, refilled by one copy each from pinned host memory), the decode
launches run on the split grid sized for the runner's max_context (a sequence's splits past its own context exit
at once; no per-step work list), and rows past the live batch are padding that writes to and reads from a
scratch block the runner reserves from the block manager.

The cache keeps its begin / write / attend interface: the runner hands it PagedMetadata whose device fields are
views of the persistent buffers and whose host context lengths are max_context for every row, which is what fixes
the decode grid. Pools of the model dtype and INT8 format "int8" (per-token scales) are supported; format
"int8-kchannel" plans its staging writes on the host each forward and is not captured.
"""

from __future__ import annotations

import numpy as np
import torch

from .block_manager import BlockManager
from .paged_cache import PagedKVCache, PagedMetadata, PerSequence

SCRATCH_SEQ = -(1 << 40)  # the runner's own sequence id in the block manager: the padding rows' block


def _not_kept(i: int):
    raise RuntimeError("per-sequence block lists are not kept by the graph runner (its rows are decode rows)")


class DecodeGraphRunner:
    """Replays captured decode steps of `model` through `cache` for batches of up to max_batch sequences whose
    contexts stay within max_context tokens."""

    def __init__(self, model, cache: PagedKVCache, manager: BlockManager, max_batch: int, max_context: int,
                 buckets: list[int] | None = None):
        if not cache.on_gpu or cache.attn_backend not in ("hip", "triton"):
            raise ValueError("graph capture needs a GPU cache on the HIP backend")
        if getattr(cache, "fmt", "int8") != "int8":
            raise ValueError("format int8-kchannel plans staging writes per forward and cannot be captured")
        if max_batch < 1 or max_context < 1:
            raise ValueError("max_batch and max_context must be positive")
        self.model, self.cache, self.manager = model, cache, manager
        self.max_batch, self.max_context = max_batch, max_context
        B = cache.block_size
        self.B, self.width = B, -(-max_context // B)
        self.buckets = sorted(buckets or [b for b in (1, 2, 4, 8, 16, 32, 64, 128, 256, 512, 1024, 2048)
                                          if b < max_batch] + [max_batch])
        if self.buckets[-1] < max_batch or self.buckets[0] < 1:
            raise ValueError("buckets must cover 1 .. max_batch")
        manager.allocate(SCRATCH_SEQ, 1)
        self.scratch_block = int(manager.table_array(SCRATCH_SEQ)[0])
        dev = cache.device
        n = max_batch
        # int64: ids, positions, slots, slot blocks, slot offsets, last-token rows; int32: tables, context lengths
        self._h64 = torch.empty(6 * n, dtype=torch.int64, pin_memory=True)
        self._h32 = torch.empty(n * self.width + n, dtype=torch.int32, pin_memory=True)
        self._n64, self._n32 = self._h64.numpy(), self._h32.numpy()  # numpy views of the pinned buffers
        self._d64 = torch.empty(6 * n, dtype=torch.int64, device=dev)
        self._d32 = torch.empty(n * self.width + n, dtype=torch.int32, device=dev)
        self._copied = torch.cuda.Event()
        self._graphs: dict[int, tuple[torch.cuda.CUDAGraph, torch.Tensor]] = {}
        self._pool = None
        self._stream = torch.cuda.Stream(device=dev)  # capture stream (default priority)
        self._fill_padding(0)
        self._upload()

    # ---- persistent metadata ------------------------------------------------------------------------------------

    def _views(self, bucket: int):
        n, w = self.max_batch, self.width
        d64, d32 = self._d64, self._d32
        return (d64[:bucket], d64[n:n + bucket], d64[2 * n:2 * n + bucket], d64[3 * n:3 * n + bucket],
                d64[4 * n:4 * n + bucket], d64[5 * n:5 * n + bucket],
                d32[:bucket * w].view(bucket, w), d32[n * w:n * w + bucket])

    def _meta(self, bucket: int) -> PagedMetadata:
        ids, pos, slots, blocks, offs, last, bt, ctx = self._views(bucket)
        no_rows = PerSequence(bucket, _not_kept)
        return PagedMetadata(
            num_tokens=bucket, query_starts=list(range(bucket + 1)), context_lens=[self.max_context] * bucket,
            positions=pos, slots_cpu=[], slot_mapping=slots, slot_blocks=blocks, slot_offsets=offs,
            block_ids=no_rows, block_ids_cpu=no_rows, block_tables=bt, context_lens_t=ctx, last_token_indices=last)

    def _fill_padding(self, first: int) -> None:
        """Rows first .. max_batch - 1: token 0 at position 0 in slot 0 of the scratch block, one key of context."""
        n, w, h64, h32 = self.max_batch, self.width, self._n64, self._n32
        h64[first:n] = 0
        h64[n + first:2 * n] = 0
        h64[2 * n + first:3 * n] = self.scratch_block * self.B
        h64[3 * n + first:4 * n] = self.scratch_block
        h64[4 * n + first:5 * n] = 0
        h64[5 * n + first:6 * n] = np.arange(first, n)
        bt = h32[:n * w].reshape(n, w)
        bt[first:] = -1
        bt[first:, 0] = self.scratch_block
        h32[n * w + first:n * w + n] = 1

    def _upload(self) -> None:
        self._d64.copy_(self._h64, non_blocking=True)
        self._d32.copy_(self._h32, non_blocking=True)
        self._copied.record()

    def _fill(self, seq_ids: list[int]) -> None:
        """This step's rows: each sequence's newest token (its slot already appended) at position len - 1."""
        self._copied.synchronize()  # the previous step's copy has left the pinned buffers
        n, w, B, b = self.max_batch, self.width, self.B, len(seq_ids)
        h64, h32 = self._n64, self._n32
        bt = h32[:n * w].reshape(n, w)
        lens = np.empty(b, dtype=np.int64)
        blocks = np.empty(b, dtype=np.int64)
        for i, s in enumerate(seq_ids):
            ctx = self.manager.seq_len(s)
            if not 1 <= ctx <= self.max_context:
                raise ValueError(f"sequence {s}: context {ctx} outside 1 .. {self.max_context}")
            table = self.manager.table_array(s)
            nb = -(-ctx // B)
            bt[i, :nb] = table[:nb]
            bt[i, nb:] = -1
            lens[i] = ctx
            blocks[i] = table[(ctx - 1) // B]
        p = lens - 1
        h64[n:n + b] = p
        h64[2 * n:2 * n + b] = blocks * B + p % B
        h64[3 * n:3 * n + b] = blocks
        h64[4 * n:4 * n + b] = p % B
        h64[5 * n:5 * n + b] = np.arange(b)
        h32[n * w:n * w + b] = lens

    # ---- capture and replay -------------------------------------------------------------------------------------

    def _bucket(self, b: int) -> int:
        for k in self.buckets:
            if k >= b:
                return k
        raise ValueError(f"batch {b} exceeds max_batch {self.max_batch}")

    def _forward(self, bucket: int) -> torch.Tensor:
        ids, pos = self._views(bucket)[:2]
        return self.model.forward(ids, pos, self.cache, self._meta(bucket))

    def capture(self, bucket: int) -> None:
        """Record the decode step of `bucket` rows (one eager warm-up step on the capture stream first, which
        builds the launch plans and the split workspace outside the graph). Reads and writes only the scratch
        block when the persistent buffers hold padding."""
        if bucket in self._graphs:
            return
        self._copied.synchronize()
        self._fill_padding(0)
        self._upload()
        s = self._stream
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            self._forward(bucket)
        s.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, pool=self._pool, stream=s):
            logits = self._forward(bucket)
        torch.cuda.current_stream().wait_stream(s)
        if self._pool is None:
            self._pool = g.pool()
        self._graphs[bucket] = (g, logits)

    def step(self, seq_ids: list[int], input_ids: torch.Tensor, graph: bool = True) -> torch.Tensor:
        """Logits [len(seq_ids), vocab] of one decode step: row i is sequence seq_ids[i]'s newest token
        (input_ids[i], at position manager.seq_len(s) - 1; the caller has appended its slot). graph=False runs the
        same static-shape step eagerly (the graph's reference)."""
        b = len(seq_ids)
        if input_ids.shape != (b,):
            raise ValueError("one input id per sequence")
        bucket = self._bucket(b)
        if graph and bucket not in self._graphs:
            self.capture(bucket)
        self._fill(seq_ids)
        self._fill_padding(b)
        self._upload()
        # the token ids go device to device (the previous step's argmax need not visit the host)
        self._d64[:b].copy_(input_ids.to(self._d64.device, torch.int64), non_blocking=True)
        if not graph:
            return self._forward(bucket)[:b]
        g, logits = self._graphs[bucket]
        g.replay()
        return logits[:b]

    def close(self) -> None:
        """Drop the graphs and return the scratch block to the manager."""
        self._graphs.clear()
        self.manager.free(SCRATCH_SEQ)
