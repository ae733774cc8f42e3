"""Decode steps replayed from HIP graphs: the whole forward of a batch of one-token rows (embedding, every layer's
GEMMs, the HIP store and paged-decode launches, the LM head) captured once per batch-size bucket and replayed after
one small upload and one metadata launch.

The reference launches every kernel of a decode step from Python (about 800 launches per step for Qwen2.5-0.5B,
reference README.md:144,172 and docs/implementation-plan.md:126), so small-batch steps are bound by launch
overhead. Capture needs every launch to be shape-static and every pointer fixed: the metadata lives in persistent
device buffers, derived before each replay from the device block tables by one sipa_paged_metadata launch (the
host uploads only the step's (table row, position) pairs); the decode launches run on the split grid sized for
the runner's max_context (a sequence's splits past its own context exit at once; no per-step work list); and
rows past the live batch are padding that writes to and reads from a scratch block the runner reserves from the
block manager.

The cache keeps its begin / write / attend interface: the runner hands it PagedMetadata whose device fields are
views of the persistent buffers and whose host context lengths are max_context for every row, which is what fixes
the decode grid. Pools of the model dtype and both INT8 formats are supported. Format "int8-kchannel" keeps each
sequence's partial last block of K in a bf16 staging slot; its per-step staging plan (slot per row, the block
each row's slot is quantized into, the tail slot the decode reads) is kept by the cache's host bookkeeping as in
an eager forward and uploaded with the step's other host data, and the captured write stages every row and
quantizes every row's slot, into the row's block when the row completes it and into the scratch block otherwise.
"""

from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import _hip
from .block_manager import BlockManager
from .device_tables import DeviceBlockTables
from .hip_decode import decode_workspace_bytes, reserve_workspace
from .paged_cache import PagedKVCache, PagedMetadata, PerSequence

SCRATCH_SEQ = -(1 << 40)  # the runner's own sequence id in the block manager: the padding rows' block


def _not_kept(i: int):
    raise RuntimeError("per-sequence block lists are not kept by the graph runner (its rows are decode rows)")


class DecodeGraphRunner:
    """Replays captured decode steps of `model` through `cache` for batches of up to max_batch sequences whose
    contexts stay within max_context tokens. The block tables live on the device (`device_tables`, made here for
    up to max_seqs live sequences when not given), and each step's metadata is derived there by one
    sipa_paged_metadata launch into the graph's persistent buffers."""

    def __init__(self, model, cache: PagedKVCache, manager: BlockManager, max_batch: int, max_context: int,
                 buckets: list[int] | None = None, device_tables: DeviceBlockTables | None = None,
                 max_seqs: int | None = None):
        if not cache.on_gpu or cache.attn_backend not in ("hip", "triton"):
            raise ValueError("graph capture needs a GPU cache on the HIP backend")
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
        dev = cache.device
        self._own_tables = device_tables is None
        if device_tables is None:
            device_tables = DeviceBlockTables(manager, dev, max_seqs or 4 * max_batch + 1, self.width)
        if device_tables.max_blocks < self.width:
            raise ValueError(f"device tables of {device_tables.max_blocks} blocks cannot hold {max_context} tokens")
        self.tables = device_tables
        manager.allocate(SCRATCH_SEQ, 1)
        n = max_batch
        # persistent step buffers. int64: ids, positions, slots, slot blocks, slot offsets, last-token rows;
        # int32: block tables [n, width], context lengths
        self._d64 = torch.zeros(6 * n, dtype=torch.int64, device=dev)
        self._d32 = torch.empty(n * self.width + n, dtype=torch.int32, device=dev)
        # the step's (row, start, query start) triples, uploaded in one copy from pinned memory
        self._hinfo = torch.empty(3 * n + 1, dtype=torch.int32, pin_memory=True)
        self._ninfo = self._hinfo.numpy()
        self._dinfo = torch.empty(3 * n + 1, dtype=torch.int32, device=dev)
        self._copied = torch.cuda.Event()
        self._kchannel = getattr(cache, "fmt", None) == "int8-kchannel"
        self._plan = None
        if self._kchannel:
            # format B's staging plan: int64 stage slots, quantization sources, quantization destinations
            # [3n] and int32 tail slots [n], one pinned copy each; rows 0 .. n - 1 are the stage writes' sources
            self._hplan = torch.empty(3 * n, dtype=torch.int64, pin_memory=True)
            self._htail = torch.empty(n, dtype=torch.int32, pin_memory=True)
            self._dplan = torch.zeros(3 * n, dtype=torch.int64, device=dev)
            self._dtail = torch.zeros(n, dtype=torch.int32, device=dev)
            self._plan = (torch.arange(n, dtype=torch.int64, device=dev), self._dplan[:n], self._dplan[n:2 * n],
                          self._dplan[2 * n:], self._dtail)
        # per bucket: the graph, its logits buffer, and the split workspace its decode launches write
        self._graphs: dict[int, tuple[torch.cuda.CUDAGraph, torch.Tensor, torch.Tensor | None]] = {}
        self._pool = None
        self._stream = torch.cuda.Stream(device=dev)  # capture stream (default priority)
        # A graph keeps the raw address of the capture stream's split workspace. The buffer is sized here for the
        # largest bucket's decode launches, so no later capture replaces it while earlier graphs still use it.
        cfg = cache.cfg
        mode = {"int8": 1, "int8-kchannel": 2}.get(getattr(cache, "fmt", None), 0)
        self._ws_bytes = max(decode_workspace_bytes(b, cfg.num_q_heads, cfg.num_kv_heads, cfg.head_dim, max_context,
                                                    mode) for b in self.buckets)
        self._workspace = reserve_workspace(torch.device(dev), self._stream.cuda_stream, self._ws_bytes)
        self._prepare([], max_batch)

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

    def _prepare(self, seq_ids: list[int], bucket: int) -> None:
        """Write the metadata of a step over seq_ids (each sequence's newest token, its slot already appended, at
        position len - 1) padded to `bucket` rows into the persistent buffers: rows past the batch read and write
        position 0 of the runner's scratch sequence."""
        b = len(seq_ids)
        m = self.manager
        lens = np.fromiter((m.seq_len(s) for s in seq_ids), dtype=np.int64, count=b)
        bad = np.flatnonzero((lens < 1) | (lens > self.max_context))
        if bad.size:
            i = int(bad[0])
            raise ValueError(f"sequence {seq_ids[i]}: context {lens[i]} outside 1 .. {self.max_context}")
        self._copied.synchronize()  # the previous step's copy has left the pinned buffer
        info = self._ninfo
        info[:b] = np.fromiter((self.tables.row(s) for s in seq_ids), dtype=np.int64, count=b)
        info[b:bucket] = self.tables.row(SCRATCH_SEQ)
        info[bucket:bucket + b] = lens - 1
        info[bucket + b:2 * bucket] = 0
        info[2 * bucket:3 * bucket + 1] = np.arange(bucket + 1)
        self._dinfo[:3 * bucket + 1].copy_(self._hinfo[:3 * bucket + 1], non_blocking=True)
        if self._kchannel:
            self._stage_plan(seq_ids, lens, bucket)
        self._copied.record()
        self.tables.sync()
        ids, pos, slots, blocks, offs, last, bt, ctx = self._views(bucket)
        p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
        _hip.check(_hip.lib().sipa_paged_metadata(
            p(self.tables.table), self.tables.table.stride(0), self.tables.max_seqs, self.tables.max_blocks,
            p(self._dinfo), bucket, bucket, self.B, self.width, p(pos), p(slots), p(blocks), p(offs), p(last),
            p(bt), p(ctx), _hip.stream_of(self._d64)), "graph runner metadata")

    def _stage_plan(self, seq_ids: list[int], lens: np.ndarray, bucket: int) -> None:
        """Format B: the step's staging plan from the cache's slot bookkeeping (row i writes position lens[i] - 1
        of its sequence; padding rows write offset 0 of the scratch block, whose staging slot stays held),
        uploaded into the persistent plan buffers."""
        B, m, n = self.B, self.manager, self.max_batch
        blocks = [int(m.table_array(s)[(int(L) - 1) // B]) for s, L in zip(seq_ids, lens)]
        offsets = [(int(L) - 1) % B for L in lens]
        scratch = int(m.table_array(SCRATCH_SEQ)[0])
        pad = bucket - len(seq_ids)
        slots, src, dst, tails = self.cache.plan_static_decode(blocks + [scratch] * pad, offsets + [0] * pad,
                                                               scratch)
        h = self._hplan.numpy()
        h[:bucket], h[n:n + bucket], h[2 * n:2 * n + bucket] = slots, src, dst
        self._htail.numpy()[:bucket] = tails
        self._dplan.copy_(self._hplan, non_blocking=True)
        self._dtail.copy_(self._htail, non_blocking=True)

    # ---- capture and replay -------------------------------------------------------------------------------------

    def _bucket(self, b: int) -> int:
        for k in self.buckets:
            if k >= b:
                return k
        raise ValueError(f"batch {b} exceeds max_batch {self.max_batch}")

    def _forward(self, bucket: int) -> torch.Tensor:
        ids, pos = self._views(bucket)[:2]
        if self._plan is None:
            return self.model.forward(ids, pos, self.cache, self._meta(bucket))
        self.cache.use_static_plan(self._plan)  # only this forward's begin() takes the persistent plan
        try:
            return self.model.forward(ids, pos, self.cache, self._meta(bucket))
        finally:
            self.cache.use_static_plan(None)

    def capture(self, bucket: int) -> None:
        """Record the decode step of `bucket` rows (one eager warm-up step on the capture stream first, which
        builds the launch plans and the split workspace outside the graph). Reads and writes only the scratch
        block when the persistent buffers hold padding."""
        if bucket in self._graphs:
            return
        self._prepare([], bucket)
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
        plan = getattr(self.cache, "_plan", None)  # the decode plan the captured layers launched
        ws = getattr(plan, "workspace", None)
        if ws is not None and ws.data_ptr() != self._workspace.data_ptr():
            raise RuntimeError("the captured decode used a split workspace the runner did not reserve")
        self._graphs[bucket] = (g, logits, ws)

    def step(self, seq_ids: list[int], input_ids: torch.Tensor, graph: bool = True) -> torch.Tensor:
        """Logits [len(seq_ids), vocab] of one decode step: row i is sequence seq_ids[i]'s newest token
        (input_ids[i], at position manager.seq_len(s) - 1; the caller has appended its slot). graph=False runs the
        same static-shape step eagerly (the graph's reference)."""
        b = len(seq_ids)
        if input_ids.shape != (b,):
            raise ValueError("one input id per sequence")
        if len(set(seq_ids)) != b:
            raise ValueError("a decode step holds each sequence once")
        bucket = self._bucket(b)
        if graph and bucket not in self._graphs:
            self.capture(bucket)
        self._prepare(seq_ids, bucket)
        # the token ids go device to device (the previous step's argmax need not visit the host)
        self._d64[:b].copy_(input_ids.to(self._d64.device, torch.int64), non_blocking=True)
        if not graph:
            return self._forward(bucket)[:b]
        g, logits, _ = self._graphs[bucket]
        g.replay()
        return logits[:b]

    def close(self) -> None:
        """Drop the graphs, return the scratch block to the manager, and detach device tables made here."""
        self._graphs.clear()
        self.manager.free(SCRATCH_SEQ)
        if self._own_tables:
            self.tables.close()
