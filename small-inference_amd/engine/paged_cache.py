"""Paged KV cache: the block pool, per-forward packed metadata, and the begin / write / attend interface the
model calls (drop-in for the reference's engine/paged_cache.py:28-180).

Pool layout per layer: K and V as [H_kv, num_blocks, block_size, d] ([2, N, 16, 64] for Qwen2.5-0.5B); one
(head, block) is 16 x 64 x 2 B = 2 KiB contiguous in HBM, the unit the decode kernel streams. A token's slot
(block * B + offset) addresses [:, block, offset] in every layer.

Backends (attn_backend, mutable after construction):
  "hip"    decode rows (one new token per sequence) go through the HIP paged-decode kernel in one launch per
           layer, and rows with several new tokens (prefill chunks) through the HIP paged-prefill kernel in one
           more, both reading blocks in place; shapes the prefill kernel does not cover use the gather path.
  "triton" the reference's name for the same in-place decode backend: selects the HIP kernel, so callers that
           pass it (the reference's ContinuousEngine defaults to it) run unchanged.
  "gather" every sequence gathers its blocks and runs attention() (the reference's default).
On a GPU pool, write() scatters K and V with one HIP store launch; a CPU pool uses torch indexing.
"""

from __future__ import annotations

from collections.abc import Callable, Sequence
from dataclasses import dataclass

import numpy as np
import torch

from .attention import attention
from .block_manager import BlockManager
from .config import ModelConfig

BACKENDS = ("gather", "hip", "triton")
KERNEL_BACKENDS = ("hip", "triton")


class PerSequence(Sequence):
    """A per-sequence list whose entries are made on first access and kept: the kernel path of a forward reads
    none of them, the gather path only its own sequences'. Indexes, iterates and compares like a list."""

    def __init__(self, n: int, make: Callable[[int], object]):
        self._n, self._make = n, make
        self._made: dict[int, object] = {}

    def __len__(self) -> int:
        return self._n

    def __getitem__(self, i):
        if isinstance(i, slice):
            return [self[j] for j in range(*i.indices(self._n))]
        if i < 0:
            i += self._n
        if not 0 <= i < self._n:
            raise IndexError(i)
        if i not in self._made:
            self._made[i] = self._make(i)
        return self._made[i]

    def __eq__(self, other) -> bool:
        return list(self) == list(other)

    def __repr__(self) -> str:
        return repr(list(self))


@dataclass
class PagedMetadata:
    """What a forward needs to read and write the paged cache: CPU lists for host-side loops, device tensors for
    the kernels. Built once per forward, shared by every layer."""
    num_tokens: int
    query_starts: list[int]  # [num_seqs + 1]: sequence i's new tokens are rows query_starts[i]:query_starts[i+1]
    context_lens: list[int]  # [num_seqs]: tokens in the cache after this forward's writes
    positions: torch.Tensor  # [T] absolute position of each new token
    slots_cpu: list[int]  # [T] the same slots on the CPU
    slot_mapping: torch.Tensor  # [T] int64 slot of each new token
    slot_blocks: torch.Tensor  # [T] slot // block_size
    slot_offsets: torch.Tensor  # [T] slot % block_size
    block_ids: Sequence  # per sequence: its first ceil(context_len / B) blocks, int64 on the device (made on access)
    block_ids_cpu: Sequence  # the same as lists on the CPU (made on access)
    block_tables: torch.Tensor  # [num_seqs, max_blocks] int32, padded with -1 (the kernel-facing form)
    context_lens_t: torch.Tensor  # [num_seqs] int32 on the device
    last_token_indices: torch.Tensor  # [num_seqs] row of each sequence's last new token

    @property
    def num_seqs(self) -> int:
        """Sequences in this forward."""
        return len(self.context_lens)


def build_metadata(manager: BlockManager, batch: list[tuple[int, int, int]],
                   device: str | torch.device) -> PagedMetadata:
    """Metadata for a forward over batch = [(seq_id, start, n), ...]: n new tokens per sequence at positions
    start .. start + n - 1, whose slots the manager already holds. Afterwards each context is start + n tokens.

    Same contents as the reference's (engine/paged_cache.py:55-90). The tables come from the manager's int32
    mirrors with array copies, and the device arrays travel in two host-to-device copies (one int64, one int32),
    so a batch of 512 long sequences costs about a millisecond of host time instead of tens."""
    B = manager.block_size
    S = len(batch)
    if S == 0:
        raise ValueError("a forward needs at least one sequence")
    # This package's BlockManager keeps an int32 mirror of every table; a manager with only the reference's
    # block_table() list (engine/block_manager.py:106-108) works too, at the cost of one conversion per sequence.
    table_of = getattr(manager, "table_array", None)
    if table_of is None:
        def table_of(seq_id: int) -> np.ndarray:
            return np.asarray(manager.block_table(seq_id), dtype=np.int32)
    starts, lens, tables = [0], [], []
    positions: list[int] = []
    slot_list: list[int] = []
    for seq_id, start, n in batch:
        if n < 1:
            raise ValueError(f"sequence {seq_id}: a forward needs at least one new token")
        ctx = start + n
        held = manager.seq_len(seq_id)
        if held < ctx:
            raise ValueError(f"sequence {seq_id} holds {held} tokens, forward needs {ctx}")
        if start < 0:
            raise ValueError(f"sequence {seq_id}: negative start {start}")
        table = table_of(seq_id)[:(ctx + B - 1) // B]
        if n == 1:  # a decode row: one slot, no array work
            positions.append(start)
            slot_list.append(int(table[start // B]) * B + start % B)
        else:
            p = np.arange(start, ctx, dtype=np.int64)
            positions.extend(p.tolist())
            slot_list.extend((table[p // B].astype(np.int64) * B + p % B).tolist())
        starts.append(starts[-1] + n)
        lens.append(ctx)
        tables.append(table)
    T = len(positions)
    width = max(t.shape[0] for t in tables)
    # One int64 upload: positions, slots, slot blocks, slot offsets, last-token rows.
    slots = np.asarray(slot_list, dtype=np.int64)
    i64 = np.concatenate([np.asarray(positions, dtype=np.int64), slots, slots // B, slots % B,
                          np.asarray(starts[1:], dtype=np.int64) - 1])
    # One int32 upload: the -1 padded block tables, then the context lengths.
    i32 = np.full(S * width + S, -1, dtype=np.int32)
    bt = i32[:S * width].reshape(S, width)
    for i, t in enumerate(tables):
        bt[i, :t.shape[0]] = t
    i32[S * width:] = lens
    d64 = torch.from_numpy(i64).to(device)
    d32 = torch.from_numpy(i32).to(device)
    return PagedMetadata(
        num_tokens=T,
        query_starts=starts,
        context_lens=lens,
        positions=d64[:T],
        slots_cpu=slot_list,
        slot_mapping=d64[T:2 * T],
        slot_blocks=d64[2 * T:3 * T],
        slot_offsets=d64[3 * T:4 * T],
        block_ids=PerSequence(S, lambda i: torch.from_numpy(tables[i].astype(np.int64)).to(device)),
        block_ids_cpu=PerSequence(S, lambda i: tables[i].tolist()),
        block_tables=d32[:S * width].view(S, width),
        context_lens_t=d32[S * width:],
        last_token_indices=d64[4 * T:],
    )


class PagedKVCache:
    def __init__(self, cfg: ModelConfig, num_blocks: int, block_size: int, device: str | torch.device,
                 dtype: torch.dtype, attn_backend: str = "gather"):
        """K and V pools of [layers, H_kv, num_blocks, block_size, d]; contents are garbage until written."""
        if attn_backend not in BACKENDS:
            raise ValueError(f"attn_backend must be one of {BACKENDS}")
        self.attn_backend = attn_backend
        self.cfg, self.num_blocks, self.block_size, self.dtype = cfg, num_blocks, block_size, dtype
        self.device = torch.device(device)
        self._allocate((cfg.num_layers, cfg.num_kv_heads, num_blocks, block_size, cfg.head_dim), device, dtype)
        self.meta: PagedMetadata | None = None
        self._decode = None
        self._prefill_launch = None
        self._plan = None
        self._plan_scale = None
        self._arange = torch.empty(0, dtype=torch.int64, device=device)

    def _allocate(self, shape: tuple, device: str | torch.device, dtype: torch.dtype) -> None:
        """K and V pools in the model dtype (the INT8 cache overrides this)."""
        self.k = torch.empty(shape, device=device, dtype=dtype)
        self.v = torch.empty(shape, device=device, dtype=dtype)

    @staticmethod
    def blocks_for_budget(cfg: ModelConfig, budget_bytes: int, block_size: int, bytes_per_elem: int = 2) -> int:
        """Blocks that fit in budget_bytes (2 GiB -> 10,922 blocks of 16 tokens for 0.5B in bf16)."""
        return budget_bytes // (block_size * cfg.kv_bytes_per_token(bytes_per_elem))

    @property
    def on_gpu(self) -> bool:
        return self.device.type == "cuda"

    def begin(self, n_tokens: int, meta: PagedMetadata | None) -> None:
        """Start a forward over n_tokens new tokens described by meta."""
        if meta is None or meta.num_tokens != n_tokens:
            raise ValueError("a paged forward needs metadata for exactly its tokens")
        self.meta = meta
        self._decode = None
        self._prefill_launch = None
        self._plan = None  # decode launch parameters, built by the first attend() of the forward
        if self.attn_backend not in KERNEL_BACKENDS:
            return
        if not self.on_gpu:
            raise ValueError(f"attn_backend {self.attn_backend!r} runs the HIP kernel and needs a GPU pool")
        per_seq = [meta.query_starts[i + 1] - meta.query_starts[i] for i in range(meta.num_seqs)]
        dec = [i for i, n in enumerate(per_seq) if n == 1]
        self._prefill = [i for i, n in enumerate(per_seq) if n > 1]
        if self._prefill and self._prefill_kernel_ok(max(meta.context_lens[i] for i in self._prefill)):
            # Multi-token rows run the paged prefill kernel in place of gather-then-attend: one launch per layer
            # for all of them, with this subset of the metadata built once per forward.
            pf = self._prefill
            host = [meta.query_starts[i] for i in pf] + [per_seq[i] for i in pf]
            rows = torch.tensor(host, dtype=torch.int32).to(self.device, non_blocking=True)
            if len(pf) == meta.num_seqs:
                bt, ctx = meta.block_tables, meta.context_lens_t
            else:
                idx = torch.tensor(pf, device=meta.positions.device)
                bt, ctx = meta.block_tables[idx], meta.context_lens_t[idx]
            from .hip_prefill import prefill_splits

            max_ctx = max(meta.context_lens[i] for i in pf)
            cfg = self.cfg
            splits = prefill_splits(cfg.num_q_heads, cfg.num_kv_heads, cfg.head_dim, [per_seq[i] for i in pf], max_ctx)
            self._prefill_launch = (bt, ctx, rows[:len(pf)], rows[len(pf):], max_ctx, max(per_seq[i] for i in pf),
                                    splits)
            self._prefill_seqs = pf
            self._prefill = []
        if dec:
            # Once per forward, shared by every layer: the decode rows and their slice of the metadata.
            if len(dec) == meta.num_seqs:
                rows, bt, ctx = None, meta.block_tables, meta.context_lens_t
            else:
                idx = torch.tensor(dec, device=meta.positions.device)
                rows, bt, ctx = meta.last_token_indices[idx], meta.block_tables[idx], meta.context_lens_t[idx]
            self._decode = (rows, bt, ctx, [meta.context_lens[i] for i in dec])
            self._decode_seqs = dec

    def write(self, layer: int, k: torch.Tensor, v: torch.Tensor) -> None:
        """Scatter this forward's k, v [T, H_kv, d] into their slots."""
        m = self.meta
        if self.on_gpu:
            from .hip_quant import store_tokens

            store_tokens(k, m.slot_blocks, m.slot_offsets, self.k[layer], x2=v, pool2=self.v[layer])
            return
        self.k[layer][:, m.slot_blocks, m.slot_offsets] = k.transpose(0, 1)
        self.v[layer][:, m.slot_blocks, m.slot_offsets] = v.transpose(0, 1)

    def gather(self, layer: int, seq: int) -> tuple[torch.Tensor, torch.Tensor]:
        """Sequence seq's K, V as [H_kv, context_len, d] copies."""
        m, (Hkv, d) = self.meta, (self.cfg.num_kv_heads, self.cfg.head_dim)
        ctx, blocks = m.context_lens[seq], m.block_ids[seq]
        k = self.k[layer][:, blocks].view(Hkv, -1, d)[:, :ctx]
        v = self.v[layer][:, blocks].view(Hkv, -1, d)[:, :ctx]
        return k, v

    def _key_positions(self, n: int) -> torch.Tensor:
        if self._arange.numel() < n:
            self._arange = torch.arange(max(n, 2 * self._arange.numel()), device=self.device)
        return self._arange[:n]

    def _attend_gather(self, layer: int, i: int, q: torch.Tensor, positions: torch.Tensor,
                       scale: float) -> torch.Tensor:
        """Reference attention for sequence i's rows of q over its gathered context."""
        m = self.meta
        a, b = m.query_starts[i], m.query_starts[i + 1]
        k, v = self.gather(layer, i)
        return attention(q[a:b], k, v, positions[a:b], self._key_positions(m.context_lens[i]), scale)

    def _prefill_kernel_ok(self, max_context: int) -> bool:
        """Whether this forward's multi-token rows can run the paged prefill kernel (bf16 model, bf16 or INT8 pool,
        16-token blocks, head_dim 64/128, group <= 8, contexts <= 32768)."""
        from .hip_prefill import prefill_supported

        cfg = self.cfg
        return prefill_supported(self.dtype, self.k.dtype, self.block_size, cfg.head_dim,
                                 cfg.num_q_heads // cfg.num_kv_heads, max_context)

    def _attend_prefill(self, layer: int, q: torch.Tensor, scale: float, out: torch.Tensor) -> None:
        """Multi-token rows of the forward, written into their rows of out [T, Hq, d] by the prefill kernel."""
        from .hip_prefill import paged_prefill_attention

        bt, ctx, qs, ql, max_ctx, max_q, splits = self._prefill_launch
        paged_prefill_attention(q, self.k[layer], self.v[layer], bt, ctx, qs, ql, scale, max_ctx, max_q, out=out,
                                num_splits=splits, quant=self._prefill_quant(layer))

    def _prefill_quant(self, layer: int):
        """Extra prefill-kernel inputs of INT8 caches; None for the model-dtype pool."""
        return None

    def attend(self, layer: int, q: torch.Tensor, positions: torch.Tensor, scale: float) -> torch.Tensor:
        """Attention of every sequence in the forward over its own context. Returns [T, Hq * d]."""
        m = self.meta
        T, Hq, d = q.shape
        if self._decode is None:
            if self._prefill_launch is not None:  # only multi-token rows, all on the prefill kernel
                out = torch.empty(T, Hq, d, device=q.device, dtype=q.dtype)
                self._attend_prefill(layer, q, scale, out)
                return out.view(T, Hq * d)
            outs = [self._attend_gather(layer, i, q, positions, scale) for i in range(m.num_seqs)]
            return outs[0] if len(outs) == 1 else torch.cat(outs)
        from .hip_decode import DecodePlan

        rows, bt, ctx, lens = self._decode
        q_dec = q if rows is None else q[rows]
        quant = self._kernel_quant(layer)
        if self._plan is None or self._plan_scale != scale:  # first layer of the forward: validate once
            # The host-side lengths let a ragged batch run from a work list (built once, used by every layer).
            self._plan = DecodePlan(q_dec, self.k[layer], self.v[layer], bt, ctx, scale, max(lens), quant=quant,
                                    host_context_lens=lens)
            self._plan_scale = scale
            dec = self._plan()
        else:
            dec = self._plan(q=q_dec, k_cache=self.k[layer], v_cache=self.v[layer], quant=quant)
        if rows is None:
            return dec.view(T, Hq * d)
        out = torch.empty(T, Hq * d, device=q.device, dtype=q.dtype)
        out[rows] = dec.view(-1, Hq * d)
        if self._prefill_launch is not None:
            self._attend_prefill(layer, q, scale, out.view(T, Hq, d))
        for i in self._prefill:
            out[m.query_starts[i]:m.query_starts[i + 1]] = self._attend_gather(layer, i, q, positions, scale)
        return out

    def _kernel_quant(self, layer: int):
        """Extra kernel inputs of INT8 caches; None for the model-dtype pool."""
        return None
