"""INT8 paged KV caches: same pool and interface as PagedKVCache at about half the bytes (drop-in for the
reference's engine/quant_cache.py:28-196).

Format "int8" (per token): K and V int8 [layers, H_kv, N, B, d], one fp16 scale per (token, head) each,
[layers, H_kv, N, B]. 6,336 B/token for 0.5B instead of 12,288.

Format "int8-kchannel" (per-channel K): V as above; K int8 with one fp16 scale per (block, head, channel),
[layers, H_kv, N, d], over the block's 16 tokens. A block's channel scales exist only once its 16th token does,
so each sequence's partial last block of K lives in a bf16 staging slot ([layers, H_kv, n_stage, B, d]); the
forward that writes a block's 16th token quantizes the block from staging into the pool and frees the slot; a
block one forward writes whole (prefill-chunk interiors) is quantized straight from that forward's K. A
sequence holds at most 2 slots at once, so n_stage = 2 * max_num_seqs suffices. 6,624 B/token for full blocks.

On a GPU pool every write is fused HIP work (engine/hip_quant.py): V (and format A's K) per token, format B's
staging scatter, its completed blocks from staging and its whole blocks from the forward's rows, all bit-exact
with the torch quantizer (engine/quant.py), which CPU pools and fused_writes = False use. Decode reads go
through the HIP decode kernel with dequantization fused into the loads (QuantKV modes 1 / 2).
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from .block_manager import BlockManager
from .config import ModelConfig
from .hip_decode import QuantKV
from .paged_cache import PagedKVCache, PagedMetadata
from .quant import dequantize, quantize_per_channel, quantize_per_token

FORMATS = ("bf16", "int8", "int8-kchannel")

# Pool bytes per (token, KV head, layer) as a function of (head_dim d, block size B); K and V together.
_BYTES_PER_HEAD_TOKEN = {
    "bf16": lambda d, B: 4 * d,                      # K and V in bf16
    "int8": lambda d, B: 2 * (d + 2),                # int8 K and V, an fp16 scale each
    "int8-kchannel": lambda d, B: (d + 2) + d + 2 * d / B,  # V as "int8"; K codes and d fp16 scales per block
}


def kv_bytes_per_token(cfg: ModelConfig, fmt: str, block_size: int = 16) -> float:
    """Pool bytes per token: 12,288 / 6,336 / 6,624 for 0.5B (bf16 / int8 / int8-kchannel, 16-token blocks)."""
    return cfg.num_layers * cfg.num_kv_heads * _BYTES_PER_HEAD_TOKEN[fmt](cfg.head_dim, block_size)


def blocks_for_budget(cfg: ModelConfig, fmt: str, budget_bytes: int, block_size: int, n_stage: int = 0) -> int:
    """Blocks that fit in budget_bytes after n_stage bf16 staging slots (format B)."""
    staging = 2 * n_stage * cfg.num_layers * cfg.num_kv_heads * block_size * cfg.head_dim
    return int((budget_bytes - staging) // (block_size * kv_bytes_per_token(cfg, fmt, block_size)))


class StagingBook:
    """Host bookkeeping of format B's staging slots: which slot holds which partial block.

    slot_of maps block id -> slot; free is the stack of idle slots, top at the end of the list, so a fresh book
    hands out slot 0 first and a returned slot is the next one handed out. Both are mutated in place (the cache
    exposes them as _stage_of and _free_stage)."""

    def __init__(self, n_stage: int):
        self.n_stage = n_stage
        self.slot_of: dict[int, int] = {}
        self.free: list[int] = list(range(n_stage))[::-1]

    def assign(self, blocks) -> None:
        """Give each of blocks (none of them holding a slot) the next idle slot, in order."""
        blocks = list(blocks)
        if len(blocks) > len(self.free):
            raise RuntimeError(f"the forward needs {len(blocks)} more INT8 staging slots than the {len(self.free)} "
                               f"idle of {self.n_stage}; construct the cache with a larger n_stage")
        for b in blocks:
            self.slot_of[b] = self.free.pop()

    def slot(self, block: int) -> int:
        """The block's slot, assigned on first use."""
        if block not in self.slot_of:
            self.assign([block])
        return self.slot_of[block]

    def release(self, blocks) -> None:
        """Blocks that left staging (quantized into the pool, or freed by the block manager) return their slots,
        in the order given; blocks without a slot are ignored."""
        for b in blocks:
            s = self.slot_of.pop(b, None)
            if s is not None:
                self.free.append(s)


@dataclass
class _StagingPlan:
    """Format B's writes for one forward, as host arrays (uploaded together). Row indices refer to the forward's
    tokens; blocks and slots to the pool and the staging pool."""
    staged_rows: np.ndarray   # tokens whose K goes to a staging slot ...
    staged_slots: np.ndarray  # ... this slot ...
    staged_offs: np.ndarray   # ... at this offset
    done_blocks: np.ndarray   # blocks whose last token this forward writes: quantized from ...
    done_slots: np.ndarray    # ... their staging slot
    whole_blocks: np.ndarray  # blocks this forward writes entirely, never staged: quantized from ...
    whole_rows: np.ndarray    # ... these rows, B per block
    tails: np.ndarray         # per sequence: slot of its partial last block, -1 when that block is full


def plan_staging(book: StagingBook, slots_cpu: list[int], query_starts: list[int], context_lens: list[int],
                 B: int) -> _StagingPlan:
    """Classify the blocks a forward writes (reference engine/quant_cache.py:84-122, same outcome): in order of
    their first token, a block that is written entirely by this forward and holds no slot is quantized directly;
    every other block goes through staging (a slot assigned on its first staged token) and is quantized from its
    slot, which is then released, when this forward writes its last offset. Slots are assigned before any is
    released, so no slot serves two blocks within one forward."""
    slots = np.asarray(slots_cpu, dtype=np.int64)
    blk, off = slots // B, slots % B
    uniq, first, inv, count = np.unique(blk, return_index=True, return_inverse=True, return_counts=True)
    order = np.argsort(first, kind="stable")          # unique blocks by first token
    rank = np.empty_like(order)
    rank[order] = np.arange(order.size)
    rows = np.argsort(rank[inv], kind="stable")       # token rows grouped by block, token order inside a group
    sizes = count[order]
    ends = np.cumsum(sizes)
    blocks = uniq[order]
    first_off, last_off = off[rows[ends - sizes]], off[rows[ends - 1]]
    get = book.slot_of.get
    slot_of_block = np.fromiter((get(b, -1) for b in blocks.tolist()), dtype=np.int64, count=blocks.size)
    held = slot_of_block >= 0
    whole = (first_off == 0) & (sizes == B) & ~held
    fresh = np.flatnonzero(~whole & ~held)
    book.assign(blocks[fresh].tolist())
    slot_of_block[fresh] = np.fromiter((book.slot_of[b] for b in blocks[fresh].tolist()), dtype=np.int64,
                                       count=fresh.size)
    group = np.repeat(np.arange(blocks.size), sizes)  # position of each grouped row's block
    staged = ~whole[group]
    done = ~whole & (last_off == B - 1)
    plan = _StagingPlan(rows[staged], slot_of_block[group][staged], off[rows[staged]], blocks[done],
                        slot_of_block[done], blocks[whole], rows[whole[group]], np.empty(0, dtype=np.int64))
    book.release(plan.done_blocks.tolist())
    # each sequence's last block is one of this forward's blocks; its slot (a done block's is released, but a
    # sequence whose last block is done has a full last block and no tail)
    last_block = blk[np.asarray(query_starts[1:], dtype=np.int64) - 1]
    ctx = np.asarray(context_lens, dtype=np.int64)
    slot_sorted = np.empty_like(slot_of_block)
    slot_sorted[order] = slot_of_block  # by position in uniq (sorted block ids)
    plan.tails = np.where(ctx % B != 0, slot_sorted[np.searchsorted(uniq, last_block)], -1).astype(np.int64)
    return plan


class QuantPagedKVCache(PagedKVCache):
    def __init__(self, cfg: ModelConfig, num_blocks: int, block_size: int, device: str | torch.device,
                 dtype: torch.dtype, attn_backend: str = "gather", fmt: str = "int8",
                 manager: BlockManager | None = None, n_stage: int = 128):
        """`dtype` is the model's activation dtype. Format B needs the BlockManager (to release a freed sequence's
        staging slot) and n_stage slots."""
        if fmt not in ("int8", "int8-kchannel"):
            raise ValueError(f"fmt must be int8 or int8-kchannel, got {fmt}")
        self.fmt, self.n_stage = fmt, n_stage
        super().__init__(cfg, num_blocks, block_size, device, dtype, attn_backend)
        self.fused_writes = self.on_gpu  # HIP quantize-and-store on GPU pools; torch quantizer otherwise
        self._staged = self._done = self._direct = None
        self._rows_write = None  # format B decode step: (staging slot per row, quantization block per row or None)
        self._static = None  # format B's staging plan in persistent buffers (graph-replayed decode steps)
        if fmt == "int8-kchannel":
            if manager is None:
                raise ValueError("int8-kchannel needs the BlockManager to track partial blocks")
            self._book = StagingBook(n_stage)
            self._stage_of, self._free_stage = self._book.slot_of, self._book.free
            manager.add_free_listener(self._book.release)

    def _allocate(self, shape: tuple, device: str | torch.device, dtype: torch.dtype) -> None:
        """int8 K/V, fp16 scales, and (format B) the bf16 staging slots; all zero-initialised."""
        L, H, N, B, D = shape
        per_token = (L, H, N, B)
        buffers = {"k": (shape, torch.int8), "v": (shape, torch.int8), "v_scale": (per_token, torch.float16),
                   "k_scale": (per_token if self.fmt == "int8" else (L, H, N, D), torch.float16)}
        if self.fmt == "int8-kchannel":
            buffers["stage"] = ((L, H, self.n_stage, B, D), torch.bfloat16)
        for name, (shp, dt) in buffers.items():
            setattr(self, name, torch.zeros(shp, device=device, dtype=dt))

    def use_static_plan(self, buffers: tuple | None) -> None:
        """For decode steps replayed from graphs (engine/graph_runner.py): begin() binds format B's staging plan to
        persistent device buffers (rows int64 [n] = 0 .. n - 1, stage slots, done sources, done destinations, all
        int64 [n], and tail slots int32 [n]), which the caller fills from plan_static_decode() before each step,
        instead of building it per forward. None returns to per-forward plans."""
        self._static = buffers

    def plan_static_decode(self, blocks: list[int], offsets: list[int],
                           scratch_block: int) -> tuple[list[int], list[int], list[int], list[int]]:
        """Host side of a fixed-shape decode step whose row i writes one token at (blocks[i], offsets[i]): per row
        its block's staging slot (allocated on the block's first staged token), the slot and block of the
        block quantization (the row writing a block's last token quantizes it from its slot into the block and
        gives the slot back; every other row's quantization goes to scratch_block, which only padding rows read),
        and its tail slot (-1 once the block is full). Same slots and values as begin() plans for the same rows."""
        last = self.block_size - 1
        slots = [self._book.slot(b) for b in blocks]
        completes = [off == last for off in offsets]
        dst = [b if c else scratch_block for b, c in zip(blocks, completes)]
        tails = [-1 if c else s for s, c in zip(slots, completes)]
        self._book.release([b for b, c in zip(blocks, completes) if c])
        return slots, list(slots), dst, tails

    def begin(self, n_tokens: int, meta: PagedMetadata | None) -> None:
        """Base bookkeeping, then (format B) the staging plan of every block this forward writes."""
        super().begin(n_tokens, meta)
        if self.fmt != "int8-kchannel":
            return
        if self._static is not None:  # a graph-replayed decode step: every row staged, every block quantized
            rows, slots, src, dst, tails = self._static
            T = meta.num_tokens
            self._staged = (rows[:T], slots[:T], meta.slot_offsets)
            self._done = (dst[:T], src[:T])
            self._direct = None
            self._rows_write = (slots[:T], dst[:T])
            self._tails = self._tails_dec = self._tails_pf = tails[:T]
            return
        plan = plan_staging(self._book, meta.slots_cpu, meta.query_starts, meta.context_lens, self.block_size)
        # The whole plan in one host array and one asynchronous copy from pinned memory (separate uploads from
        # pageable lists would each hold the host until the device has caught up).
        parts = (plan.staged_rows, plan.staged_slots, plan.staged_offs, plan.done_blocks, plan.done_slots,
                 plan.whole_blocks, plan.whole_rows, plan.tails)
        flat = torch.from_numpy(np.concatenate(parts))
        dev = meta.positions.device
        if dev.type == "cuda":
            flat = flat.pin_memory().to(dev, non_blocking=True)
        views = torch.split(flat, [p.size for p in parts])
        self._staged = views[0:3] if plan.staged_rows.size else None
        self._done = views[3:5] if plan.done_blocks.size else None
        self._direct = views[5:7] if plan.whole_blocks.size else None
        # A decode step (every row staged, in row order, each in a slot of its own) takes the one-launch write; a
        # row then quantizes its slot when it writes the block's last offset, as the plan's done list says.
        T = plan.staged_rows.size
        decode_step = (plan.whole_blocks.size == 0 and T == meta.num_tokens
                       and np.array_equal(plan.staged_rows, np.arange(T))
                       and np.unique(plan.staged_slots).size == T)
        self._rows_write = (views[1], None) if decode_step and T else None
        self._tails = views[7].to(torch.int32)
        self._tails_dec = self._rows_of(self._tails, getattr(self, "_decode_seqs", None), self._decode, dev)
        self._tails_pf = self._rows_of(self._tails, getattr(self, "_prefill_seqs", None), self._prefill_launch, dev)

    def _rows_of(self, per_seq: torch.Tensor, seqs: list[int] | None, used, dev) -> torch.Tensor:
        """per_seq restricted to the sequences a kernel launch of this forward covers (all of them: itself)."""
        if used is None or seqs is None or len(seqs) == per_seq.numel():
            return per_seq
        return per_seq[torch.tensor(seqs, device=dev)]

    # ---- writes ------------------------------------------------------------------------------------------------

    def write(self, layer: int, k: torch.Tensor, v: torch.Tensor) -> None:
        """Quantize and store this forward's k, v [T, H_kv, d]."""
        if self.fused_writes:
            self._write_fused(layer, k, v)
        else:
            self._write_torch(layer, k, v)

    def _token_store(self, codes_pool: torch.Tensor, scale_pool: torch.Tensor, x: torch.Tensor) -> None:
        """Per-token quantization of x [T, H, d] into one layer's pools at this forward's slots."""
        codes, scales = quantize_per_token(x)
        where = (slice(None), self.meta.slot_blocks, self.meta.slot_offsets)
        codes_pool[where] = codes.transpose(0, 1)
        scale_pool[where] = scales.transpose(0, 1)

    def _k_block_sources(self, layer: int, k16: torch.Tensor):
        """(destination blocks, their [H, n, B, d] bf16 tiles) for the K blocks format B quantizes this forward:
        completed blocks from their staging slots, whole blocks from the forward's rows."""
        if self._done is not None:
            blocks, slots = self._done
            yield blocks, self.stage[layer][:, slots]
        if self._direct is not None:
            blocks, rows = self._direct
            H, d = k16.shape[1], k16.shape[2]
            yield blocks, k16[rows].view(-1, self.block_size, H, d).permute(2, 0, 1, 3)

    def _write_torch(self, layer: int, k: torch.Tensor, v: torch.Tensor) -> None:
        """write() with the torch quantizer (CPU pools, or fused_writes = False)."""
        self._token_store(self.v[layer], self.v_scale[layer], v)
        if self.fmt == "int8":
            self._token_store(self.k[layer], self.k_scale[layer], k)
            return
        # Staging holds bf16, and whole blocks are rounded to bf16 too: a block's codes do not depend on whether
        # it was staged token by token or written in one forward.
        k16 = k.to(torch.bfloat16)
        if self._staged is not None:
            rows, slots, offs = self._staged
            self.stage[layer][:, slots, offs] = k16[rows].transpose(0, 1)
        for blocks, tiles in self._k_block_sources(layer, k16):
            codes, scales = quantize_per_channel(tiles, dim=2)  # one scale per (head, block, channel)
            self.k[layer][:, blocks] = codes
            self.k_scale[layer][:, blocks] = scales

    def _write_fused(self, layer: int, k: torch.Tensor, v: torch.Tensor) -> None:
        """write() through the HIP kernels: one launch per step below."""
        from .hip_quant import (kchan_write_rows, quantize_store_block_rows, quantize_store_blocks,
                                quantize_store_tokens, store_tokens)

        m = self.meta
        if self.fmt == "int8":  # V and K in one launch
            quantize_store_tokens(v, m.slot_blocks, m.slot_offsets, self.v[layer], self.v_scale[layer],
                                  x2=k, q_pool2=self.k[layer], s_pool2=self.k_scale[layer])
            return
        if self._rows_write is not None:  # a decode step: V, the K staging store and completed blocks in one launch
            slots, dst = self._rows_write
            kchan_write_rows(k, v, m.slot_blocks, m.slot_offsets, slots, dst, self.v[layer], self.v_scale[layer],
                             self.k[layer], self.k_scale[layer], self.stage[layer])
            return
        quantize_store_tokens(v, m.slot_blocks, m.slot_offsets, self.v[layer], self.v_scale[layer])
        if self._staged is not None:
            rows, slots, offs = self._staged
            store_tokens(k, slots, offs, self.stage[layer], rows=rows)
        if self._done is not None:
            blocks, slots = self._done
            quantize_store_blocks(self.stage[layer], slots, blocks, self.k[layer], self.k_scale[layer])
        if self._direct is not None:
            blocks, rows = self._direct
            quantize_store_block_rows(k, rows, blocks, self.k[layer], self.k_scale[layer])

    # ---- reads -------------------------------------------------------------------------------------------------

    def gather(self, layer: int, seq: int) -> tuple[torch.Tensor, torch.Tensor]:
        """Sequence seq's dequantized K, V as [H_kv, context_len, d] in the model dtype."""
        meta, B = self.meta, self.block_size
        n, ids = meta.context_lens[seq], meta.block_ids[seq]
        H, d = self.cfg.num_kv_heads, self.cfg.head_dim
        # Scales broadcast over the channels (per token) or over the tokens of a block (per channel).
        v = dequantize(self.v[layer][:, ids], self.v_scale[layer][:, ids].unsqueeze(-1), self.dtype)
        k_axis = -1 if self.fmt == "int8" else 2
        k = dequantize(self.k[layer][:, ids], self.k_scale[layer][:, ids].unsqueeze(k_axis), self.dtype)
        if self.fmt == "int8-kchannel" and n % B:  # the partial last block is in its staging slot
            slot = self._stage_of[meta.block_ids_cpu[seq][-1]]
            k[:, -1] = self.stage[layer][:, slot].to(self.dtype)
        return k.reshape(H, -1, d)[:, :n], v.reshape(H, -1, d)[:, :n]

    def _prefill_quant(self, layer: int) -> QuantKV:
        """Scales (and format B's staging, with the tail slots of the forward's multi-token rows) for the prefill
        kernel, which dequantizes K/V as gather() does."""
        if self.fmt == "int8":
            return QuantKV(1, self.k_scale[layer], self.v_scale[layer])
        return QuantKV(2, self.k_scale[layer], self.v_scale[layer], self.stage[layer], self._tails_pf)

    def _kernel_quant(self, layer: int) -> QuantKV:
        """Scales (and format B's staging) for the decode kernel."""
        if self.fmt == "int8":
            return QuantKV(1, self.k_scale[layer], self.v_scale[layer])
        return QuantKV(2, self.k_scale[layer], self.v_scale[layer], self.stage[layer], self._tails_dec)
