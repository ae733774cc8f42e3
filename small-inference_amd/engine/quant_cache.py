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

import torch

from .block_manager import BlockManager
from .config import ModelConfig
from .hip_decode import QuantKV
from .paged_cache import PagedKVCache, PagedMetadata
from .quant import dequantize, quantize_per_channel, quantize_per_token

FORMATS = ("bf16", "int8", "int8-kchannel")


def kv_bytes_per_token(cfg: ModelConfig, fmt: str, block_size: int = 16) -> float:
    """Pool bytes per token: 12,288 / 6,336 / 6,624 for 0.5B (bf16 / int8 / int8-kchannel, 16-token blocks)."""
    d = cfg.head_dim
    per_head_layer = {"bf16": 4 * d, "int8": 2 * (d + 2), "int8-kchannel": (d + 2) + d + 2 * d / block_size}[fmt]
    return cfg.num_layers * cfg.num_kv_heads * per_head_layer


def blocks_for_budget(cfg: ModelConfig, fmt: str, budget_bytes: int, block_size: int, n_stage: int = 0) -> int:
    """Blocks that fit in budget_bytes after n_stage bf16 staging slots (format B)."""
    stage_bytes = n_stage * cfg.num_layers * cfg.num_kv_heads * block_size * cfg.head_dim * 2
    return int((budget_bytes - stage_bytes) // (block_size * kv_bytes_per_token(cfg, fmt, block_size)))


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
        self._static = None  # format B's staging plan in persistent buffers (graph-replayed decode steps)
        if fmt == "int8-kchannel":
            if manager is None:
                raise ValueError("int8-kchannel needs the BlockManager to track partial blocks")
            self._stage_of: dict[int, int] = {}  # block id -> staging slot
            self._free_stage = list(reversed(range(n_stage)))  # LIFO, slot 0 handed out first
            manager.add_free_listener(self._release_blocks)

    def _allocate(self, shape: tuple, device: str | torch.device, dtype: torch.dtype) -> None:
        """int8 K/V, fp16 scales, and (format B) the bf16 staging slots; all zero-initialised."""
        L, H, N, B, D = shape
        self.k = torch.zeros(shape, device=device, dtype=torch.int8)
        self.v = torch.zeros(shape, device=device, dtype=torch.int8)
        self.v_scale = torch.zeros(L, H, N, B, device=device, dtype=torch.float16)
        if self.fmt == "int8":
            self.k_scale = torch.zeros(L, H, N, B, device=device, dtype=torch.float16)
        else:
            self.k_scale = torch.zeros(L, H, N, D, device=device, dtype=torch.float16)
            self.stage = torch.zeros(L, H, self.n_stage, B, D, device=device, dtype=torch.bfloat16)

    def _release_blocks(self, blocks: list[int]) -> None:
        """BlockManager listener: freed blocks give back their staging slots."""
        for b in blocks:
            slot = self._stage_of.pop(b, None)
            if slot is not None:
                self._free_stage.append(slot)

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
        B = self.block_size
        slots, src, dst, tails, done = [], [], [], [], []
        for b, off in zip(blocks, offsets):
            slot = self._stage_of.get(b)
            if slot is None:
                if not self._free_stage:
                    raise RuntimeError("out of INT8 staging slots; raise n_stage")
                slot = self._stage_of[b] = self._free_stage.pop()
            slots.append(slot)
            src.append(slot)
            if off == B - 1:
                dst.append(b)
                tails.append(-1)
                done.append(b)
            else:
                dst.append(scratch_block)
                tails.append(slot)
        for b in done:
            self._free_stage.append(self._stage_of.pop(b))
        return slots, src, dst, tails

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
            self._tails = self._tails_dec = self._tails_pf = tails[:T]
            return
        B, dev = self.block_size, meta.positions.device
        rows_of: dict[int, list[tuple[int, int]]] = {}  # block -> [(token row, offset)] in token order
        for row, slot in enumerate(meta.slots_cpu):
            rows_of.setdefault(slot // B, []).append((row, slot % B))
        staged_rows, staged_slots, staged_offs, done, direct, direct_rows = [], [], [], [], [], []
        for b, items in rows_of.items():
            whole = items[0][1] == 0 and len(items) == B
            if whole and b not in self._stage_of:
                direct.append(b)  # written whole by this forward: quantized straight from k, never staged
                direct_rows.extend(r for r, _ in items)
                continue
            if b not in self._stage_of:
                if not self._free_stage:
                    raise RuntimeError("out of INT8 staging slots; raise n_stage")
                self._stage_of[b] = self._free_stage.pop()
            slot = self._stage_of[b]
            staged_rows.extend(r for r, _ in items)
            staged_slots.extend([slot] * len(items))
            staged_offs.extend(o for _, o in items)
            if items[-1][1] == B - 1:
                done.append(b)

        done_slots = [self._stage_of[b] for b in done]
        for b in done:  # free now: nothing reassigns a slot before the next forward's begin()
            self._free_stage.append(self._stage_of.pop(b))
        # Per sequence: the staging slot of its partial last block, -1 if the last block is full (the last block
        # is the one holding the sequence's last new token).
        last_slots = [meta.slots_cpu[e - 1] for e in meta.query_starts[1:]]
        tails = [self._stage_of[last_slots[i] // B] if ctx % B else -1 for i, ctx in enumerate(meta.context_lens)]
        # The whole plan in one host array and one asynchronous copy from pinned memory (separate uploads from
        # pageable lists would each hold the host until the device has caught up).
        parts = (staged_rows, staged_slots, staged_offs, done, done_slots, direct, direct_rows, tails)
        flat = torch.tensor([x for part in parts for x in part], dtype=torch.int64)
        if dev.type == "cuda":
            flat = flat.pin_memory().to(dev, non_blocking=True)
        views = torch.split(flat, [len(part) for part in parts])
        self._staged = views[0:3] if staged_rows else None
        self._done = views[3:5] if done else None
        self._direct = views[5:7] if direct else None
        self._tails = views[7].to(torch.int32)
        if self._decode is not None and len(self._decode_seqs) != meta.num_seqs:
            self._tails_dec = self._tails[torch.tensor(self._decode_seqs, device=dev)]
        else:
            self._tails_dec = self._tails
        if self._prefill_launch is not None and len(self._prefill_seqs) != meta.num_seqs:
            self._tails_pf = self._tails[torch.tensor(self._prefill_seqs, device=dev)]
        else:
            self._tails_pf = self._tails

    def write(self, layer: int, k: torch.Tensor, v: torch.Tensor) -> None:
        """Quantize and store this forward's k, v [T, H_kv, d]."""
        if self.fused_writes:
            self._write_fused(layer, k, v)
            return
        m = self.meta
        vq, vs = quantize_per_token(v)
        self.v[layer][:, m.slot_blocks, m.slot_offsets] = vq.transpose(0, 1)
        self.v_scale[layer][:, m.slot_blocks, m.slot_offsets] = vs.t()
        if self.fmt == "int8":
            kq, ks = quantize_per_token(k)
            self.k[layer][:, m.slot_blocks, m.slot_offsets] = kq.transpose(0, 1)
            self.k_scale[layer][:, m.slot_blocks, m.slot_offsets] = ks.t()
            return
        # Every path quantizes the bf16-rounded K, so a block's int8 contents do not depend on its chunking.
        if self._staged is not None:
            rows, slots, offs = self._staged
            self.stage[layer][:, slots, offs] = k[rows].transpose(0, 1).to(torch.bfloat16)
        if self._done is not None:
            blocks, slots = self._done
            kq, ks = quantize_per_channel(self.stage[layer][:, slots], dim=2)  # [H, n, B, d] over the B tokens
            self.k[layer][:, blocks] = kq
            self.k_scale[layer][:, blocks] = ks
        if self._direct is not None:
            blocks, rows = self._direct
            H, d = k.shape[1], k.shape[2]
            whole = k[rows].view(-1, self.block_size, H, d).permute(2, 0, 1, 3).to(torch.bfloat16)  # [H, n, B, d]
            kq, ks = quantize_per_channel(whole, dim=2)
            self.k[layer][:, blocks] = kq
            self.k_scale[layer][:, blocks] = ks

    def _write_fused(self, layer: int, k: torch.Tensor, v: torch.Tensor) -> None:
        """write() through the HIP kernels: one launch per step below."""
        from .hip_quant import quantize_store_block_rows, quantize_store_blocks, quantize_store_tokens, store_tokens

        m = self.meta
        if self.fmt == "int8":  # V and K in one launch
            quantize_store_tokens(v, m.slot_blocks, m.slot_offsets, self.v[layer], self.v_scale[layer],
                                  x2=k, q_pool2=self.k[layer], s_pool2=self.k_scale[layer])
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

    def gather(self, layer: int, seq: int) -> tuple[torch.Tensor, torch.Tensor]:
        """Sequence seq's dequantized K, V as [H_kv, context_len, d] in the model dtype."""
        m, (H, d), B = self.meta, (self.cfg.num_kv_heads, self.cfg.head_dim), self.block_size
        ctx, blocks = m.context_lens[seq], m.block_ids[seq]
        v = dequantize(self.v[layer][:, blocks], self.v_scale[layer][:, blocks][..., None], self.dtype)
        if self.fmt == "int8":
            k = dequantize(self.k[layer][:, blocks], self.k_scale[layer][:, blocks][..., None], self.dtype)
        else:
            k = dequantize(self.k[layer][:, blocks], self.k_scale[layer][:, blocks][:, :, None], self.dtype)
            if ctx % B:
                k[:, -1] = self.stage[layer][:, self._stage_of[m.block_ids_cpu[seq][-1]]].to(self.dtype)
        return k.view(H, -1, d)[:, :ctx], v.view(H, -1, d)[:, :ctx]

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
