"""Seeded test inputs shared by the parity tests: fragmented block pools (the reference tests' fill-then-free-in-
random-order pattern, reference tests/test_paged.py:23-32 and tests/test_decode_kernel.py:21-39) and decode cases.
"""

from __future__ import annotations

import numpy as np
import torch

from engine.block_manager import BlockManager
from oracle import paged_ref

HEADS = {"0.5B": (14, 2, 64), "1.5B": (12, 2, 128)}
RAGGED = [1, 15, 16, 17, 33, 100, 1000]


def fragmented_manager(num_blocks: int, block_size: int, gen: torch.Generator) -> BlockManager:
    """A manager whose free stack is shuffled: every later allocation gets a scattered, non-monotonic table."""
    m = BlockManager(num_blocks, block_size)
    for s in range(num_blocks):
        m.allocate(1_000_000 + s, block_size)
    for s in torch.randperm(num_blocks, generator=gen).tolist():
        m.free(1_000_000 + s)
    return m


def make_case(lengths, Hq, Hkv, D, B, dtype, seed=0, device="cuda", spare=2):
    """q [S, Hq, D], pools [Hkv, N, B, D] ~ N(0, 1) in `dtype` on `device`, -1 padded int32 tables over a
    fragmented pool of spare x the needed blocks, int32 context lengths. Returns (q, k, v, bt, ctx, tables)."""
    g = torch.Generator().manual_seed(seed)
    need = sum(-(-n // B) for n in lengths)
    m = fragmented_manager(max(need * spare, 1), B, g)
    for i, n in enumerate(lengths):
        m.allocate(i, n)
    tables = [m.block_table(i) for i in range(len(lengths))]
    bt = torch.from_numpy(paged_ref.padded_tables(tables, lengths, B)).to(device)
    k = torch.randn(Hkv, m.num_blocks, B, D, generator=g).to(device, dtype)
    v = torch.randn(Hkv, m.num_blocks, B, D, generator=g).to(device, dtype)
    q = torch.randn(len(lengths), Hq, D, generator=g).to(device, dtype)
    ctx = torch.tensor(lengths, dtype=torch.int32, device=device)
    return q, k, v, bt, ctx, tables


def as_np32(t: torch.Tensor) -> np.ndarray:
    """A tensor's values as a float32 numpy array on the CPU (bf16 widens exactly)."""
    return t.detach().float().cpu().numpy()


def oracle_decode(q, k, v, tables, lengths, scale, dtype=np.float64):
    """The oracle's gather-then-attend on CPU copies of the inputs."""
    return paged_ref.decode(as_np32(q), as_np32(k), as_np32(v), tables, lengths, scale, dtype)


def compact_pool(k: torch.Tensor, tables: list[list[int]], lengths: list[int], B: int):
    """Copy only the blocks the tables use to the CPU and renumber the tables: (pool [Hkv, n_used, B, D] fp32,
    new tables). Lets the oracle check cases whose full pool is too large for host memory."""
    used = sorted({b for t, n in zip(tables, lengths) for b in t[:-(-n // B)]})
    remap = {b: i for i, b in enumerate(used)}
    idx = torch.tensor(used, dtype=torch.int64, device=k.device)
    small = k.index_select(1, idx).float().cpu().numpy()
    return small, [[remap[b] for b in t[:-(-n // B)]] for t, n in zip(tables, lengths)]


def bf16_half_ulp(x: np.ndarray) -> np.ndarray:
    """Half a bf16 unit in the last place at |x| (8 significant bits): the rounding error any bf16 output may
    carry on top of the arithmetic's own error."""
    ax = np.maximum(np.abs(np.asarray(x, dtype=np.float64)), 2.0 ** -126)
    return 2.0 ** (np.floor(np.log2(ax)) - 8)


def bf16_error_beyond_rounding(got: np.ndarray, ref: np.ndarray) -> float:
    """max |got - ref| - half_ulp_bf16(got): how far a bf16 output lies from the reference beyond its own output
    rounding (<= the error of the fp32 result before rounding)."""
    return float((np.abs(got - ref) - bf16_half_ulp(got)).max())
