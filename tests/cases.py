"""Seeded test inputs shared by the parity tests: fragmented block pools (the reference tests' fill-then-free-in-
random-order pattern, reference tests/test_paged.py:23-32 and tests/test_decode_kernel.py:21-39) and decode cases.
"""

from __future__ import annotations

import json
import os

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


def ramp_scores(q, k, tables, lengths, B, direction, q0=64.0, span=8.0):
    """Scores that trend across the keys: channel 0 of every key goes linearly from -span to +span over its
    sequence's positions (reversed for direction -1) and channel 0 of every query is q0, so that with head_dim 64
    (scale 1/8) a score moves by about 4 in the exp2 domain every 64 keys. Direction 0: a spike instead, channel
    0 zero but for the key at two thirds of each sequence, which gets +span (about 90 above the other scores in
    the exp2 domain). q and k are modified in place."""
    q[..., 0] = q0
    kk = k.float()
    for s, n in enumerate(lengths):
        pos = torch.arange(n)
        blk = torch.tensor(tables[s][:-(-n // B)])[pos // B]
        if direction == 0:
            x = torch.zeros(n)
            x[2 * n // 3] = span
        else:
            x = direction * (2.0 * span * pos / max(n - 1, 1) - span)
        kk[:, blk, pos % B, 0] = x.to(kk)
    k.copy_(kk.to(k.dtype))


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


def oracle_cache_decode(cache, layer: int, q: np.ndarray, tables: list[list[int]], lengths: list[int], scale: float,
                        tails: list[int] | None = None) -> np.ndarray:
    """The oracle's fp32 decode of one layer of a cache for the given sequences (tables, lengths), q [S, Hq, D]:
    only the blocks the tables use are copied to the host; INT8 pools are dequantized as the reference's gather
    path does (per-token scales; format "int8-kchannel" with per-(block, channel) K scales and each partial last
    block of K from its staging slot, tails[i], -1 when the last block is full)."""
    B = cache.block_size
    used = sorted({b for t, n in zip(tables, lengths) for b in t[:-(-n // B)]})
    remap = {b: i for i, b in enumerate(used)}
    idx = torch.tensor(used, dtype=torch.int64, device=cache.k.device)
    t2 = [[remap[b] for b in t[:-(-n // B)]] for t, n in zip(tables, lengths)]

    def take(x):
        return x[layer].index_select(1, idx).float().cpu().numpy()

    fmt = getattr(cache, "fmt", "bf16")
    if fmt == "bf16":
        kp, vp = take(cache.k), take(cache.v)
    else:
        vp = paged_ref.dequant_tokens(take(cache.v), take(cache.v_scale))
        kp = paged_ref.dequant_tokens(take(cache.k), take(cache.k_scale)) if fmt == "int8" else None
    if fmt == "int8-kchannel":
        kq, ks, stage = take(cache.k), take(cache.k_scale), cache.stage[layer].float().cpu().numpy()
    out = np.empty(q.shape, dtype=np.float32)
    for i, n in enumerate(lengths):
        if fmt == "int8-kchannel":
            k_i = paged_ref.gather_kchannel(kq, ks, stage, t2[i], n, int(tails[i]))
        else:
            k_i = paged_ref.gather(kp, t2[i], n)
        out[i] = paged_ref.attend_one(q[i], k_i, paged_ref.gather(vp, t2[i], n), scale, np.float32)
    return out


def bf16_bracket(ref: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """The two bf16 values that bracket each element of ref (equal to ref where it is a bf16 value): (lower,
    upper), each as float64."""
    ref = np.asarray(ref, dtype=np.float64)
    mag = np.abs(ref)
    t = mag.astype(np.float32).view(np.uint32) & np.uint32(0xFFFF0000)  # |ref| in fp32, truncated to bf16
    step = np.uint32(0x10000)
    cand = [np.where(t >= step, t - step, t), t, np.minimum(t + step, np.uint32(0x7F800000))]
    vals = [c.view(np.float32).astype(np.float64) for c in cand]
    lo = np.max([np.where(v <= mag, v, -np.inf) for v in vals], axis=0)
    hi = np.min([np.where(v >= mag, v, np.inf) for v in vals], axis=0)
    sign = np.where(ref < 0, -1.0, 1.0)
    return np.where(ref < 0, sign * hi, sign * lo), np.where(ref < 0, sign * lo, sign * hi)


def assert_decode_close(got, ref, what: str = "decode", atol: float = 8e-3) -> float:
    """The north-star bound on a bf16 attention output against the fp32 oracle plus the output's own rounding:
    every element within atol (8e-3) of the oracle, or equal to one of the two bf16 values that bracket the
    oracle's value (a result the exact output could round to). Prints the raw max-abs error, how many elements
    needed the rounding clause and the |ref| percentiles; with SIPA_PARITY_LOG set, appends them as a JSON line to
    that file. Returns the raw max-abs."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    err = np.abs(got - ref)
    near = err <= atol
    lo, hi = bf16_bracket(ref)
    rounded = (got == lo) | (got == hi)
    clause = ~near & rounded
    bad = ~near & ~rounded
    raw = float(err.max()) if err.size else 0.0
    mag = np.abs(ref)
    q = np.percentile(mag, [50, 99, 100]) if mag.size else [0, 0, 0]
    stats = {"case": what, "max_abs": raw, "elements": int(err.size), "rounding_clause": int(clause.sum()),
             "ref_abs_p50": float(q[0]), "ref_abs_p99": float(q[1]), "ref_abs_max": float(q[2])}
    print(f"{what}: max-abs {raw:.2e}; {stats['rounding_clause']} of {err.size} elements past {atol} are the "
          f"bf16 rounding of the oracle; |ref| median {q[0]:.2f}, p99 {q[1]:.2f}, max {q[2]:.2f}", flush=True)
    log = os.environ.get("SIPA_PARITY_LOG")
    if log:
        with open(log, "a") as f:
            f.write(json.dumps(stats) + "\n")
    if bad.any():
        i = int(np.flatnonzero(bad.ravel())[0])
        raise AssertionError(f"{what}: {int(bad.sum())} elements off by more than {atol} and not a bf16 rounding of "
                             f"the oracle, e.g. got {got.ravel()[i]!r} for {ref.ravel()[i]!r}")
    return raw
