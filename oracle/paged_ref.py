"""CPU oracle of the paged-attention decode path. TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this package, and only as the
checker; the product (small-inference_amd/) never does and fails loudly without its HIP library.

Every function restates the reference's algorithm on the CPU (numpy, or torch on the CPU for the timed baseline)
and cites the reference file:line it follows. Pinning (tests/test_oracle.py): the reference's own known answers
(slot_mapping, block tables, budgets), torch's library routines (scaled_dot_product_attention, torch.round,
.to(float16)), brute force on tiny inputs, closed forms (uniform and one-hot softmax) and invariants (split
merging, round-trip bounds).
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "liboracle_quant.so"
QMAX = 127  # reference engine/quant.py:19


# ---- block-table indexing ----------------------------------------------------------------------------------------

def slots(table: list[int], start: int, end: int, block_size: int) -> list[int]:
    """Slots of positions [start, end): table[p // B] * B + p % B (reference engine/block_manager.py:118-123)."""
    return [table[p // block_size] * block_size + p % block_size for p in range(start, end)]


def padded_tables(tables: list[list[int]], lengths: list[int], block_size: int) -> np.ndarray:
    """[S, width] int32 block tables, each cut to ceil(len / B) blocks and padded with -1
    (reference engine/paged_cache.py:72-74,87)."""
    cut = [t[:-(-n // block_size)] for t, n in zip(tables, lengths)]
    width = max(len(t) for t in cut)
    return np.array([t + [-1] * (width - len(t)) for t in cut], dtype=np.int32)


def metadata(tables: dict[int, list[int]], batch: list[tuple[int, int, int]], block_size: int) -> dict:
    """Packed per-forward metadata for batch [(seq, start, n)] (reference engine/paged_cache.py:55-90):
    query_starts, context_lens, positions, slot_mapping, slot_blocks, slot_offsets, block_tables (-1 padded),
    last_token_indices."""
    B = block_size
    positions, slot_list, qs, ctx, cut = [], [], [0], [], []
    for seq, start, n in batch:
        positions += list(range(start, start + n))
        slot_list += slots(tables[seq], start, start + n, B)
        qs.append(qs[-1] + n)
        ctx.append(start + n)
        cut.append(tables[seq][:-(-(start + n) // B)])
    width = max(len(t) for t in cut)
    return {
        "query_starts": qs, "context_lens": ctx, "positions": positions, "slot_mapping": slot_list,
        "slot_blocks": [s // B for s in slot_list], "slot_offsets": [s % B for s in slot_list],
        "block_tables": [t + [-1] * (width - len(t)) for t in cut],
        "last_token_indices": [e - 1 for e in qs[1:]],
    }


# ---- gather-then-attend ------------------------------------------------------------------------------------------

def gather(pool: np.ndarray, table, ctx: int) -> np.ndarray:
    """One sequence's [Hkv, ctx, D] from a [Hkv, N, B, D] pool (reference engine/paged_cache.py:141-147)."""
    Hkv, _, B, D = pool.shape
    nb = -(-ctx // B)
    return pool[:, np.asarray(table[:nb], dtype=np.int64)].reshape(Hkv, nb * B, D)[:, :ctx]


def attend_one(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float, dtype=np.float64) -> np.ndarray:
    """Decode attention of one query token, q [Hq, D] over k, v [Hkv, n, D]: query head h uses KV head h // g,
    out = softmax(scale q k^T) v with the softmax in `dtype` (reference engine/attention.py:6-28 with T = 1)."""
    Hq, D = q.shape
    Hkv = k.shape[0]
    g = Hq // Hkv
    qg = q.astype(dtype).reshape(Hkv, g, D)
    s = np.matmul(qg, k.astype(dtype).transpose(0, 2, 1)) * dtype(scale)  # [Hkv, g, n]
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=-1, keepdims=True)
    return np.matmul(p, v.astype(dtype)).reshape(Hq, D)


def decode(q, k_pool, v_pool, tables, lengths, scale, dtype=np.float64) -> np.ndarray:
    """[S, Hq, D] paged decode: gather each sequence's K/V through its table, attend (the reference's gather
    backend, engine/paged_cache.py:149-162)."""
    out = np.empty(q.shape, dtype=dtype)
    for i, n in enumerate(lengths):
        out[i] = attend_one(q[i], gather(k_pool, tables[i], n), gather(v_pool, tables[i], n), scale, dtype)
    return out


def prefill(q, k_pool, v_pool, tables, context_lens, query_starts, query_lens, scale, dtype=np.float64):
    """Causal attention of multi-token rows over the paged context (the reference's gather path for prefill
    chunks, engine/paged_cache.py:149-155 with engine/attention.py:6-28): sequence s's new tokens are rows
    query_starts[s] .. + query_lens[s] - 1 of q [T, Hq, D], at positions ctx - n .. ctx - 1 (ctx =
    context_lens[s], n = query_lens[s]); the token at position p sees keys 0 .. p. Returns [T, Hq, D] in dtype
    (rows of no sequence are zero)."""
    T, Hq, D = q.shape
    out = np.zeros((T, Hq, D), dtype=dtype)
    for s, (ctx, q0, n) in enumerate(zip(context_lens, query_starts, query_lens)):
        k = gather(k_pool, tables[s], ctx).astype(dtype)
        v = gather(v_pool, tables[s], ctx).astype(dtype)
        Hkv = k.shape[0]
        g = Hq // Hkv
        qs = q[q0:q0 + n].astype(dtype).reshape(n, Hkv, g, D).transpose(1, 2, 0, 3)  # [Hkv, g, n, D]
        sc = np.matmul(qs, k.transpose(0, 2, 1)[:, None]) * dtype(scale)              # [Hkv, g, n, ctx]
        pos = np.arange(ctx - n, ctx)[:, None]
        sc = np.where(np.arange(ctx)[None, :] <= pos, sc, -np.inf)
        sc = sc - sc.max(axis=-1, keepdims=True)
        p = np.exp(sc)
        p /= p.sum(axis=-1, keepdims=True)
        out[q0:q0 + n] = np.matmul(p, v[:, None]).transpose(2, 0, 1, 3).reshape(n, Hq, D)
    return out


# ---- INT8 dequantize-then-attend ---------------------------------------------------------------------------------

def dequant_tokens(q_pool: np.ndarray, s_pool: np.ndarray) -> np.ndarray:
    """int8 [H, N, B, D] x per-token scales [H, N, B] -> fp32 (reference engine/quant.py:46-48,
    engine/quant_cache.py:183-185)."""
    return q_pool.astype(np.float32) * s_pool.astype(np.float32)[..., None]


def dequant_channels(q_pool: np.ndarray, s_pool: np.ndarray) -> np.ndarray:
    """int8 [H, N, B, D] x per-(block, channel) scales [H, N, D] -> fp32 (reference engine/quant_cache.py:186-187)."""
    return q_pool.astype(np.float32) * s_pool.astype(np.float32)[:, :, None, :]


def gather_kchannel(kq, ksc, stage, table, ctx: int, tail_slot: int) -> np.ndarray:
    """Format-B K of one sequence [H, ctx, D] in fp32: full blocks dequantized with their channel scales, the
    partial last block (ctx % B != 0) taken from its bf16 staging slot (reference engine/quant_cache.py:186-190)."""
    H, _, B, D = kq.shape
    nb = -(-ctx // B)
    blocks = np.asarray(table[:nb], dtype=np.int64)
    k = dequant_channels(kq[:, blocks], ksc[:, blocks])
    if ctx % B:
        k[:, -1] = stage[:, tail_slot].astype(np.float32)
    return k.reshape(H, nb * B, D)[:, :ctx]


# ---- split-K merge -----------------------------------------------------------------------------------------------

def split_state(q, k, v, scale, dtype=np.float64):
    """Unnormalised softmax state of one split: (m [Hq], l [Hq], acc [Hq, D]) with m = max score,
    l = sum exp(s - m), acc = sum exp(s - m) v (reference engine/triton_decode.py:118-131,133-137)."""
    Hq, D = q.shape
    Hkv = k.shape[0]
    g = Hq // Hkv
    s = np.matmul(q.astype(dtype).reshape(Hkv, g, D), k.astype(dtype).transpose(0, 2, 1)).reshape(Hq, -1) * scale
    m = s.max(axis=-1)
    p = np.exp(s - m[:, None])
    acc = np.matmul(p.reshape(Hkv, g, -1), v.astype(dtype)).reshape(Hq, D)
    return m, p.sum(axis=-1), acc


def combine(ms, ls, accs):
    """Merge split states: M = max_j m_j; out = sum_j e^(m_j - M) acc_j / sum_j e^(m_j - M) l_j
    (reference engine/triton_decode.py:20-24,144-161)."""
    ms, ls, accs = np.asarray(ms), np.asarray(ls), np.asarray(accs)
    M = ms.max(axis=0)
    w = np.exp(ms - M)
    return (w[..., None] * accs).sum(axis=0) / (w * ls).sum(axis=0)[..., None]


# ---- quantizer (plain C, with a numpy restatement beside it) ----------------------------------------------------

_lib = None


def _load():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is missing: run oracle/build.py (or __graft_entry__.build())")
        lib = ctypes.CDLL(str(LIB_PATH))
        lib.oracle_quantize_groups.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
                                               ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p]
        lib.oracle_f32_to_f16.argtypes = [ctypes.c_float]
        lib.oracle_f32_to_f16.restype = ctypes.c_uint16
        _lib = lib
    return _lib


def quantize_groups_c(x: np.ndarray, axis: int) -> tuple[np.ndarray, np.ndarray]:
    """Symmetric absmax INT8 over `axis` of fp32 x with fp16 scales, through the C oracle. Returns (int8 codes of
    x's shape, fp16 scales with `axis` removed) (reference engine/quant.py:22-43)."""
    x = np.ascontiguousarray(np.moveaxis(np.asarray(x, dtype=np.float32), axis, -1))
    n = x.shape[-1]
    groups = x.size // n if n else 0
    q = np.empty(x.shape, dtype=np.int8)
    s = np.empty(x.shape[:-1], dtype=np.uint16)
    _load().oracle_quantize_groups(x.ctypes.data, groups, n, n, 1, q.ctypes.data, s.ctypes.data)
    return np.moveaxis(q, -1, axis), s.view(np.float16)


def quantize_per_token(x: np.ndarray):
    """One scale per vector over the last axis (reference engine/quant.py:34-37)."""
    return quantize_groups_c(x, -1)


def quantize_per_channel(x: np.ndarray, axis: int):
    """One scale per position of every other axis, over `axis` (reference engine/quant.py:40-43)."""
    return quantize_groups_c(x, axis)


def quantize_groups_np(x: np.ndarray, axis: int) -> tuple[np.ndarray, np.ndarray]:
    """numpy restatement of the same quantizer: float32 IEEE division, astype(float16) rounds to nearest even,
    np.rint rounds half to even."""
    x = np.asarray(x, dtype=np.float32)
    s16 = (np.abs(x).max(axis=axis, keepdims=True) / np.float32(QMAX)).astype(np.float16)
    s32 = s16.astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        q = np.where(s32 > 0, np.rint(x / np.where(s32 > 0, s32, np.float32(1))), np.float32(0))
    return np.clip(q, -QMAX, QMAX).astype(np.int8), np.squeeze(s16, axis=axis)


def f32_to_f16_bits_c(values) -> np.ndarray:
    """The C oracle's binary32 -> binary16 conversion, element by element (for pinning it)."""
    lib = _load()
    return np.array([lib.oracle_f32_to_f16(float(v)) for v in np.asarray(values, dtype=np.float32).ravel()],
                    dtype=np.uint16)


# ---- bf16 helpers --------------------------------------------------------------------------------------------------

def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round fp32 values to bf16 (nearest even; past the largest bf16, infinity) and return them as fp32. NaN
    stays NaN (the integer rounding below would carry a signalling NaN's payload into the exponent)."""
    x = np.asarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    r = (((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint32) << 16).view(np.float32)
    return np.where(np.isnan(x), np.float32(np.nan), r).astype(np.float32)


# ---- timed CPU baseline (torch on the host cores) -------------------------------------------------------------------

def decode_torch_cpu(q, k_pool, v_pool, tables, lengths, scale):
    """fp32 gather-then-attend on the CPU with torch (reference engine/paged_cache.py:141-155 and
    engine/attention.py:18-28 for T = 1): per sequence, copy its blocks out of the pool, then bmm -> softmax ->
    bmm with the group stacked along M. Inputs are torch CPU tensors; returns [S, Hq, D] fp32."""
    import torch

    S, Hq, D = q.shape
    Hkv, _, B, _ = k_pool.shape
    g = Hq // Hkv
    out = torch.empty(S, Hq, D, dtype=torch.float32)
    for i, n in enumerate(lengths):
        nb = -(-n // B)
        blocks = tables[i, :nb].long()
        k = k_pool[:, blocks].reshape(Hkv, nb * B, D)[:, :n].float()
        v = v_pool[:, blocks].reshape(Hkv, nb * B, D)[:, :n].float()
        qg = q[i].float().reshape(Hkv, g, D)
        p = torch.softmax(torch.bmm(qg, k.transpose(1, 2)) * scale, dim=-1)
        out[i] = torch.bmm(p, v).reshape(Hq, D)
    return out
