"""Fused INT8 quantize-and-store and plain scatter-store on MI355X through libsmallinf_hip.so: the drop-in for the
reference's engine/triton_quant.py (quantize_store_tokens, quantize_store_blocks; reference :61-84), plus the two
stores the reference leaves to torch ops (the pool scatter of engine/paged_cache.py:135-139 and format B's
staging and whole-block writes, engine/quant_cache.py:165-177).

The quantizer is bit-exact with engine/quant.py: scale = fp16(absmax / 127), code = clamp(rint(x / scale),
-127, 127) with IEEE fp32 division and round-half-even; a zero scale gives zero codes.
"""

from __future__ import annotations

import ctypes

import torch

from . import _hip


def _i64(t: torch.Tensor) -> torch.Tensor:
    """Index vectors go to the kernels as contiguous int64."""
    return t if (t.dtype == torch.int64 and t.is_contiguous()) else t.to(torch.int64).contiguous()


def _require(ok: bool, msg: str) -> None:
    """The kernels index the pools with the shapes given here: a mismatch is refused before any launch."""
    if not ok:
        raise ValueError(msg)


def _token_pools(x: torch.Tensor, q_pool: torch.Tensor, s_pool: torch.Tensor) -> None:
    T, H, D = x.shape
    _require(q_pool.dim() == 4 and q_pool.shape[0] == H and q_pool.shape[3] == D,
             f"q_pool {tuple(q_pool.shape)} must be [H={H}, N, B, D={D}]")
    _require(tuple(s_pool.shape) == tuple(q_pool.shape[:3]),
             f"s_pool {tuple(s_pool.shape)} must be [H, N, B] = {tuple(q_pool.shape[:3])}")
    _require(q_pool.dtype == torch.int8 and s_pool.dtype == torch.float16, "q_pool must be int8 and s_pool fp16")
    _require(q_pool.is_contiguous() and s_pool.is_contiguous(), "the pools must be contiguous")


def quantize_store_tokens(x: torch.Tensor, blocks: torch.Tensor, offsets: torch.Tensor, q_pool: torch.Tensor,
                          s_pool: torch.Tensor, *, x2: torch.Tensor | None = None, q_pool2: torch.Tensor | None = None,
                          s_pool2: torch.Tensor | None = None) -> None:
    """x [T, H, D] (rows may be strided; last dim contiguous) -> q_pool [H, N, B, D] int8 and s_pool [H, N, B]
    fp16 at (blocks[t], offsets[t]). With x2, q_pool2, s_pool2 (the other of K and V, same shapes) both pairs are
    stored in the same launch, equal bit for bit to two calls. One launch."""
    T, H, D = x.shape
    if T == 0:
        return
    _require(x.stride(-1) == 1, "x needs a contiguous last dim")
    _require(blocks.numel() == T and offsets.numel() == T, f"{T} tokens need {T} blocks and offsets")
    _token_pools(x, q_pool, s_pool)
    _hip.require_gpu(x, blocks, offsets, q_pool, s_pool)
    blocks, offsets = _i64(blocks), _i64(offsets)
    if x2 is not None:
        if q_pool2 is None or s_pool2 is None:
            raise ValueError("x2 needs q_pool2 and s_pool2")
        if x2.shape != x.shape or x2.dtype != x.dtype or x2.stride(-1) != 1:
            raise ValueError("x2 must match x in shape and dtype, last dim contiguous")
        if (q_pool2.shape, q_pool2.stride(), q_pool2.dtype) != (q_pool.shape, q_pool.stride(), q_pool.dtype) or \
                (s_pool2.shape, s_pool2.stride(), s_pool2.dtype) != (s_pool.shape, s_pool.stride(), s_pool.dtype):
            raise ValueError("the second pools must match the first in shape, strides and dtype")
        _hip.require_gpu(x2, q_pool2, s_pool2)
        rc = _hip.lib().sipa_quantize_store_tokens_kv(
            x.data_ptr(), x2.data_ptr(), _hip.dtype_code(x.dtype), x.stride(0), x.stride(1), x2.stride(0),
            x2.stride(1), T, H, D, blocks.data_ptr(), offsets.data_ptr(), q_pool.data_ptr(), q_pool2.data_ptr(),
            q_pool.stride(0), q_pool.stride(1), q_pool.shape[2], s_pool.data_ptr(), s_pool2.data_ptr(),
            s_pool.stride(0), s_pool.stride(1), _hip.stream_of(x))
        _hip.check(rc, "quantize_store_tokens")
        return
    rc = _hip.lib().sipa_quantize_store_tokens(
        x.data_ptr(), _hip.dtype_code(x.dtype), x.stride(0), x.stride(1), T, H, D, blocks.data_ptr(),
        offsets.data_ptr(), q_pool.data_ptr(), q_pool.stride(0), q_pool.stride(1), q_pool.shape[2],
        s_pool.data_ptr(), s_pool.stride(0), s_pool.stride(1), _hip.stream_of(x))
    _hip.check(rc, "quantize_store_tokens")


def quantize_store_blocks(src_pool: torch.Tensor, src: torch.Tensor, dst: torch.Tensor, q_pool: torch.Tensor,
                          s_pool: torch.Tensor) -> None:
    """Blocks src_pool[:, src[i]] ([H, n_src, B, D], e.g. bf16 staging) -> q_pool[:, dst[i]] int8 with per-channel
    scales s_pool[:, dst[i]] ([H, N, D] fp16). One launch."""
    if src.numel() == 0:
        return
    H, _, B, D = src_pool.shape
    _require(src.numel() == dst.numel(), f"{src.numel()} sources for {dst.numel()} destinations")
    _require(q_pool.dim() == 4 and (q_pool.shape[0], q_pool.shape[2], q_pool.shape[3]) == (H, B, D),
             f"q_pool {tuple(q_pool.shape)} must be [H={H}, N, B={B}, D={D}]")
    _require(tuple(s_pool.shape) == (H, q_pool.shape[1], D), f"s_pool {tuple(s_pool.shape)} must be [H, N, D]")
    _require(q_pool.dtype == torch.int8 and s_pool.dtype == torch.float16, "q_pool must be int8 and s_pool fp16")
    _require(src_pool.is_contiguous() and q_pool.is_contiguous() and s_pool.is_contiguous(),
             "the pools must be contiguous")
    _hip.require_gpu(src_pool, src, dst, q_pool, s_pool)
    src, dst = _i64(src), _i64(dst)
    rc = _hip.lib().sipa_quantize_store_blocks(
        src_pool.data_ptr(), _hip.dtype_code(src_pool.dtype), src_pool.stride(0), src_pool.stride(1),
        src_pool.stride(2), src.data_ptr(), dst.data_ptr(), src.numel(), H, B, D, q_pool.data_ptr(),
        q_pool.stride(0), q_pool.stride(1), s_pool.data_ptr(), s_pool.stride(0), s_pool.stride(1),
        _hip.stream_of(src_pool))
    _hip.check(rc, "quantize_store_blocks")


def quantize_store_block_rows(x: torch.Tensor, rows: torch.Tensor, dst: torch.Tensor, q_pool: torch.Tensor,
                              s_pool: torch.Tensor) -> None:
    """Whole blocks taken from rows of x [T, H, D]: block i is rows[i*B : (i+1)*B] (B = q_pool's block size),
    rounded to bf16, then quantized per channel into q_pool[:, dst[i]], s_pool[:, dst[i]]. One launch."""
    if dst.numel() == 0:
        return
    H, _, B, D = q_pool.shape
    _require(x.dim() == 3 and x.shape[1] == H and x.shape[2] == D and x.stride(-1) == 1,
             f"x {tuple(x.shape)} must be [T, H={H}, D={D}] with a contiguous last dim")
    _require(tuple(s_pool.shape) == (H, q_pool.shape[1], D), f"s_pool {tuple(s_pool.shape)} must be [H, N, D]")
    _require(q_pool.dtype == torch.int8 and s_pool.dtype == torch.float16, "q_pool must be int8 and s_pool fp16")
    _require(q_pool.is_contiguous() and s_pool.is_contiguous(), "the pools must be contiguous")
    _require(rows.numel() == dst.numel() * B, f"{rows.numel()} rows for {dst.numel()} blocks of {B}")
    _hip.require_gpu(x, rows, dst, q_pool, s_pool)
    rows, dst = _i64(rows), _i64(dst)
    rc = _hip.lib().sipa_quantize_store_block_rows(
        x.data_ptr(), _hip.dtype_code(x.dtype), x.stride(0), x.stride(1), rows.data_ptr(), dst.data_ptr(),
        dst.numel(), H, B, D, q_pool.data_ptr(), q_pool.stride(0), q_pool.stride(1), s_pool.data_ptr(),
        s_pool.stride(0), s_pool.stride(1), _hip.stream_of(x))
    _hip.check(rc, "quantize_store_block_rows")


def store_tokens(x: torch.Tensor, blocks: torch.Tensor, offsets: torch.Tensor, pool: torch.Tensor,
                 rows: torch.Tensor | None = None, x2: torch.Tensor | None = None,
                 pool2: torch.Tensor | None = None) -> None:
    """pool[:, blocks[i], offsets[i]] = x[rows[i] if rows is not None else i] (x [T, H, D], pool [H, N, B, D]),
    converted to the pool's dtype with round-to-nearest-even; (x2, pool2) in the same launch (x2 may have other
    strides than x, as K and V views of a fused projection do). One launch."""
    n = blocks.numel()
    if n == 0:
        return
    T, H, D = x.shape
    _require(x.stride(-1) == 1 and pool.stride(-1) == 1, "x and the pool need a contiguous last dim")
    _require(pool.dim() == 4 and pool.shape[0] == H and pool.shape[3] == D,
             f"pool {tuple(pool.shape)} must be [H={H}, N, B, D={D}]")
    _require(offsets.numel() == n, f"{n} blocks but {offsets.numel()} offsets")
    _require(n <= T if rows is None else rows.numel() == n, "one source row per stored token")
    if x2 is not None:
        _require(x2.shape == x.shape and x2.stride(-1) == 1 and x2.dtype == x.dtype,
                 "x2 must match x in shape and dtype, last dim contiguous")
        _require(pool2 is not None and pool2.shape == pool.shape and pool2.stride() == pool.stride() and
                 pool2.dtype == pool.dtype, "pool2 must match the pool in shape, strides and dtype")
        _hip.require_gpu(x2, pool2)
    _hip.require_gpu(x, blocks, offsets, pool)
    blocks, offsets = _i64(blocks), _i64(offsets)
    rows = None if rows is None else _i64(rows)
    rc = _hip.lib().sipa_store_tokens(
        x.data_ptr(), _hip.ptr(x2), _hip.dtype_code(x.dtype), x.stride(0), x.stride(1),
        x.stride(0) if x2 is None else x2.stride(0), x.stride(1) if x2 is None else x2.stride(1), _hip.ptr(rows), n, H, D,
        blocks.data_ptr(), offsets.data_ptr(), pool.data_ptr(), _hip.ptr(pool2), _hip.dtype_code(pool.dtype),
        pool.stride(0), pool.stride(1), pool.stride(2), _hip.stream_of(x))
    _hip.check(rc, "store_tokens")


def kchan_write_rows(k: torch.Tensor, v: torch.Tensor, blocks: torch.Tensor, offsets: torch.Tensor,
                     stage_slots: torch.Tensor, quant_dst: torch.Tensor | None, v_pool: torch.Tensor,
                     v_scale: torch.Tensor, k_pool: torch.Tensor, k_scale: torch.Tensor, stage: torch.Tensor) -> None:
    """Format B's writes of a decode step in one launch (no reference counterpart; the reference's cache makes
    three calls, engine/quant_cache.py:161-170): row t's V quantized per token at (blocks[t], offsets[t]), its K
    rounded to bf16 into stage[:, stage_slots[t], offsets[t]], and, when quant_dst[t] >= 0 (quant_dst None: when
    offsets[t] is the block's last offset, into blocks[t]), the slot's block quantized per channel into
    k_pool / k_scale. Equal bit for bit to quantize_store_tokens + store_tokens + quantize_store_blocks when no
    two rows share a staging slot."""
    T, H, D = v.shape
    if T == 0:
        return
    _require(k.shape == v.shape and k.dtype == v.dtype, "k and v must match in shape and dtype")
    _require(k.stride(-1) == 1 and v.stride(-1) == 1, "k and v need a contiguous last dim")
    _require(blocks.numel() == T and offsets.numel() == T and stage_slots.numel() == T,
             f"{T} rows need {T} blocks, offsets and staging slots")
    _require(quant_dst is None or quant_dst.numel() == T, f"quant_dst needs {T} entries")
    _token_pools(v, v_pool, v_scale)
    N, B = v_pool.shape[1], v_pool.shape[2]
    _require(tuple(k_pool.shape) == tuple(v_pool.shape) and k_pool.dtype == torch.int8 and k_pool.is_contiguous(),
             f"k_pool {tuple(k_pool.shape)} must be int8 {tuple(v_pool.shape)}, contiguous")
    _require(tuple(k_scale.shape) == (H, N, D) and k_scale.dtype == torch.float16 and k_scale.is_contiguous(),
             f"k_scale {tuple(k_scale.shape)} must be fp16 [H={H}, N={N}, D={D}], contiguous")
    _require(stage.dim() == 4 and (stage.shape[0], stage.shape[2], stage.shape[3]) == (H, B, D)
             and stage.dtype == torch.bfloat16 and stage.stride(-1) == 1,
             f"stage {tuple(stage.shape)} must be bf16 [H={H}, n_stage, B={B}, D={D}]")
    _hip.require_gpu(k, v, blocks, offsets, stage_slots, v_pool, v_scale, k_pool, k_scale, stage)
    blocks, offsets, stage_slots = _i64(blocks), _i64(offsets), _i64(stage_slots)
    if quant_dst is not None:
        _hip.require_gpu(quant_dst)
        quant_dst = _i64(quant_dst)
    p = _hip.KchanWriteParams()
    p.k, p.v, p.x_dtype = k.data_ptr(), v.data_ptr(), _hip.dtype_code(v.dtype)
    p.k_stride_t, p.k_stride_h, p.v_stride_t, p.v_stride_h = k.stride(0), k.stride(1), v.stride(0), v.stride(1)
    p.T, p.H, p.D, p.B = T, H, D, B
    p.blocks, p.offsets, p.stage_slots = blocks.data_ptr(), offsets.data_ptr(), stage_slots.data_ptr()
    p.quant_dst = quant_dst.data_ptr() if quant_dst is not None else None
    p.v_pool, p.v_scale, p.k_pool, p.k_scale = v_pool.data_ptr(), v_scale.data_ptr(), k_pool.data_ptr(), k_scale.data_ptr()
    p.q_stride_h, p.q_stride_n = v_pool.stride(0), v_pool.stride(1)
    p.vs_stride_h, p.vs_stride_n = v_scale.stride(0), v_scale.stride(1)
    p.ks_stride_h, p.ks_stride_n = k_scale.stride(0), k_scale.stride(1)
    p.stage, p.st_stride_h, p.st_stride_n, p.st_stride_b = stage.data_ptr(), stage.stride(0), stage.stride(1), stage.stride(2)
    _hip.check(_hip.lib().sipa_kchan_write_rows(ctypes.byref(p), _hip.stream_of(v)), "kchan_write_rows")
