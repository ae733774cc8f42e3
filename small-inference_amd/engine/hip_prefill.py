"""Paged attention for multi-token rows (prefill chunks) through libsmallinf_hip.so: the rows the reference
serves with its gather path (engine/paged_cache.py:149-155,174-175 with engine/attention.py:6-28), computed in
place from the block pool by one launch for all sequences of a forward.
"""

from __future__ import annotations

import ctypes

import torch

from . import _hip
from .hip_decode import reserve_workspace  # one split workspace per (device, stream) serves decode and prefill

# wg_layout names, indexed by their SIPA_PREFILL_* values
WG_LAYOUTS = ("auto", "w4x2", "w8x1", "w16x1", "w16h2")


def prefill_supported(q_dtype: torch.dtype, pool_dtype: torch.dtype, block_size: int, head_dim: int, group: int,
                      max_context: int) -> bool:
    """Whether the prefill kernel covers this shape (bf16 q; bf16 or int8 pool; 16-token blocks, head_dim 64/128,
    GQA group <= 8, contexts <= 32768); callers use the gather path otherwise."""
    return (q_dtype == torch.bfloat16 and pool_dtype in (torch.bfloat16, torch.int8) and block_size == 16 and
            head_dim in (64, 128) and group <= 8 and 0 < max_context <= 32768)


def _scale_dtype(t: torch.Tensor) -> int:
    if t.dtype == torch.float16:
        return _hip.F16
    if t.dtype == torch.float32:
        return _hip.F32
    raise ValueError(f"scales must be fp16 or fp32, got {t.dtype}")


def prefill_splits(num_q_heads: int, num_kv_heads: int, head_dim: int, query_lens: list[int], max_context: int,
                   cu_count: int = 0) -> int:
    """Key splits per query tile for a call whose sequences have these new-token counts (library policy)."""
    tiles = sum(-(-n // 16) for n in query_lens)
    return _hip.lib().sipa_prefill_splits(num_q_heads, num_kv_heads, head_dim, tiles, max_context, cu_count)


def paged_prefill_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, block_tables: torch.Tensor,
                            context_lens: torch.Tensor, query_starts: torch.Tensor, query_lens: torch.Tensor,
                            scale: float, max_context: int, max_query_len: int,
                            out: torch.Tensor | None = None, *, num_splits: int | None = None,
                            host_query_lens: list[int] | None = None, quant=None,
                            merge_path: str = "auto", wg_layout: str = "auto") -> torch.Tensor:
    """Causal attention of every sequence's new tokens over its paged context.

    q [T, Hq, D] bf16 (rows may be strided, last dim contiguous); k_cache, v_cache [Hkv, N, 16, D] bf16 (int8 with
    quant), one layer of the pool with this forward's K/V already written; block_tables
    [S, >= ceil(max_context / 16)] int32; context_lens [S] int32 (after the writes); query_starts, query_lens [S]
    int32: sequence s's new tokens are rows query_starts[s] .. + query_lens[s] - 1 of q at positions
    context_lens[s] - query_lens[s] ..; max_context and
    max_query_len are the host-known maxima. Writes those rows of out ([T, Hq, D], q's dtype; other rows are left
    as they are) and returns out. Each 16-token query tile's keys are cut into num_splits splits (default: the
    library's policy over host_query_lens when given, else over S x ceil(max_query_len / 16) tiles).
    INT8 pools take quant (engine.hip_decode.QuantKV: mode 1 per-token scales, mode 2 per-channel K scales with
    format B's staging and tail slots, which must then cover these S sequences); K/V are dequantized as the
    reference's gather path does, q * s in fp32 rounded to bf16.
    merge_path: "auto" merges a query tile's key splits from the L2 of the XCD they ran on when they shared one
    (the kernel places them so), through memory otherwise; "memory" always through memory. Same bits either way.
    wg_layout: the workgroup layout, waves x column tiles (a query head and 16 tokens) per wave: "w4x2", "w8x1",
    "w16x1", "w16h2" (16 waves over 8 column tiles and two consecutive key splits, combined in the workgroup;
    format B pools take the first two), or "auto", the library's choice by grid size and context
    (sipa_prefill_params.wg_layout). "w4x2" and "w8x1" give the same bits, "w16x1" too with one split.
    """
    S = block_tables.shape[0]
    T, Hq, D = q.shape
    Hkv, N, B, _ = k_cache.shape
    if out is None:
        out = torch.empty_like(q)
    pool_dtype = torch.int8 if quant is not None else torch.bfloat16
    if q.dtype != torch.bfloat16 or k_cache.dtype != pool_dtype or v_cache.dtype != pool_dtype:
        raise ValueError("the prefill kernel needs bf16 q and bf16 pools, or int8 pools with quant")
    for t in (block_tables, context_lens, query_starts, query_lens):
        if t.dtype != torch.int32:
            raise ValueError("block tables, context lengths and query rows must be int32")
    for t in (context_lens, query_starts, query_lens):
        if t.dim() != 1 or not t.is_contiguous() or t.numel() < S:
            raise ValueError("context lengths and query rows must be contiguous [num_seqs] vectors")
    if q.stride(-1) != 1 or out.stride(-1) != 1 or out.shape != q.shape or out.dtype != q.dtype:
        raise ValueError("q and out must be [T, Hq, D] of one dtype with a contiguous last dim")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()) or block_tables.stride(-1) != 1:
        raise ValueError("pools and block tables must be contiguous")
    _hip.require_gpu(q, k_cache, v_cache, block_tables, context_lens, query_starts, query_lens, out)
    p = _hip.PrefillParams()
    p.struct_size = ctypes.sizeof(_hip.PrefillParams)
    p.num_seqs, p.num_tokens, p.num_q_heads, p.num_kv_heads, p.head_dim, p.block_size = S, T, Hq, Hkv, D, B
    p.num_blocks, p.max_context, p.max_query_len, p.scale = N, max_context, max_query_len, float(scale)
    p.q, p.q_stride_t, p.q_stride_h = q.data_ptr(), q.stride(0), q.stride(1)
    p.k_cache, p.v_cache = k_cache.data_ptr(), v_cache.data_ptr()
    p.kv_stride_h, p.kv_stride_n = k_cache.stride(0), k_cache.stride(1)
    p.block_tables, p.bt_stride_s, p.bt_width = block_tables.data_ptr(), block_tables.stride(0), block_tables.shape[1]
    p.context_lens, p.query_starts = context_lens.data_ptr(), query_starts.data_ptr()
    p.query_lens = query_lens.data_ptr()
    p.out, p.out_stride_t, p.out_stride_h = out.data_ptr(), out.stride(0), out.stride(1)
    if quant is not None:
        if quant.mode not in (1, 2):
            raise ValueError(f"QuantKV mode {quant.mode}")
        p.kv_mode = quant.mode
        ks, vs = quant.k_scale, quant.v_scale
        p.k_scale, p.k_scale_dtype, p.ks_stride_h, p.ks_stride_n = ks.data_ptr(), _scale_dtype(ks), *ks.stride()[:2]
        p.v_scale, p.v_scale_dtype, p.vs_stride_h, p.vs_stride_n = vs.data_ptr(), _scale_dtype(vs), *vs.stride()[:2]
        if quant.mode == 2:
            st, tails = quant.stage, quant.tail_slots
            if st is None or tails is None or st.dtype != torch.bfloat16 or tails.dtype != torch.int32:
                raise ValueError("format B needs bf16 staging and int32 tail slots")
            if tails.numel() < S or not tails.is_contiguous():
                raise ValueError("tail slots must be a contiguous vector covering every sequence")
            p.stage, p.st_stride_h, p.st_stride_n, p.st_stride_b = st.data_ptr(), *st.stride()[:3]
            p.num_stage, p.tail_slots = st.shape[1], tails.data_ptr()
            _hip.require_gpu(q, st, tails)
        _hip.require_gpu(q, ks, vs)
    lib = _hip.lib()
    if num_splits is None:
        lens = host_query_lens if host_query_lens is not None else [max_query_len] * S
        num_splits = prefill_splits(Hq, Hkv, D, lens, max_context)
    p.num_splits = num_splits
    if merge_path not in ("auto", "memory"):
        raise ValueError(f"merge_path {merge_path!r} is neither 'auto' nor 'memory'")
    p.merge_path = 1 if merge_path == "memory" else 0
    if wg_layout not in WG_LAYOUTS:
        raise ValueError(f"wg_layout {wg_layout!r} is not one of {', '.join(WG_LAYOUTS)}")
    p.wg_layout = WG_LAYOUTS.index(wg_layout)
    stream = _hip.stream_of(q)
    nbytes = lib.sipa_prefill_workspace_bytes(S, Hq, Hkv, D, max_query_len, max_context, num_splits)
    if nbytes > 0:
        ws = reserve_workspace(q.device, stream, nbytes)
        p.workspace, p.workspace_bytes = ws.data_ptr(), ws.numel()
    _hip.check(lib.sipa_prefill(ctypes.byref(p), stream), "paged_prefill_attention")
    return out
