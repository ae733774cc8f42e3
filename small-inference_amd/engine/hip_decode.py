"""Paged decode attention on MI355X through libsmallinf_hip.so: the drop-in for the reference's
engine/triton_decode.py (paged_decode_attention, choose_splits, QuantKV; reference :164-238).

One query token per sequence, K/V read in place from the [Hkv, N, B, D] pool of one layer through the block
tables. The split count comes from the GPU's CU count instead of the reference's 20-SM constants: at most one
(sequence, KV head, split) workgroup per CU, splits of at most 2048 tokens (so that long sequences spread over
several CUs) and, for small batches, not so short that the merge's round trips outweigh the streaming they save
(the library's sipa_choose_splits_for). A split past a sequence's end does no work; the last split workgroup of a
(sequence, KV head) to finish merges the partials (combine="fused"), or a second kernel does (combine="kernel").

Kernels: bf16 queries with 16-token blocks and head_dim 64/128 run the MFMA kernels (bf16 pools, and both INT8
formats with fp16 or constant scales); everything else (fp32 models, other block sizes or head dims) runs the
VALU kernel. impl="valu" / "mfma" forces one.
"""

from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass

import numpy as np
import torch

from . import _hip

TILE = 64  # split chunks are multiples of 64 tokens; the block size must divide it (as in the reference)
DEFAULT_CU_COUNT = 256  # MI355X; used when no GPU is visible (host-side planning only)


@dataclass
class QuantKV:
    """INT8 side inputs of one layer. mode 1: k_scale, v_scale [Hkv, N, B] (per token). mode 2: k_scale
    [Hkv, N, D] (per block and channel; a zero block stride gives per-(head, channel) scales), v_scale [Hkv, N, B],
    stage [Hkv, n_stage, B, D] bf16 holding each sequence's partial last block of K, tail_slots [S] int32 (the
    sequence's staging slot, -1 if its last block is full). Scales are fp16 (the caches') or fp32."""
    mode: int
    k_scale: torch.Tensor
    v_scale: torch.Tensor
    stage: torch.Tensor | None = None
    tail_slots: torch.Tensor | None = None


_cu_counts: dict[int, int] = {}


def device_cu_count(device: torch.device | int | None = None) -> int:
    """CU count of a GPU (cached); DEFAULT_CU_COUNT when no GPU is visible."""
    if not torch.cuda.is_available():
        return DEFAULT_CU_COUNT
    if device is None:
        idx = torch.cuda.current_device()
    else:
        d = torch.device("cuda", device) if isinstance(device, int) else torch.device(device)
        idx = d.index if d.index is not None else torch.cuda.current_device()
    if idx not in _cu_counts:
        n = _hip.lib().sipa_device_cu_count(idx)
        if n <= 0:
            _hip.check(n, "sipa_device_cu_count")
        _cu_counts[idx] = n
    return _cu_counts[idx]


def choose_splits(num_seqs: int, num_kv_heads: int, max_context: int, cu_count: int | None = None) -> int:
    """Splits per sequence for a bf16/fp32 call: at most one workgroup per CU, splits of at most 2048 tokens and
    at least 512 past 8 splits (short contexts: up to 8 splits of at least 128 tokens)."""
    cu = device_cu_count() if cu_count is None else cu_count
    return int(_hip.lib().sipa_choose_splits(num_seqs, num_kv_heads, max_context, cu))


INT8_MAX_SPLIT = 4096  # the INT8 kernels stage a split's token scales in LDS: splits of at most this many tokens


def build_work_list(context_lens: list[int], num_kv_heads: int, cu_count: int | None = None,
                    items_per_cu: int = 3, max_piece: int = 0) -> tuple[np.ndarray, int]:
    """Work list for a ragged batch from host-side context lengths: ([n, 8] int32 items, largest split count of
    a pair). Each (sequence, KV head) pair is cut into near-equal pieces of about sum(ctx) * Hkv /
    (cu_count * items_per_cu) tokens (at most max_piece; 0: 32768); items are ordered longest first. Three items
    per CU measured best on MI355X (C3 ragged 256: 30.4 -> 29.4 us against two; 512 x U[1024, 16384]: 390 -> 382 us;
    four to six were no better)."""
    cu = device_cu_count() if cu_count is None else cu_count
    ctx = np.ascontiguousarray(context_lens, dtype=np.int32)
    lib, maxs = _hip.lib(), ctypes.c_int32(0)
    n = lib.sipa_build_work_list(ctx.ctypes.data, len(ctx), num_kv_heads, cu, items_per_cu, max_piece, None, 0,
                                 None)
    if n < 0:
        _hip.check(n, "build_work_list")
    items = np.zeros((n, 8), dtype=np.int32)
    rc = lib.sipa_build_work_list(ctx.ctypes.data, len(ctx), num_kv_heads, cu, items_per_cu, max_piece,
                                  items.ctypes.data, n, ctypes.byref(maxs))
    if rc < 0:
        _hip.check(rc, "build_work_list")
    return items, int(maxs.value)


def check_work_list(items: np.ndarray, num_seqs: int, num_kv_heads: int, max_context: int, num_splits: int) -> None:
    """Raise ValueError unless a host work list is consistent (sipa_check_work_list): each pair's splits listed
    once, in order, with one split count; ranges inside [0, max_context)."""
    items = np.ascontiguousarray(items, dtype=np.int32)
    _hip.check(_hip.lib().sipa_check_work_list(items.ctypes.data, items.shape[0], num_seqs, num_kv_heads, max_context,
                                              num_splits), "work list")


def is_ragged(context_lens: list[int]) -> bool:
    """Whether a batch gains from a work list: its lengths are far from uniform (total under 80% of
    num_seqs * max_context)."""
    return len(context_lens) > 1 and sum(context_lens) < 0.8 * len(context_lens) * max(context_lens)


def split_plan(max_context: int, num_splits: int) -> tuple[int, int]:
    """(splits actually launched, tokens per split) for a requested split count: chunks are rounded up to a
    multiple of 64 tokens and splits that would be empty for every sequence are dropped."""
    chunk = int(_hip.lib().sipa_split_chunk(max_context, num_splits))
    return math.ceil(max_context / chunk), chunk


def split_grid(num_seqs: int, num_kv_heads: int, max_context: int, num_splits: int, kv_mode: int = 0):
    """(splits, chunk, chunk_old, n_old): the split grid a call launches on the MFMA kernels without a work list:
    the first n_old splits of every sequence hold chunk_old tokens, the others chunk (sipa_decode_split_grid)."""
    c, co, no = ctypes.c_int32(0), ctypes.c_int32(0), ctypes.c_int32(0)
    n = _hip.lib().sipa_decode_split_grid(num_seqs, num_kv_heads, max_context, num_splits, kv_mode, ctypes.byref(c),
                                          ctypes.byref(co), ctypes.byref(no))
    if n < 0:
        _hip.check(n, "split grid")
    return int(n), int(c.value), int(co.value), int(no.value)


# Workspace (split partials + merge counters) per (device, stream): zero-filled once, the kernels leave the
# counters zero again, so later calls on the same stream reuse it without a memset.
_workspaces: dict[tuple[int, int], torch.Tensor] = {}


def reserve_workspace(device: torch.device, stream: int, nbytes: int) -> torch.Tensor:
    """The split workspace of (device, stream), at least nbytes (and 1 MiB) long. A larger request replaces the
    stream's buffer with a new zeroed one; the old one lives on only while something holds it, so code that keeps
    raw addresses beyond a call (captured graphs) must keep the tensor this returned, or reserve the largest size
    it will need before it records any address."""
    device = torch.device(device)
    index = device.index if device.index is not None else torch.cuda.current_device()
    key = (index, stream)
    ws = _workspaces.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=torch.device("cuda", index))
        _workspaces[key] = ws
    return ws


def grid_splits(num_seqs: int, num_kv_heads: int, max_context: int, quant_mode: int = 0,
                cu_count: int | None = None) -> int:
    """The split count a decode plan requests on the (sequence, KV head, split) grid when none is given: the
    library's policy for the kernel family, and for INT8 pools pieces of at most INT8_MAX_SPLIT tokens."""
    cu = device_cu_count() if cu_count is None else cu_count
    req = int(_hip.lib().sipa_choose_splits_for(num_seqs, num_kv_heads, max_context, cu, quant_mode))
    if quant_mode:
        req = max(req, math.ceil(max_context / INT8_MAX_SPLIT))
    return req


def decode_workspace_bytes(num_seqs: int, num_q_heads: int, num_kv_heads: int, head_dim: int, max_context: int,
                           quant_mode: int = 0, num_splits: int | None = None, cu_count: int | None = None) -> int:
    """Workspace bytes a grid decode of these shapes needs (num_splits None: the policy's split count)."""
    req = num_splits or grid_splits(num_seqs, num_kv_heads, max_context, quant_mode, cu_count)
    return int(_hip.lib().sipa_decode_workspace_bytes(num_seqs, num_q_heads, num_kv_heads, head_dim, req))


class DecodePlan:
    """Validated launch parameters of one paged decode, reusable across layers and steps of the same shapes.

    Building a plan does every shape, dtype and stride check and fills the C parameter block once; calling it
    swaps in the per-call tensors (q, the layer's pools and scales, out) and costs one ctypes call and one kernel
    launch. paged_decode_attention() builds a plan and runs it once; the caches build one per forward in begin()
    and run it for every layer.
    """

    def __init__(self, q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, block_tables: torch.Tensor,
                 context_lens: torch.Tensor, scale: float, max_context: int, num_splits: int | None = None,
                 quant: QuantKV | None = None, *, impl: str = "auto", combine: str = "fused",
                 host_context_lens: list[int] | None = None, work_list: str = "auto"):
        S, Hq, D = q.shape
        Hkv, N, B, _ = k_cache.shape
        # The reference asserts these (engine/triton_decode.py:201,211): AssertionError, raised explicitly so that
        # python -O keeps the checks.
        if not (q.stride(-1) == 1 and k_cache.is_contiguous() and v_cache.is_contiguous() and
                block_tables.stride(-1) == 1):
            raise AssertionError("q needs a contiguous last dim, the pools must be contiguous")
        if TILE % B:
            raise AssertionError(f"block size {B} must divide the {TILE}-token tile")
        _hip.require_gpu(q, k_cache, v_cache, block_tables, context_lens)
        if block_tables.dtype != torch.int32 or context_lens.dtype != torch.int32:
            raise ValueError("block_tables and context_lens must be int32")
        # the kernels load every sequence's table entries up to max_context before they read its length
        if block_tables.dim() != 2 or block_tables.shape[0] < S or block_tables.shape[1] * B < max_context:
            raise ValueError(f"block_tables {tuple(block_tables.shape)} must hold {S} rows of at least "
                             f"ceil({max_context} / {B}) entries")
        if context_lens.numel() < S:
            raise ValueError(f"context_lens holds {context_lens.numel()} lengths for {S} sequences")
        if impl not in _hip.IMPL or combine not in _hip.COMBINE:
            raise ValueError(f"impl {impl!r} / combine {combine!r}")
        self.shape, self.dtype, self.device = (S, Hq, D), q.dtype, q.device
        self.pool_shape, self.pool_dtype = tuple(k_cache.shape), k_cache.dtype
        self.quant_mode = 0 if quant is None else quant.mode
        self._keep = [block_tables, context_lens.contiguous()]  # tensors the parameter block points into
        self.lib = _hip.lib()
        self.stream = _hip.stream_of(q)
        if work_list not in ("auto", "on", "off"):
            raise ValueError(f"work_list {work_list!r}")
        use_list = work_list == "on" or (work_list == "auto" and num_splits is None and
                                         host_context_lens is not None and is_ragged(host_context_lens))
        if use_list and host_context_lens is None:
            raise ValueError("work_list='on' needs host_context_lens")
        self.items = None
        self.workspace = None
        self.chunk_old = self.n_old = 0  # the split grid's longer splits (see split_grid)
        if use_list:
            if len(host_context_lens) != S or max(host_context_lens, default=0) > max_context:
                raise ValueError("host_context_lens must hold S lengths, none above max_context")
            items, max_splits = build_work_list(host_context_lens, Hkv, device_cu_count(q.device),
                                                max_piece=0 if quant is None else INT8_MAX_SPLIT)
            check_work_list(items, S, Hkv, max_context, max_splits)
            self.items = torch.from_numpy(items).to(q.device)
            self._keep.append(self.items)
            self.requested = self.splits = max_splits
            self.chunk = None
        else:
            # The library's policy for this kernel family (the INT8 kernels run two workgroups per CU), and INT8
            # work in pieces of at most INT8_MAX_SPLIT tokens.
            self.requested = num_splits or grid_splits(S, Hkv, max_context, self.quant_mode, device_cu_count(q.device))
            if quant is not None:
                self.requested = max(self.requested, math.ceil(max_context / INT8_MAX_SPLIT))
            self.splits, self.chunk = split_plan(max_context, self.requested)
            if S > 0:
                _, chunk, self.chunk_old, self.n_old = split_grid(S, Hkv, max_context, self.requested, self.quant_mode)
                if self.n_old:
                    self.chunk = chunk

        p = self.params = _hip.DecodeParams()
        p.struct_size = ctypes.sizeof(_hip.DecodeParams)
        p.num_seqs, p.num_q_heads, p.num_kv_heads, p.head_dim, p.block_size = S, Hq, Hkv, D, B
        p.num_blocks, p.max_context, p.num_splits = N, max_context, self.requested
        p.q_dtype = _hip.dtype_code(q.dtype)
        p.impl, p.combine = _hip.IMPL[impl], _hip.COMBINE[combine]
        p.scale = float(scale)
        p.block_tables, p.bt_stride_s, p.bt_width = block_tables.data_ptr(), block_tables.stride(0), \
            block_tables.shape[1]
        p.context_lens = self._keep[1].data_ptr()
        p.kv_mode = self.quant_mode
        if self.items is not None:
            p.work_items, p.num_items = self.items.data_ptr(), self.items.shape[0]
        if quant is None:
            if k_cache.dtype != q.dtype or v_cache.dtype != q.dtype:
                raise ValueError("without `quant` the pool must be in q's dtype")
        else:
            if k_cache.dtype != torch.int8 or v_cache.dtype != torch.int8:
                raise ValueError("INT8 modes need int8 pools")
            if quant.mode not in (1, 2):
                raise ValueError(f"QuantKV.mode must be 1 or 2, got {quant.mode}")
            if quant.mode == 2:
                if quant.stage is None or quant.tail_slots is None:
                    raise ValueError("mode 2 needs stage and tail_slots")
                if quant.tail_slots.dtype != torch.int32:
                    raise ValueError("tail_slots must be int32")
                if quant.tail_slots.numel() < S:
                    raise ValueError(f"tail_slots holds {quant.tail_slots.numel()} slots for {S} sequences")
                tails = quant.tail_slots.contiguous()
                self._keep.append(tails)
                p.tail_slots = tails.data_ptr()
                self.num_stage = p.num_stage = quant.stage.shape[1]
        if S > 0 and self.splits > 1:
            nbytes = int(self.lib.sipa_decode_workspace_bytes(S, Hq, Hkv, D, self.requested))
            ws = reserve_workspace(q.device, self.stream, nbytes)
            self.workspace = ws
            self._keep.append(ws)
            p.workspace, p.workspace_bytes = ws.data_ptr(), ws.numel()
        self._bind(q, k_cache, v_cache, quant)

    def _bind(self, q, k_cache, v_cache, quant) -> None:
        """Point the parameter block at this call's tensors (same shapes and dtypes as the plan's)."""
        if tuple(q.shape) != self.shape or q.dtype != self.dtype or q.stride(-1) != 1:
            raise ValueError("q does not match the plan")
        if tuple(k_cache.shape) != self.pool_shape or tuple(v_cache.shape) != self.pool_shape or \
                k_cache.dtype != self.pool_dtype or v_cache.dtype != self.pool_dtype or \
                not (k_cache.is_contiguous() and v_cache.is_contiguous()):
            raise ValueError("the pools do not match the plan")
        self._q, self._k, self._v, self._quant = q, k_cache, v_cache, quant
        p = self.params
        p.q, p.q_stride_s, p.q_stride_h = q.data_ptr(), q.stride(0), q.stride(1)
        p.k_cache, p.v_cache = k_cache.data_ptr(), v_cache.data_ptr()
        p.kv_stride_h, p.kv_stride_n = k_cache.stride(0), k_cache.stride(1)
        if self.quant_mode:
            ks, vs = quant.k_scale, quant.v_scale
            if ks.stride(-1) != 1 or vs.stride(-1) != 1:
                raise ValueError("scales need a contiguous last dim")
            p.k_scale, p.k_scale_dtype, p.ks_stride_h, p.ks_stride_n = \
                ks.data_ptr(), _hip.dtype_code(ks.dtype), ks.stride(0), ks.stride(1)
            p.v_scale, p.v_scale_dtype, p.vs_stride_h, p.vs_stride_n = \
                vs.data_ptr(), _hip.dtype_code(vs.dtype), vs.stride(0), vs.stride(1)
            if self.quant_mode == 2:
                st = quant.stage
                if st.dtype != torch.bfloat16 or st.stride(-1) != 1:
                    raise ValueError("stage must be bf16 with a contiguous last dim")
                if st.shape[1] != self.num_stage:
                    raise ValueError("stage does not match the plan's staging slots")
                p.stage, p.st_stride_h, p.st_stride_n, p.st_stride_b = \
                    st.data_ptr(), st.stride(0), st.stride(1), st.stride(2)

    def __call__(self, q: torch.Tensor | None = None, k_cache: torch.Tensor | None = None,
                 v_cache: torch.Tensor | None = None, quant: QuantKV | None = None,
                 out: torch.Tensor | None = None) -> torch.Tensor:
        """Run the decode; tensors left as None keep the ones last bound. Returns out ([S, Hq, D], q's dtype)."""
        if q is not None or k_cache is not None or v_cache is not None or quant is not None:
            self._bind(q if q is not None else self._q, k_cache if k_cache is not None else self._k,
                       v_cache if v_cache is not None else self._v, quant if quant is not None else self._quant)
        if out is None:
            out = torch.empty(self.shape, device=self.device, dtype=self.dtype)
        elif tuple(out.shape) != self.shape or out.dtype != self.dtype or out.stride(-1) != 1:
            raise ValueError("out must be [S, Hq, D] in q's dtype with a contiguous last dim")
        if self.shape[0] == 0:
            return out
        p = self.params
        p.out, p.out_stride_s, p.out_stride_h = out.data_ptr(), out.stride(0), out.stride(1)
        _hip.check(self.lib.sipa_decode(ctypes.byref(p), self.stream), "paged_decode_attention")
        return out

    def launch_raw(self, k_ptr: int, v_ptr: int, out_ptr: int) -> int:
        """Lowest-overhead launch for benchmarks: swap the pool and output addresses only (pools with the bound
        shapes, strides and dtypes; out a contiguous [S, Hq, D] tensor in q's dtype) and return the C return
        code."""
        p = self.params
        p.k_cache, p.v_cache, p.out = k_ptr, v_ptr, out_ptr
        p.out_stride_s, p.out_stride_h = self.shape[1] * self.shape[2], self.shape[2]
        return self.lib.sipa_decode(ctypes.byref(p), self.stream)


def paged_decode_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, block_tables: torch.Tensor,
                           context_lens: torch.Tensor, scale: float, max_context: int,
                           num_splits: int | None = None, quant: QuantKV | None = None, *, impl: str = "auto",
                           combine: str = "fused", out: torch.Tensor | None = None,
                           host_context_lens: list[int] | None = None, work_list: str = "auto") -> torch.Tensor:
    """Attention of one query token per sequence over its paged context.

    q [S, Hq, D] (rows may be strided, last dim contiguous); k_cache, v_cache [Hkv, N, B, D], one layer of the
    pool, contiguous (int8 when `quant` is given); block_tables [S, max_blocks] int32; context_lens [S] int32 (each
    >= 1, the new token included); max_context = max(context_lens), known on the host. num_splits None picks from
    the CU count. Returns [S, Hq, D] in q's dtype (written into `out` if given).

    host_context_lens: the same lengths as a host list, when the caller has them (the caches do). A ragged batch
    then runs from a work list (work_list="auto"; "on" forces it, "off" keeps the split grid): near-equal pieces,
    longest first, always merged by the last-arriving workgroup.
    """
    plan = DecodePlan(q, k_cache, v_cache, block_tables, context_lens, scale, max_context, num_splits, quant,
                      impl=impl, combine=combine, host_context_lens=host_context_lens, work_list=work_list)
    return plan(out=out)
