#!/usr/bin/env python3
"""Paged-decode HBM throughput on one MI355X: the reference's headline kernel benchmark on its named config.

Metric: paged-decode HBM GB/s and fraction of the 8 TB/s peak, and µs per call. Workload (config
C2): one layer of Qwen2.5-0.5B attention (14 query heads, 2 KV heads, head_dim 64), 16-token blocks, batch 32 x
8192 context, bf16 N(0, 1) Q/K/V from a fixed seed, block tables a random permutation of a 32768-block pool. A step
is one pass over the pool's rotated layers: one paged_decode_attention call per layer (8 calls by default, as a
decode step makes one call per layer), each over the whole batch with the CU-count split policy and the fused split
merge. `value` (GB/s) and `config.us_per_call` are per call; `ms_per_step` covers the step's calls.

Every timed region follows W warm-up calls and at least 0.3 s of back-to-back calls of the same kind, so that the
GPU runs at the clocks sustained work gets (an idle GPU clocks down). Bytes per call are algorithmic: K and V actually read from the pool plus Q and O (512 B per token + 3,584 B per
sequence for 0.5B); block tables and split partials are not counted. Calls rotate over 8 layers of a
[8, 2, 32768, 16, 64] pool so each call streams memory the previous calls did not touch (the 256 MB MALL cannot
serve it). Inputs are resident in HBM before the timed region.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--details/--no-details] [--no-cpu]

Prints one JSON line. `roofline.achieved` divides the bytes by the decode kernel's average duration from HIP
events around each launch; `cpu_baseline` times the CPU oracle's torch gather-then-attend (fp32) on the same
inputs on this machine's host cores; `details` holds the other configs (single pass, batch 1, C1, C3, C4 INT8
modes, the store kernels, the VALU kernel, the read-only streaming ceiling).
"""

from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parent
for _p in (ROOT, ROOT / "small-inference_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

PEAK_GBS = 8000.0  # MI355X HBM3E
METRIC = "paged-decode HBM GB/s & % of 8 TB/s peak (B=32, 8k ctx, bf16/INT8); µs/call"
TRAFFIC_FILE = ROOT / "profiles" / "decode_c2_traffic.json"


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


# ---- workloads -------------------------------------------------------------------------------------------------

class Decode:
    """A paged-decode workload: pools of `layers` layers on the GPU, one DecodePlan, algorithmic bytes per call."""

    def __init__(self, name, q, k, v, bt, ctx_t, lengths, scale, bytes_per_call, splits=None, quant=None,
                 impl="auto", combine="fused", meta=None, work_list="auto"):
        from engine.hip_decode import DecodePlan

        self.name, self.q, self.k, self.v, self.bt, self.ctx_t = name, q, k, v, bt, ctx_t
        self.lengths, self.scale, self.bytes = lengths, scale, bytes_per_call
        self.quant = quant  # per-layer list of QuantKV or None
        self.layers = k.shape[0]
        self.out = torch.empty_like(q)
        # One plan per layer, each bound to its layer's pools and scales: a call is one ctypes call + one launch.
        self.plans = [DecodePlan(q, k[i], v[i], bt, ctx_t, scale, max(lengths), splits,
                                 None if quant is None else quant[i], impl=impl, combine=combine,
                                 host_context_lens=list(lengths), work_list=work_list)
                      for i in range(self.layers)]
        self.plan = self.plans[0]
        self.k_ptrs = [k[i].data_ptr() for i in range(self.layers)]
        self.v_ptrs = [v[i].data_ptr() for i in range(self.layers)]
        self.out_ptr = self.out.data_ptr()
        self.meta = dict(meta or {}, splits=self.plan.splits, chunk=self.plan.chunk, impl=impl, combine=combine)
        if self.plan.n_old:
            self.meta.update(longer_splits=self.plan.n_old, longer_split_tokens=self.plan.chunk_old)
        if self.plan.items is not None:
            self.meta.update(work_items=int(self.plan.items.shape[0]), combine="fused")

    def call(self, i: int) -> None:
        layer = i % self.layers
        rc = self.plans[layer].launch_raw(self.k_ptrs[layer], self.v_ptrs[layer], self.out_ptr)
        if rc:
            from engine import _hip
            _hip.check(rc, self.name)


# Seconds of back-to-back calls before each timed region, after the `warmup` calls: a GPU left idle lowers its
# clocks, and a few calls do not raise them again (one 512-token prefill chunk at 8K context took 34.6-35.5 µs a
# call timed after 1 s idle, 33.1 after 10 warm-up calls, 30.9 after 0.5 s of calls).
WARM_S = 0.3
LAST_WARM_CALLS = 0  # calls time_calls made before its last timed region began


def time_calls(fn, steps: int, warmup: int, per_launch: bool, warm_s: float = WARM_S):
    """(ms per call over a back-to-back region, mean µs per call from event pairs around each call or None).
    Warm-up: `warmup` calls, then more until `warm_s` seconds of calls have run; their count is left in
    LAST_WARM_CALLS."""
    global LAST_WARM_CALLS
    t0, i = time.perf_counter(), 0
    while i < warmup or time.perf_counter() - t0 < warm_s:
        fn(i)
        i += 1
        if i % 32 == 0:
            torch.cuda.synchronize()  # the host stays within 32 calls of the GPU
    torch.cuda.synchronize()
    LAST_WARM_CALLS = i
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(steps):
        fn(warmup + i)
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    kern_us = None
    if per_launch:
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
        for i, (a, b) in enumerate(evs):
            a.record()
            fn(warmup + steps + i)
            b.record()
        torch.cuda.synchronize()
        kern_us = statistics.mean(a.elapsed_time(b) for a, b in evs) * 1e3
    return ms, kern_us


def lifo_tables(num_blocks: int, lengths: list[int], B: int, seed: int) -> list[list[int]]:
    """Block tables from a fragmented pool: fill it with one-block sequences, free them in a seeded random order,
    then allocate the sequences (the reference tests' LIFO-scattering pattern)."""
    from engine.block_manager import BlockManager

    m = BlockManager(num_blocks, B)
    g = torch.Generator().manual_seed(seed)
    for s in range(num_blocks):
        m.allocate(1 << 30 | s, B)
    for s in torch.randperm(num_blocks, generator=g).tolist():
        m.free(1 << 30 | s)
    for i, n in enumerate(lengths):
        m.allocate(i, n)
    return [m.block_table(i) for i in range(len(lengths))]


def padded(tables: list[list[int]], lengths: list[int], B: int) -> torch.Tensor:
    cut = [t[:-(-n // B)] for t, n in zip(tables, lengths)]
    w = max(len(t) for t in cut)
    return torch.tensor([t + [-1] * (w - len(t)) for t in cut], dtype=torch.int32, device="cuda")


def bf16_decode(name, lengths, N, Hq=14, Hkv=2, D=64, B=16, layers=8, seed=0, tables=None, splits=None,
                impl="auto", combine="fused", work_list="auto"):
    """bf16 pools [layers, Hkv, N, B, D] ~ N(0, 1), q ~ N(0, 1), scale 1/sqrt(D)."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    k = torch.randn(layers, Hkv, N, B, D, device="cuda", dtype=torch.bfloat16, generator=g)
    v = torch.randn(layers, Hkv, N, B, D, device="cuda", dtype=torch.bfloat16, generator=g)
    q = torch.randn(len(lengths), Hq, D, device="cuda", dtype=torch.bfloat16, generator=g)
    if tables is None:
        perm = torch.randperm(N, generator=torch.Generator().manual_seed(seed))
        tables, at = [], 0
        for n in lengths:
            nb = -(-n // B)
            tables.append(perm[at:at + nb].tolist())
            at += nb
    bt = padded(tables, lengths, B)
    ctx_t = torch.tensor(lengths, dtype=torch.int32, device="cuda")
    nbytes = 2 * Hkv * D * 2 * sum(lengths) + 2 * Hq * D * 2 * len(lengths)
    wl = Decode(name, q, k, v, bt, ctx_t, lengths, D ** -0.5, nbytes, splits, impl=impl, combine=combine,
                meta={"batch": len(lengths), "context": max(lengths), "pool_blocks": N}, work_list=work_list)
    wl.tables = tables
    return wl


def measure(wl, steps, warmup, per_launch=True) -> dict:
    """us per call over a back-to-back region (the figure that agrees with rocprof), its GB/s and fraction of the
    8 TB/s peak, and the per-call time with an event pair around each launch."""
    ms, pair_us = time_calls(wl.call, steps, warmup, per_launch)
    r = {"us_per_call": round(ms * 1e3, 2), "gb_s": round(wl.bytes / (ms * 1e-3) / 1e9, 1),
         "frac_of_peak": round(wl.bytes / (ms * 1e-3) / 1e9 / PEAK_GBS, 4), "bytes_per_call": wl.bytes}
    if pair_us is not None:
        r["event_pair_us"] = round(pair_us, 2)
    r.update(wl.meta)
    log(f"[bench] {wl.name}: {json.dumps(r)}")
    return r


def check_against_oracle(wl, layer=0, max_seqs=32) -> float:
    """Max-abs error of the GPU output for `layer` against the oracle's fp32 gather-then-attend (first seqs)."""
    import numpy as np
    from oracle import paged_ref

    wl.call(layer)  # rotation index == layer for the first `layers` calls
    torch.cuda.synchronize()
    got = wl.out.float().cpu().numpy()
    S = min(max_seqs, len(wl.lengths))
    err = 0.0
    for s in range(S):
        n, t = wl.lengths[s], wl.tables[s]
        idx = torch.tensor(t[:-(-n // wl.k.shape[3])], device="cuda")
        kk = wl.k[layer].index_select(1, idx).float().cpu().numpy()
        vv = wl.v[layer].index_select(1, idx).float().cpu().numpy()
        ref = paged_ref.attend_one(wl.q[s].float().cpu().numpy(), kk.reshape(kk.shape[0], -1, kk.shape[-1])[:, :n],
                                   vv.reshape(vv.shape[0], -1, vv.shape[-1])[:, :n], wl.scale, np.float32)
        err = max(err, float(np.abs(got[s] - ref).max()))
    return err


def cpu_baseline(wl, budget_s: float) -> dict:
    """The CPU oracle's torch fp32 gather-then-attend on the same inputs (layer 0), on the host cores."""
    from oracle import paged_ref

    threads = torch.get_num_threads()
    B = wl.k.shape[3]
    used = sorted({b for t, n in zip(wl.tables, wl.lengths) for b in t[:-(-n // B)]})
    remap = {b: i for i, b in enumerate(used)}
    idx = torch.tensor(used, dtype=torch.int64, device="cuda")
    k_cpu = wl.k[0].index_select(1, idx).cpu()
    v_cpu = wl.v[0].index_select(1, idx).cpu()
    tables = [[remap[b] for b in t[:-(-n // B)]] for t, n in zip(wl.tables, wl.lengths)]
    bt = torch.tensor([t + [-1] * (max(map(len, tables)) - len(t)) for t in tables], dtype=torch.int64)
    q_cpu = wl.q.cpu()
    times = []
    t_end = time.perf_counter() + budget_s
    out = None
    while len(times) < 5 or (time.perf_counter() < t_end and len(times) < 200):
        t0 = time.perf_counter()
        out = paged_ref.decode_torch_cpu(q_cpu, k_cpu, v_cpu, bt, wl.lengths, wl.scale)
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    wl.call(0)
    torch.cuda.synchronize()
    err = float((wl.out.float().cpu() - out).abs().max())
    r = {"value": round(wl.bytes / med / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
         "us_per_call": round(med * 1e6, 1), "reps": len(times), "max_abs_vs_gpu": round(err, 5),
         "sample": f"the full C2 batch ({len(wl.lengths)} x {max(wl.lengths)}), layer 0, oracle/paged_ref.py "
                   f"decode_torch_cpu (fp32 gather-then-attend, torch {threads} threads), median of {len(times)}"}
    log(f"[bench] cpu_baseline: {json.dumps(r)}")
    return r


def cpu_path(wl, budget_s: float = 2.0) -> dict:
    """The CPU oracle's fp32 gather-then-attend on a detail workload's layer 0 (the INT8 pools dequantized on the
    CPU inside the timed call, as the reference's gather path dequantizes): median time and GB/s over the same
    algorithmic bytes, beside the GPU figure."""
    from oracle import paged_ref

    B = wl.k.shape[3]
    used = sorted({b for t, n in zip(wl.tables, wl.lengths) for b in t[:-(-n // B)]})
    remap = {b: i for i, b in enumerate(used)}
    idx = torch.tensor(used, dtype=torch.int64, device="cuda")
    kq, vq = wl.k[0].index_select(1, idx).cpu(), wl.v[0].index_select(1, idx).cpu()
    tables = [[remap[b] for b in t[:-(-n // B)]] for t, n in zip(wl.tables, wl.lengths)]
    bt = torch.tensor([t + [-1] * (max(map(len, tables)) - len(t)) for t in tables], dtype=torch.int64)
    q = wl.q.cpu()
    if wl.quant is None:
        def run():
            return paged_ref.decode_torch_cpu(q, kq, vq, bt, wl.lengths, wl.scale)
    else:
        qk = wl.quant[0]
        ks, vs = qk.k_scale.index_select(1, idx).cpu(), qk.v_scale.index_select(1, idx).cpu()

        def run():
            k = kq.float() * (ks.float()[..., None] if qk.mode == 1 else ks.float()[:, :, None, :])
            v = vq.float() * vs.float()[..., None]
            return paged_ref.decode_torch_cpu(q, k, v, bt, wl.lengths, wl.scale)
    times, t_end = [], time.perf_counter() + budget_s
    while len(times) < 3 or (time.perf_counter() < t_end and len(times) < 50):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    return {"cpu_us_per_call": round(med * 1e6, 1), "cpu_gb_s": round(wl.bytes / med / 1e9, 3),
            "cpu_threads": torch.get_num_threads(), "cpu_reps": len(times)}


# ---- detail workloads ----------------------------------------------------------------------------------------------

def int8_decode(name, fmt, lengths, N, Hq=12, Hkv=2, D=128, B=16, layers=4, seed=0, impl="auto",
                f32_channel_scales=False, work_list="auto", splits=None):
    """1.5B-shaped INT8 pools built by the HIP quantize-and-store kernels from bf16 K ~ N(0, 1) with 4 of 128
    channels per head scaled by U[20, 68] and V ~ N(0, 1) (config C4)."""
    from engine.hip_decode import QuantKV
    from engine.hip_quant import quantize_store_blocks, quantize_store_tokens

    g = torch.Generator(device="cuda").manual_seed(seed)
    cpu_g = torch.Generator().manual_seed(seed)
    kq = torch.empty(layers, Hkv, N, B, D, dtype=torch.int8, device="cuda")
    vq = torch.empty_like(kq)
    vs = torch.empty(layers, Hkv, N, B, dtype=torch.float16, device="cuda")
    ks = torch.empty(layers, Hkv, N, B if fmt == "int8" else D, dtype=torch.float16, device="cuda")
    tok_blocks = torch.arange(N * B, device="cuda") // B
    tok_offs = torch.arange(N * B, device="cuda") % B
    for layer in range(layers):
        chan_scale = torch.ones(Hkv, 1, 1, D)
        for h in range(Hkv):
            ch = torch.randperm(D, generator=cpu_g)[:4]
            chan_scale[h, 0, 0, ch] = 20 + 48 * torch.rand(4, generator=cpu_g)
        kb = (torch.randn(Hkv, N, B, D, device="cuda", generator=g) * chan_scale.cuda()).bfloat16()
        vb = torch.randn(Hkv, N, B, D, device="cuda", generator=g).bfloat16()
        as_tokens = lambda x: x.permute(1, 2, 0, 3).reshape(N * B, Hkv, D)  # noqa: E731  (a strided view)
        quantize_store_tokens(as_tokens(vb), tok_blocks, tok_offs, vq[layer], vs[layer])
        if fmt == "int8":
            quantize_store_tokens(as_tokens(kb), tok_blocks, tok_offs, kq[layer], ks[layer])
        else:
            ids = torch.arange(N, device="cuda")
            quantize_store_blocks(kb, ids, ids, kq[layer], ks[layer])
        del kb, vb
    q = torch.randn(len(lengths), Hq, D, device="cuda", dtype=torch.bfloat16, generator=g)
    perm = torch.randperm(N, generator=cpu_g)
    tables, at = [], 0
    for n in lengths:
        nb = -(-n // B)
        tables.append(perm[at:at + nb].tolist())
        at += nb
    bt = padded(tables, lengths, B)
    ctx_t = torch.tensor(lengths, dtype=torch.int32, device="cuda")
    if fmt == "int8":
        quant = [QuantKV(1, ks[i], vs[i]) for i in range(layers)]
        per_token = 2 * Hkv * (D + 2)
    else:
        stage = torch.zeros(Hkv, 4, B, D, dtype=torch.bfloat16, device="cuda")
        tails = torch.full((len(lengths),), -1, dtype=torch.int32, device="cuda")  # 4096 is block-aligned
        if f32_channel_scales:  # the literal reading of C4(a): one fp32 scale per (head, channel), block stride 0
            kscale = [ks[i][:, :1].float().expand(Hkv, N, D) for i in range(layers)]
        else:
            kscale = [ks[i] for i in range(layers)]
        quant = [QuantKV(2, kscale[i], vs[i], stage, tails) for i in range(layers)]
        per_token = Hkv * (D + 2) + Hkv * (D + 2 * D / B)
    nbytes = int(per_token * sum(lengths)) + 2 * Hq * D * 2 * len(lengths)
    wl = Decode(name, q, kq, vq, bt, ctx_t, lengths, D ** -0.5, nbytes, splits, quant, impl=impl, work_list=work_list,
                meta={"batch": len(lengths), "context": max(lengths), "format": fmt,
                      "k_scales": "fp32 per (head, channel)" if f32_channel_scales else "fp16 per (block, channel)"
                      if fmt != "int8" else "fp16 per token"})
    wl.tables = tables
    return wl


def store_bench(steps: int) -> dict:
    """C3's bf16 store of one new K/V token for each of 256 sequences, and C4's INT8 quantize-and-store of 64 new
    tokens (K and V, 1.5B), with the C4 codes checked bit-exact against the C oracle."""
    import numpy as np
    from engine.hip_quant import quantize_store_tokens, store_tokens
    from oracle import paged_ref

    res = {}
    g = torch.Generator(device="cuda").manual_seed(7)
    # C3: 256 tokens of [2, 64] bf16 K and V into partially filled last blocks of a 200k-block pool
    N = 200_000
    pk = torch.zeros(2, N, 16, 64, dtype=torch.bfloat16, device="cuda")
    pv = torch.zeros_like(pk)
    x = torch.randn(256, 2, 64, device="cuda", dtype=torch.bfloat16, generator=g)
    y = torch.randn(256, 2, 64, device="cuda", dtype=torch.bfloat16, generator=g)
    blocks = torch.randperm(N, generator=torch.Generator().manual_seed(7))[:256].cuda()
    offs = torch.randint(1, 16, (256,), generator=torch.Generator().manual_seed(8)).cuda()
    ms, kus = time_calls(lambda i: store_tokens(x, blocks, offs, pk, x2=y, pool2=pv), steps, 20, True)
    ok = bool(torch.equal(pk[:, blocks, offs], x.transpose(0, 1)) and torch.equal(pv[:, blocks, offs],
                                                                                  y.transpose(0, 1)))
    res["c3_store_bf16"] = {"us_per_call": round(ms * 1e3, 2), "kernel_us": round(kus, 2), "tokens": 256,
                            "bytes_per_call": 4 * 256 * 2 * 64 * 2, "exact": ok}
    # C4: 64 new tokens, K and V [64, 2, 128] bf16, per-token INT8 into a 32768-block pool
    N = 32768
    qk = torch.zeros(2, N, 16, 128, dtype=torch.int8, device="cuda")
    qv = torch.zeros_like(qk)
    sk = torch.zeros(2, N, 16, dtype=torch.float16, device="cuda")
    sv = torch.zeros_like(sk)
    kx = (torch.randn(64, 2, 128, device="cuda", generator=g) * 3).bfloat16()
    vx = torch.randn(64, 2, 128, device="cuda", generator=g).bfloat16()
    blocks = torch.randperm(N, generator=torch.Generator().manual_seed(9))[:64].cuda()
    offs = torch.randint(0, 16, (64,), generator=torch.Generator().manual_seed(10)).cuda()

    def qs(i):
        quantize_store_tokens(kx, blocks, offs, qk, sk)
        quantize_store_tokens(vx, blocks, offs, qv, sv)

    def check() -> bool:
        exact = True
        for xx, qq, ss in ((kx, qk, sk), (vx, qv, sv)):
            q_ref, s_ref = paged_ref.quantize_per_token(xx.float().cpu().numpy())
            exact &= bool(np.array_equal(qq[:, blocks, offs].transpose(0, 1).cpu().numpy(), q_ref))
            exact &= bool(np.array_equal(ss[:, blocks, offs].t().cpu().numpy().view(np.uint16),
                                         s_ref.view(np.uint16)))
        return exact

    ms, kus = time_calls(qs, steps, 20, True)
    exact = check()
    # the same K and V in one launch (the cache's per-token write)
    for t in (qk, qv, sk, sv):
        t.zero_()
    ms1, kus1 = time_calls(lambda i: quantize_store_tokens(vx, blocks, offs, qv, sv, x2=kx, q_pool2=qk, s_pool2=sk),
                           steps, 20, True)
    res["c4_quantize_store_64"] = {"us_per_call": round(ms * 1e3, 2), "kernel_us_2_launches": round(kus, 2),
                                   "us_per_call_one_launch": round(ms1 * 1e3, 2),
                                   "kernel_us_one_launch": round(kus1, 2), "tokens": 64,
                                   "bit_exact_vs_oracle": exact and check(),
                                   "bytes_per_call": 2 * (64 * 2 * 128 * 2 + 64 * 2 * 128 + 64 * 2 * 2)}
    log(f"[bench] stores: {json.dumps(res)}")
    return res


def prefill_bench(steps: int, warmup: int) -> dict:
    """Multi-token rows (prefill) with 0.5B shapes: the HIP paged prefill kernel against the reference's gather
    path (per sequence: gather K/V out of the pool, engine/attention.py's bmm-softmax-bmm in bf16) on the same
    inputs. Cases: 4 fresh 2048-token prompts, and one 512-token chunk at 8K context. Reports µs per call, the
    causal attention TFLOP/s (4 D Hq flops per visible (query, key) pair) and the max-abs difference between the
    two paths."""
    from engine.attention import attention
    from engine.hip_prefill import paged_prefill_attention

    from engine.hip_decode import QuantKV
    from engine.quant import quantize_per_token

    Hq, Hkv, D, B, N = 14, 2, 64, 16, 32768
    res = {}
    for name, ctx, qlen, int8 in (("prefill_4x2048_fresh", [2048] * 4, [2048] * 4, False),
                                  ("prefill_512_at_8k", [8192], [512], False),
                                  ("prefill_512_at_8k_int8", [8192], [512], True)):
        g = torch.Generator(device="cuda").manual_seed(3)
        k = torch.randn(Hkv, N, B, D, device="cuda", dtype=torch.bfloat16, generator=g)
        v = torch.randn(Hkv, N, B, D, device="cuda", dtype=torch.bfloat16, generator=g)
        quant = None
        if int8:  # per-token INT8 pools (format "int8"); the gather path dequantizes them to bf16 per call
            (kq, ks), (vq, vs) = quantize_per_token(k), quantize_per_token(v)
            quant = QuantKV(1, ks, vs)
        T = sum(qlen)
        q = torch.randn(T, Hq, D, device="cuda", dtype=torch.bfloat16, generator=g)
        tables = lifo_tables(N, ctx, B, 3)
        bt = padded(tables, ctx, B)
        starts = [sum(qlen[:i]) for i in range(len(qlen))]
        i32 = lambda xs: torch.tensor(xs, dtype=torch.int32, device="cuda")  # noqa: E731
        c, st, ln = i32(ctx), i32(starts), i32(qlen)
        out = torch.empty_like(q)
        scale = D ** -0.5

        def kern(i):
            if quant is None:
                paged_prefill_attention(q, k, v, bt, c, st, ln, scale, max(ctx), max(qlen), out=out)
            else:
                paged_prefill_attention(q, kq, vq, bt, c, st, ln, scale, max(ctx), max(qlen), out=out, quant=quant)

        blocks = [torch.tensor(t[:-(-n // B)], device="cuda") for t, n in zip(tables, ctx)]
        kpos = torch.arange(max(ctx), device="cuda")

        def gather_path(i):
            outs = []
            for s in range(len(ctx)):
                if quant is None:
                    kk = k[:, blocks[s]].view(Hkv, -1, D)[:, :ctx[s]]
                    vv = v[:, blocks[s]].view(Hkv, -1, D)[:, :ctx[s]]
                else:  # engine/quant_cache.py gather(): dequantize the sequence's blocks to the model dtype
                    kk = (kq[:, blocks[s]].float() * ks[:, blocks[s]].float()[..., None]).bfloat16()
                    vv = (vq[:, blocks[s]].float() * vs[:, blocks[s]].float()[..., None]).bfloat16()
                    kk, vv = kk.view(Hkv, -1, D)[:, :ctx[s]], vv.view(Hkv, -1, D)[:, :ctx[s]]
                qpos = torch.arange(ctx[s] - qlen[s], ctx[s], device="cuda")
                outs.append(attention(q[starts[s]:starts[s] + qlen[s]], kk, vv, qpos, kpos[:ctx[s]], scale))
            return torch.cat(outs)

        ms, kus = time_calls(kern, steps, warmup, True)
        gms, _ = time_calls(gather_path, max(3, steps // 10), 2, False)
        diff = (out.float().view(T, -1) - gather_path(0).float()).abs().max().item()
        pairs = sum(sum(n - m + r + 1 for r in range(m)) for n, m in zip(ctx, qlen))
        flops = 4 * D * Hq * pairs
        res[name] = {"us_per_call": round(ms * 1e3, 2), "kernel_us": round(kus, 2),
                     "tflop_s": round(flops / (ms * 1e-3) / 1e12, 1),
                     "frac_of_bf16_mfma_peak": round(flops / (ms * 1e-3) / 2.5e15, 4),
                     "gather_path_us": round(gms * 1e3, 1), "speedup_vs_gather": round(gms / ms, 2),
                     "max_abs_vs_gather_path": round(diff, 5), "tokens": T, "context": ctx,
                     "pool": "int8 per-token" if int8 else "bf16"}
        del k, v
        torch.cuda.empty_cache()
    log(f"[bench] prefill: {json.dumps(res)}")
    return res


def paged_read_floor(wl, steps: int, warmup: int) -> dict:
    """The same call's HBM reads without the decode arithmetic or the split merge (csrc/probe.hip
    sipa_probe_paged_read: the same grid or work list, block-table staging, two 32-token tiles in flight per wave,
    and the INT8 kernels' scale reads: per-token rows, or format B's per-channel K rows and per-token V rows): the
    floor a decode kernel of this layout reaches on this access pattern."""
    lib = ctypes.CDLL(str(ROOT / "small-inference_amd" / "build" / "libsmallinf_probe.so"))
    vp, i32, i64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64
    lib.sipa_probe_paged_read.argtypes = [vp, vp, vp, vp, vp, i64, i32, i32, i32, i32, i32, i32, vp, i32, i64, i64,
                                          i64, i64, i32, i64, i64, i32, i32, vp, vp]
    lib.sipa_probe_paged_read.restype = i32
    sink = torch.zeros(1 << 16, dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    k0, esz = wl.k[0], wl.k.element_size()
    Hkv, N, B, D = k0.shape
    ctx = max(wl.lengths)
    plan = wl.plan
    items = plan.items
    if items is None:
        assert min(wl.lengths) == ctx, "the grid floor takes a uniform batch"
    mode = 0 if wl.quant is None else wl.quant[0].mode

    def call(i):
        layer = i % wl.layers
        ks = vs = None
        ks_sh = ks_sn = vs_sh = vs_sn = ks_row = vs_row = 0
        if mode:
            q = wl.quant[layer]
            ks, vs = q.k_scale.data_ptr(), q.v_scale.data_ptr()
            vs_sh, vs_sn, vs_row = q.v_scale.stride(0) * 2, q.v_scale.stride(1) * 2, B * 2
            ks_sh, ks_sn = q.k_scale.stride(0) * q.k_scale.element_size(), q.k_scale.stride(1) * q.k_scale.element_size()
            ks_row = (B if mode == 1 else D) * q.k_scale.element_size()
        rc = lib.sipa_probe_paged_read(wl.k[layer].data_ptr(), wl.v[layer].data_ptr(), ks, vs, wl.bt.data_ptr(),
                                       wl.bt.stride(0), len(wl.lengths), Hkv, ctx, plan.chunk or 0, plan.chunk_old,
                                       plan.n_old, None if items is None else items.data_ptr(),
                                       0 if items is None else items.shape[0], k0.stride(0) * esz,
                                       k0.stride(1) * esz, ks_sh, ks_sn, ks_row, vs_sh, vs_sn, vs_row, D * esz,
                                       sink.data_ptr(), stream)
        if rc:
            raise RuntimeError(f"sipa_probe_paged_read: {rc}")

    ms, _ = time_calls(call, steps, warmup, per_launch=False)
    r = {"us_per_call": round(ms * 1e3, 2), "gb_s": round(wl.bytes / (ms * 1e-3) / 1e9, 1),
         "frac_of_peak": round(wl.bytes / (ms * 1e-3) / 1e9 / PEAK_GBS, 4), "splits": plan.splits,
         "scales": ["none", "per token", "per channel K, per token V"][mode],
         "grid": "work list" if items is not None else ("two-length splits" if plan.n_old else "equal splits")}
    log(f"[bench] {wl.name} paged-read floor: {json.dumps(r)}")
    return r


def stream_ceiling(steps: int) -> dict:
    """Read-only streaming ceiling of this GPU from the probe library (1 GiB buffers, 4 rotating)."""
    lib = ctypes.CDLL(str(ROOT / "small-inference_amd" / "build" / "libsmallinf_probe.so"))
    lib.sipa_probe_read.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int32,
                                    ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p]
    nbytes = 1 << 30
    bufs = [torch.empty(nbytes, dtype=torch.uint8, device="cuda") for _ in range(4)]
    sink = torch.zeros(1 << 16, dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    best, sweep = {}, []
    for wgs in (256, 512, 1024, 2048, 4096):
        for unroll in (4, 8, 16):
            for nt in (0, 1):
                def rd(i, wgs=wgs, unroll=unroll, nt=nt):
                    if lib.sipa_probe_read(bufs[i % 4].data_ptr(), nbytes, sink.data_ptr(), wgs, unroll, nt,
                                           stream):
                        raise RuntimeError("probe read launch failed")
                ms, kus = time_calls(rd, max(8, steps // 20), 4, True, warm_s=0.0)  # the sweep runs back to back
                gbs = nbytes / (kus * 1e-6) / 1e9
                sweep.append((wgs, unroll, nt, round(gbs, 1)))
                if gbs > best.get("gb_s", 0):
                    best = {"gb_s": round(gbs, 1), "workgroups": wgs, "loads_in_flight_per_lane": unroll,
                            "nontemporal": nt, "bytes": nbytes, "frac_of_peak": round(gbs / PEAK_GBS, 4)}
    best["sweep"] = sweep
    log(f"[bench] stream ceiling: {json.dumps(best)}")
    del bufs
    return best


def c3_context_lengths() -> list[int]:
    """C3's 256 ragged context lengths: seeded log-normal around 600 tokens, clipped to [16, 8192]."""
    import numpy as np

    rng = np.random.default_rng(0)
    return np.clip(np.rint(rng.lognormal(math.log(600), 1.0, 256)), 16, 8192).astype(int).tolist()


def details(steps: int, warmup: int) -> dict:
    out = {}
    c2 = bf16_decode("c2_single_pass", [8192] * 32, 32768, splits=1)
    out["c2_single_pass"] = measure(c2, steps, warmup)
    out["c2_single_pass"]["max_abs_vs_oracle"] = round(check_against_oracle(c2), 5)
    out["c2_separate_combine"] = measure(bf16_decode("c2_separate_combine", [8192] * 32, 32768, combine="kernel"),
                                         steps, warmup)
    out["c2_valu"] = measure(bf16_decode("c2_valu", [8192] * 32, 32768, impl="valu"), steps // 2, warmup)
    del c2
    torch.cuda.empty_cache()
    for splits, label in ((1, "single_pass"), (None, "split")):
        out[f"c2_batch1_{label}"] = measure(bf16_decode(f"c2_batch1_{label}", [8192], 8192, layers=64,
                                                        splits=splits), steps, warmup)
    c1_lengths = [1024]
    c1 = bf16_decode("c1", c1_lengths, 4096, layers=64, tables=lifo_tables(4096, c1_lengths, 16, 0))
    c1.scale = 1 / 8
    out["c1_1x1024"] = measure(c1, steps, warmup)
    out["c1_1x1024"]["max_abs_vs_oracle"] = round(check_against_oracle(c1), 5)
    out["c1_1x1024"].update(cpu_path(c1))
    c3_lengths = c3_context_lengths()
    for key, wlist in (("c3_ragged256", "auto"), ("c3_ragged256_split_grid", "off")):
        c3 = bf16_decode(key, c3_lengths, 200_000, layers=4, work_list=wlist)
        out[key] = measure(c3, steps, warmup)
        out[key]["sum_context"] = int(sum(c3_lengths))
        out[key]["max_abs_vs_oracle_first32"] = round(check_against_oracle(c3), 5)
        if wlist == "auto":
            out[key].update(cpu_path(c3))
            out[key]["paged_read_floor"] = paged_read_floor(c3, steps, warmup)
        del c3
        torch.cuda.empty_cache()
    torch.cuda.empty_cache()
    c4_lengths = [4096] * 64
    for fmt, f32s, key in (("int8", False, "c4b_int8_per_token"), ("int8-kchannel", False, "c4a_int8_kchannel"),
                           ("int8-kchannel", True, "c4a_int8_kchannel_f32_head_channel_scales")):
        wl = int8_decode(key, fmt, c4_lengths, 32768, f32_channel_scales=f32s)
        out[key] = measure(wl, steps, warmup)
        if not f32s:
            out[key].update(cpu_path(wl))
            out[key]["paged_read_floor"] = paged_read_floor(wl, steps, warmup)
        del wl
        torch.cuda.empty_cache()
    out.update(store_bench(steps))
    out.update(prefill_bench(steps, warmup))
    out["graph_decode_steps"] = graph_step_bench()
    out["stream_read_ceiling"] = stream_ceiling(steps)
    torch.cuda.empty_cache()
    for fmt in ("bf16", "int8"):
        try:
            out[f"c5_decode_step_{fmt}"] = decode_step_bench(fmt=fmt)
        except (RuntimeError, torch.OutOfMemoryError) as e:  # a box with less free HBM than the pool needs
            out[f"c5_decode_step_{fmt}"] = {"error": str(e)[:200]}
        torch.cuda.empty_cache()
    return out


def decode_step_bench(steps: int = 5, warmup: int = 2, batch: int = 512, pool_fraction: float = 0.85,
                      fmt: str = "bf16", seed: int = 0) -> dict:
    """Config C5: packed decode steps of a random-init Qwen2.5-0.5B-shaped model (engine/model.py, torch GEMMs)
    through the paged cache with the HIP store and decode kernels, batch 512, contexts ~ U[1024, 16384], over a
    pool sized to `pool_fraction` of free HBM with scattered block ids. Reports host metadata time, GPU step time,
    tokens/s and the share of the step spent in the 24 decode-attention launches."""
    import random
    import time

    from engine.block_manager import BlockManager
    from engine.config import QWEN2_5_0_5B as cfg
    from engine.device_tables import DeviceBlockTables
    from engine.model import Qwen2Model
    from engine.paged_cache import PagedKVCache, build_metadata
    from engine.quant_cache import QuantPagedKVCache, kv_bytes_per_token

    rng = random.Random(seed)
    ctx = [rng.randint(1024, 16384) for _ in range(batch)]
    B = 16
    free, _ = torch.cuda.mem_get_info()
    per_block = int(B * kv_bytes_per_token(cfg, fmt))
    N = int(free * pool_fraction) // per_block
    need = sum(-(-(n + steps + warmup) // B) for n in ctx)
    if N < need:
        raise RuntimeError(f"pool of {N} blocks cannot hold the batch ({need} blocks)")
    m = BlockManager(N, B)
    rng.shuffle(m._free)  # a long-running pool: every table scattered over the whole pool
    if fmt == "bf16":
        cache = PagedKVCache(cfg, N, B, "cuda", torch.bfloat16, attn_backend="triton")
    else:
        cache = QuantPagedKVCache(cfg, N, B, "cuda", torch.bfloat16, "triton", fmt, m, n_stage=2 * batch)
    gen = torch.Generator(device="cuda").manual_seed(seed)
    for t in (cache.k, cache.v):  # the contexts' K/V: unit-variance values (the INT8 pools: random codes)
        if t.dtype == torch.int8:
            t.random_(-127, 128, generator=gen)
        else:
            t.normal_(generator=gen)
    if fmt != "bf16":
        for t in (cache.k_scale, cache.v_scale):
            t.fill_(1.0 / 64)
    for s, n in enumerate(ctx):
        m.allocate(s, n)
    model = Qwen2Model(cfg, "cuda", torch.bfloat16, seed=seed, max_positions=16384 + steps + warmup + 1)
    ids = torch.randint(0, cfg.vocab_size, (batch,), device="cuda", generator=gen)
    dev_tables = DeviceBlockTables(m, "cuda", max_seqs=batch, max_blocks=-(-(16384 + steps + warmup + 1) // B))
    host_ms, dev_ms, gpu_ms, attn_ms = [], [], [], []
    for step in range(warmup + steps):
        batch_desc = []
        for s in range(batch):
            m.append_slot(s)
            batch_desc.append((s, ctx[s], 1))
            ctx[s] += 1
        t0 = time.perf_counter()
        meta_host = build_metadata(m, batch_desc, "cuda")  # the reference's host-side builder (for its time)
        t1 = time.perf_counter()
        meta = dev_tables.build(batch_desc)  # the device-side builder drives the step
        t2 = time.perf_counter()
        del meta_host
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        logits = model.forward(ids, meta.positions, cache, meta)
        ids = logits.argmax(-1)
        e1.record()
        torch.cuda.synchronize()
        if step < warmup:
            continue
        host_ms.append((t1 - t0) * 1e3)
        dev_ms.append((t2 - t1) * 1e3)
        gpu_ms.append(e0.elapsed_time(e1))
        # The same step's 24 decode launches alone, through the plan the forward built (q from a random tensor).
        plan = cache._plan
        q = torch.randn(batch, cfg.num_q_heads, cfg.head_dim, device="cuda", dtype=torch.bfloat16, generator=gen)
        out = torch.empty_like(q)
        a0, a1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a0.record()
        for layer in range(cfg.num_layers):
            plan(q=q, k_cache=cache.k[layer], v_cache=cache.v[layer], quant=cache._kernel_quant(layer), out=out)
        a1.record()
        torch.cuda.synchronize()
        attn_ms.append(a0.elapsed_time(a1))
    med = lambda xs: sorted(xs)[len(xs) // 2]  # noqa: E731
    g, h, dm, a = med(gpu_ms), med(host_ms), med(dev_ms), med(attn_ms)
    kv_bytes = 2 * cfg.num_layers * cfg.num_kv_heads * cfg.head_dim * (2 if fmt == "bf16" else 1) * sum(ctx)
    r = {"format": fmt, "batch": batch, "context_mean": round(sum(ctx) / batch), "pool_blocks": N,
         "pool_gb": round(N * per_block / 1e9, 1), "gpu_step_ms": round(g, 3),
         "host_metadata_ms": round(h, 3), "device_metadata_host_ms": round(dm, 3),
         "tokens_per_s_gpu": round(batch / (g * 1e-3)), "tokens_per_s_with_host": round(batch / ((g + dm) * 1e-3)),
         "tokens_per_s_with_host_builder": round(batch / ((g + h) * 1e-3)),
         "attention_ms": round(a, 3), "attention_share": round(a / g, 3),
         "attention_kv_gb_s": round(kv_bytes / (a * 1e-3) / 1e9, 1), "work_list": plan.items is not None,
         "steps": steps}
    log(f"[bench] c5_decode_step_{fmt}: {json.dumps(r)}")
    return r


def graph_step_bench(batches=(1, 8, 64), steps: int = 20, warmup: int = 3, seed: int = 0, fmt: str = "bf16") -> dict:
    """Decode steps of a random-init Qwen2.5-0.5B-shaped model (24 layers) at small batches, contexts ~ U[512, 2048],
    pool in `fmt` (bf16, int8 or int8-kchannel): the ordinary eager step (build_metadata, ~300 launches from
    Python) against the same step replayed from a HIP graph (engine/graph_runner.py: one metadata copy, one
    replay). Wall time per step, synchronised each step as a serving loop is (it needs the sampled tokens), host
    work included."""
    import random
    import time

    from engine.block_manager import BlockManager
    from engine.config import QWEN2_5_0_5B as cfg
    from engine.graph_runner import DecodeGraphRunner
    from engine.model import Qwen2Model
    from engine.paged_cache import PagedKVCache, build_metadata
    from engine.quant_cache import QuantPagedKVCache

    res = {}
    model = Qwen2Model(cfg, "cuda", torch.bfloat16, seed=seed, max_positions=4096)
    N, B = 16384, 16
    for batch in batches:
        rng = random.Random(seed + batch)
        m = BlockManager(N, B)
        rng.shuffle(m._free)
        if fmt == "bf16":
            cache = PagedKVCache(cfg, N, B, "cuda", torch.bfloat16, attn_backend="triton")
            cache.k.normal_()
            cache.v.normal_()
        else:
            cache = QuantPagedKVCache(cfg, N, B, "cuda", torch.bfloat16, "triton", fmt, m, n_stage=2 * batch + 2)
            cache.k.random_(-127, 128)
            cache.v.random_(-127, 128)
            cache.k_scale.fill_(1 / 64)
            cache.v_scale.fill_(1 / 64)
            if fmt == "int8-kchannel":
                cache.stage.normal_()
        ctx = [rng.randint(512, 2048) for _ in range(batch)]
        for s, n in enumerate(ctx):
            m.allocate(s, n)
        runner = DecodeGraphRunner(model, cache, m, max_batch=batch, max_context=4096, buckets=[batch])
        seqs = list(range(batch))
        ids = torch.zeros(batch, dtype=torch.long, device="cuda")
        times = {}
        for mode in ("eager", "graph"):
            ts = []
            for i in range(warmup + steps):
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                for s in seqs:
                    m.append_slot(s)
                if mode == "eager":
                    meta = build_metadata(m, [(s, m.seq_len(s) - 1, 1) for s in seqs], "cuda")
                    logits = model.forward(ids, meta.positions, cache, meta)
                else:
                    logits = runner.step(seqs, ids)
                ids = logits.argmax(-1)
                torch.cuda.synchronize()
                if i >= warmup:
                    ts.append((time.perf_counter() - t0) * 1e3)
            times[mode] = sorted(ts)[len(ts) // 2]
        runner.close()
        res[f"batch{batch}"] = {"eager_step_ms": round(times["eager"], 3), "graph_step_ms": round(times["graph"], 3),
                                "speedup": round(times["eager"] / times["graph"], 2),
                                "graph_tokens_per_s": round(batch / (times["graph"] * 1e-3)),
                                "context_mean": round(sum(ctx) / batch)}
        del cache, runner
        torch.cuda.empty_cache()
    log(f"[bench] graph decode steps ({fmt}): {json.dumps(res)}")
    return res


def calibrate_copy(mib: int) -> int:
    """A plain device copy of a known size, 10 launches: rocprof's per-dispatch FETCH_SIZE and WRITE_SIZE of this
    kernel against its exact byte count give the scale factor applied to the decode kernel's counters."""
    lib = ctypes.CDLL(str(ROOT / "small-inference_amd" / "build" / "libsmallinf_probe.so"))
    lib.sipa_probe_copy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_void_p]
    nbytes = mib << 20
    src = torch.randint(0, 255, (nbytes,), dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    stream = torch.cuda.current_stream().cuda_stream
    for _ in range(10):
        if lib.sipa_probe_copy(dst.data_ptr(), src.data_ptr(), nbytes, 2048, stream):
            raise RuntimeError("probe copy launch failed")
    torch.cuda.synchronize()
    assert torch.equal(src, dst)
    print(json.dumps({"kernel": "probe_copy_kernel", "bytes_read": nbytes, "bytes_written": nbytes, "launches": 10}))
    return 0


# ---- main ------------------------------------------------------------------------------------------------------------

def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100, help="timed steps (each one call per rotated layer)")
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--layers", type=int, default=8, help="pool layers the calls rotate over (defeats the MALL)")
    ap.add_argument("--splits", type=int, default=None, help="force a split count (default: CU-count policy)")
    ap.add_argument("--impl", default="auto", choices=["auto", "mfma", "mfma_pbf16", "valu", "valu_stream", "valu_dot2"])
    ap.add_argument("--combine", default="fused", choices=["fused", "kernel"])
    ap.add_argument("--details", dest="details", action="store_true", default=True)
    ap.add_argument("--no-details", dest="details", action="store_false")
    ap.add_argument("--no-cpu", dest="cpu", action="store_false", default=True)
    ap.add_argument("--cpu-budget", type=float, default=10.0, help="seconds of CPU-baseline timing")
    ap.add_argument("--prefill", action="store_true", help="only run the paged prefill kernel against the "
                    "gather path")
    ap.add_argument("--graph", action="store_true", help="only run small-batch decode steps, eager against HIP "
                    "graph replay")
    ap.add_argument("--c5", action="store_true", help="only run config C5 (decode steps of a random-init 0.5B "
                    "model at batch 512 through the paged cache) and print its JSON")
    ap.add_argument("--c4", action="store_true", help="only run config C4 (INT8 decode, 1.5B shape, 64 x 4096: "
                    "per-token, then per-channel K) for --steps calls each and print its JSON")
    ap.add_argument("--c3", action="store_true", help="only run config C3 (bf16 decode of 256 ragged sequences "
                    "on the work list) for --steps calls and print its JSON")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="only run the probe library's plain copy kernel over MIB MiB, 10 times (the reference "
                         "point for rocprof's FETCH_SIZE / WRITE_SIZE counters), and print its byte count")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU: this build runs the paged-decode kernels on a single MI355X and has no "
              f"multi-GPU path (asked for --gpus {args.gpus}, WORLD_SIZE {world}). Run with --gpus 1.",
              file=sys.stderr)
        return 2

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    torch.cuda.set_device(0)
    if args.calibrate_copy:
        return calibrate_copy(args.calibrate_copy)
    if args.prefill:
        print(json.dumps(prefill_bench(args.steps, args.warmup)), flush=True)
        return 0
    if args.graph:
        print(json.dumps({f: graph_step_bench(fmt=f) for f in ("bf16", "int8", "int8-kchannel")}), flush=True)
        return 0
    if args.c4:
        res = {}
        for fmt, key in (("int8", "c4b_int8_per_token"), ("int8-kchannel", "c4a_int8_kchannel")):
            if args.impl not in ("auto", "mfma") and fmt != "int8":
                continue  # the VALU streaming kernels cover the per-token format only
            wl = int8_decode(key, fmt, [4096] * 64, 32768, impl=args.impl, splits=args.splits)
            res[key] = measure(wl, args.steps, args.warmup, per_launch=False)
            # each format runs its own kernel, so the indices count that kernel's dispatches
            log(f"[bench] c4 {key} timed region: decode dispatches {LAST_WARM_CALLS} to "
                f"{LAST_WARM_CALLS + args.steps - 1}")
            if args.impl in ("auto", "mfma"):
                res[key]["paged_read_floor"] = paged_read_floor(wl, args.steps, args.warmup)
            del wl
            torch.cuda.empty_cache()
        print(json.dumps(res), flush=True)
        return 0
    if args.c3:
        wl = bf16_decode("c3_ragged256", c3_context_lengths(), 200_000, layers=4, impl=args.impl,
                         splits=args.splits)
        res = measure(wl, args.steps, args.warmup, per_launch=False)
        log(f"[bench] c3 timed region: decode dispatches {LAST_WARM_CALLS} to {LAST_WARM_CALLS + args.steps - 1}")
        if args.impl in ("auto", "mfma"):
            res["paged_read_floor"] = paged_read_floor(wl, args.steps, args.warmup)
        print(json.dumps({"c3_ragged256": res}), flush=True)
        return 0
    if args.c5:
        res = {}
        for fmt in ("bf16", "int8", "int8-kchannel"):
            res[fmt] = decode_step_bench(fmt=fmt)
            torch.cuda.empty_cache()
        print(json.dumps({"c5_decode_step": res}), flush=True)
        return 0
    from engine.hip_decode import device_cu_count

    cu = device_cu_count()
    log(f"[bench] device {torch.cuda.get_device_name(0)}, {cu} CUs")

    wl = bf16_decode("c2", [8192] * 32, 32768, layers=args.layers, splits=args.splits, impl=args.impl,
                     combine=args.combine)
    # The timed region: K steps of `layers` back-to-back launches each on the launch stream, HIP events at both
    # ends. Each call is one kernel (the split merge is fused), so region / (K x layers) is the kernel's average
    # duration plus the dispatch gap between consecutive kernels; rocprofv3's kernel trace of the same command
    # agrees to about 1%.
    calls = args.steps * args.layers
    ms, _ = time_calls(wl.call, calls, args.warmup * args.layers, per_launch=False)  # ms per call
    # No decode call precedes the warm-up, so these are the timed calls' places among the process's decode
    # dispatches (0-based, launch order): a kernel trace can average exactly the timed region.
    log(f"[bench] c2 timed region: decode dispatches {LAST_WARM_CALLS} to {LAST_WARM_CALLS + calls - 1}")
    kern_us = ms * 1e3
    _, pair_us = time_calls(wl.call, min(args.steps, 200), 0, per_launch=True)
    value = wl.bytes / (ms * 1e-3) / 1e9
    achieved = wl.bytes / (kern_us * 1e-6) / 1e9
    err = check_against_oracle(wl)
    log(f"[bench] c2: {kern_us:.2f} us/call over the timed region ({pair_us:.2f} us with an event pair around "
        f"each launch), {value:.1f} GB/s, max-abs vs oracle {err:.2e}, splits {wl.plan.splits} x {wl.plan.chunk}")

    traffic = None
    if TRAFFIC_FILE.exists():
        traffic = json.loads(TRAFFIC_FILE.read_text()).get("hbm_bytes_per_launch")
    result = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms * args.layers, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) Q/K/V, random-permutation block tables)",
        "config": {"workload": "C2: bf16 paged decode, batch 32 x 8192 context, Qwen2.5-0.5B attention shape "
                               "(14 q / 2 kv heads, head_dim 64), 16-token blocks, 32768-block pool",
                   "batch": 32, "context": 8192, "block_size": 16, "q_heads": 14, "kv_heads": 2, "head_dim": 64,
                   "splits": wl.plan.splits, "split_tokens": wl.plan.chunk, "impl": args.impl,
                   "combine": args.combine, "layers_rotated": args.layers, "cu_count": cu,
                   "bytes_per_call": wl.bytes, "us_per_call": round(ms * 1e3, 2), "calls_per_step": args.layers,
                   "timed_calls": calls,
                   "max_abs_vs_fp32_oracle": round(err, 5)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / PEAK_GBS, 4), "traffic": traffic,
                     "kernel_us": round(kern_us, 2), "event_pair_us": round(pair_us, 2),
                     "kernel": "sipa::decode_mfma_bf16<64, 2>" if args.impl != "valu"
                     else "sipa::decode_valu<1, 0, 64>",
                     "paged_read_floor": paged_read_floor(wl, calls, args.warmup * args.layers)},
    }
    if args.cpu:
        result["cpu_baseline"] = cpu_baseline(wl, args.cpu_budget)
    del wl
    torch.cuda.empty_cache()
    if args.details:
        result["details"] = details(max(50, args.steps // 2), max(10, args.warmup // 2))
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
