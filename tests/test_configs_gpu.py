"""Parity at the full sizes of the BASELINE configurations C1–C4, against the CPU oracle.

The other GPU tests pin the kernels on small and edge-case inputs; these run the shapes the benchmark measures:
C1 1 x 1024 (0.5B heads, LIFO-scattered tables, scale 1/8), C2 32 x 8192 (0.5B, a random permutation of a
32768-block pool), C3 256 ragged sequences (log-normal, median 600, sigma 1.0, clipped to [16, 8192], over a
200,000-block pool) with the fused store of one new token per sequence before the decode, C4 64 x 4096 INT8 in
both formats (1.5B heads, four outlier K channels per head scaled by U[20, 68]).

Tolerances, written here: every bf16 output element within 8e-3 of the oracle's fp32 gather-then-attend (the
north-star bound) or equal to one of the two bf16 values that bracket the oracle's value (the output's own
rounding, which matters for C4, whose outlier channels make |out| reach a few units). Every path the library picks
for these shapes is covered: single pass, the CU-count split grid with the fused merge and with the separate
merge kernel, and the ragged work list.
"""

import math

import numpy as np
import pytest
import torch

from cases import HEADS, as_np32, assert_decode_close, compact_pool
from engine.hip_decode import paged_decode_attention
from engine.hip_quant import store_tokens
from oracle import paged_ref

pytestmark = pytest.mark.gpu


def permuted_tables(num_blocks: int, lengths: list[int], B: int, seed: int) -> list[list[int]]:
    """Each sequence's blocks taken in turn from one random permutation of the pool (the bench's tables)."""
    perm = torch.randperm(num_blocks, generator=torch.Generator().manual_seed(seed)).tolist()
    tables, at = [], 0
    for n in lengths:
        nb = -(-n // B)
        tables.append(perm[at:at + nb])
        at += nb
    assert at <= num_blocks
    return tables


def bf16_pools(Hkv, N, B, D, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    k = torch.randn(Hkv, N, B, D, device="cuda", dtype=torch.bfloat16, generator=g)
    v = torch.randn(Hkv, N, B, D, device="cuda", dtype=torch.bfloat16, generator=g)
    return k, v, g


def oracle_fp32(q, k, v, tables, lengths, scale):
    """fp32 gather-then-attend over only the blocks the tables use (copied to the host)."""
    B = k.shape[2]
    kk, t2 = compact_pool(k, tables, lengths, B)
    vv, _ = compact_pool(v, tables, lengths, B)
    return paged_ref.decode(as_np32(q), kk, vv, t2, lengths, scale, np.float32)


def check(out, ref, what):
    err = float(np.abs(as_np32(out).astype(np.float64) - ref).max())
    print(f"{what}: max-abs {err:.2e}", flush=True)
    assert err <= 8e-3, f"{what}: max-abs {err:.3e} against the fp32 oracle"


def run_paths(q, k, v, bt, ctx, tables, lengths, scale, paths):
    ref = oracle_fp32(q, k, v, tables, lengths, scale)
    for name, kw in paths:
        print(f"case {name} S={len(lengths)} max_ctx={max(lengths)}", flush=True)
        out = paged_decode_attention(q, k, v, bt, ctx, scale, max(lengths), host_context_lens=lengths, **kw)
        torch.cuda.synchronize()
        check(out, ref, name)


def test_c1_single_sequence_1024():
    """C1: 1 x 1024 over a 4096-block pool whose free list was scattered (the reference tests' LIFO pattern)."""
    from cases import fragmented_manager

    Hq, Hkv, D = HEADS["0.5B"]
    m = fragmented_manager(4096, 16, torch.Generator().manual_seed(11))
    m.allocate(0, 1024)
    tables, lengths = [m.block_table(0)], [1024]
    k, v, g = bf16_pools(Hkv, 4096, 16, D, 1)
    q = torch.randn(1, Hq, D, device="cuda", dtype=torch.bfloat16, generator=g)
    bt = torch.tensor(tables, dtype=torch.int32, device="cuda")
    ctx = torch.tensor(lengths, dtype=torch.int32, device="cuda")
    run_paths(q, k, v, bt, ctx, tables, lengths, 1 / 8,
              [("c1 single pass", dict(num_splits=1)), ("c1 auto splits", {})])


def test_c2_batch32_8192():
    """C2: 32 x 8192, single pass, the CU-count split grid (fused merge and separate merge kernel)."""
    Hq, Hkv, D = HEADS["0.5B"]
    lengths = [8192] * 32
    tables = permuted_tables(32768, lengths, 16, 2)
    k, v, g = bf16_pools(Hkv, 32768, 16, D, 2)
    q = torch.randn(32, Hq, D, device="cuda", dtype=torch.bfloat16, generator=g)
    bt = torch.tensor(tables, dtype=torch.int32, device="cuda")
    ctx = torch.tensor(lengths, dtype=torch.int32, device="cuda")
    run_paths(q, k, v, bt, ctx, tables, lengths, D ** -0.5,
              [("c2 single pass", dict(num_splits=1)), ("c2 split grid", {}),
               ("c2 separate merge", dict(combine="kernel"))])


def test_c2_batch1_8192():
    """C2's batch-1 case, 1 x 8192 over an 8192-block pool (the bench's split-K gain case): single pass, the CU-count
    split grid (16 splits) with the fused merge, the separate merge kernel, and a forced 32-way split."""
    Hq, Hkv, D = HEADS["0.5B"]
    lengths = [8192]
    tables = permuted_tables(8192, lengths, 16, 4)
    k, v, g = bf16_pools(Hkv, 8192, 16, D, 4)
    q = torch.randn(1, Hq, D, device="cuda", dtype=torch.bfloat16, generator=g)
    bt = torch.tensor(tables, dtype=torch.int32, device="cuda")
    ctx = torch.tensor(lengths, dtype=torch.int32, device="cuda")
    run_paths(q, k, v, bt, ctx, tables, lengths, D ** -0.5,
              [("c2 batch 1 single pass", dict(num_splits=1)), ("c2 batch 1 split grid", {}),
               ("c2 batch 1 separate merge", dict(combine="kernel")), ("c2 batch 1 32 splits", dict(num_splits=32))])


def test_c3_ragged_256_with_fused_store():
    """C3: 256 log-normal lengths over a 200,000-block pool. One new K/V token per sequence goes into its
    partially filled last block with the store kernel first (the step's write), then the decode reads it: the
    work list (the default for a ragged batch) and the split grid."""
    Hq, Hkv, D = HEADS["0.5B"]
    rng = np.random.default_rng(0)
    lengths = np.clip(np.rint(rng.lognormal(math.log(600), 1.0, 256)), 16, 8192).astype(int).tolist()
    tables = permuted_tables(200_000, lengths, 16, 3)
    k, v, g = bf16_pools(Hkv, 200_000, 16, D, 3)
    # the step's new tokens: position ctx - 1 of every sequence, written through the store kernel
    pos = torch.tensor([n - 1 for n in lengths], dtype=torch.int64)
    blocks = torch.tensor([t[(n - 1) // 16] for t, n in zip(tables, lengths)], dtype=torch.int64)
    new_k = torch.randn(256, Hkv, D, device="cuda", dtype=torch.bfloat16, generator=g)
    new_v = torch.randn(256, Hkv, D, device="cuda", dtype=torch.bfloat16, generator=g)
    store_tokens(new_k, blocks.cuda(), (pos % 16).cuda(), k, x2=new_v, pool2=v)
    torch.cuda.synchronize()
    assert torch.equal(k[:, blocks, pos % 16].transpose(0, 1), new_k)
    assert torch.equal(v[:, blocks, pos % 16].transpose(0, 1), new_v)
    q = torch.randn(256, Hq, D, device="cuda", dtype=torch.bfloat16, generator=g)
    bt = torch.from_numpy(paged_ref.padded_tables(tables, lengths, 16)).cuda()
    ctx = torch.tensor(lengths, dtype=torch.int32, device="cuda")
    run_paths(q, k, v, bt, ctx, tables, lengths, D ** -0.5,
              [("c3 work list", dict(work_list="on")), ("c3 split grid", dict(work_list="off"))])


@pytest.mark.parametrize("fmt", ["int8", "int8-kchannel"])
def test_c4_int8_64x4096(fmt):
    """C4: 64 x 4096 with the 1.5B heads over pools filled by the fused quantize-and-store kernels (through the
    cache's writes), against the oracle's dequantize-then-attend; the split grid and the work list."""
    from test_quant_gpu import int8_case

    Hq, Hkv, D = HEADS["1.5B"]
    lengths = [4096] * 64
    q, cache, meta, quant, k32, v32 = int8_case(Hq, Hkv, D, lengths, fmt, seed=9)
    ref = np.stack([paged_ref.attend_one(as_np32(q[s]), k32[s], v32[s], D ** -0.5, np.float32)
                    for s in range(len(lengths))])
    for name, kw in (("grid", {}), ("work list", dict(host_context_lens=lengths, work_list="on"))):
        print(f"case c4 {fmt} {name}", flush=True)
        out = paged_decode_attention(q, cache.k[0], cache.v[0], meta.block_tables, meta.context_lens_t,
                                     D ** -0.5, max(lengths), quant=quant, **kw)
        assert_decode_close(out.double().cpu().numpy(), ref, f"c4 {fmt} {name}")
