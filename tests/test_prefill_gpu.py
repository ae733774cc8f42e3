"""Parity of the HIP paged prefill kernel (multi-token rows attending causally over the paged context) with the
CPU oracle, on the shapes the reference serves: fresh prompts and mid-context chunks, ragged chunk lengths around
the 16-token tile and 32-key tile boundaries, shuffled block tables, GQA groups 1 .. 8, head_dim 64 and 128.

Tolerances, written here: against the fp32 oracle, the decode kernels' bar (`cases.assert_decode_close`): every
element within 8e-3, or one of the two bf16 values that bracket the oracle's value (the output's own rounding,
which alone exceeds 8e-3 for |out| >= 4); the kernel rounds probabilities to bf16 before P.V as the reference's
own path does (engine/attention.py:22-27). rtol/atol 1e-2 against fp64 beside it; a torch fp32 reference on the
GPU for the long-context case.
"""

import numpy as np
import pytest
import torch

from cases import as_np32, assert_decode_close, bf16_bracket, fragmented_manager, ramp_scores
from engine.hip_prefill import paged_prefill_attention
from oracle import paged_ref

pytestmark = pytest.mark.gpu

# (Hq, Hkv, D); groups of 1 .. 4 query heads put 2 .. 8 16-token subtiles in one unit
SHAPES = {"0.5B": (14, 2, 64), "1.5B": (12, 2, 128), "g4": (32, 8, 128), "g8": (16, 2, 64), "g1": (4, 4, 64),
          "g2": (8, 4, 64), "g3": (6, 2, 128)}
SENTINEL = 7.0


def make_prefill(ctx, qlen, Hq, Hkv, D, seed=0, gap=0, device="cuda"):
    """Pools over a fragmented manager, -1 padded tables, q rows packed with `gap` unused rows between sequences.
    Returns q, k, v, bt, ctx, starts, lens (device int32) and the tables, row starts and T."""
    B = 16
    g = torch.Generator().manual_seed(seed)
    need = sum(-(-n // B) for n in ctx)
    m = fragmented_manager(max(2 * need, 1), B, g)
    for i, n in enumerate(ctx):
        m.allocate(i, n)
    tables = [m.block_table(i) for i in range(len(ctx))]
    starts, T = [], 0
    for n in qlen:
        starts.append(T)
        T += n + gap
    k = torch.randn(Hkv, m.num_blocks, B, D, generator=g).to(device, torch.bfloat16)
    v = torch.randn(Hkv, m.num_blocks, B, D, generator=g).to(device, torch.bfloat16)
    q = torch.randn(T, Hq, D, generator=g).to(device, torch.bfloat16)

    def i32(x):
        return torch.tensor(x, dtype=torch.int32, device=device)

    bt = torch.from_numpy(paged_ref.padded_tables(tables, ctx, B)).to(device)
    return q, k, v, bt, i32(ctx), i32(starts), i32(qlen), tables, starts, T


def assert_bf16_close(got, ref, what="prefill"):
    """The decode tests' bar (`cases.assert_decode_close`): every element within 8e-3 of the fp32 oracle, or one of
    the two bf16 values that bracket the oracle's value."""
    assert_decode_close(got, ref, what)


def check(ctx, qlen, shape, seed=0, gap=0, splits=None):
    Hq, Hkv, D = SHAPES[shape]
    print(f"case ctx={ctx[:6]} qlen={qlen[:6]} shape={shape} seed={seed} gap={gap} splits={splits}", flush=True)
    q, k, v, bt, c, st, ln, tables, starts, T = make_prefill(ctx, qlen, Hq, Hkv, D, seed, gap)
    scale = D ** -0.5
    out = torch.full_like(q, SENTINEL)
    paged_prefill_attention(q, k, v, bt, c, st, ln, scale, max(ctx), max(qlen), out=out, num_splits=splits,
                            host_query_lens=qlen)
    torch.cuda.synchronize()
    got = out.double().cpu().numpy()
    args = (as_np32(q), as_np32(k), as_np32(v), tables, ctx, starts, qlen, scale)
    ref32, ref64 = paged_ref.prefill(*args, dtype=np.float32), paged_ref.prefill(*args, dtype=np.float64)
    rows = np.concatenate([np.arange(s, s + n) for s, n in zip(starts, qlen)])
    other = np.setdiff1d(np.arange(T), rows)
    assert_bf16_close(got[rows], ref32[rows])
    np.testing.assert_allclose(got[rows], ref64[rows], rtol=1e-2, atol=1e-2)
    assert (got[other] == SENTINEL).all(), "rows of no sequence were written"
    return out


@pytest.mark.parametrize("shape", list(SHAPES))
def test_fresh_prompts(shape):
    """First chunks (context == new tokens) of ragged lengths around the tile boundaries."""
    lens = [1, 2, 15, 16, 17, 31, 32, 33, 64, 100]
    check(lens, lens, shape)


@pytest.mark.parametrize("shape", ["0.5B", "1.5B", "g8", "g4", "g3", "g2", "g1"])
@pytest.mark.parametrize("seed", [0, 1])
@pytest.mark.parametrize("splits", [1, 4, None], ids=["one_split", "split256", "auto"])
def test_mid_context_chunks(shape, seed, splits):
    """Chunks after a cached prefix (chunked prefill): prefix lengths on and off block and tile boundaries; key
    splits of 256 keys put split starts inside query tiles (tokens that see none of a split's keys)."""
    ctx = [300, 1000, 33, 16, 48, 517, 129, 280]
    qlen = [64, 7, 33, 1, 32, 500, 16, 30]
    check(ctx, qlen, shape, seed, gap=3, splits=splits)


@pytest.mark.parametrize("shape", ["0.5B", "1.5B"])
@pytest.mark.parametrize("splits", [2, 7, 32])
def test_split_counts(shape, splits):
    """A long chunk over a longer prefix at several split counts (32: more splits than 256-key chunks allow)."""
    check([3000, 700], [700, 300], shape, seed=splits, splits=splits)


def test_single_token_rows_equal_decode():
    """One-token chunks are decode rows: the prefill kernel agrees with the oracle's decode at every length."""
    lens = [1, 15, 16, 17, 33, 100, 1000]
    check(lens, [1] * len(lens), "0.5B")


@pytest.mark.parametrize("shape", ["0.5B", "1.5B"])
def test_long_context_chunk_against_torch(shape):
    """A 512-token chunk at 8K context (and a 2K prompt) against torch fp32 attention on the GPU, row blocks at a
    time; repeated launches give identical bits."""
    Hq, Hkv, D = SHAPES[shape]
    ctx, qlen = [8192, 2048], [512, 2048]
    print(f"case long ctx={ctx} qlen={qlen} shape={shape}", flush=True)
    q, k, v, bt, c, st, ln, tables, starts, T = make_prefill(ctx, qlen, Hq, Hkv, D, seed=5)
    scale = D ** -0.5
    out = paged_prefill_attention(q, k, v, bt, c, st, ln, scale, max(ctx), max(qlen))
    again = paged_prefill_attention(q, k, v, bt, c, st, ln, scale, max(ctx), max(qlen))
    torch.cuda.synchronize()
    assert torch.equal(out, again)
    G = Hq // Hkv
    for s in range(2):
        idx = torch.tensor(tables[s][:-(-ctx[s] // 16)], device="cuda", dtype=torch.int64)
        kk = k.index_select(1, idx).reshape(Hkv, -1, D)[:, :ctx[s]].float().repeat_interleave(G, 0)
        vv = v.index_select(1, idx).reshape(Hkv, -1, D)[:, :ctx[s]].float().repeat_interleave(G, 0)
        for r0 in range(0, qlen[s], 256):
            r1 = min(r0 + 256, qlen[s])
            qq = q[starts[s] + r0:starts[s] + r1].float().permute(1, 0, 2)                 # [Hq, rows, D]
            sc = torch.matmul(qq, kk.transpose(1, 2).contiguous()) * scale
            pos = torch.arange(ctx[s] - qlen[s] + r0, ctx[s] - qlen[s] + r1, device="cuda")[:, None]
            sc = sc.masked_fill(torch.arange(ctx[s], device="cuda")[None, :] > pos, float("-inf"))
            want = torch.matmul(torch.softmax(sc, -1), vv).permute(1, 0, 2)
            assert_bf16_close(out[starts[s] + r0:starts[s] + r1].double().cpu().numpy(),
                              want.double().cpu().numpy(), f"seq {s} rows {r0}..{r1}")


@pytest.mark.parametrize("shape", ["0.5B", "1.5B"])
def test_chunk_at_8k_splits_against_torch(shape):
    """The reference scheduler's default step (one 512-token chunk) at 8K context runs split (the policy gives
    8 splits of 1024 keys on 256 CUs): torch fp32 on the GPU agrees, and launches with the workspace reused (split
    counts 8, 3, 8) give the same bits each time the split count repeats."""
    Hq, Hkv, D = SHAPES[shape]
    ctx, qlen = [8192], [512]
    print(f"case chunk at 8k shape={shape}", flush=True)
    q, k, v, bt, c, st, ln, tables, starts, T = make_prefill(ctx, qlen, Hq, Hkv, D, seed=6)
    scale = D ** -0.5
    run = lambda n: paged_prefill_attention(q, k, v, bt, c, st, ln, scale, 8192, 512, num_splits=n)  # noqa: E731
    a, b, a2 = run(8), run(3), run(8)
    mem = paged_prefill_attention(q, k, v, bt, c, st, ln, scale, 8192, 512, num_splits=8, merge_path="memory")
    # 16 waves over key halves: each workgroup combines two of the 8 key chunks, then 4 splits merge
    hx = [paged_prefill_attention(q, k, v, bt, c, st, ln, scale, 8192, 512, num_splits=8, wg_layout="w16h2",
                                  merge_path=path) for path in ("auto", "memory")]
    torch.cuda.synchronize()
    assert torch.equal(a, a2)
    assert torch.equal(a, mem)  # the L2 merge and the merge through memory give the same bits
    assert torch.equal(hx[0], hx[1])
    G = Hq // Hkv
    idx = torch.tensor(tables[0], device="cuda", dtype=torch.int64)
    kk = k.index_select(1, idx).reshape(Hkv, -1, D)[:, :8192].float().repeat_interleave(G, 0)
    vv = v.index_select(1, idx).reshape(Hkv, -1, D)[:, :8192].float().repeat_interleave(G, 0)
    qq = q.float().permute(1, 0, 2)
    sc = torch.matmul(qq, kk.transpose(1, 2).contiguous()) * scale
    pos = torch.arange(8192 - 512, 8192, device="cuda")[:, None]
    sc = sc.masked_fill(torch.arange(8192, device="cuda")[None, :] > pos, float("-inf"))
    want = torch.matmul(torch.softmax(sc, -1), vv).permute(1, 0, 2).double().cpu().numpy()
    for got in (a, b, hx[0]):
        assert_bf16_close(got.double().cpu().numpy(), want, "chunk at 8k")


def test_strided_q_view():
    """q as a view into a fused QKV projection (row stride past Hq * D) and a head-strided out."""
    Hq, Hkv, D = SHAPES["0.5B"]
    ctx, qlen = [70, 40], [70, 24]
    q, k, v, bt, c, st, ln, tables, starts, T = make_prefill(ctx, qlen, Hq, Hkv, D, seed=3)
    fused = torch.zeros(T, (Hq + 2 * Hkv) * D, dtype=torch.bfloat16, device="cuda")
    fused[:, :Hq * D] = q.reshape(T, -1)
    qv = fused[:, :Hq * D].view(T, Hq, D)
    out = paged_prefill_attention(qv, k, v, bt, c, st, ln, D ** -0.5, max(ctx), max(qlen))
    ref = paged_prefill_attention(q.contiguous(), k, v, bt, c, st, ln, D ** -0.5, max(ctx), max(qlen))
    torch.cuda.synchronize()
    assert torch.equal(out, ref)


def test_workspace_shared_with_decode_in_any_order():
    """Decode and prefill split calls of growing sizes share one workspace: the merge counters live in a region no
    call writes partials into, so a call with more (sequence, head) pairs than the last never reads old partials
    as counters. Prefill (16 splits, 8 units) -> decode (200 sequences, 4 splits) -> prefill (150 units) ->
    the first prefill again, bit-identical."""
    from cases import make_case, oracle_decode
    from engine.hip_decode import paged_decode_attention

    first = check([4096], [64], "0.5B", seed=11)
    Hq, Hkv, D = SHAPES["0.5B"]
    lengths = [1000] * 200
    q, k, v, bt, ctx, tables = make_case(lengths, Hq, Hkv, D, 16, torch.bfloat16, seed=12)
    print("case decode 200 x 1000 splits=4 after a prefill split call", flush=True)
    out = paged_decode_attention(q, k, v, bt, ctx, D ** -0.5, 1000, num_splits=4, work_list="off")
    torch.cuda.synchronize()
    ref = oracle_decode(q, k, v, tables, lengths, D ** -0.5, np.float32)
    assert np.abs(out.double().cpu().numpy() - ref).max() <= 8e-3
    check([3000] * 3, [400] * 3, "0.5B", seed=13)
    again = check([4096], [64], "0.5B", seed=11)
    assert torch.equal(first, again)


def int8_pools(k, v, fmt, ctx, tables, g):
    """Quantize bf16 pools with the reference's quantizer (engine/quant.py): per-token K and V (format "int8"), or
    per-(block, channel) K (format "int8-kchannel") with each sequence's partial last block of K in a bf16 staging
    slot and its int8 codes overwritten with noise (so only the staging can give the right answer). Returns the
    QuantKV, the int8 pools, and the bf16 pools the reference's gather path would attend over."""
    from engine.hip_decode import QuantKV
    from engine.quant import dequantize, quantize_per_channel, quantize_per_token

    vq, vs = quantize_per_token(v)
    v_deq = dequantize(vq, vs[..., None], torch.bfloat16)
    if fmt == "int8":
        kq, ks = quantize_per_token(k)
        return QuantKV(1, ks, vs), kq, vq, dequantize(kq, ks[..., None], torch.bfloat16), v_deq
    kq, ks = quantize_per_channel(k, dim=2)
    k_deq = dequantize(kq, ks[:, :, None], torch.bfloat16)
    Hkv, _, B, D = k.shape
    stage = torch.zeros(Hkv, len(ctx) + 1, B, D, dtype=torch.bfloat16, device=k.device)
    tails = []
    for s, (n, t) in enumerate(zip(ctx, tables)):
        if n % B == 0:
            tails.append(-1)
            continue
        blk = t[n // B]
        stage[:, s + 1] = k[:, blk]  # the staged partial block, in the model dtype
        kq[:, blk] = torch.randint(-127, 128, kq[:, blk].shape, generator=g, device=k.device, dtype=torch.int8)
        k_deq[:, blk] = k[:, blk]
        tails.append(s + 1)
    tails = torch.tensor(tails, dtype=torch.int32, device=k.device)
    return QuantKV(2, ks, vs, stage, tails), kq, vq, k_deq, v_deq


@pytest.mark.parametrize("fmt", ["int8", "int8-kchannel"])
@pytest.mark.parametrize("shape", ["0.5B", "1.5B", "g4"])
@pytest.mark.parametrize("splits", [1, None], ids=["one_split", "auto"])
def test_int8_pools(fmt, shape, splits):
    """INT8 pools: the kernel dequantizes as the reference's gather path (q * s in fp32, rounded to bf16; format B's
    partial last block from staging), so its output equals, bit for bit, the bf16 kernel's on those dequantized
    pools, and is within the bf16 bounds of the oracle on them; keys with outlier channels (x 20 .. 68)."""
    Hq, Hkv, D = SHAPES[shape]
    ctx, qlen = [300, 1000, 33, 517, 280, 64], [64, 7, 33, 500, 30, 64]
    print(f"case int8 {fmt} shape={shape} splits={splits}", flush=True)
    q, k, v, bt, c, st, ln, tables, starts, T = make_prefill(ctx, qlen, Hq, Hkv, D, seed=21)
    g = torch.Generator(device="cuda").manual_seed(4)
    outlier = torch.ones(Hkv, 1, 1, D, device="cuda")
    outlier[:, :, :, :4] = 20 + 48 * torch.rand(Hkv, 1, 1, 4, generator=g, device="cuda")
    k = (k.float() * outlier).bfloat16()
    quant, kq, vq, k_deq, v_deq = int8_pools(k, v, fmt, ctx, tables, g)
    scale = D ** -0.5
    got = paged_prefill_attention(q, kq, vq, bt, c, st, ln, scale, max(ctx), max(qlen), num_splits=splits,
                                  quant=quant)
    ref_kernel = paged_prefill_attention(q, k_deq, v_deq, bt, c, st, ln, scale, max(ctx), max(qlen),
                                         num_splits=splits)
    torch.cuda.synchronize()
    assert torch.equal(got, ref_kernel)
    args = (as_np32(q), as_np32(k_deq), as_np32(v_deq), tables, ctx, starts, qlen, scale)
    ref32 = paged_ref.prefill(*args, dtype=np.float32)
    rows = np.concatenate([np.arange(s, s + n) for s, n in zip(starts, qlen)])
    # The outlier channels make the softmax peaked, and the kernel (like the reference's gather path) rounds the
    # probabilities to bf16 for P.V: the north-star 8e-3, or one bf16 step of the output where that is larger (the
    # two bf16 values bracketing the oracle's), plus that rounding's own error, 2^-9 sum_k p_k |v_k| (the oracle's
    # attention over |V|).
    pv_abs = paged_ref.prefill(args[0], args[1], np.abs(args[2]), *args[3:], dtype=np.float32)[rows]
    err = np.abs(got.double().cpu().numpy()[rows] - ref32[rows])
    lo, hi = bf16_bracket(ref32[rows])
    bound = np.maximum(8e-3, hi - lo) + 2 ** -9 * pv_abs
    print(f"int8 prefill: max-abs {err.max():.2e}, at most {(err / bound).max():.2f} of the bound", flush=True)
    assert (err <= bound).all(), f"max excess {(err - bound).max():.3e}"


@pytest.mark.parametrize("shape", ["0.5B", "1.5B"])
def test_kchannel_scale_layouts(shape):
    """Format B's channel scales in every layout the parameter block allows give the same output bits: fp16 rows
    (16-byte vector loads), fp32 rows (the same values), and fp16 / fp32 views whose rows are not 16-byte aligned
    (the kernel's per-scale loads); per-(head, channel) scales broadcast over blocks (block stride 0, fp32) equal
    the same scales written out per block."""
    from engine.hip_decode import QuantKV

    Hq, Hkv, D = SHAPES[shape]
    ctx, qlen = [300, 1000, 33, 517], [64, 7, 33, 200]
    print(f"case kchannel scale layouts shape={shape}", flush=True)
    q, k, v, bt, c, st, ln, tables, starts, T = make_prefill(ctx, qlen, Hq, Hkv, D, seed=23)
    g = torch.Generator(device="cuda").manual_seed(5)
    quant, kq, vq, _, _ = int8_pools(k, v, "int8-kchannel", ctx, tables, g)
    N = kq.shape[1]
    scale = D ** -0.5

    def run(ks):
        return paged_prefill_attention(q, kq, vq, bt, c, st, ln, scale, max(ctx), max(qlen),
                                       quant=QuantKV(2, ks, quant.v_scale, quant.stage, quant.tail_slots))

    def misaligned(x):  # the same values in a view whose rows start 1 element past a 16-byte boundary
        wide = torch.zeros(Hkv, N, D + 1, dtype=x.dtype, device=x.device)
        wide[:, :, 1:] = x
        return wide[:, :, 1:]

    ks16 = quant.k_scale
    base = run(ks16)
    for name, ks in (("fp32", ks16.float()), ("fp16 misaligned", misaligned(ks16)),
                     ("fp32 misaligned", misaligned(ks16.float()))):
        assert torch.equal(run(ks), base), name
    per_ch = torch.rand(Hkv, 1, D, generator=g, device="cuda") * 0.05 + 0.01  # fp32 per (head, channel)
    wide = run(per_ch.expand(Hkv, N, D))
    assert per_ch.expand(Hkv, N, D).stride(1) == 0
    assert torch.equal(wide, run(per_ch.expand(Hkv, N, D).contiguous()))
    assert torch.equal(wide, run(misaligned(per_ch.expand(Hkv, N, D).contiguous())))


@pytest.mark.parametrize("shape", ["0.5B", "1.5B", "g4", "g1"])
@pytest.mark.parametrize("splits", [2, 5, 32])
def test_merge_paths_agree(shape, splits):
    """The split merge from the XCD's L2 (units whose splits shared an XCD) and through memory (agent-coherent
    loads, every unit) give the same bits, and the memory path meets the oracle bound on its own; unit counts
    that are not multiples of 8 exercise the padded grid."""
    Hq, Hkv, D = SHAPES[shape]
    ctx, qlen = [3000, 700, 129], [700, 300, 17]
    print(f"case merge paths shape={shape} splits={splits}", flush=True)
    q, k, v, bt, c, st, ln, tables, starts, T = make_prefill(ctx, qlen, Hq, Hkv, D, seed=31)
    scale = D ** -0.5
    run = lambda path: paged_prefill_attention(q, k, v, bt, c, st, ln, scale, max(ctx), max(qlen),  # noqa: E731
                                               num_splits=splits, merge_path=path)
    auto, mem, auto2 = run("auto"), run("memory"), run("auto")
    torch.cuda.synchronize()
    assert torch.equal(auto, mem) and torch.equal(auto, auto2)
    args = (as_np32(q), as_np32(k), as_np32(v), tables, ctx, starts, qlen, scale)
    ref32 = paged_ref.prefill(*args, dtype=np.float32)
    rows = np.concatenate([np.arange(s0, s0 + n) for s0, n in zip(starts, qlen)])
    assert_bf16_close(mem.double().cpu().numpy()[rows], ref32[rows], "merge through memory")
    with pytest.raises(ValueError):
        run("l2")


@pytest.mark.parametrize("direction", [1, -1, 0], ids=["rising", "falling", "spike"])
@pytest.mark.parametrize("splits", [1, 6])
@pytest.mark.parametrize("layout", ["auto", "w16h2", "w16x1"])
def test_scores_trending_across_keys(direction, splits, layout):
    """Scores rising (or falling) by about 4 in the exp2 domain every 64 keys, or one key's score about 90 above
    the rest. Rising, some score passes the running max by more than 2^16 every few tiles, so the kernel takes
    those tiles' max and rescales, and uses the standing max for the tiles between; falling, the later
    probabilities underflow against the first tile's max; the spike's tile (whose p would overflow against the
    standing max) takes the max. The output meets the oracle's bound on every row."""
    Hq, Hkv, D = SHAPES["0.5B"]
    ctx, qlen = [3000, 700], [700, 300]
    print(f"case prefill trending scores direction={direction} splits={splits} layout={layout}", flush=True)
    q, k, v, bt, c, st, ln, tables, starts, T = make_prefill(ctx, qlen, Hq, Hkv, D, seed=71)
    ramp_scores(q, k, tables, ctx, 16, direction)
    scale = D ** -0.5
    out = paged_prefill_attention(q, k, v, bt, c, st, ln, scale, max(ctx), max(qlen), num_splits=splits,
                                  wg_layout=layout)
    torch.cuda.synchronize()
    ref32 = paged_ref.prefill(as_np32(q), as_np32(k), as_np32(v), tables, ctx, starts, qlen, scale,
                              dtype=np.float32)
    rows = np.concatenate([np.arange(s0, s0 + n) for s0, n in zip(starts, qlen)])
    assert_bf16_close(out.double().cpu().numpy()[rows], ref32[rows], "trending scores")


@pytest.mark.parametrize("shape", ["0.5B", "1.5B"])
@pytest.mark.parametrize("layout", ["auto", "w16h2"])
def test_split_partials_beyond_fp16_range(shape, layout):
    """V at 2^24 times unit scale, so that every split's O / l rows (weighted means of V rows, about 0.05 to 3 at
    unit scale) pass fp16's 65504: the fp16 partial rows are stored times 2^-e and merged back, and the output
    divided by 2^24 (exact in bf16) meets the oracle's bound at unit scale, with every value finite (unscaled
    fp16 partials would be inf)."""
    Hq, Hkv, D = SHAPES[shape]
    ctx, qlen = [3000, 700], [700, 300]
    print(f"case prefill partials beyond fp16 range {shape} {layout}", flush=True)
    q, k, v, bt, c, st, ln, tables, starts, T = make_prefill(ctx, qlen, Hq, Hkv, D, seed=61)
    scale = D ** -0.5
    out = paged_prefill_attention(q, k, v * 2.0 ** 24, bt, c, st, ln, scale, max(ctx), max(qlen), num_splits=6,
                                  wg_layout=layout)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    ref32 = paged_ref.prefill(as_np32(q), as_np32(k), as_np32(v), tables, ctx, starts, qlen, scale,
                              dtype=np.float32)
    rows = np.concatenate([np.arange(s0, s0 + n) for s0, n in zip(starts, qlen)])
    assert_bf16_close(out.double().cpu().numpy()[rows] / 2.0 ** 24, ref32[rows], "V x 2^24, divided back")


@pytest.mark.parametrize("shape", ["0.5B", "1.5B"])
@pytest.mark.parametrize("layout", ["auto", "w16h2"])
def test_l2_merge_reads_this_calls_partials(shape, layout):
    """The prefill merge from the XCD's L2: calls alternating between two inputs of one shape (the same workspace
    addresses) each give the memory-path bits of their own inputs, so no partial of an earlier call is read
    back (16 waves over key halves too: 6 key chunks, 3 workgroups a unit)."""
    Hq, Hkv, D = SHAPES[shape]
    ctx, qlen = [3000, 700], [700, 300]
    cases = [make_prefill(ctx, qlen, Hq, Hkv, D, seed=s) for s in (51, 52)]
    scale = D ** -0.5
    print(f"case prefill l2 merge alternation {shape} {layout}", flush=True)

    def run(i, path):
        q, k, v, bt, c, st, ln = cases[i][:7]
        return paged_prefill_attention(q, k, v, bt, c, st, ln, scale, max(ctx), max(qlen), num_splits=6,
                                       merge_path=path, wg_layout=layout)

    want = [run(i, "memory").clone() for i in (0, 1)]
    for rep in range(3):
        for i in (0, 1):
            got = run(i, "auto")
            torch.cuda.synchronize()
            assert torch.equal(got, want[i]), f"rep {rep} input {i}"


@pytest.mark.parametrize("shape", ["0.5B", "1.5B", "g1", "g3"])
@pytest.mark.parametrize("splits", [2, 3, 5, 7, 8, 32])
def test_key_halves_against_oracle(shape, splits):
    """16 waves over two key splits each (W16H2) at every split parity: an odd count leaves the last workgroup's
    second half without keys, and contexts that are not multiples of the split length leave it short; a chunk
    shorter than its context's prefix (mid-context rows) and one at its start (fresh rows) in one call. Held to the
    oracle bound, and the L2 and memory merges give the same bits."""
    Hq, Hkv, D = SHAPES[shape]
    ctx, qlen = [3001, 700, 129, 64], [500, 300, 17, 64]
    print(f"case key halves shape={shape} splits={splits}", flush=True)
    q, k, v, bt, c, st, ln, tables, starts, T = make_prefill(ctx, qlen, Hq, Hkv, D, seed=81)
    scale = D ** -0.5
    run = lambda path: paged_prefill_attention(q, k, v, bt, c, st, ln, scale, max(ctx), max(qlen),  # noqa: E731
                                               num_splits=splits, merge_path=path, wg_layout="w16h2")
    got, mem = run("auto"), run("memory")
    torch.cuda.synchronize()
    assert torch.equal(got, mem)
    args = (as_np32(q), as_np32(k), as_np32(v), tables, ctx, starts, qlen, scale)
    ref32 = paged_ref.prefill(*args, dtype=np.float32)
    ref64 = paged_ref.prefill(*args, dtype=np.float64)
    rows = np.concatenate([np.arange(s0, s0 + n) for s0, n in zip(starts, qlen)])
    out = got.double().cpu().numpy()[rows]
    assert_bf16_close(out, ref32[rows], "key halves")
    np.testing.assert_allclose(out, ref64[rows], rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("shape", ["0.5B", "1.5B", "g4", "g1", "g3"])
@pytest.mark.parametrize("pool", ["bf16", "int8", "int8-kchannel"])
@pytest.mark.parametrize("splits", [1, None], ids=["one_split", "auto"])
def test_wave_layouts_agree(shape, pool, splits):
    """The workgroup layouts compute every column tile with the same operations in the same order. 4 waves of two
    column tiles and 8 waves of one run the same units, so they give the same bits, each one's unused column
    tiles included. 16 waves of 16 column tiles run units of twice the tokens: with one split they give the same
    bits too (a unit's earlier tokens also run its later tokens' key tiles, fully masked for them, which must
    leave their bits alone); with several, a token whose 16-token unit saw one split may sit in a 32-token unit
    that sees two, and its row then goes through the merge's fp16 partials. There the bar is the oracle's, and
    the layouts stay within a bf16 rounding and the fp16 partial's of each other. 16 waves over two key halves
    combine each pair of key chunks in the workgroup first (its own arithmetic): held to that bar at every split
    count."""
    Hq, Hkv, D = SHAPES[shape]
    ctx, qlen = [300, 1000, 33, 517], [64, 7, 33, 200]
    print(f"case wave layouts shape={shape} pool={pool} splits={splits}", flush=True)
    q, k, v, bt, c, st, ln, tables, starts, T = make_prefill(ctx, qlen, Hq, Hkv, D, seed=61)
    quant = None
    if pool != "bf16":
        g = torch.Generator(device="cuda").manual_seed(7)
        quant, k, v, _, _ = int8_pools(k, v, pool, ctx, tables, g)
    run = lambda lay: paged_prefill_attention(q, k, v, bt, c, st, ln, D ** -0.5, max(ctx), max(qlen),  # noqa: E731
                                              num_splits=splits, quant=quant, wg_layout=lay)
    want = run("w4x2")
    layouts = ["w8x1", "auto"] + (["w16x1", "w16h2"] if pool != "int8-kchannel" else [])
    got = {lay: run(lay) for lay in layouts}
    torch.cuda.synchronize()
    assert torch.equal(got["w8x1"], want)
    if pool == "int8-kchannel":  # format B's auto layout is always w4x2
        assert torch.equal(got["auto"], want)
    else:
        rows = torch.cat([torch.arange(s, s + n) for s, n in zip(starts, qlen)]).cuda()
        for lay in ("w16x1", "w16h2", "auto"):  # auto picks w8x1 or w16x1 for these small grids
            if splits == 1 and lay != "w16h2":
                assert torch.equal(got[lay], want), lay
            else:
                a, b = got[lay][rows].float(), want[rows].float()
                bound = 2 ** -7 * torch.maximum(a.abs(), b.abs()) + 2 ** -9
                assert ((a - b).abs() <= bound).all(), f"{lay}: {((a - b).abs() - bound).max().item():.3e} over"
        if quant is None:
            scale = D ** -0.5
            args = (as_np32(q), as_np32(k), as_np32(v), tables, ctx, starts, qlen, scale)
            ref32 = paged_ref.prefill(*args, dtype=np.float32)
            npr = rows.cpu().numpy()
            for lay in ("w16x1", "w16h2"):
                assert_bf16_close(got[lay].double().cpu().numpy()[npr], ref32[npr], lay)
    with pytest.raises(ValueError):
        run("w2x4")
    if pool == "int8-kchannel":
        for lay in ("w16x1", "w16h2"):
            with pytest.raises(ValueError, match="format B"):
                run(lay)
