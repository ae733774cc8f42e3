"""Parity of the HIP paged-decode kernels with the CPU oracle (gather-then-attend), on the reference's edge cases.

Mirrors the reference's tests/test_decode_kernel.py:56-105: shuffled block tables, ragged lengths
[1, 15, 16, 17, 33, 100, 1000] in one batch, block sizes 8 / 16 / 32, both head layouts (0.5B 14/2/64, 1.5B
12/2/128), bf16 and fp32, single pass and split-K (3 splits, the CU-count policy, more splits than tokens), plus
both kernels (MFMA, VALU) and both split merges (last-arriving workgroup, separate kernel).

Tolerances, written here: fp32 1e-5 (reference tests/test_decode_kernel.py:63) against the fp64 oracle; bf16
max-abs 8e-3 against the fp32 oracle (the north-star bound for unit-variance inputs) and 1e-2 against fp64 (the
reference's), and the median relative error under 2^-8 (reference :89-94).
"""

import numpy as np
import pytest
import torch

from cases import HEADS, RAGGED, assert_decode_close, make_case, oracle_decode, ramp_scores
from engine.hip_decode import choose_splits, paged_decode_attention, split_plan

pytestmark = pytest.mark.gpu


def run(lengths, heads, B, dtype, splits, impl="auto", combine="fused", seed=0, work_list="off"):
    Hq, Hkv, D = HEADS[heads]
    q, k, v, bt, ctx, tables = make_case(lengths, Hq, Hkv, D, B, dtype, seed)
    scale = D ** -0.5
    print(f"case lengths={lengths[:8]} heads={heads} B={B} {dtype} splits={splits} impl={impl} {combine} "
          f"work_list={work_list}", flush=True)
    out = paged_decode_attention(q, k, v, bt, ctx, scale, max(lengths), num_splits=splits, impl=impl,
                                 combine=combine, host_context_lens=lengths, work_list=work_list)
    torch.cuda.synchronize()
    got = out.double().cpu().numpy()
    ref64 = oracle_decode(q, k, v, tables, lengths, scale, np.float64)
    if dtype == torch.float32:
        np.testing.assert_allclose(got, ref64, rtol=1e-5, atol=1e-5)
    else:
        ref32 = oracle_decode(q, k, v, tables, lengths, scale, np.float32)
        err = np.abs(got - ref32).max()
        assert err <= 8e-3, f"max-abs {err:.3e} vs fp32 oracle"
        np.testing.assert_allclose(got, ref64, rtol=1e-2, atol=1e-2)
    return got, ref64


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
@pytest.mark.parametrize("heads", list(HEADS))
@pytest.mark.parametrize("B", [8, 16, 32])
@pytest.mark.parametrize("splits", [1, 3, None], ids=["single", "split3", "auto"])
def test_ragged_batch_matches_oracle(dtype, heads, B, splits):
    """Ragged lengths 1 .. 1000 over shuffled tables (auto kernel choice: MFMA for bf16 with B = 16)."""
    run(RAGGED, heads, B, dtype, splits)


@pytest.mark.parametrize("heads", list(HEADS))
@pytest.mark.parametrize("impl", ["mfma", "valu"])
@pytest.mark.parametrize("combine", ["fused", "kernel"])
@pytest.mark.parametrize("splits", [1, 3, 16])
def test_kernels_and_merges(heads, impl, combine, splits):
    """Both bf16 kernels with both split merges, B = 16."""
    run(RAGGED, heads, 16, torch.bfloat16, splits, impl=impl, combine=combine)


@pytest.mark.parametrize("n", [1, 2, 31, 32, 33, 63, 64, 65, 4097])
@pytest.mark.parametrize("impl", ["mfma", "valu"])
def test_single_sequence_lengths(n, impl):
    """Batch 1 at tile, block and split boundaries, single pass and the CU-count split choice."""
    for splits in (1, None):
        run([n], "0.5B", 16, torch.bfloat16, splits, impl=impl)


@pytest.mark.parametrize("heads", list(HEADS))
def test_short_splits_each_tile_count(heads):
    """Splits of 1 to 3 32-token tiles a wave take their own load paths in the MFMA kernel (the tiles' loads in
    flight together): one sequence per length, so that the waves of its single split hold 1 (96, 100 tokens), 1 or
    2 (200), 2 or 3 (288, 300) and 3 (352, 383, 384) tiles, partial last tiles included; the same lengths in one
    batch on 3 splits and on the work list, whose items are that short too."""
    lengths = [96, 100, 200, 288, 300, 352, 383, 384]
    for n in lengths:
        run([n], heads, 16, torch.bfloat16, 1, impl="mfma")
    run(lengths, heads, 16, torch.bfloat16, 3, impl="mfma")
    run(lengths, heads, 16, torch.bfloat16, None, impl="mfma", work_list="on")


@pytest.mark.parametrize("heads", list(HEADS))
def test_context_longer_than_one_split_holds(heads):
    """A 40,000-token sequence asked for a single pass: a split stages at most 32,768 tokens of block ids, so the
    library cuts it into two and the output still matches the oracle; on the split grid and the work list."""
    run([40000, 5], heads, 16, torch.bfloat16, 1)
    run([40000, 5], heads, 16, torch.bfloat16, None, work_list="on")


@pytest.mark.parametrize("impl", ["mfma", "valu"])
def test_more_splits_than_tokens(impl):
    """Splits past a short sequence's end contribute nothing (reference tests/test_decode_kernel.py:84-86)."""
    dtype = torch.bfloat16 if impl == "mfma" else torch.float32
    run([1, 3, 2000], "0.5B", 16, dtype, 16, impl=impl)


@pytest.mark.parametrize("impl", ["mfma", "valu"])
def test_bf16_error_is_output_rounding(impl):
    """Against fp64 the bf16 kernel's median relative error stays below 2^-8 (output rounding dominates)."""
    got, ref = run(RAGGED, "0.5B", 16, torch.bfloat16, 1, impl=impl)
    rel = np.median(np.abs(got - ref) / np.maximum(np.abs(ref), 1e-3))
    print(f"\nbf16 {impl} median relative error vs fp64: {rel:.1e} (bf16 half-ulp {2 ** -9:.1e})")
    assert rel < 2 ** -8


def correctly_rounded_fraction(got: np.ndarray, ref64: np.ndarray) -> float:
    """Fraction of bf16 outputs equal to the fp64 oracle rounded to bf16 (round to nearest even)."""
    r = torch.from_numpy(ref64.astype(np.float32)).bfloat16().double().numpy()
    return float((got == r).mean())


@pytest.mark.parametrize("heads", list(HEADS))
def test_pv_product_keeps_reference_precision_of_p(heads):
    """The reference keeps P in fp32 and runs P.V in TF32, 11 significant bits of P (engine/triton_decode.py:14-18,
    206-210). Max-abs hides P's precision under the output's own bf16 rounding, so this counts outputs equal to the
    fp64 oracle rounded to bf16: with P carried to b bits that fraction is about 0.58 (b = 8), 0.89-0.93 (b = 11,
    TF32) and 0.99 (b = 16) on these shapes (numpy simulation of the same softmax with P rounded to b bits). The
    default kernel (P as a bf16 hi + lo pair) must reach 0.95; the one-term bf16-P variant must not, which shows
    the statistic separates the two."""
    lengths = [100, 777, 1000, 2048, 3000, 8192]
    Hq, Hkv, D = HEADS[heads]
    q, k, v, bt, ctx, tables = make_case(lengths, Hq, Hkv, D, 16, torch.bfloat16, seed=11)
    scale = D ** -0.5
    ref64 = oracle_decode(q, k, v, tables, lengths, scale, np.float64)
    frac = {}
    for impl in ("auto", "mfma_pbf16"):
        for splits in (1, None):
            print(f"case {heads} lengths={lengths} impl={impl} splits={splits}", flush=True)
            out = paged_decode_attention(q, k, v, bt, ctx, scale, max(lengths), num_splits=splits, impl=impl)
            torch.cuda.synchronize()
            got = out.double().cpu().numpy()
            assert np.abs(got - ref64).max() <= 8e-3
            frac[impl, splits] = correctly_rounded_fraction(got, ref64)
    print(f"\ncorrectly rounded fraction: {frac}")
    assert min(frac["auto", 1], frac["auto", None]) >= 0.95, frac
    assert max(frac["mfma_pbf16", 1], frac["mfma_pbf16", None]) < 0.8, frac


def test_split_policy_uses_cu_count():
    """The split policy reads the device's CU count and fills it: a 32 x 8k batch (64 programs) gets about one
    workgroup per CU, with splits of at most 2048 tokens."""
    from engine.hip_decode import device_cu_count

    cu = device_cu_count()
    print(f"\nCU count {cu}")
    assert cu >= 1
    s = choose_splits(32, 2, 8192, cu)
    launched, chunk = split_plan(8192, s)
    assert chunk <= 2048 and 64 * launched >= min(cu, 64 * 8192 // 256)


@pytest.mark.parametrize("impl", ["mfma", "valu"])
def test_l2_and_memory_merges_agree_past_the_cu_count(impl):
    """The fused merge reads the split partials from the XCD's L2 when every split of a pair ran there (the grid
    with sequences x KV heads a multiple of 8) and through memory otherwise. Both read the same partials in the
    same order, so 256 sequences (512 pairs: the L2 path) and the same 256 plus one more (514 pairs: memory)
    give the same bits for the 256, on grids of 2,048 workgroups, eight per CU, where a CU merges several pairs
    whose partial rows share cache lines; both match the oracle."""
    Hq, Hkv, D = HEADS["0.5B"]
    g = torch.Generator().manual_seed(17)
    lengths = torch.randint(600, 2049, (257,), generator=g).tolist()
    lengths[0] = 2048
    q, k, v, bt, ctx, tables = make_case(lengths, Hq, Hkv, D, 16, torch.bfloat16, seed=17)
    scale = D ** -0.5
    outs = []
    for S in (256, 257):
        print(f"case merge paths impl={impl} S={S} splits=4", flush=True)
        outs.append(paged_decode_attention(q[:S], k, v, bt[:S], ctx[:S], scale, 2048, num_splits=4, impl=impl))
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1][:256])
    ref = oracle_decode(q[:32], k, v, tables[:32], lengths[:32], scale, np.float32)
    assert_decode_close(outs[0][:32].double().cpu().numpy(), ref, f"merge paths {impl}")


def test_repeated_calls_reuse_workspace():
    """The fused merge's counters return to zero: ten calls on one stream give identical outputs."""
    Hq, Hkv, D = HEADS["0.5B"]
    q, k, v, bt, ctx, tables = make_case(RAGGED, Hq, Hkv, D, 16, torch.bfloat16, seed=3)
    outs = [paged_decode_attention(q, k, v, bt, ctx, D ** -0.5, max(RAGGED), num_splits=8).clone()
            for _ in range(10)]
    for o in outs[1:]:
        assert torch.equal(o, outs[0])


def test_strided_q_view():
    """q as a strided view of a fused QKV output (row stride (Hq + Hkv) * D), as the model passes it."""
    Hq, Hkv, D = HEADS["0.5B"]
    q, k, v, bt, ctx, tables = make_case(RAGGED, Hq, Hkv, D, 16, torch.bfloat16, seed=4)
    qkv = torch.zeros(len(RAGGED), Hq + 2 * Hkv, D, dtype=torch.bfloat16, device="cuda")
    qkv[:, :Hq] = q
    out = paged_decode_attention(qkv[:, :Hq], k, v, bt, ctx, D ** -0.5, max(RAGGED))
    ref = oracle_decode(q, k, v, tables, RAGGED, D ** -0.5, np.float32)
    assert np.abs(out.float().cpu().numpy() - ref).max() <= 8e-3


@pytest.mark.parametrize("heads", list(HEADS))
@pytest.mark.parametrize("impl,dtype", [("mfma", torch.bfloat16), ("valu", torch.bfloat16), ("valu", torch.float32)],
                         ids=["mfma-bf16", "valu-bf16", "valu-fp32"])
@pytest.mark.parametrize("lengths", [RAGGED, [1, 5000, 64, 65, 20000, 3, 129]], ids=["ragged", "long"])
def test_work_list_matches_oracle(heads, impl, dtype, lengths):
    """Ragged batches run from a host-built work list (near-equal pieces, longest first, merged in place)."""
    run(lengths, heads, 16, dtype, None, impl=impl, work_list="on")


def test_work_list_block_sizes():
    """Work lists with 8- and 32-token blocks (VALU kernel): pieces start on 64-token boundaries."""
    for B in (8, 32):
        run(RAGGED + [3000], "0.5B", B, torch.float32, None, work_list="on")


def test_decode_plan_replays_in_a_hip_graph():
    """A layer loop of decode launches (split merge fused, workspace allocated and zeroed before capture, no
    allocation or memset inside) captured in a HIP graph: every replay, with eager work and synchronizations in
    between, equals the eager result bit for bit."""
    from engine.hip_decode import DecodePlan

    Hq, Hkv, D = HEADS["0.5B"]
    layers = 3
    q, k, v, bt, ctx, tables = make_case(RAGGED, Hq, Hkv, D, 16, torch.bfloat16, seed=7)
    ks = [torch.randn_like(k) for _ in range(layers)]
    vs = [torch.randn_like(v) for _ in range(layers)]
    outs = [torch.empty_like(q) for _ in range(layers)]
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        plan = DecodePlan(q, ks[0], vs[0], bt, ctx, D ** -0.5, max(RAGGED), num_splits=4)
        for i in range(layers):
            plan(k_cache=ks[i], v_cache=vs[i], out=outs[i])
        stream.synchronize()
        eager = [o.clone() for o in outs]
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for i in range(layers):
                plan(k_cache=ks[i], v_cache=vs[i], out=outs[i])
        for rep in range(4):
            for o in outs:
                o.zero_()
            graph.replay()
            stream.synchronize()
            for o, e in zip(outs, eager):
                assert torch.equal(o, e), f"replay {rep}"
            plan(k_cache=ks[0], v_cache=vs[0], out=torch.empty_like(q))  # eager work between replays
            stream.synchronize()


def test_workspace_reuse_with_more_pairs():
    """Split calls on one workspace with a growing number of (sequence, KV head) pairs: 2 sequences then 300,
    both split 4 ways; the second call's merge counters must not overlap the first call's partials."""
    run([3000, 2000], "0.5B", 16, torch.bfloat16, 4)
    run([600] * 300, "0.5B", 16, torch.bfloat16, 4, seed=1)


def clamped_case(seed):
    """A batch whose tables hold ids outside the pool (past N and negative): what the kernels read instead is
    the clamped table (ids into [0, N))."""
    Hq, Hkv, D = HEADS["0.5B"]
    lengths = [700, 1500, 90]
    q, k, v, bt, ctx, tables = make_case(lengths, Hq, Hkv, D, 16, torch.bfloat16, seed=seed)
    N = k.shape[1]
    bad = bt.clone()
    fixed = [list(t) for t in tables]
    for s, j, b, c in ((0, 3, N + 5, N - 1), (1, 0, -7, 0), (1, 50, 1 << 30, N - 1), (2, 5, -1, 0)):
        bad[s, j] = b
        fixed[s][j] = c
    return q, k, v, bad, ctx, fixed, lengths


@pytest.mark.parametrize("impl,work_list,over", [("auto", "off", True), ("valu", "off", True),
                                                 ("auto", "on", False)])
def test_bad_ids_and_lengths_are_clamped(impl, work_list, over):
    """Block ids outside the pool are clamped into it and context lengths to max_context, as the prefill kernel
    does: the output is the clamped inputs' (every access stays in the pool), and the merge counters are back at
    zero afterwards (a length past max_context would otherwise report splits the grid does not have), so the
    next call on the same workspace is exact."""
    q, k, v, bad, ctx, fixed, lengths = clamped_case(seed=21)
    D, B, max_ctx = q.shape[2], k.shape[2], max(lengths)
    want_lengths = list(lengths)
    if over:  # sequence 2 reports 5500 tokens; the kernels read max_context of them, padding ids clamped to 0
        ctx = ctx.clone()
        ctx[2] = max_ctx + 4000
        want_lengths[2] = max_ctx
        fixed[2] = fixed[2] + [0] * (-(-max_ctx // B) - len(fixed[2]))
    print(f"case clamp impl={impl} work_list={work_list} over={over}", flush=True)
    kw = dict(impl=impl, host_context_lens=lengths, work_list=work_list)
    if work_list == "off":
        kw["num_splits"] = 3
    out = paged_decode_attention(q, k, v, bad, ctx, D ** -0.5, max_ctx, **kw)
    torch.cuda.synchronize()
    ref = oracle_decode(q, k, v, fixed, want_lengths, D ** -0.5, np.float32)
    assert np.abs(out.double().cpu().numpy() - ref).max() <= 8e-3
    # the same workspace, valid inputs: exact against a plan whose counters were never touched by the bad call
    q2, k2, v2, bt2, ctx2, tables2 = make_case(lengths, q.shape[1], k.shape[0], D, B, torch.bfloat16, seed=22)
    again = paged_decode_attention(q2, k2, v2, bt2, ctx2, D ** -0.5, max_ctx, **kw)
    torch.cuda.synchronize()
    ref2 = oracle_decode(q2, k2, v2, tables2, lengths, D ** -0.5, np.float32)
    assert np.abs(again.double().cpu().numpy() - ref2).max() <= 8e-3


def test_int8_bad_ids_are_clamped():
    """The INT8 kernel clamps block ids into the pool the same way (per-token scales)."""
    from engine.hip_decode import QuantKV

    q, k, v, bad, ctx, fixed, lengths = clamped_case(seed=23)
    Hkv, N, B, D = k.shape
    g = torch.Generator(device="cuda").manual_seed(23)
    kq = torch.randint(-127, 128, (Hkv, N, B, D), device="cuda", dtype=torch.int8, generator=g)
    vq = torch.randint(-127, 128, (Hkv, N, B, D), device="cuda", dtype=torch.int8, generator=g)
    ks = (torch.rand(Hkv, N, B, device="cuda", generator=g) / 64 + 1 / 256).half()
    vs = (torch.rand(Hkv, N, B, device="cuda", generator=g) / 64 + 1 / 256).half()
    print("case clamp int8", flush=True)
    out = paged_decode_attention(q, kq, vq, bad, ctx, D ** -0.5, max(lengths), num_splits=3,
                                 quant=QuantKV(1, ks, vs))
    torch.cuda.synchronize()
    kf, vf = kq.float() * ks.float()[..., None], vq.float() * vs.float()[..., None]
    ref = oracle_decode(q, kf, vf, fixed, lengths, D ** -0.5, np.float32)
    assert_decode_close(out.double().cpu().numpy(), ref, "int8 clamp")


def test_table_narrower_than_max_context_is_refused():
    """The kernels load table entries up to max_context for every sequence: a narrower table is refused on the
    host, before any launch."""
    Hq, Hkv, D = HEADS["0.5B"]
    q, k, v, bt, ctx, tables = make_case([100, 300], Hq, Hkv, D, 16, torch.bfloat16, seed=5)
    with pytest.raises(ValueError):
        paged_decode_attention(q, k, v, bt[:, :10], ctx, D ** -0.5, 300)
    with pytest.raises(ValueError):
        paged_decode_attention(q, k, v, bt, ctx[:1], D ** -0.5, 300)


@pytest.mark.parametrize("heads", list(HEADS))
@pytest.mark.parametrize("impl", ["valu_stream", "valu_dot2"])
@pytest.mark.parametrize("splits", [1, 3, None], ids=["single", "split3", "auto"])
def test_valu_streaming_kernels_match_oracle(heads, impl, splits):
    """The VALU streaming kernels (the matrix-core A/B competitors: fp32 FMAs, v_dot2 pairs) on bf16 pools, ragged
    lengths with partial blocks and tiles, against the oracle to the north-star bound."""
    run(RAGGED + [2100, 64], heads, 16, torch.bfloat16, splits, impl=impl)


@pytest.mark.parametrize("heads", list(HEADS))
def test_l2_merge_reads_this_calls_partials(heads):
    """On the split grid with S * Hkv a multiple of 8 the fused merge reads the partials from the XCD's L2. Calls
    that alternate between two batches of the same shape (the same workspace addresses) each match the oracle on
    their own inputs, so no partial of an earlier call is read back; a batch whose S * Hkv is not a multiple of 8
    (merged through memory) in between changes nothing."""
    Hq, Hkv, D = HEADS[heads]
    lengths = [700, 2100, 33, 4096, 1000, 1, 3000, 129]  # S = 8: S * Hkv = 16
    cases = [make_case(lengths, Hq, Hkv, D, 16, torch.bfloat16, seed=s) for s in (41, 42)]
    odd = make_case(lengths[:3], Hq, Hkv, D, 16, torch.bfloat16, seed=43)  # S * Hkv = 6
    refs = [oracle_decode(q, k, v, t, lengths, D ** -0.5, np.float32) for q, k, v, _, _, t in cases]
    print(f"case l2 merge alternation {heads}", flush=True)
    for rep in range(3):
        for i, (q, k, v, bt, ctx, _) in enumerate(cases):
            out = paged_decode_attention(q, k, v, bt, ctx, D ** -0.5, max(lengths), num_splits=4)
            torch.cuda.synchronize()
            assert_decode_close(out.double().cpu().numpy(), refs[i], f"l2 merge rep {rep} batch {i}")
        q, k, v, bt, ctx, _ = odd
        paged_decode_attention(q, k, v, bt, ctx, D ** -0.5, max(lengths[:3]), num_splits=4)


@pytest.mark.parametrize("direction", [1, -1, 0], ids=["rising", "falling", "spike"])
@pytest.mark.parametrize("splits", [1, 3, None], ids=["single", "split3", "auto"])
def test_scores_trending_across_keys(direction, splits):
    """Scores rising (or falling) by about 4 in the exp2 domain every 64 keys, or one key's score about 90 above
    the rest: rising, the running max is passed by more than the lazy-rescale slack every few tiles and acc and l
    are rescaled there; falling, the later probabilities underflow against the first tiles' max; the spike
    rescales once. The bf16 MFMA kernel against the fp32 oracle."""
    lengths = [3000, 700, 129, 17]
    Hq, Hkv, D = HEADS["0.5B"]
    q, k, v, bt, ctx, tables = make_case(lengths, Hq, Hkv, D, 16, torch.bfloat16, seed=71)
    ramp_scores(q, k, tables, lengths, 16, direction)
    print(f"case trending scores direction={direction} splits={splits}", flush=True)
    out = paged_decode_attention(q, k, v, bt, ctx, D ** -0.5, max(lengths), num_splits=splits, impl="mfma",
                                 host_context_lens=lengths)
    torch.cuda.synchronize()
    ref32 = oracle_decode(q, k, v, tables, lengths, D ** -0.5, np.float32)
    assert_decode_close(out.double().cpu().numpy(), ref32, "trending scores")
