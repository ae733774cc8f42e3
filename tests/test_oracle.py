"""Pinning the CPU oracle (oracle/) before it is trusted as the checker of the HIP kernels.

Each restatement is checked against something independent of its own formula:
  - the quantizer (plain C) against torch's library routines that the reference's quantizer is made of
    (torch.round, Tensor.to(float16), fp32 division; reference engine/quant.py:22-31), against the numpy
    restatement, and against the invariants the reference's tests assert (tests/test_quant.py:8-51);
  - the C binary32 -> binary16 conversion against numpy's astype(float16) over every class of input;
  - gather-then-attend against torch.nn.functional.scaled_dot_product_attention with repeated KV heads, against
    brute-force loops in fp64, and against closed forms (uniform and one-hot softmax);
  - the split merge against the unsplit softmax (the identity Flash-Decoding rests on);
  - indexing and metadata against the reference tests' known answers (tests/golden/reference_known_answers.json);
  - the bf16 rounding helper against torch's Tensor.bfloat16() over specials, ties and every exponent;
  - dequantization against the exact products (int8 x fp16 fits fp32) and the quantizer's round-trip bound
    |x - q s| <= s / 2 (reference tests/test_quant.py:8-26), per token and per channel;
  - the timed CPU baseline (torch gather-then-attend) against the fp64 oracle decode on a ragged, scattered batch.
"""

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import paged_ref

GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_known_answers.json").read_text())


# ---- quantizer ----------------------------------------------------------------------------------------------------

def torch_quantize(x: np.ndarray, axis: int):
    """The reference quantizer's arithmetic, spelled with torch's own ops (engine/quant.py:22-31)."""
    t = torch.from_numpy(x)
    s = (t.abs().amax(dim=axis, keepdim=True).float() / 127).to(torch.float16)
    sf = s.float()
    q = torch.where(sf > 0, torch.round(t.float() / torch.where(sf > 0, sf, torch.ones_like(sf))),
                    torch.zeros((), dtype=torch.float32)).clamp(-127, 127).to(torch.int8)
    return q.numpy(), s.squeeze(axis).numpy()


def edge_rows() -> np.ndarray:
    rng = np.random.default_rng(0)
    rows = [np.zeros(64), np.full(64, 1e-9), np.linspace(-7e-4, 7e-4, 64), rng.standard_normal(64) * 1e-5,
            np.array([127.0, -127.0, 63.5, -63.5] * 16)]
    s = float(np.float16(3.0 / 127))
    ties = (np.arange(64) - 32.0 + 0.5) * s
    ties[0] = 127 * s
    rows.append(ties)
    for k in range(0, 20):  # absmax / 127 right at, above and below fp16 rounding ties
        base = float(np.float16(2.0 ** -k)) * 127
        r = rng.standard_normal(64) * base / 4
        r[7] = np.nextafter(np.float32(base), np.float32(k % 3 - 1))
        rows.append(r)
    rows.append(rng.standard_normal(64) * 1e4)
    return np.stack(rows).astype(np.float32)


@pytest.mark.parametrize("case", ["random", "edges", "scaled"])
def test_quantizer_matches_torch_library_routines(case):
    rng = np.random.default_rng(1)
    if case == "random":
        x = (rng.standard_normal((257, 3, 64)) * rng.random((257, 3, 1)) * 5).astype(np.float32)
    elif case == "edges":
        x = edge_rows()[:, None, :]
    else:
        x = (rng.standard_normal((64, 2, 128)) * np.exp(rng.uniform(-12, 12, (64, 2, 1)))).astype(np.float32)
    for axis in (-1, 0):
        qc, sc = paged_ref.quantize_groups_c(x, axis)
        qt, st = torch_quantize(x, axis)
        qn, sn = paged_ref.quantize_groups_np(x, axis)
        assert np.array_equal(qc, qt) and np.array_equal(sc.view(np.uint16), st.view(np.uint16))
        assert np.array_equal(qc, qn) and np.array_equal(sc.view(np.uint16), sn.view(np.uint16))


def test_quantizer_bf16_inputs_match_torch():
    """bf16 activations (the model dtype) widen exactly to fp32 first, as x.float() does in the reference."""
    g = torch.Generator().manual_seed(3)
    xb = (torch.randn(100, 2, 64, generator=g) * 3).bfloat16()
    x = xb.float().numpy()
    qc, sc = paged_ref.quantize_per_token(x)
    from engine.quant import quantize_per_token

    qt, st = quantize_per_token(xb)
    assert np.array_equal(qc, qt.numpy()) and np.array_equal(sc.view(np.uint16), st.numpy().view(np.uint16))


def test_quantizer_invariants():
    """Reference tests/test_quant.py:8-36: codes in [-127, 127], the absmax maps to +-127, |x - q s| <= s/2
    (plus the fp16 slack), zero groups give scale 0 and zero codes."""
    rng = np.random.default_rng(0)
    x = (rng.standard_normal((37, 2, 64)) * rng.random((37, 2, 1)) * 5).astype(np.float32)
    q, s = paged_ref.quantize_per_token(x)
    s32 = s.astype(np.float32)[..., None]
    assert q.dtype == np.int8 and s.dtype == np.float16 and np.abs(q.astype(int)).max() <= 127
    assert (np.abs(q.astype(int)).max(-1) == 127).mean() > 0.9
    assert (np.abs(x - q * s32) <= s32 * 0.5 * (1 + 1e-3) + 1e-7).all()
    z = np.zeros((3, 2, 64), np.float32)
    z[1, 0] = np.linspace(-2, 2, 64)
    qz, sz = paged_ref.quantize_per_token(z)
    assert sz[0, 0] == 0 and sz[2, 1] == 0 and (qz[0] == 0).all()


def test_per_channel_axis_semantics():
    """quantize_per_channel(x, axis) gives one scale per position of the other axes (the block's channels)."""
    rng = np.random.default_rng(2)
    x = (rng.standard_normal((2, 3, 16, 64)) * rng.random((1, 1, 1, 64)) * 3).astype(np.float32)
    q, s = paged_ref.quantize_per_channel(x, axis=2)
    assert q.shape == x.shape and s.shape == (2, 3, 64)
    for h in range(2):
        for b in range(3):
            qq, ss = paged_ref.quantize_per_token(np.ascontiguousarray(x[h, b].T))
            assert np.array_equal(q[h, b], qq.T) and np.array_equal(s[h, b], ss)


def test_f16_conversion_matches_numpy():
    rng = np.random.default_rng(4)
    specials = np.array([0.0, -0.0, 2 ** -24, 2 ** -25, 1.5 * 2 ** -25, 2 ** -14, 2 ** -14 - 2 ** -25,
                         65504.0, 65519.99, 65520.0, 1e6, np.inf, -np.inf, 1.0 + 2 ** -11, 1.0 + 3 * 2 ** -11,
                         6.1e-5, 5.96e-8], np.float32)
    vals = np.concatenate([specials, rng.standard_normal(20000).astype(np.float32) *
                           np.exp2(rng.uniform(-30, 18, 20000)).astype(np.float32)])
    got = paged_ref.f32_to_f16_bits_c(vals)
    with np.errstate(over="ignore"):  # values past 65520 overflow to inf, as they should
        want = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


# ---- attention --------------------------------------------------------------------------------------------------

def sdpa_reference(q, k, v, scale):
    """torch's scaled_dot_product_attention with KV heads repeated over their query groups (fp64)."""
    Hq, Hkv = q.shape[0], k.shape[0]
    kk = torch.from_numpy(k).double().repeat_interleave(Hq // Hkv, 0)
    vv = torch.from_numpy(v).double().repeat_interleave(Hq // Hkv, 0)
    out = torch.nn.functional.scaled_dot_product_attention(torch.from_numpy(q).double()[:, None], kk, vv,
                                                           scale=scale)
    return out[:, 0].numpy()


@pytest.mark.parametrize("Hq,Hkv,D,n", [(14, 2, 64, 1), (14, 2, 64, 37), (12, 2, 128, 300), (6, 2, 16, 5)])
def test_attend_matches_sdpa(Hq, Hkv, D, n):
    rng = np.random.default_rng(n)
    q, k, v = rng.standard_normal((Hq, D)), rng.standard_normal((Hkv, n, D)), rng.standard_normal((Hkv, n, D))
    ref = sdpa_reference(q, k, v, D ** -0.5)
    np.testing.assert_allclose(paged_ref.attend_one(q, k, v, D ** -0.5, np.float64), ref, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(paged_ref.attend_one(q, k, v, D ** -0.5, np.float32), ref, rtol=1e-5, atol=1e-5)


def test_attend_matches_brute_force():
    rng = np.random.default_rng(9)
    Hq, Hkv, D, n = 4, 2, 8, 5
    q, k, v = rng.standard_normal((Hq, D)), rng.standard_normal((Hkv, n, D)), rng.standard_normal((Hkv, n, D))
    out = np.zeros((Hq, D))
    for h in range(Hq):
        kv = h // (Hq // Hkv)
        e = [np.exp(0.3 * sum(q[h, d] * k[kv, t, d] for d in range(D))) for t in range(n)]
        for d in range(D):
            out[h, d] = sum(e[t] * v[kv, t, d] for t in range(n)) / sum(e)
    np.testing.assert_allclose(paged_ref.attend_one(q, k, v, 0.3, np.float64), out, rtol=1e-12)


def test_attend_closed_forms():
    rng = np.random.default_rng(10)
    k, v = rng.standard_normal((2, 50, 16)), rng.standard_normal((2, 50, 16))
    uniform = paged_ref.attend_one(np.zeros((6, 16)), k, v, 1.0, np.float64)  # q = 0: every weight 1/n
    np.testing.assert_allclose(uniform, np.repeat(v.mean(axis=1), 3, axis=0), rtol=1e-12)
    k2 = np.zeros((2, 50, 16))
    k2[:, 17, 0] = 1.0
    q = np.zeros((6, 16))
    q[:, 0] = 1e4  # one key dominates
    np.testing.assert_allclose(paged_ref.attend_one(q, k2, v, 1.0, np.float64), np.repeat(v[:, 17], 3, axis=0))


@pytest.mark.parametrize("cuts", [[], [1], [63, 64], [5, 100, 101, 300]])
def test_split_merge_equals_unsplit(cuts):
    """Splitting the context and merging (m, l, acc) states gives the unsplit softmax (engine/triton_decode.py:20-24)."""
    rng = np.random.default_rng(len(cuts))
    Hq, Hkv, D, n = 14, 2, 64, 400
    q, k, v = rng.standard_normal((Hq, D)), rng.standard_normal((Hkv, n, D)), rng.standard_normal((Hkv, n, D))
    bounds = [0] + cuts + [n]
    states = [paged_ref.split_state(q, k[:, a:b], v[:, a:b], 0.125) for a, b in zip(bounds, bounds[1:])]
    merged = paged_ref.combine(*zip(*states))
    np.testing.assert_allclose(merged, paged_ref.attend_one(q, k, v, 0.125, np.float64), rtol=1e-12, atol=1e-12)


def test_gather_and_decode_follow_the_block_table():
    """Paged gather reads [:, table[p // B], p % B] (reference engine/paged_cache.py:3-5,141-147): equal to the
    contiguous sequence it was scattered from."""
    rng = np.random.default_rng(11)
    Hkv, N, B, D, n = 2, 12, 4, 8, 11
    seq_k = rng.standard_normal((Hkv, n, D))
    table = [7, 2, 9]
    pool = rng.standard_normal((Hkv, N, B, D))
    for p in range(n):
        pool[:, table[p // B], p % B] = seq_k[:, p]
    np.testing.assert_array_equal(paged_ref.gather(pool, table, n), seq_k)
    q = rng.standard_normal((1, 6, D))
    np.testing.assert_allclose(paged_ref.decode(q, pool, pool, [table], [n], 0.5)[0],
                               paged_ref.attend_one(q[0], seq_k, seq_k, 0.5))


def scatter_sequences(rng, lengths, Hkv, D, B, N):
    """Random pool [Hkv, N, B, D] holding sequences of these lengths through shuffled block tables; returns the
    pool, the tables and the contiguous [Hkv, n, D] sequences."""
    pool = rng.standard_normal((Hkv, N, B, D))
    free = list(rng.permutation(N))
    tables, seqs = [], []
    for n in lengths:
        t = [int(free.pop()) for _ in range(-(-n // B))]
        x = rng.standard_normal((Hkv, n, D))
        for p in range(n):
            pool[:, t[p // B], p % B] = x[:, p]
        tables.append(t)
        seqs.append(x)
    return pool, tables, seqs


def test_prefill_fresh_sequence_matches_sdpa_causal():
    """A sequence's first chunk (context == new tokens) is torch's causal scaled_dot_product_attention."""
    rng = np.random.default_rng(13)
    Hq, Hkv, D, B, n = 6, 2, 16, 4, 23
    kp, tables, ks = scatter_sequences(rng, [n], Hkv, D, B, 12)
    vp, _, _ = scatter_sequences(np.random.default_rng(13), [n], Hkv, D, B, 12)  # same tables, other values
    vs = paged_ref.gather(vp, tables[0], n)
    q = rng.standard_normal((n, Hq, D))
    got = paged_ref.prefill(q, kp, vp, tables, [n], [0], [n], 0.3)
    qt = torch.from_numpy(q).permute(1, 0, 2)                                         # [Hq, n, D]
    kk = torch.from_numpy(ks[0]).repeat_interleave(Hq // Hkv, 0)
    vv = torch.from_numpy(vs).repeat_interleave(Hq // Hkv, 0)
    want = torch.nn.functional.scaled_dot_product_attention(qt, kk, vv, is_causal=True, scale=0.3)
    np.testing.assert_allclose(got, want.permute(1, 0, 2).numpy(), rtol=1e-12, atol=1e-12)


def test_prefill_chunk_rows_are_decode_rows():
    """Mid-context chunks of a packed batch: row r of sequence s (position ctx - n + r) equals one-token attention
    over keys 0 .. its position; rows of no sequence stay zero."""
    rng = np.random.default_rng(14)
    Hq, Hkv, D, B = 8, 2, 8, 4
    ctx, qlen = [9, 30, 5], [4, 17, 1]
    pool, tables, seqs = scatter_sequences(rng, ctx, Hkv, D, B, 20)
    starts = [0, 6, 23]                      # rows 4, 5 and 24.. belong to no sequence
    q = rng.standard_normal((26, Hq, D))
    got = paged_ref.prefill(q, pool, pool, tables, ctx, starts, qlen, 0.25)
    for s in range(3):
        for r in range(qlen[s]):
            n = ctx[s] - qlen[s] + r + 1
            want = paged_ref.attend_one(q[starts[s] + r], seqs[s][:, :n], seqs[s][:, :n], 0.25)
            np.testing.assert_allclose(got[starts[s] + r], want, rtol=1e-12, atol=1e-12)
    assert not got[[4, 5, 24, 25]].any()


def test_kchannel_gather_reads_tail_from_staging():
    rng = np.random.default_rng(12)
    H, N, B, D, n = 2, 6, 4, 8, 10  # 2 full blocks + 2 staged tokens
    kq = rng.integers(-127, 128, (H, N, B, D)).astype(np.int8)
    ks = rng.random((H, N, D)).astype(np.float16)
    stage = rng.standard_normal((H, 3, B, D)).astype(np.float32)
    k = paged_ref.gather_kchannel(kq, ks, stage, [4, 1, 5], n, 2)
    np.testing.assert_array_equal(k[:, :4], kq[:, 4].astype(np.float32) * ks[:, 4][:, None, :].astype(np.float32))
    np.testing.assert_array_equal(k[:, 8:], stage[:, 2, :2])


# ---- indexing and metadata: the reference tests' known answers ------------------------------------------------------

def test_metadata_known_answer():
    ka = GOLDEN["metadata_packed_batch"]
    # The tables the reference scenario produces (blocks handed out 0, 1, 2, 3, then 4), per its own test.
    tables = {0: [0, 4], 1: [1, 2, 3]}
    meta = paged_ref.metadata(tables, [tuple(b) for b in ka["batch"]], ka["block_size"])
    for key in ("query_starts", "context_lens", "positions", "slot_mapping", "slot_blocks", "slot_offsets",
                "block_tables", "last_token_indices"):
        assert meta[key] == ka[key], key
    padded = paged_ref.padded_tables([tables[0], tables[1]], meta["context_lens"], ka["block_size"])
    assert padded.dtype == np.int32 and padded.tolist() == ka["block_tables"]


def test_slots_known_answer():
    ka = GOLDEN["block_manager_allocate_append"]
    assert paged_ref.slots([0, 1], 0, 6, 4) == ka["ops"][0][3]
    assert paged_ref.slots([0, 1, 2, 3], 9, 14, 4) == ka["ops"][4][3]


def test_per_channel_beats_per_token_with_outlier_channels():
    """The reference's motivation for format B (tests/test_quant.py:39-50): with a few outlier channels, per-channel
    scales over a block's tokens lose less than per-token scales over a token's channels."""
    rng = np.random.default_rng(15)
    x = rng.standard_normal((2, 64, 16, 128)).astype(np.float32)
    x[..., :4] *= 40.0
    qt, st = paged_ref.quantize_per_token(x)
    qc, sc = paged_ref.quantize_per_channel(x, axis=2)
    err_t = np.linalg.norm(paged_ref.dequant_tokens(qt, st) - x) / np.linalg.norm(x)
    err_c = np.linalg.norm(paged_ref.dequant_channels(qc, sc) - x) / np.linalg.norm(x)
    assert err_c < err_t / 2, (err_c, err_t)


# ---- bf16 rounding, dequantization, the CPU baseline ---------------------------------------------------------------

def test_bf16_round_matches_torch():
    """bf16_round == torch's fp32 -> bf16 -> fp32 bit for bit: specials, subnormals, the largest finite values
    (round to infinity), exact ties with even and odd lower neighbours, and random values over every exponent."""
    rng = np.random.default_rng(21)
    f32 = np.float32
    specials = np.array([0.0, -0.0, np.inf, -np.inf, 1.0, -1.0, np.finfo(f32).max, -np.finfo(f32).max,
                         np.finfo(f32).tiny, 1e-45, -1e-45, 3.0e38, 65504.0], dtype=f32)
    lower = rng.integers(0, 1 << 15, 4000, dtype=np.uint32) << 16 | (rng.integers(0, 256, 4000, dtype=np.uint32) << 23)
    ties = (lower.astype(np.uint32) | 0x8000).view(f32)  # exactly halfway between two bf16 neighbours
    near = np.concatenate([(lower | 0x7FFF).view(f32), (lower | 0x8001).view(f32)])
    with np.errstate(over="ignore"):  # the largest draws overflow to infinity: a case of their own
        wide = (rng.standard_normal(20000) * 2.0 ** rng.integers(-149, 128, 20000)).astype(f32)
    x = np.concatenate([specials, ties, near, wide])
    x = x[np.isfinite(x) | np.isinf(x)]
    want = torch.from_numpy(x.copy()).bfloat16().float().numpy()
    got = paged_ref.bf16_round(x)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert np.isnan(paged_ref.bf16_round(np.array([np.nan, np.float32(np.nan) * -1], dtype=f32))).all()
    snan = np.array([0x7F800001, 0xFF800123], dtype=np.uint32).view(f32)
    assert np.isnan(paged_ref.bf16_round(snan)).all()


@pytest.mark.parametrize("seed", range(3))
def test_dequantize_is_exact_and_inverts_the_quantizer(seed):
    """dequant_tokens / dequant_channels equal the exact products q * s (an int8 code times an fp16 scale is
    exact in fp32) with each scale on its own axis, and undo the quantizer to within half a step:
    |x - q s| <= s / 2 for every element (the reference's round-trip invariant, tests/test_quant.py:8-26)."""
    rng = np.random.default_rng(30 + seed)
    x = (rng.standard_normal((2, 9, 16, 64)) * rng.random((2, 9, 16, 1)) * 4).astype(np.float32)
    x[..., :3] *= 30.0  # outlier channels
    x[1, 4, 7] = 0.0    # a zero vector (scale 0, codes 0)
    qt, st = paged_ref.quantize_per_token(x)
    dt = paged_ref.dequant_tokens(qt, st)
    assert dt.dtype == np.float32 and dt.shape == x.shape
    assert np.array_equal(dt.astype(np.float64), qt.astype(np.float64) * st.astype(np.float64)[..., None])
    assert (np.abs(x.astype(np.float64) - dt) <= st.astype(np.float64)[..., None] / 2).all()
    assert not dt[1, 4, 7].any()
    qc, sc = paged_ref.quantize_per_channel(x, axis=2)  # [H, N, D] scales over each block's 16 tokens
    dc = paged_ref.dequant_channels(qc, sc)
    assert dc.dtype == np.float32 and dc.shape == x.shape
    assert np.array_equal(dc.astype(np.float64), qc.astype(np.float64) * sc.astype(np.float64)[:, :, None, :])
    assert (np.abs(x.astype(np.float64) - dc) <= sc.astype(np.float64)[:, :, None, :] / 2).all()


def test_cpu_baseline_matches_oracle_decode():
    """decode_torch_cpu (the timed CPU baseline: torch gather-then-attend in fp32) equals the fp64 oracle decode on
    a ragged batch over a scattered pool with partial last blocks and GQA groups of 7."""
    rng = np.random.default_rng(40)
    Hq, Hkv, D, B = 14, 2, 64, 16
    lengths = [1, 15, 16, 17, 33, 100, 1000, 257]
    nbs = [-(-n // B) for n in lengths]
    perm = rng.permutation(3 * sum(nbs)).tolist()
    tables, at = [], 0
    for nb in nbs:
        tables.append(perm[at:at + nb])
        at += nb
    N = len(perm)
    k = rng.standard_normal((Hkv, N, B, D)).astype(np.float32)
    v = rng.standard_normal((Hkv, N, B, D)).astype(np.float32)
    q = rng.standard_normal((len(lengths), Hq, D)).astype(np.float32)
    bt = torch.from_numpy(paged_ref.padded_tables(tables, lengths, B).astype(np.int64))
    got = paged_ref.decode_torch_cpu(torch.from_numpy(q), torch.from_numpy(k), torch.from_numpy(v), bt, lengths,
                                     D ** -0.5).numpy()
    want = paged_ref.decode(q, k, v, tables, lengths, D ** -0.5, np.float64)
    np.testing.assert_allclose(got, want, rtol=2e-5, atol=2e-6)
