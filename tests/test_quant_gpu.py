"""INT8 on the GPU: fused quantize-and-store is bit-exact with the C oracle, and the INT8 decode modes match the
oracle's dequantize-then-attend.

Mirrors the reference's tests/test_quant_cache.py:221-259 (kernel vs fp64 attention over the cache's own
dequantized K/V: lengths [1, 15, 16, 17, 33, 100, 700], outlier channels 1 + 5 * (c % 13 == 0), chunked writes
[37, n - 37], both formats, B 8 / 16 / 32, fp32 / bf16, single / auto splits; tolerances 1e-4 fp32 and 2e-2
bf16 as there, plus the north-star 8e-3 max-abs for bf16 against the fp32 oracle) and :351-410 (fused writes
bit-exact, from a strided view with a zero vector, blocks, whole chunked fills).
"""

import numpy as np
import pytest
import torch

from cases import HEADS, as_np32, assert_decode_close
from engine.block_manager import BlockManager
from engine.config import ModelConfig
from engine.hip_decode import paged_decode_attention
from engine.hip_quant import (kchan_write_rows, quantize_store_block_rows, quantize_store_blocks,
                              quantize_store_tokens, store_tokens)
from engine.paged_cache import build_metadata
from engine.quant_cache import QuantPagedKVCache
from oracle import paged_ref

pytestmark = pytest.mark.gpu
FMTS = ["int8", "int8-kchannel"]


def bits16(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(a).view(np.uint16)


# ---- quantize-and-store, bit-exact ------------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16], ids=["bf16", "fp32", "fp16"])
@pytest.mark.parametrize("D", [16, 64, 128])
def test_token_quantization_is_exact(dtype, D):
    """Per-token codes and fp16 scales equal the oracle's, from a strided view, including a zero vector."""
    g = torch.Generator().manual_seed(0)
    big = (torch.randn(37, 16, D, generator=g) * 3).to("cuda", dtype)
    x = big[:, 14:]  # [37, 2, D], row stride 16 * D
    x[5, 1] = 0
    N, B = 20, 16
    blocks = torch.randperm(N, generator=g)[:3].repeat_interleave(B)[:37].cuda()
    offsets = (torch.arange(37) % B).cuda()
    qp = torch.zeros(2, N, B, D, dtype=torch.int8, device="cuda")
    sp = torch.zeros(2, N, B, dtype=torch.float16, device="cuda")
    print(f"case tokens {dtype} D={D}", flush=True)
    quantize_store_tokens(x, blocks, offsets, qp, sp)
    q_ref, s_ref = paged_ref.quantize_per_token(as_np32(x))
    assert np.array_equal(qp[:, blocks, offsets].transpose(0, 1).cpu().numpy(), q_ref)
    assert np.array_equal(bits16(sp[:, blocks, offsets].t().cpu().numpy()), bits16(s_ref))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
@pytest.mark.parametrize("D", [64, 128])
def test_token_quantization_of_k_and_v_in_one_launch(dtype, D):
    """The two-pair launch (V and K views of one fused projection, different strides from the pools') stores
    what two single calls store, bit for bit, and both equal the oracle."""
    g = torch.Generator().manual_seed(1)
    qkv = (torch.randn(41, 18, D, generator=g) * 3).to("cuda", dtype)  # [T, Hq + 2 Hkv, D]
    k, v = qkv[:, 14:16], qkv[:, 16:18]
    v[7, 0] = 0
    N, B = 24, 16
    blocks = torch.randperm(N, generator=g)[:3].repeat_interleave(B)[:41].cuda()
    offsets = (torch.arange(41) % B).cuda()
    pools = [torch.zeros(2, N, B, D, dtype=torch.int8, device="cuda") for _ in range(4)]
    scales = [torch.zeros(2, N, B, dtype=torch.float16, device="cuda") for _ in range(4)]
    print(f"case tokens kv {dtype} D={D}", flush=True)
    quantize_store_tokens(v, blocks, offsets, pools[0], scales[0], x2=k, q_pool2=pools[1], s_pool2=scales[1])
    quantize_store_tokens(v, blocks, offsets, pools[2], scales[2])
    quantize_store_tokens(k, blocks, offsets, pools[3], scales[3])
    torch.cuda.synchronize()
    for a, b in ((0, 2), (1, 3)):
        assert torch.equal(pools[a], pools[b]) and torch.equal(scales[a].view(torch.int16), scales[b].view(torch.int16))
    for x, i in ((v, 0), (k, 1)):
        q_ref, s_ref = paged_ref.quantize_per_token(as_np32(x))
        assert np.array_equal(pools[i][:, blocks, offsets].transpose(0, 1).cpu().numpy(), q_ref)
        assert np.array_equal(bits16(scales[i][:, blocks, offsets].t().cpu().numpy()), bits16(s_ref))
    with pytest.raises(ValueError):  # a second pool of another shape
        quantize_store_tokens(v, blocks, offsets, pools[0], scales[0], x2=k, q_pool2=pools[1][:1],
                              s_pool2=scales[1])


def test_token_quantization_edge_values():
    """Scales that round to zero or to fp16 subnormals, exact .5 ties of x / s, values at the +-127 edge, and
    absmax near fp16 rounding ties: codes and scales still equal the oracle's."""
    rows = []
    rows.append(np.zeros(64, np.float32))                                   # scale 0
    rows.append(np.full(64, 1e-9, np.float32))                              # absmax/127 underflows fp16
    rows.append(np.linspace(-7e-4, 7e-4, 64).astype(np.float32))            # subnormal fp16 scale
    s = np.float32(np.float16(3.0 / 127))                                   # a representable scale
    ties = (np.arange(64, dtype=np.float32) - 32.0 + 0.5) * s              # x / s lands on .5
    ties[0] = 127 * s
    rows.append(ties.astype(np.float32))
    for k in range(4, 16):                                                  # absmax / 127 near fp16 ties
        base = np.float32(np.float16(2.0 ** -k)) * 127
        r = np.random.default_rng(k).standard_normal(64).astype(np.float32) * base / 4
        r[3] = np.nextafter(base, np.float32(0)) if k % 2 else np.nextafter(base, np.float32(1))
        rows.append(r)
    rows.append(np.array([127.0, -127.0, 63.5, -63.5] * 16, np.float32))
    x_np = np.stack(rows)[:, None, :]  # [T, 1, 64]
    T = x_np.shape[0]
    x = torch.from_numpy(x_np).cuda()
    blocks = torch.arange(T, device="cuda") // 16
    offsets = torch.arange(T, device="cuda") % 16
    nb = -(-T // 16)
    qp = torch.zeros(1, nb, 16, 64, dtype=torch.int8, device="cuda")
    sp = torch.zeros(1, nb, 16, dtype=torch.float16, device="cuda")
    quantize_store_tokens(x, blocks, offsets, qp, sp)
    q_ref, s_ref = paged_ref.quantize_per_token(x_np)
    assert np.array_equal(qp[:, blocks, offsets].transpose(0, 1).cpu().numpy(), q_ref)
    assert np.array_equal(bits16(sp[:, blocks, offsets].t().cpu().numpy()), bits16(s_ref))


@pytest.mark.parametrize("D", [64, 128])
def test_block_quantization_is_exact(D):
    """Per-channel blocks from bf16 staging equal the oracle's codes and channel scales."""
    g = torch.Generator().manual_seed(1)
    stage = (torch.randn(2, 8, 16, D, generator=g) * torch.rand(1, 1, 1, D, generator=g) * 4).bfloat16().cuda()
    src = torch.tensor([3, 0, 6], device="cuda")
    dst = torch.tensor([11, 2, 7], device="cuda")
    qp = torch.zeros(2, 12, 16, D, dtype=torch.int8, device="cuda")
    sp = torch.zeros(2, 12, D, dtype=torch.float16, device="cuda")
    quantize_store_blocks(stage, src, dst, qp, sp)
    q_ref, s_ref = paged_ref.quantize_per_channel(as_np32(stage[:, src]), axis=2)
    assert np.array_equal(qp[:, dst].cpu().numpy(), q_ref)
    assert np.array_equal(bits16(sp[:, dst].cpu().numpy()), bits16(s_ref))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
def test_block_rows_quantization_is_exact(dtype):
    """Whole blocks from rows of a forward's K are rounded to bf16, then quantized per channel."""
    g = torch.Generator().manual_seed(2)
    B, D = 16, 64
    x = (torch.randn(48, 2, D, generator=g) * 2).to("cuda", dtype)
    rows = torch.tensor(list(range(16, 48)), device="cuda")
    dst = torch.tensor([5, 1], device="cuda")
    qp = torch.zeros(2, 8, B, D, dtype=torch.int8, device="cuda")
    sp = torch.zeros(2, 8, D, dtype=torch.float16, device="cuda")
    quantize_store_block_rows(x, rows, dst, qp, sp)
    tiles = paged_ref.bf16_round(as_np32(x[16:48])).reshape(2, B, 2, D).transpose(2, 0, 1, 3)  # [H, n, B, D]
    q_ref, s_ref = paged_ref.quantize_per_channel(tiles, axis=2)
    assert np.array_equal(qp[:, dst].cpu().numpy(), q_ref)
    assert np.array_equal(bits16(sp[:, dst].cpu().numpy()), bits16(s_ref))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
def test_store_tokens_is_exact(dtype):
    """The scatter store writes exactly the values (and the bf16 rounding of fp32 values) into their slots."""
    g = torch.Generator().manual_seed(3)
    x = torch.randn(40, 2, 64, generator=g).to("cuda", dtype)
    y = torch.randn(40, 2, 64, generator=g).to("cuda", dtype)
    blocks = torch.randperm(30, generator=g)[:40 // 16 + 1].repeat_interleave(16)[:40].cuda()
    offsets = (torch.arange(40) % 16).cuda()
    pk = torch.zeros(2, 30, 16, 64, dtype=dtype, device="cuda")
    pv = torch.zeros_like(pk)
    store_tokens(x, blocks, offsets, pk, x2=y, pool2=pv)
    assert torch.equal(pk[:, blocks, offsets], x.transpose(0, 1))
    assert torch.equal(pv[:, blocks, offsets], y.transpose(0, 1))
    # K and V as views of one fused projection output with different row strides (as the model passes them)
    fused = torch.randn(40, 19, 64, generator=g).to("cuda", dtype)
    k_view, v_view = fused[:, 14:16], fused[:, 17:19]
    assert k_view.stride() != x.stride()
    store_tokens(x, blocks, offsets, pk, x2=v_view, pool2=pv)
    assert torch.equal(pk[:, blocks, offsets], x.transpose(0, 1))
    assert torch.equal(pv[:, blocks, offsets], v_view.transpose(0, 1))
    store_tokens(k_view, blocks, offsets, pk, x2=v_view, pool2=pv)
    assert torch.equal(pk[:, blocks, offsets], k_view.transpose(0, 1))
    stage = torch.zeros(2, 4, 16, 64, dtype=torch.bfloat16, device="cuda")
    rows = torch.tensor([7, 3, 9], device="cuda")
    store_tokens(x, torch.tensor([2, 2, 0], device="cuda"), torch.tensor([5, 6, 15], device="cuda"), stage,
                 rows=rows)
    assert torch.equal(stage[:, [2, 2, 0], [5, 6, 15]], x[rows].transpose(0, 1).bfloat16())


# ---- INT8 caches: fused writes and decode ------------------------------------------------------------------------

def make_cache(fmt, num_blocks, B, dtype, cfg, n_stage=32):
    m = BlockManager(num_blocks, B)
    return m, QuantPagedKVCache(cfg, num_blocks, B, "cuda", dtype, "hip", fmt, m, n_stage=n_stage)


def write_chunks(m, cache, seq, k, v, chunks, layer=0):
    """Append k, v [n, H, d] for `seq` in the given chunk sizes, one forward (begin + write) per chunk."""
    pos = m.seq_len(seq) if seq in m.seq_ids() else 0
    if seq not in m.seq_ids():
        m.allocate(seq, 0)
    i = 0
    for n in chunks:
        m.append_slots(seq, n)
        meta = build_metadata(m, [(seq, pos, n)], cache.k.device)
        cache.begin(n, meta)
        cache.write(layer, k[i:i + n], v[i:i + n])
        pos, i = pos + n, i + n


def tiny_cfg(Hq, Hkv, D):
    return ModelConfig(vocab_size=10, hidden_size=Hq * D, intermediate_size=16, num_layers=1, num_q_heads=Hq,
                       num_kv_heads=Hkv, head_dim=D)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16], ids=["bf16", "fp32", "fp16"])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("explicit_dst", [False, True], ids=["dst_from_offsets", "dst_given"])
def test_kchan_write_rows_equals_the_three_calls(dtype, D, explicit_dst):
    """Format B's one-launch decode write (V per token, K staged as bf16, completed blocks quantized per channel)
    leaves every pool equal bit for bit to quantize_store_tokens + store_tokens + quantize_store_blocks, for rows
    in slots of their own, with offsets 0, 15 (block completed) and between, over staging slots holding earlier
    tokens; with explicit destinations, some rows quantize into blocks of their own choosing, others into none."""
    g = torch.Generator().manual_seed(11)
    H, N, B, n_stage, T = 2, 64, 16, 24, 13
    big = (torch.randn(T, 2 * H, D, generator=g) * 3).to("cuda", dtype)
    k, v = big[:, :H], big[:, H:]  # strided rows
    blocks = torch.randperm(N, generator=g)[:T].cuda()
    offsets = torch.tensor([15, 0, 7, 15, 3, 15, 14, 1, 15, 9, 15, 12, 2]).cuda()
    slots = torch.randperm(n_stage, generator=g)[:T].cuda()
    stage0 = (torch.randn(H, n_stage, B, D, generator=g) * 2).bfloat16().cuda()
    pools0 = [torch.randint(-127, 128, (H, N, B, D), generator=g, dtype=torch.int8).cuda(),
              torch.rand(H, N, B, generator=g).half().cuda(),
              torch.randint(-127, 128, (H, N, B, D), generator=g, dtype=torch.int8).cuda(),
              torch.rand(H, N, D, generator=g).half().cuda()]
    if explicit_dst:
        dst = torch.full((T,), -1, dtype=torch.int64)
        dst[::2] = torch.randperm(N, generator=g)[:(T + 1) // 2]
        dst = dst.cuda()
    else:
        dst = None
    # the three calls
    vq, vs, kq, ks = (t.clone() for t in pools0)
    stage = stage0.clone()
    quantize_store_tokens(v, blocks, offsets, vq, vs)
    store_tokens(k, slots, offsets, stage)
    quantize = dst >= 0 if explicit_dst else offsets == B - 1
    quantize_store_blocks(stage, slots[quantize], (dst if explicit_dst else blocks)[quantize], kq, ks)
    # one launch
    vq2, vs2, kq2, ks2 = (t.clone() for t in pools0)
    stage2 = stage0.clone()
    kchan_write_rows(k, v, blocks, offsets, slots, dst, vq2, vs2, kq2, ks2, stage2)
    torch.cuda.synchronize()
    assert int(quantize.sum()) >= 5
    for a, b in ((vq, vq2), (vs, vs2), (kq, kq2), (ks, ks2), (stage, stage2)):
        assert torch.equal(a, b)


def test_kchan_decode_steps_match_torch_cache():
    """Several sequences decoding together through format B's cache: the one-launch decode write (taken for every
    step after the prefill) leaves the same pools, scales and staging as the torch quantizer path over 40 steps,
    with blocks completing at different steps and a sequence freed and replaced midway."""
    cfg = tiny_cfg(14, 2, 64)
    g = torch.Generator().manual_seed(5)
    prompts = {0: 5, 1: 16, 2: 29, 3: 1}
    states = []
    for fused in (False, True):
        m, cache = make_cache("int8-kchannel", 64, 16, torch.bfloat16, cfg, n_stage=16)
        cache.fused_writes = fused
        gg = torch.Generator().manual_seed(6)
        pos = {}
        for s, n in prompts.items():
            kv = torch.randn(2, n, 2, 64, generator=gg).bfloat16().cuda()
            write_chunks(m, cache, s, kv[0], kv[1], [n])
            pos[s] = n
        used_fused = 0
        for step in range(40):
            if step == 17:  # sequence 1 finishes; sequence 9 starts with a 3-token prompt
                m.free(1)
                del pos[1]
                kv = torch.randn(2, 3, 2, 64, generator=gg).bfloat16().cuda()
                write_chunks(m, cache, 9, kv[0], kv[1], [3])
                pos[9] = 3
            seqs = sorted(pos)
            for s in seqs:
                m.append_slots(s, 1)
            meta = build_metadata(m, [(s, pos[s], 1) for s in seqs], "cuda")
            cache.begin(len(seqs), meta)
            used_fused += cache._rows_write is not None
            kv = torch.randn(2, len(seqs), 2, 64, generator=gg).bfloat16().cuda()
            cache.write(0, kv[0], kv[1])
            for s in seqs:
                pos[s] += 1
        torch.cuda.synchronize()
        assert used_fused == 40
        states.append([cache.k.clone(), cache.v.clone(), cache.k_scale.clone(), cache.v_scale.clone(),
                       cache.stage.clone()])
    for a, b in zip(*states):
        assert torch.equal(a, b)


@pytest.mark.parametrize("fmt", FMTS)
def test_fused_cache_writes_match_reference_cache(fmt):
    """A chunked fill [5, 40, 1, 1, 30, 1, 5] (partial, interior, single-token, boundary) through the fused HIP
    writes leaves the same pools as the torch quantizer path (reference tests/test_quant_cache.py:392-410)."""
    cfg = tiny_cfg(14, 2, 64)
    g = torch.Generator().manual_seed(2)
    k = torch.randn(83, 2, 64, generator=g).bfloat16().cuda()
    v = torch.randn(83, 2, 64, generator=g).bfloat16().cuda()
    pools = []
    for fused in (False, True):
        m, cache = make_cache(fmt, 12, 16, torch.bfloat16, cfg)
        cache.fused_writes = fused
        write_chunks(m, cache, 0, k, v, [5, 40, 1, 1, 30, 1, 5])
        torch.cuda.synchronize()
        pools.append([cache.k.clone(), cache.v.clone(), cache.k_scale.clone(), cache.v_scale.clone()]
                     + ([cache.stage.clone()] if fmt == "int8-kchannel" else []))
    for a, b in zip(*pools):
        assert torch.equal(a, b)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("heads", list(HEADS))
@pytest.mark.parametrize("B", [8, 16, 32])
@pytest.mark.parametrize("splits", [1, None], ids=["single", "auto"])
def test_kernel_matches_dequantized_reference(dtype, fmt, heads, B, splits):
    """The decode kernel with fused dequantization equals attention over the cache's own dequantized K/V, for a
    ragged batch with partial last blocks (format B reads them from staging)."""
    Hq, Hkv, D = HEADS[heads]
    lengths = [1, 15, 16, 17, 33, 100, 700]
    m, cache = make_cache(fmt, sum(-(-n // B) for n in lengths) * 2, B, dtype, tiny_cfg(Hq, Hkv, D))
    g = torch.Generator().manual_seed(0)
    for s in range(len(lengths)):
        m.allocate(s, 0)
    outlier = 1 + 5 * (torch.arange(D) % 13 == 0)
    for s, n in enumerate(lengths):
        k = (torch.randn(n, Hkv, D, generator=g) * outlier).to("cuda", dtype)
        v = torch.randn(n, Hkv, D, generator=g).to("cuda", dtype)
        write_chunks(m, cache, s, k, v, [n] if n < 50 else [37, n - 37])
    meta = build_metadata(m, [(s, n - 1, 1) for s, n in enumerate(lengths)], "cuda")
    cache.begin(len(lengths), meta)
    q = torch.randn(len(lengths), Hq, D, generator=g).to("cuda", dtype)
    print(f"case {fmt} {heads} B={B} {dtype} splits={splits}", flush=True)
    out = paged_decode_attention(q, cache.k[0], cache.v[0], meta.block_tables, meta.context_lens_t, D ** -0.5,
                                 max(lengths), num_splits=splits, quant=cache._kernel_quant(0))
    got = out.double().cpu().numpy()
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    # The oracle's fp32 dequantization of the cache's own int8 pools (what the kernel computes with).
    kq, vq = cache.k[0].cpu().numpy(), cache.v[0].cpu().numpy()
    ks, vs = cache.k_scale[0].cpu().numpy(), cache.v_scale[0].cpu().numpy()
    v_deq = paged_ref.dequant_tokens(vq, vs)
    k_deq = paged_ref.dequant_tokens(kq, ks) if fmt == "int8" else None
    if fmt == "int8-kchannel":
        stage, tails = as_np32(cache.stage[0]), cache._tails_dec.cpu().numpy()
    for s, n in enumerate(lengths):
        kd, vd = cache.gather(0, s)  # dequantized in the model dtype, as the reference's gather
        ref64 = paged_ref.attend_one(as_np32(q[s]), as_np32(kd), as_np32(vd), D ** -0.5, np.float64)
        np.testing.assert_allclose(got[s], ref64, rtol=tol, atol=tol, err_msg=f"sequence {s} (length {n})")
        if dtype == torch.bfloat16:
            table = meta.block_ids_cpu[s]
            k32 = paged_ref.gather(k_deq, table, n) if fmt == "int8" else \
                paged_ref.gather_kchannel(kq, ks, stage, table, n, int(tails[s]))
            ref32 = paged_ref.attend_one(as_np32(q[s]), k32, paged_ref.gather(v_deq, table, n), D ** -0.5,
                                         np.float32)
            assert np.abs(got[s] - ref32).max() <= 8e-3, f"sequence {s}"


# ---- INT8 decode kernels, forced: MFMA and VALU, both formats, and constant channel scales ------------------------

def int8_case(Hq, Hkv, D, lengths, fmt, seed, const_channels=False, v_mag=1.0, k_mag=1.0):
    """INT8 pools built by the HIP quantizers (through the cache), outlier channels in K, and the oracle's fp32
    dequantized K/V per sequence. Returns (q, cache, meta, k32 list, v32 list). The closing step re-writes every
    sequence's last token, so format B stages one block per sequence: twice as many staging slots as sequences
    (the reference engine's n_stage = 2 max_num_seqs)."""
    B = 16
    m, cache = make_cache(fmt, sum(-(-n // B) for n in lengths) * 2, B, torch.bfloat16, tiny_cfg(Hq, Hkv, D),
                          n_stage=max(32, 2 * len(lengths)))
    g = torch.Generator().manual_seed(seed)
    outlier = torch.ones(Hkv, D)
    for h in range(Hkv):
        outlier[h, torch.randperm(D, generator=g)[:4]] = 20 + 48 * torch.rand(4, generator=g)
    for s in range(len(lengths)):
        m.allocate(s, 0)
    for s, n in enumerate(lengths):
        k = (torch.randn(n, Hkv, D, generator=g) * outlier * k_mag).to("cuda", torch.bfloat16)
        v = (torch.randn(n, Hkv, D, generator=g) * v_mag).to("cuda", torch.bfloat16)
        write_chunks(m, cache, s, k, v, [n] if n < 50 else [37, n - 37])
    meta = build_metadata(m, [(s, n - 1, 1) for s, n in enumerate(lengths)], "cuda")
    cache.begin(len(lengths), meta)
    q = torch.randn(len(lengths), Hq, D, generator=g).to("cuda", torch.bfloat16)
    kq, vq = cache.k[0].cpu().numpy(), cache.v[0].cpu().numpy()
    ks, vs = cache.k_scale[0].cpu().numpy(), cache.v_scale[0].cpu().numpy()
    quant = cache._kernel_quant(0)
    if const_channels:
        # one fp32 scale per (head, channel) for every block: re-quantize K with it (zero block stride)
        chan = (np.abs(paged_ref.dequant_channels(kq, ks)).max(axis=(1, 2)) / 127).astype(np.float32)  # [H, D]
        chan = np.maximum(chan, 1e-6)
        kq = np.clip(np.rint(paged_ref.dequant_channels(kq, ks) / chan[:, None, None, :]), -127, 127).astype(np.int8)
        cache.k[0].copy_(torch.from_numpy(kq))
        ks_t = torch.from_numpy(chan).cuda()[:, None, :].expand(Hkv, cache.k.shape[2], D)
        quant = type(quant)(2, ks_t, quant.v_scale, quant.stage, quant.tail_slots)
        k_deq = kq.astype(np.float32) * chan[:, None, None, :]
    v_deq = paged_ref.dequant_tokens(vq, vs)
    if fmt == "int8":
        k_deq = paged_ref.dequant_tokens(kq, ks)
    k32, v32 = [], []
    tails = cache._tails_dec.cpu().numpy() if fmt == "int8-kchannel" else None
    stage = as_np32(cache.stage[0]) if fmt == "int8-kchannel" else None
    for s, n in enumerate(lengths):
        table = meta.block_ids_cpu[s]
        if fmt == "int8" or const_channels:
            kk = paged_ref.gather(k_deq, table, n)
            if fmt == "int8-kchannel" and n % B:  # the partial last block still comes from staging
                kk = kk.copy()
                kk[:, (n // B) * B:] = stage[:, int(tails[s]), :n % B]
        else:
            kk = paged_ref.gather_kchannel(kq, ks, stage, table, n, int(tails[s]))
        k32.append(kk)
        v32.append(paged_ref.gather(v_deq, table, n))
    return q, cache, meta, quant, k32, v32


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("heads", list(HEADS))
@pytest.mark.parametrize("impl", ["mfma", "valu"])
@pytest.mark.parametrize("splits", [1, 3, None, "list"], ids=["single", "split3", "auto", "worklist"])
def test_int8_kernels_match_oracle(fmt, heads, impl, splits):
    """Both INT8 kernels against the oracle's fp32 dequantize-then-attend, outlier K channels (4 per head scaled
    by U[20, 68], as config C4), ragged lengths with partial last blocks: every element within 8e-3 of the oracle or
    a bf16 rounding of it; the fp32-output VALU kernel within 8e-3 everywhere."""
    Hq, Hkv, D = HEADS[heads]
    lengths = [1, 15, 16, 17, 33, 100, 700, 2100]
    q, cache, meta, quant, k32, v32 = int8_case(Hq, Hkv, D, lengths, fmt, seed=5)
    print(f"case {fmt} {heads} {impl} splits={splits}", flush=True)
    lists = dict(host_context_lens=lengths, work_list="on") if splits == "list" else {}
    if splits == "list":
        splits = None
    out = paged_decode_attention(q, cache.k[0], cache.v[0], meta.block_tables, meta.context_lens_t, D ** -0.5,
                                 max(lengths), num_splits=splits, quant=quant, impl=impl, **lists)
    got = out.double().cpu().numpy()
    ref = np.stack([paged_ref.attend_one(as_np32(q[s]), k32[s], v32[s], D ** -0.5, np.float32)
                    for s in range(len(lengths))])
    # 8e-3 max-abs, or one of the two bf16 values bracketing the oracle's (outlier channels make
    # the softmax peaked and |out| reach a few units, where half a bf16 unit of the output approaches 8e-3).
    assert_decode_close(got, ref, f"int8 {fmt} {heads} {impl} splits={splits}")
    if impl == "valu":  # the same case with an fp32 query and output: the fp32 math itself, no rounding allowance
        out32 = paged_decode_attention(q.float(), cache.k[0], cache.v[0], meta.block_tables, meta.context_lens_t,
                                       D ** -0.5, max(lengths), num_splits=splits, quant=quant, **lists)
        err32 = np.abs(out32.double().cpu().numpy() - ref).max()
        assert err32 <= 8e-3, f"fp32 max-abs {err32:.3e}"


@pytest.mark.parametrize("heads", list(HEADS))
@pytest.mark.parametrize("impl", ["valu_stream", "valu_dot2"])
@pytest.mark.parametrize("splits", [1, None], ids=["single", "auto"])
def test_int8_valu_streaming_kernels_match_oracle(heads, impl, splits):
    """The VALU streaming kernels on per-token INT8 pools (codes used with a +128 bias that the score and the
    output remove again), against the oracle's dequantize-then-attend with outlier K channels."""
    Hq, Hkv, D = HEADS[heads]
    lengths = [1, 15, 16, 17, 33, 100, 700, 2100]
    q, cache, meta, quant, k32, v32 = int8_case(Hq, Hkv, D, lengths, "int8", seed=15)
    print(f"case int8 {heads} {impl} splits={splits}", flush=True)
    out = paged_decode_attention(q, cache.k[0], cache.v[0], meta.block_tables, meta.context_lens_t, D ** -0.5,
                                 max(lengths), num_splits=splits, quant=quant, impl=impl)
    ref = np.stack([paged_ref.attend_one(as_np32(q[s]), k32[s], v32[s], D ** -0.5, np.float32)
                    for s in range(len(lengths))])
    assert_decode_close(out.double().cpu().numpy(), ref, f"int8 {heads} {impl} splits={splits}")


@pytest.mark.parametrize("fmt", FMTS)
def test_int8_context_longer_than_one_split_holds(fmt):
    """The INT8 kernels stage the token scales of at most 4,096 tokens per split: a 9,000-token sequence asked
    for a single pass is cut into three splits (and into pieces of at most 4,096 tokens on the work list)."""
    Hq, Hkv, D = HEADS["1.5B"]
    lengths = [9000, 17]
    q, cache, meta, quant, k32, v32 = int8_case(Hq, Hkv, D, lengths, fmt, seed=8)
    ref = np.stack([paged_ref.attend_one(as_np32(q[s]), k32[s], v32[s], D ** -0.5, np.float32)
                    for s in range(len(lengths))])
    for splits, lists in ((1, {}), (None, dict(host_context_lens=lengths, work_list="on"))):
        print(f"case {fmt} lengths {lengths} splits={splits} {lists.get('work_list', 'grid')}", flush=True)
        out = paged_decode_attention(q, cache.k[0], cache.v[0], meta.block_tables, meta.context_lens_t, D ** -0.5,
                                     max(lengths), num_splits=splits, quant=quant, impl="mfma", **lists)
        got = out.double().cpu().numpy()
        assert_decode_close(got, ref, f"int8 {fmt} long context splits={splits}")


@pytest.mark.parametrize("heads", list(HEADS))
@pytest.mark.parametrize("impl", ["mfma", "valu"])
def test_int8_constant_channel_scales(heads, impl):
    """Format B with one fp32 K scale per (head, channel) shared by every block (a zero block stride): the
    literal reading of config C4(a)."""
    Hq, Hkv, D = HEADS[heads]
    lengths = [1, 17, 64, 300, 1000]
    q, cache, meta, quant, k32, v32 = int8_case(Hq, Hkv, D, lengths, "int8-kchannel", seed=6,
                                               const_channels=True)
    assert quant.k_scale.stride(1) == 0 and quant.k_scale.dtype == torch.float32
    out = paged_decode_attention(q, cache.k[0], cache.v[0], meta.block_tables, meta.context_lens_t, D ** -0.5,
                                 max(lengths), quant=quant, impl=impl)
    got = out.double().cpu().numpy()
    ref = np.stack([paged_ref.attend_one(as_np32(q[s]), k32[s], v32[s], D ** -0.5, np.float32)
                    for s in range(len(lengths))])
    assert_decode_close(got, ref, f"int8 constant channel scales {heads} {impl}")


@pytest.mark.parametrize("impl", ["mfma", "valu"])
def test_kchannel_tail_slots_are_clamped_and_counted(impl):
    """Format B's tail slots come from the caller: a slot past the staging pool reads the pool's last slot (the
    kernels clamp it; wrong results, no access outside the staging pool), and a tail_slots vector shorter than the
    batch is refused on the host."""
    from engine.hip_decode import QuantKV

    Hq, Hkv, D = HEADS["0.5B"]
    lengths = [17, 100, 33]
    q, cache, meta, quant, k32, v32 = int8_case(Hq, Hkv, D, lengths, "int8-kchannel", seed=12)
    n_stage = cache.stage.shape[2]
    bad_tails = torch.tensor([n_stage + 5, 2 ** 30, -1], dtype=torch.int32, device="cuda")
    print(f"case tail clamp {impl}", flush=True)
    out = paged_decode_attention(q, cache.k[0], cache.v[0], meta.block_tables, meta.context_lens_t, D ** -0.5,
                                 max(lengths), num_splits=1, impl=impl,
                                 quant=QuantKV(2, quant.k_scale, quant.v_scale, quant.stage, bad_tails))
    torch.cuda.synchronize()
    # the oracle with the clamped slots: the last staging slot for the first two sequences, none for the third
    kq, ks = cache.k[0].cpu().numpy(), cache.k_scale[0].cpu().numpy()
    stage = as_np32(cache.stage[0])
    ref = []
    for s, (n, t) in enumerate(zip(lengths, [n_stage - 1, n_stage - 1, -1])):
        table = meta.block_ids_cpu[s]
        if t < 0:  # a -1 tail reads the quantized blocks only (the partial block's rows come from the pool)
            kk = paged_ref.gather(paged_ref.dequant_channels(kq, ks), table, n)
        else:
            kk = paged_ref.gather_kchannel(kq, ks, stage, table, n, t)
        ref.append(paged_ref.attend_one(as_np32(q[s]), kk, v32[s], D ** -0.5, np.float32))
    assert_decode_close(out.double().cpu().numpy(), np.stack(ref), f"tail clamp {impl}")
    with pytest.raises(ValueError):
        paged_decode_attention(q, cache.k[0], cache.v[0], meta.block_tables, meta.context_lens_t, D ** -0.5,
                               max(lengths), quant=QuantKV(2, quant.k_scale, quant.v_scale, quant.stage,
                                                           bad_tails[:2]))


@pytest.mark.parametrize("fmt,const", [("int8", False), ("int8-kchannel", False), ("int8-kchannel", True)],
                         ids=["per_token", "kchannel", "kchannel_const"])
@pytest.mark.parametrize("heads", list(HEADS))
def test_int8_mfma_query_magnitudes(fmt, const, heads):
    """The INT8 MFMA kernels hold the query in fp16: heads whose |q| reaches 3e5 (past fp16's 65504) or stays
    under 1e-6 (fp16 subnormals) are scaled by a power of two first, so they meet the same bound against the
    oracle's fp32 attention as ordinary heads; every other head of the same call keeps its plain scale."""
    Hq, Hkv, D = HEADS[heads]
    lengths = [1, 17, 300, 1000]
    q, cache, meta, quant, k32, v32 = int8_case(Hq, Hkv, D, lengths, fmt, seed=8, const_channels=const)
    mag = torch.ones(Hq, 1, device="cuda")
    mag[0], mag[1], mag[-1] = 3e5 / 4, 1e-7, 300.0  # |q| about 4 sigma: 3e5, 4e-7, 1.2e3
    q = (q.float() * mag).bfloat16()
    print(f"case int8 query magnitudes {fmt} const={const} {heads}", flush=True)
    out = paged_decode_attention(q, cache.k[0], cache.v[0], meta.block_tables, meta.context_lens_t, D ** -0.5,
                                 max(lengths), quant=quant, impl="mfma")
    got = out.double().cpu().numpy()
    assert np.isfinite(got).all()
    ref = np.stack([paged_ref.attend_one(as_np32(q[s]), k32[s], v32[s], D ** -0.5, np.float32)
                    for s in range(len(lengths))])
    assert_decode_close(got, ref, f"int8 query magnitudes {fmt} const={const} {heads}")


@pytest.mark.parametrize("v_mag", [2.0 ** -8, 2.0 ** -14], ids=["v_2^-8", "v_2^-14"])
@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("heads", list(HEADS))
def test_int8_mfma_small_v_scales(v_mag, fmt, heads):
    """The INT8 MFMA kernels form P' = p s_v in fp16, whose exponent range is far narrower than the reference's
    fp32 P' (engine/triton_decode.py:126-130): V of magnitude 2^-8 (scales about 1e-4) or 2^-14 (fp16-subnormal
    scales) would put most P' among fp16 subnormals. Each split scales p by a power of two chosen from its largest
    V scale, so the output divided by the V magnitude meets the unit-scale bound against the oracle's fp32
    dequantize-then-attend of the same cache, divided likewise (the factor is a power of two: exact)."""
    Hq, Hkv, D = HEADS[heads]
    lengths = [1, 17, 300, 1000, 3000]
    q, cache, meta, quant, k32, v32 = int8_case(Hq, Hkv, D, lengths, fmt, seed=21, v_mag=v_mag)
    ref = np.stack([paged_ref.attend_one(as_np32(q[s]), k32[s], v32[s], D ** -0.5, np.float32)
                    for s in range(len(lengths))])
    for splits in (1, None):
        print(f"case int8 small V {v_mag:g} {fmt} {heads} splits={splits}", flush=True)
        out = paged_decode_attention(q, cache.k[0], cache.v[0], meta.block_tables, meta.context_lens_t, D ** -0.5,
                                     max(lengths), num_splits=splits, quant=quant, impl="mfma")
        got = out.double().cpu().numpy()
        assert np.isfinite(got).all()
        assert_decode_close(got / v_mag, ref / v_mag, f"int8 V x {v_mag:g} {fmt} {heads} splits={splits}")


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("heads", list(HEADS))
def test_int8_mfma_small_k_scales(fmt, heads):
    """K of magnitude 2^-12 with the query 2^12 larger (the same scores): format B's channel scales of the
    ordinary channels are then fp16 subnormals (about 8e-6) and the per-token format's token scales small, so the
    query's fp16 product with the scale (format B: an exact high part and a low part from one fused multiply-add)
    runs where its high part may itself be inexact. The output meets the unit-scale bound against the oracle's
    fp32 dequantize-then-attend of the same cache and query."""
    Hq, Hkv, D = HEADS[heads]
    lengths = [1, 17, 300, 1000, 3000]
    q, cache, meta, quant, k32, v32 = int8_case(Hq, Hkv, D, lengths, fmt, seed=23, k_mag=2.0 ** -12)
    q = (q.float() * 2.0 ** 12).bfloat16()  # exact: a power of two
    ref = np.stack([paged_ref.attend_one(as_np32(q[s]), k32[s], v32[s], D ** -0.5, np.float32)
                    for s in range(len(lengths))])
    for splits in (1, None):
        print(f"case int8 small K {fmt} {heads} splits={splits}", flush=True)
        out = paged_decode_attention(q, cache.k[0], cache.v[0], meta.block_tables, meta.context_lens_t, D ** -0.5,
                                     max(lengths), num_splits=splits, quant=quant, impl="mfma")
        got = out.double().cpu().numpy()
        assert np.isfinite(got).all()
        assert_decode_close(got, ref, f"int8 K x 2^-12 {fmt} {heads} splits={splits}")


@pytest.mark.parametrize("fmt", FMTS)
def test_c4_quantize_store_of_64_new_tokens_is_exact(fmt):
    """Config C4's write: 64 sequences of the 1.5B shape (2 KV heads, head_dim 128) each append one token through
    the cache, K with 4 of 128 channels per head scaled by U[20, 68] (C4's outlier channels), K and V strided views
    of one fused projection output, one with a zero vector. Codes and fp16 scale bits equal the oracle's quantizer
    (reference tests/test_quant_cache.py:246-266): per token for V and format A's K; for format B's K, the staged
    bf16 rows of a partial block, and the per-channel codes and scales of every block the new token completes,
    over that block's 16 rows."""
    Hq, Hkv, D, B, S = 12, 2, 128, 16, 64
    g = torch.Generator().manual_seed(31)
    outlier = torch.ones(Hkv, D)
    for h in range(Hkv):
        outlier[h, torch.randperm(D, generator=g)[:4]] = 20 + 48 * torch.rand(4, generator=g)
    before = torch.randint(0, 48, (S,), generator=g).tolist()
    for s in range(0, S, 4):
        before[s] = 16 * (s % 3) + 15  # these sequences' new token completes a block
    m, cache = make_cache(fmt, S * 4 + 8, B, torch.bfloat16, tiny_cfg(Hq, Hkv, D), n_stage=2 * S)
    hist_k = {}
    for s, n in enumerate(before):
        m.allocate(s, 0)
        kx = (torch.randn(max(n, 1), Hkv, D, generator=g) * outlier).bfloat16()
        hist_k[s] = kx[:n]
        if n:
            write_chunks(m, cache, s, kx[:n].cuda(), torch.randn(n, Hkv, D, generator=g).bfloat16().cuda(), [n])
    qkv = torch.randn(S, Hq + 2 * Hkv, D, generator=g)
    qkv[:, Hq:Hq + Hkv] *= outlier
    qkv = qkv.bfloat16().cuda()
    k_new, v_new = qkv[:, Hq:Hq + Hkv], qkv[:, Hq + Hkv:]
    k_new[9, 1] = 0
    v_new[9, 0] = 0
    for s in range(S):
        m.append_slots(s, 1)
    meta = build_metadata(m, [(s, before[s], 1) for s in range(S)], "cuda")
    print(f"case c4 store {fmt} sequences={S} completed blocks={sum(1 for n in before if n % B == B - 1)}", flush=True)
    cache.begin(S, meta)
    cache.write(0, k_new, v_new)
    torch.cuda.synchronize()
    slots = np.asarray(meta.slot_mapping.cpu().numpy(), dtype=np.int64)
    blk, off = torch.from_numpy(slots // B).cuda(), torch.from_numpy(slots % B).cuda()
    v_ref, vs_ref = paged_ref.quantize_per_token(as_np32(v_new))
    assert np.array_equal(cache.v[0][:, blk, off].transpose(0, 1).cpu().numpy(), v_ref)
    assert np.array_equal(bits16(cache.v_scale[0][:, blk, off].t().cpu().numpy()), bits16(vs_ref))
    if fmt == "int8":
        k_ref, ks_ref = paged_ref.quantize_per_token(as_np32(k_new))
        assert np.array_equal(cache.k[0][:, blk, off].transpose(0, 1).cpu().numpy(), k_ref)
        assert np.array_equal(bits16(cache.k_scale[0][:, blk, off].t().cpu().numpy()), bits16(ks_ref))
        return
    kq, ks, stage = cache.k[0].cpu().numpy(), cache.k_scale[0].cpu().numpy(), cache.stage[0].cpu()
    done = 0
    for s in range(S):
        b, o = int(slots[s] // B), int(slots[s] % B)
        rows = torch.cat([hist_k[s][before[s] - o:], k_new[s:s + 1].cpu()])  # the block's rows so far, [o + 1, H, D]
        if o == B - 1:  # completed: quantized per channel from its 16 bf16 rows
            q_ref, s_ref = paged_ref.quantize_per_channel(as_np32(rows.transpose(0, 1)), axis=1)
            assert np.array_equal(kq[:, b], q_ref), s
            assert np.array_equal(bits16(ks[:, b]), bits16(s_ref)), s
            done += 1
        else:  # partial: the rows wait in the block's staging slot, rounded to bf16
            slot = cache._stage_of[b]
            assert torch.equal(stage[:, slot, :o + 1], rows.transpose(0, 1)), s
    assert done == sum(1 for n in before if n % B == B - 1) >= S // 4


def test_kchannel_two_class_split_grid_with_ragged_lengths():
    """Format B on a grid of exactly two workgroups per CU (64 sequences x 2 KV heads x 4 splits on 256 CUs) takes
    splits of two lengths: the first CU-count workgroups (the earlier-dispatched of each CU's pair) get the longer
    ones. Sequences whose contexts end inside the long splits, at their boundaries and inside the short ones all
    match the oracle's dequantize-then-attend, through the fused merge and the separate combine kernel."""
    from engine.hip_decode import device_cu_count

    cu = device_cu_count()
    if cu % 128:
        pytest.skip(f"{cu} CUs: 128 (sequence, KV head) pairs do not divide the CU count")
    Hq, Hkv, D = HEADS["1.5B"]
    g = torch.Generator().manual_seed(41)
    lengths = torch.randint(1, 4097, (64,), generator=g).tolist()
    lengths[:8] = [4096, 1, 1280, 1281, 2560, 2561, 3000, 17]
    q, cache, meta, quant, k32, v32 = int8_case(Hq, Hkv, D, lengths, "int8-kchannel", seed=42)
    ref = np.stack([paged_ref.attend_one(as_np32(q[s]), k32[s], v32[s], D ** -0.5, np.float32)
                    for s in range(len(lengths))])
    from engine.hip_decode import split_grid

    splits, chunk, chunk_old, n_old = split_grid(64, Hkv, 4096, 2 * cu // 128, 2)
    print(f"grid: {splits} splits, {n_old} of {chunk_old} tokens, the rest {chunk}", flush=True)
    assert splits == 2 * cu // 128 and n_old == cu // 128 and chunk_old > chunk and chunk_old % 128 == 0
    assert n_old * chunk_old + (splits - n_old) * chunk >= 4096
    assert split_grid(64, Hkv, 4096, 2 * cu // 128, 1)[3] == 0  # the per-token format keeps equal splits
    for combine in ("fused", "kernel"):
        print(f"case kchannel two-class grid, 64 ragged sequences, {combine}", flush=True)
        out = paged_decode_attention(q, cache.k[0], cache.v[0], meta.block_tables, meta.context_lens_t, D ** -0.5,
                                     4096, num_splits=2 * cu // 128, quant=quant, impl="mfma", combine=combine)
        assert_decode_close(out.double().cpu().numpy(), ref, f"kchannel two-class grid {combine}")
