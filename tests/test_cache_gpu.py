"""The drop-in interface end to end on the GPU: begin / write / attend of PagedKVCache and QuantPagedKVCache with
attn_backend "triton" (the reference engine's default name, served by the HIP kernels) over mixed batches of
decode rows and prefill chunks, as engine/model.py:145-146 drives it (reference tests/test_paged.py:186-205).

Checked against the oracle: each row's softmax attention over the cache contents gathered back to fp32 (for the
INT8 caches, the dequantized contents), causal within a chunk. Tolerances: fp32 caches 1e-5; bf16 decode rows
(the HIP decode kernel) 8e-3 max-abs; bf16 prefill rows (the HIP prefill kernel) within 8e-3 or a bf16 rounding
of the oracle (`cases.assert_decode_close`), for the INT8 caches over the gather at the model dtype, since the
prefill kernel dequantizes K/V to bf16 as the reference's gather path does (engine/quant_cache.py:179-190).
"""

import numpy as np
import pytest
import torch

from cases import assert_decode_close, fragmented_manager
from engine.config import ModelConfig
from engine.paged_cache import PagedKVCache, build_metadata
from engine.quant_cache import QuantPagedKVCache
from oracle import paged_ref

pytestmark = pytest.mark.gpu

CFG = {64: ModelConfig(vocab_size=97, hidden_size=896, intermediate_size=64, num_layers=2, num_q_heads=14,
                       num_kv_heads=2, head_dim=64),
       128: ModelConfig(vocab_size=97, hidden_size=1536, intermediate_size=64, num_layers=2, num_q_heads=12,
                        num_kv_heads=2, head_dim=128)}


def forward(m, cache, batch, layer, gen, dtype):
    """One forward over batch [(seq, start, n)]: metadata, begin, write random k/v, attend random q."""
    cfg = cache.cfg
    meta = build_metadata(m, batch, "cuda")
    T = meta.num_tokens
    cache.begin(T, meta)
    k = torch.randn(T, cfg.num_kv_heads, cfg.head_dim, generator=gen).to("cuda", dtype)
    v = torch.randn(T, cfg.num_kv_heads, cfg.head_dim, generator=gen).to("cuda", dtype)
    q = torch.randn(T, cfg.num_q_heads, cfg.head_dim, generator=gen).to("cuda", dtype)
    cache.write(layer, k, v)
    out = cache.attend(layer, q, meta.positions, cfg.head_dim ** -0.5)
    return meta, q, out


def reference(cache, meta, q, layer, gather_dtype=torch.float32):
    """Oracle: per sequence, gather the cache back (INT8 caches dequantized to gather_dtype) and attend causally
    in fp32."""
    cfg, d = cache.cfg, cache.cfg.head_dim
    saved, cache.dtype = cache.dtype, gather_dtype
    try:
        rows = []
        for i in range(meta.num_seqs):
            k, v = cache.gather(layer, i)
            k, v = k.float().cpu().numpy(), v.float().cpu().numpy()
            a, b = meta.query_starts[i], meta.query_starts[i + 1]
            ctx = meta.context_lens[i]
            for r in range(a, b):
                n = ctx - (b - 1 - r)  # causal: the row at position ctx - 1 - (b - 1 - r) sees n keys
                rows.append(paged_ref.attend_one(q[r].float().cpu().numpy(), k[:, :n], v[:, :n], d ** -0.5,
                                                 np.float32))
    finally:
        cache.dtype = saved
    return np.stack(rows).reshape(len(rows), cfg.num_q_heads * d)


def check_rows(cache, meta, q, out, layer, dtype, what):
    ref = reference(cache, meta, q, layer)
    got = out.float().cpu().numpy()
    err = np.abs(got - ref)
    chunk = {r for a, b in zip(meta.query_starts, meta.query_starts[1:]) if b - a > 1 for r in range(a, b)}
    dec = np.array([r not in chunk for r in range(meta.num_tokens)])
    if dtype == torch.float32:
        assert err.max() <= 1e-5, f"{what}: {err.max():.3e}"
        return
    if dec.any():
        assert err[dec].max() <= 8e-3, f"{what}: decode rows {err[dec].max():.3e}"
    if not (~dec).any():
        return
    if isinstance(cache, QuantPagedKVCache):
        # the prefill kernel dequantizes K/V to the model dtype, as the reference's gather() does: the oracle
        # over that gather is held to the same bar
        ref = reference(cache, meta, q, layer, gather_dtype=dtype)
    assert_decode_close(got[~dec], ref[~dec], f"{what}: chunk rows")


def run_mixed(make_cache, dtype, D, seed):
    gen = torch.Generator().manual_seed(seed)
    m = fragmented_manager(256, 16, gen)
    cache = make_cache(m)
    print(f"case {type(cache).__name__} {getattr(cache, 'fmt', 'model')} {dtype} D={D} seed={seed}", flush=True)
    for layer in range(2):  # prompts only
        for s, n in ((1, 70), (2, 300), (3, 16)):
            if s not in m.seq_ids():
                m.allocate(s, n)
        meta, q, out = forward(m, cache, [(1, 0, 70), (2, 0, 300), (3, 0, 16)], layer, gen, dtype)
        torch.cuda.synchronize()
        check_rows(cache, meta, q, out, layer, dtype, f"prompts layer {layer}")
    for step in range(3):  # decode steps mixed with a prefill chunk of a new sequence
        for s in (1, 2, 3):
            m.append_slot(s)
        batch = [(1, m.seq_len(1) - 1, 1), (2, m.seq_len(2) - 1, 1), (3, m.seq_len(3) - 1, 1)]
        if step == 1:
            m.allocate(4, 0)
            m.append_slots(4, 21)
            batch.insert(1, (4, 0, 21))
        for layer in range(2):
            meta, q, out = forward(m, cache, batch, layer, gen, dtype)
            torch.cuda.synchronize()
            check_rows(cache, meta, q, out, layer, dtype, f"step {step} layer {layer}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
@pytest.mark.parametrize("D", [64, 128])
def test_paged_cache_mixed_batches(dtype, D):
    run_mixed(lambda m: PagedKVCache(CFG[D], 256, 16, "cuda", dtype, attn_backend="triton"), dtype, D, seed=D)


@pytest.mark.parametrize("fmt", ["int8", "int8-kchannel"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
@pytest.mark.parametrize("D", [64, 128])
def test_quant_cache_mixed_batches(fmt, dtype, D):
    run_mixed(lambda m: QuantPagedKVCache(CFG[D], 256, 16, "cuda", dtype, "triton", fmt, m, n_stage=16),
              dtype, D, seed=7 + D)


def test_model_mixed_batch_kernel_vs_gather():
    """The reference's tiny model shape (tests/tiny_model.py:7-10: 2 layers, 6 query heads over 2 KV heads, so a
    GQA group of 3, head_dim 16, hidden 96, MLP 160) in fp32 over 4-token blocks drives the cache as the reference's
    model does (fused QKV views as K and V, per-layer write then attend): one prefill chunk and two decode rows in
    one packed forward; the kernel backend's logits equal the gather backend's to fp32 summation order (reference
    tests/test_paged.py:186-205, which sets attn_backend after construction, as here)."""
    from engine.model import Qwen2Model

    tiny = ModelConfig(vocab_size=97, hidden_size=96, intermediate_size=160, num_layers=2, num_q_heads=6,
                       num_kv_heads=2, head_dim=16, rope_theta=10_000.0, max_position_embeddings=256)
    model = Qwen2Model(tiny, "cuda", torch.float32, seed=1, max_positions=128, std=0.1)
    outs = {}
    for backend in ("gather", "triton"):
        m = fragmented_manager(32, 4, torch.Generator().manual_seed(2))
        cache = PagedKVCache(tiny, 32, 4, "cuda", torch.float32)
        cache.attn_backend = backend
        for s, n in ((1, 9), (2, 30)):
            m.allocate(s, n)
            meta = build_metadata(m, [(s, 0, n)], "cuda")
            model.forward(torch.arange(n, device="cuda") % 97, meta.positions, cache, meta)
        m.allocate(0, 13)
        m.append_slot(1)
        m.append_slot(2)
        meta = build_metadata(m, [(1, 9, 1), (0, 0, 13), (2, 30, 1)], "cuda")
        ids = torch.tensor([5] + list(range(20, 33)) + [7], device="cuda")
        outs[backend] = model.forward(ids, meta.positions, cache, meta, last_only=False)
    torch.testing.assert_close(outs["triton"], outs["gather"], rtol=1e-5, atol=1e-5)
