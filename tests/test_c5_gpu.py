"""Config C5 on the GPU: the packed decode step of a Qwen2.5-0.5B-shaped model at batch 512 with contexts
U[1024, 16384], through the caches' begin / write / attend (the reference's step: engine/continuous.py:55-68
driving engine/model.py:145-146,167; its model-level checks: tests/test_paged.py:99-130).

- One layer at C5's batch over pools larger than 2^31 bytes (block offsets past the int32 range are read), for the
  bf16 cache and the per-token INT8 cache: the step's new K/V land in their slots (bit-exact, INT8 codes and scales
  equal the oracle's quantizer), and 32 sampled sequences' attention equals the oracle's fp32 gather-then-attend
  (INT8 dequantized as the reference's gather path does) to the north-star bound.
- The full 24-layer step (random-init weights, torch GEMMs): logits are finite, every layer's attention output
  inside the step equals a separate paged_decode_attention call on the same q and pools bit for bit, and the first
  and last layers' outputs equal the oracle on 32 sampled sequences.
"""

import numpy as np
import pytest
import torch

from cases import as_np32, assert_decode_close, oracle_cache_decode
from engine.block_manager import BlockManager
from engine.config import QWEN2_5_0_5B, ModelConfig
from engine.hip_decode import paged_decode_attention
from engine.model import Qwen2Model
from engine.paged_cache import PagedKVCache, build_metadata
from engine.quant_cache import QuantPagedKVCache
from oracle import paged_ref

pytestmark = pytest.mark.gpu

BATCH = 512


def c5_lengths(seed: int) -> list[int]:
    """Contexts after the step's new token, U[1024, 16384]."""
    return np.random.default_rng(seed).integers(1024, 16385, BATCH).tolist()


def scattered_manager(num_blocks: int, seed: int) -> BlockManager:
    """A manager whose free stack is a random permutation of the pool (the reference's tests reorder the free
    list the same way, reference tests/test_block_manager.py:61-66): tables reach every part of the pool."""
    m = BlockManager(num_blocks, 16)
    m._free[:] = np.random.default_rng(seed).permutation(num_blocks).tolist()
    return m


def step_metadata(m: BlockManager, lengths: list[int]):
    """Every sequence holds lengths[i] - 1 tokens, then gains the step's token: one decode row each."""
    for s, n in enumerate(lengths):
        m.allocate(s, n - 1)
        m.append_slot(s)
    return build_metadata(m, [(s, n - 1, 1) for s, n in enumerate(lengths)], "cuda")


def sample_rows(lengths: list[int], seed: int) -> list[int]:
    rng = np.random.default_rng(seed)
    rows = set(rng.choice(len(lengths), 30, replace=False).tolist())
    rows |= {int(np.argmax(lengths)), int(np.argmin(lengths))}
    return sorted(rows)


@pytest.mark.parametrize("fmt", ["bf16", "int8"])
def test_c5_layer_over_a_pool_past_2gib(fmt):
    cfg = ModelConfig(vocab_size=512, hidden_size=896, intermediate_size=256, num_layers=1, num_q_heads=14,
                      num_kv_heads=2, head_dim=64)
    Hq, Hkv, D = 14, 2, 64
    # blocks per layer so that one layer's K pool passes 2^31 bytes (bf16: 4 KiB per block over 2 heads; int8: 2 KiB)
    N = 600_000 if fmt == "bf16" else 1_200_000
    lengths = c5_lengths(7)
    m = scattered_manager(N, 7)
    meta = step_metadata(m, lengths)
    if fmt == "bf16":
        cache = PagedKVCache(cfg, N, 16, "cuda", torch.bfloat16, attn_backend="triton")
    else:
        cache = QuantPagedKVCache(cfg, N, 16, "cuda", torch.bfloat16, "triton", "int8", m)
    assert cache.k[0].numel() * cache.k.element_size() > 2 ** 31
    g = torch.Generator(device="cuda").manual_seed(7)
    if fmt == "bf16":
        cache.k.normal_(generator=g)
        cache.v.normal_(generator=g)
    else:
        cache.k.random_(-127, 128, generator=g)
        cache.v.random_(-127, 128, generator=g)
        cache.k_scale.uniform_(1 / 128, 1 / 32, generator=g)
        cache.v_scale.uniform_(1 / 128, 1 / 32, generator=g)
    tables = [m.block_table(s) for s in range(BATCH)]
    top = max(b for t, n in zip(tables, lengths) for b in t[:-(-n // 16)])
    per_block = 16 * D * cache.k.element_size()
    assert (Hkv - 1) * N * per_block + top * per_block > 2 ** 31  # head 1's rows of high blocks sit past 2 GiB
    k_new = torch.randn(BATCH, Hkv, D, device="cuda", dtype=torch.bfloat16, generator=g)
    v_new = torch.randn(BATCH, Hkv, D, device="cuda", dtype=torch.bfloat16, generator=g)
    q = torch.randn(BATCH, Hq, D, device="cuda", dtype=torch.bfloat16, generator=g)
    print(f"case c5 layer {fmt}: N={N}, max block id {top}, sum ctx {sum(lengths)}", flush=True)
    cache.begin(BATCH, meta)
    cache.write(0, k_new, v_new)
    out = cache.attend(0, q, meta.positions, D ** -0.5)
    torch.cuda.synchronize()
    assert out.shape == (BATCH, Hq * D)
    # the step's writes, bit for bit
    blk, off = meta.slot_blocks, meta.slot_offsets
    if fmt == "bf16":
        assert torch.equal(cache.k[0][:, blk, off].transpose(0, 1), k_new)
        assert torch.equal(cache.v[0][:, blk, off].transpose(0, 1), v_new)
    else:
        for new, codes, scales in ((k_new, cache.k, cache.k_scale), (v_new, cache.v, cache.v_scale)):
            q_ref, s_ref = paged_ref.quantize_per_token(as_np32(new))
            assert np.array_equal(codes[0][:, blk, off].transpose(0, 1).cpu().numpy(), q_ref)
            got_s = scales[0][:, blk, off].t().cpu().numpy()
            assert np.array_equal(got_s.view(np.uint16), s_ref.view(np.uint16))
    rows = sample_rows(lengths, 8)
    ref = oracle_cache_decode(cache, 0, as_np32(q[rows]), [tables[r] for r in rows], [lengths[r] for r in rows],
                              D ** -0.5)
    assert_decode_close(as_np32(out.view(BATCH, Hq, D)[rows]), ref, f"c5 layer {fmt}")


class RecordingCache(PagedKVCache):
    """PagedKVCache that keeps each layer's q and attention output of the last forward."""

    def begin(self, n_tokens, meta):
        super().begin(n_tokens, meta)
        self.seen = {}

    def attend(self, layer, q, positions, scale):
        out = super().attend(layer, q, positions, scale)
        self.seen[layer] = (q.clone(), out.clone(), scale)
        return out


def test_c5_full_decode_step():
    cfg = QWEN2_5_0_5B
    Hq, D = cfg.num_q_heads, cfg.head_dim
    lengths = c5_lengths(11)
    N = sum(-(-n // 16) for n in lengths) + 1024
    m = scattered_manager(N, 11)
    meta = step_metadata(m, lengths)
    cache = RecordingCache(cfg, N, 16, "cuda", torch.bfloat16, attn_backend="triton")
    g = torch.Generator(device="cuda").manual_seed(11)
    cache.k.normal_(generator=g)
    cache.v.normal_(generator=g)
    model = Qwen2Model(cfg, "cuda", torch.bfloat16, seed=11, max_positions=16400, std=0.02)
    ids = torch.randint(0, cfg.vocab_size, (BATCH,), device="cuda", generator=g)
    print(f"case c5 full step: {cfg.num_layers} layers, pool {N} blocks, sum ctx {sum(lengths)}", flush=True)
    logits = model.forward(ids, meta.positions, cache, meta)
    torch.cuda.synchronize()
    assert logits.shape == (BATCH, cfg.vocab_size)
    assert torch.isfinite(logits.float()).all()
    assert sorted(cache.seen) == list(range(cfg.num_layers))
    tables = [m.block_table(s) for s in range(BATCH)]
    rows = sample_rows(lengths, 12)
    for layer in range(cfg.num_layers):
        q, out, scale = cache.seen[layer]
        again = paged_decode_attention(q, cache.k[layer], cache.v[layer], meta.block_tables, meta.context_lens_t,
                                       scale, max(lengths), host_context_lens=lengths)
        assert torch.equal(again.view(BATCH, Hq * D), out), f"layer {layer}: in-step attention differs"
        if layer in (0, cfg.num_layers - 1):
            ref = oracle_cache_decode(cache, layer, as_np32(q[rows]), [tables[r] for r in rows],
                                      [lengths[r] for r in rows], scale)
            assert_decode_close(as_np32(out.view(BATCH, Hq, D)[rows]), ref, f"c5 full step layer {layer}")
