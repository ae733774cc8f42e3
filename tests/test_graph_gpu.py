"""Decode steps replayed from HIP graphs (engine/graph_runner.py) against the same steps run eagerly.

Checks: a replayed step gives the same logits, bit for bit, as the same static-shape step run eagerly on the same
cache state (the same kernels with the same launch parameters), and matches the ordinary eager forward
(build_metadata, per-step split choice) within bf16 tolerance; replays alternate with eager work and batch sizes
change between buckets, and every replay is checked (graph replays have produced wrong results after the first
on this platform when a captured node misbehaves); the INT8 per-token cache is captured too.
"""

import pytest
import torch

from cases import fragmented_manager
from engine.config import ModelConfig
from engine.graph_runner import DecodeGraphRunner
from engine.model import Qwen2Model
from engine.paged_cache import PagedKVCache, build_metadata
from engine.quant_cache import QuantPagedKVCache

pytestmark = pytest.mark.gpu

CFG = ModelConfig(vocab_size=512, hidden_size=896, intermediate_size=256, num_layers=2, num_q_heads=14,
                  num_kv_heads=2, head_dim=64)


def setup(fmt, lengths, seed=0, num_blocks=512):
    gen = torch.Generator().manual_seed(seed)
    m = fragmented_manager(num_blocks, 16, gen)
    if fmt == "bf16":
        cache = PagedKVCache(CFG, num_blocks, 16, "cuda", torch.bfloat16, attn_backend="triton")
    else:
        cache = QuantPagedKVCache(CFG, num_blocks, 16, "cuda", torch.bfloat16, "triton", fmt, m, n_stage=16)
    g = torch.Generator(device="cuda").manual_seed(seed)
    for t in (cache.k, cache.v):
        if t.dtype == torch.int8:
            t.random_(-127, 128, generator=g)
        else:
            t.normal_(generator=g)
    if fmt != "bf16":
        cache.k_scale.fill_(1 / 64)
        cache.v_scale.fill_(1 / 64)
    for s, n in enumerate(lengths):
        m.allocate(s, n)
    model = Qwen2Model(CFG, "cuda", torch.bfloat16, seed=seed, max_positions=4096, std=0.05)
    return m, cache, model


@pytest.mark.parametrize("fmt", ["bf16", "int8"])
def test_replay_matches_eager_steps(fmt):
    lengths = [5, 300, 17, 1000, 64]
    m, cache, model = setup(fmt, lengths)
    runner = DecodeGraphRunner(model, cache, m, max_batch=8, max_context=2048)
    g = torch.Generator(device="cuda").manual_seed(1)
    batches = [[0, 1, 2, 3, 4], [1, 3, 4], [0, 1, 2, 3, 4], [4], [0, 1, 2, 3, 4]]  # buckets 8, 4, 8, 1, 8
    for step, seqs in enumerate(batches):
        for s in seqs:
            m.append_slot(s)
        ids = torch.randint(0, CFG.vocab_size, (len(seqs),), device="cuda", generator=g)
        print(f"case {fmt} step {step} batch {len(seqs)}", flush=True)
        got = runner.step(seqs, ids).clone()
        torch.cuda.synchronize()
        # the same static-shape step eagerly (it rewrites the same K/V values for the new tokens)
        ref = runner.step(seqs, ids, graph=False)
        torch.cuda.synchronize()
        assert torch.equal(got, ref), f"step {step}: replay differs from the eager static step"
        # the ordinary forward: per-step metadata and split choice, so the decode launches sum in another order;
        # through two bf16 layers that moves a few logits by a few bf16 steps
        meta = build_metadata(m, [(s, m.seq_len(s) - 1, 1) for s in seqs], "cuda")
        plain = model.forward(ids, meta.positions, cache, meta).float()
        torch.cuda.synchronize()
        scale = plain.abs().max().item()
        torch.testing.assert_close(got.float(), plain, rtol=0.02, atol=0.02 * scale)
        assert (got.float() - plain).abs().mean().item() <= 2e-3 * scale
    runner.close()


def test_replays_interleaved_with_eager_work():
    """The same captured step replayed five times with eager torch work and syncs in between: every replay
    equals the eager result."""
    lengths = [40, 700, 129]
    m, cache, model = setup("bf16", lengths, seed=3)
    runner = DecodeGraphRunner(model, cache, m, max_batch=4, max_context=1024, buckets=[4])
    for s in range(3):
        m.append_slot(s)
    ids = torch.tensor([3, 7, 11], device="cuda")
    ref = runner.step([0, 1, 2], ids, graph=False).clone()
    for i in range(5):
        print(f"case replay {i}", flush=True)
        junk = torch.randn(1 << 20, device="cuda").sum()  # eager work between replays
        got = runner.step([0, 1, 2], ids)
        torch.cuda.synchronize()
        assert torch.isfinite(junk)
        assert torch.equal(got, ref), f"replay {i} differs"
    runner.close()


def test_runner_rejects_what_it_cannot_capture():
    m, cache, model = setup("int8-kchannel", [10])
    with pytest.raises(ValueError):
        DecodeGraphRunner(model, cache, m, max_batch=2, max_context=64)
    m2, cache2, model2 = setup("bf16", [3000])
    runner = DecodeGraphRunner(model2, cache2, m2, max_batch=2, max_context=1024)
    m2.append_slot(0)
    with pytest.raises(ValueError):  # context past max_context
        runner.step([0], torch.tensor([1], device="cuda"))
    with pytest.raises(ValueError):  # more rows than max_batch
        runner.step([0, 0, 0], torch.tensor([1, 2, 3], device="cuda"))
    runner.close()
