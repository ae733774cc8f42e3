"""Decode steps replayed from HIP graphs (engine/graph_runner.py) against the same steps run eagerly.

Checks: a replayed step gives the same logits, bit for bit, as the same static-shape step run eagerly on the same
cache state (the same kernels with the same launch parameters), and matches the ordinary eager forward
(build_metadata, per-step split choice) within bf16 tolerance; replays alternate with eager work and batch sizes
change between buckets, and every replay is checked (graph replays have produced wrong results after the first
on this platform when a captured node misbehaves); both INT8 caches are captured too. Each step runs three times
from the same cache state (pools, scales, staging and the staging-slot bookkeeping are saved and restored): the
replay, the eager static step and the ordinary forward. Format "int8-kchannel" frees a block's staging slot in
the step that completes the block, so a step is not repeatable without the restore; the lengths make blocks
complete (and new ones start) during the steps.
"""

import pytest
import torch

from cases import fragmented_manager
from engine.config import ModelConfig
from engine.graph_runner import SCRATCH_SEQ, DecodeGraphRunner
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
    for t in (cache.k, cache.v) + ((cache.stage,) if fmt == "int8-kchannel" else ()):
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


def snapshot(cache):
    names = [n for n in ("k", "v", "k_scale", "v_scale", "stage") if hasattr(cache, n)]
    books = (dict(cache._stage_of), list(cache._free_stage)) if hasattr(cache, "_stage_of") else None
    return {n: getattr(cache, n).clone() for n in names}, books


def restore(cache, snap):
    tensors, books = snap
    for n, t in tensors.items():
        getattr(cache, n).copy_(t)
    if books is not None:
        cache._stage_of.clear()
        cache._stage_of.update(books[0])
        cache._free_stage[:] = books[1]


@pytest.mark.parametrize("fmt", ["bf16", "int8", "int8-kchannel"])
def test_replay_matches_eager_steps(fmt):
    # sequence 1 completes a block in step 0, sequence 4 in step 3 and starts one in step 4, sequence 0 in step 4
    lengths = [13, 303, 17, 1005, 60]
    m, cache, model = setup(fmt, lengths)
    runner = DecodeGraphRunner(model, cache, m, max_batch=8, max_context=2048)
    scratch = int(m.table_array(SCRATCH_SEQ)[0])
    keep_blocks = torch.ones(cache.k.shape[2], dtype=torch.bool, device="cuda")
    keep_blocks[scratch] = False
    if fmt == "int8-kchannel":
        keep_slots = torch.ones(cache.n_stage, dtype=torch.bool, device="cuda")
        keep_slots[cache._stage_of[scratch]] = False
    g = torch.Generator(device="cuda").manual_seed(1)
    batches = [[0, 1, 2, 3, 4], [1, 3, 4], [0, 1, 2, 3, 4], [4], [0, 1, 2, 3, 4]]  # buckets 8, 4, 8, 1, 8
    for step, seqs in enumerate(batches):
        for s in seqs:
            m.append_slot(s)
        ids = torch.randint(0, CFG.vocab_size, (len(seqs),), device="cuda", generator=g)
        print(f"case {fmt} step {step} batch {len(seqs)}", flush=True)
        before = snapshot(cache)
        got = runner.step(seqs, ids).clone()
        torch.cuda.synchronize()
        after = snapshot(cache)
        # the same static-shape step eagerly from the same state: same logits and same cache contents
        restore(cache, before)
        ref = runner.step(seqs, ids, graph=False)
        torch.cuda.synchronize()
        assert torch.equal(got, ref), f"step {step}: replay differs from the eager static step"
        eager = snapshot(cache)
        assert after[1] == eager[1], f"step {step}: staging bookkeeping differs"
        # outside the scratch block and its staging slot (the padding rows', which a capture's warm-up writes)
        for n, t in after[0].items():
            keep = keep_slots if n == "stage" else keep_blocks
            assert torch.equal(t[:, :, keep], eager[0][n][:, :, keep]), f"step {step}: cache {n} differs"
        restore(cache, before)
        # the ordinary forward: per-step metadata and split choice, so the decode launches sum in another order;
        # through two bf16 layers that moves a few logits by a few bf16 steps
        meta = build_metadata(m, [(s, m.seq_len(s) - 1, 1) for s in seqs], "cuda")
        plain = model.forward(ids, meta.positions, cache, meta).float()
        torch.cuda.synchronize()
        scale = plain.abs().max().item()
        torch.testing.assert_close(got.float(), plain, rtol=0.02, atol=0.02 * scale)
        assert (got.float() - plain).abs().mean().item() <= 2e-3 * scale
        if fmt == "int8-kchannel":  # the plan's slots and tails are the ones the eager forward planned
            assert (dict(cache._stage_of), list(cache._free_stage)) == after[1]
    runner.close()
    if fmt == "int8-kchannel":  # closing gives back the scratch block's staging slot
        assert scratch not in cache._stage_of
        assert len(cache._free_stage) + len(cache._stage_of) == cache.n_stage


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
    m = fragmented_manager(64, 16, torch.Generator().manual_seed(0))
    gather = PagedKVCache(CFG, 64, 16, "cuda", torch.bfloat16, attn_backend="gather")
    with pytest.raises(ValueError):  # the gather backend launches per sequence: nothing to capture
        DecodeGraphRunner(Qwen2Model(CFG, "cuda", torch.bfloat16, seed=0, max_positions=64), gather, m,
                          max_batch=2, max_context=64)
    m2, cache2, model2 = setup("bf16", [3000])
    runner = DecodeGraphRunner(model2, cache2, m2, max_batch=2, max_context=1024)
    m2.append_slot(0)
    with pytest.raises(ValueError):  # context past max_context
        runner.step([0], torch.tensor([1], device="cuda"))
    with pytest.raises(ValueError):  # a sequence twice in one step
        runner.step([0, 0], torch.tensor([1, 2], device="cuda"))
    m2.allocate(1, 10)
    m2.allocate(2, 10)
    with pytest.raises(ValueError):  # more rows than max_batch
        runner.step([0, 1, 2], torch.tensor([1, 2, 3], device="cuda"))
    runner.close()
