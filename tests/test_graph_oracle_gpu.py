"""Decode steps replayed from HIP graphs (engine/graph_runner.py) against the CPU oracle.

Every replayed step's attention output of every layer is recorded inside the graph (the test's cache copies q and
the attention output of each layer into persistent buffers, so the copies are captured too) and compared with the
oracle's fp32 gather-then-attend over the cache's pools after the step (bf16, and both INT8 formats dequantized as
the reference's gather path does), to the north-star bound (tests/cases.py assert_decode_close). The reference's
motivation for capturing the decode step is launch overhead (reference README.md:144,
docs/implementation-plan.md:126); replays must compute what the reference's attention computes.

Also the split workspace a graph records: buckets captured in increasing size (the larger ones need a larger split
workspace) and then replayed in any order, with the caching allocator's freed memory reused in between, keep their
results (a graph whose workspace was freed and reused would write partials and merge counters into foreign memory).
"""

import numpy as np
import pytest
import torch

from cases import as_np32, assert_decode_close, fragmented_manager, oracle_cache_decode
from engine.config import ModelConfig
from engine.graph_runner import DecodeGraphRunner
from engine.hip_decode import decode_workspace_bytes
from engine.model import Qwen2Model
from engine.paged_cache import PagedKVCache
from engine.quant_cache import QuantPagedKVCache

pytestmark = pytest.mark.gpu

CFG = ModelConfig(vocab_size=512, hidden_size=896, intermediate_size=256, num_layers=2, num_q_heads=14,
                  num_kv_heads=2, head_dim=64)


def recording(cls):
    """A cache class whose attend() also copies q and its output into persistent buffers (captured with the
    step when the step is captured)."""

    class Recording(cls):
        rec_q = rec_o = None

        def record(self, rows: int) -> None:
            L, Hq, D = self.cfg.num_layers, self.cfg.num_q_heads, self.cfg.head_dim
            self.rec_q = torch.zeros(L, rows, Hq, D, dtype=torch.bfloat16, device=self.device)
            self.rec_o = torch.zeros(L, rows, Hq * D, dtype=torch.bfloat16, device=self.device)

        def attend(self, layer, q, positions, scale):
            out = super().attend(layer, q, positions, scale)
            if self.rec_q is not None:
                T = q.shape[0]
                self.rec_q[layer, :T].copy_(q)
                self.rec_o[layer, :T].copy_(out)
            return out

    return Recording


def make(fmt, num_blocks, seed, n_stage=64):
    m = fragmented_manager(num_blocks, 16, torch.Generator().manual_seed(seed))
    if fmt == "bf16":
        cache = recording(PagedKVCache)(CFG, num_blocks, 16, "cuda", torch.bfloat16, attn_backend="triton")
    else:
        cache = recording(QuantPagedKVCache)(CFG, num_blocks, 16, "cuda", torch.bfloat16, "triton", fmt, m,
                                             n_stage=n_stage)
    g = torch.Generator(device="cuda").manual_seed(seed)
    for t in (cache.k, cache.v) + ((cache.stage,) if fmt == "int8-kchannel" else ()):
        if t.dtype == torch.int8:
            t.random_(-127, 128, generator=g)
        else:
            t.normal_(generator=g)
    if fmt != "bf16":
        cache.k_scale.uniform_(1 / 128, 1 / 32, generator=g)
        cache.v_scale.uniform_(1 / 128, 1 / 32, generator=g)
    model = Qwen2Model(CFG, "cuda", torch.bfloat16, seed=seed, max_positions=20000, std=0.05)
    return m, cache, model


def tails_of(cache, m, seqs):
    """Format B: each sequence's staging slot of its partial last block after the step (-1 when full)."""
    if getattr(cache, "fmt", None) != "int8-kchannel":
        return None
    out = []
    for s in seqs:
        n = m.seq_len(s)
        out.append(cache._stage_of[m.block_table(s)[(n - 1) // 16]] if n % 16 else -1)
    return out


def check_step(cache, m, seqs, what, sample=None):
    """Every layer's recorded attention output of the step over seqs against the oracle (rows `sample`, or all)."""
    torch.cuda.synchronize()
    rows = list(range(len(seqs))) if sample is None else sample
    sel = [seqs[i] for i in rows]
    tables, lengths = [m.block_table(s) for s in sel], [m.seq_len(s) for s in sel]
    tails = tails_of(cache, m, sel)
    D = CFG.head_dim
    for layer in range(CFG.num_layers):
        q = as_np32(cache.rec_q[layer, rows])
        ref = oracle_cache_decode(cache, layer, q, tables, lengths, D ** -0.5, tails)
        got = as_np32(cache.rec_o[layer, rows]).reshape(ref.shape)
        assert_decode_close(got, ref, f"{what} layer {layer}")


@pytest.mark.parametrize("fmt", ["bf16", "int8", "int8-kchannel"])
def test_replayed_steps_match_oracle(fmt):
    """Replays of three buckets (1, 4, 8), each step checked layer by layer against the oracle; blocks complete
    and new ones start during the steps (format B quantizes them from staging inside the graph)."""
    lengths = [13, 303, 17, 1005, 60, 2000, 31]
    m, cache, model = make(fmt, 700, seed=1)
    for s, n in enumerate(lengths):
        m.allocate(s, n)
    runner = DecodeGraphRunner(model, cache, m, max_batch=8, max_context=4096, buckets=[1, 4, 8])
    cache.record(8)
    g = torch.Generator(device="cuda").manual_seed(2)
    batches = [[0, 1, 2, 3, 4, 5, 6], [1, 3, 4], [5], [0, 1, 2, 3, 4, 5, 6], [2, 6, 0], [3]]
    for step, seqs in enumerate(batches):
        for s in seqs:
            m.append_slot(s)
        ids = torch.randint(0, CFG.vocab_size, (len(seqs),), device="cuda", generator=g)
        print(f"case {fmt} step {step} batch {len(seqs)}", flush=True)
        logits = runner.step(seqs, ids)
        torch.cuda.synchronize()
        assert torch.isfinite(logits.float()).all()
        check_step(cache, m, seqs, f"{fmt} step {step}")
    runner.close()


def test_bucket_workspaces_survive_larger_captures():
    """Bucket 1 is captured first, then bucket 64, whose decode needs a split workspace of more than 1 MiB at
    max_context 16384 (the smallest buffer the workspace holder allocates); bucket 1 is replayed afterwards, with
    freed allocator memory overwritten in between, and every replay matches the oracle."""
    Hq, Hkv, D = CFG.num_q_heads, CFG.num_kv_heads, CFG.head_dim
    need1 = decode_workspace_bytes(1, Hq, Hkv, D, 16384)
    need64 = decode_workspace_bytes(64, Hq, Hkv, D, 16384)
    print(f"workspace bytes: bucket 1 {need1}, bucket 64 {need64}", flush=True)
    assert need64 > (1 << 20) > need1
    rng = np.random.default_rng(3)
    lengths = rng.integers(100, 3000, 48).tolist()
    m, cache, model = make("bf16", sum(-(-n // 16) + 2 for n in lengths) + 64, seed=3)
    for s, n in enumerate(lengths):
        m.allocate(s, n)
    runner = DecodeGraphRunner(model, cache, m, max_batch=64, max_context=16384, buckets=[1, 64])
    cache.record(64)
    g = torch.Generator(device="cuda").manual_seed(4)
    junk = []
    for step, seqs in enumerate([[7], list(range(48)), [11], [7, 30, 2] + list(range(40, 48)), [0]]):
        for s in seqs:
            m.append_slot(s)
        ids = torch.randint(0, CFG.vocab_size, (len(seqs),), device="cuda", generator=g)
        print(f"case workspace step {step} batch {len(seqs)}", flush=True)
        runner.step(seqs, ids)
        check_step(cache, m, seqs, f"workspace step {step}")
        # churn the caching allocator: free blocks get reused by new tensors filled with garbage
        junk.clear()
        torch.cuda.empty_cache()
        junk.extend(torch.full((1 << 18,), -7.0, device="cuda") for _ in range(16))
    runner.close()


def test_c5_shaped_buckets_captured_in_increasing_size():
    """C5-like shapes (0.5B heads, contexts U[1024, 16384], up to 512 sequences): buckets 8, 64 and 512 captured
    in that order, then each replayed; 32 sampled rows of every replay checked against the oracle."""
    rng = np.random.default_rng(5)
    lengths = rng.integers(1024, 16385, 512).tolist()
    need = sum(-(-(n + 4) // 16) for n in lengths) + 64
    m, cache, model = make("bf16", need, seed=5)
    for s, n in enumerate(lengths):
        m.allocate(s, n)
    runner = DecodeGraphRunner(model, cache, m, max_batch=512, max_context=16400, buckets=[8, 64, 512])
    cache.record(512)
    g = torch.Generator(device="cuda").manual_seed(6)
    order = [8, 64, 512, 8, 512, 64]
    for step, b in enumerate(order):
        seqs = rng.choice(512, size=b, replace=False).tolist()
        for s in seqs:
            m.append_slot(s)
        ids = torch.randint(0, CFG.vocab_size, (b,), device="cuda", generator=g)
        print(f"case c5-shaped step {step} batch {b}", flush=True)
        runner.step(seqs, ids)
        sample = sorted(rng.choice(b, size=min(32, b), replace=False).tolist())
        check_step(cache, m, seqs, f"c5-shaped step {step} (batch {b})", sample)
    runner.close()
