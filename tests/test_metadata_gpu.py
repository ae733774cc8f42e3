"""Per-forward metadata derived on the device (engine/device_tables.py, sipa_paged_metadata) against the oracle's
restatement of the reference's builder (oracle/paged_ref.py metadata, reference engine/paged_cache.py:55-90) and
against the host builder build_metadata: every field equal, bit for bit, for decode batches, prefill chunks and
mixed batches over fragmented pools; and a model forward driven by the device metadata gives the same logits as one
driven by the host metadata."""

import random

import pytest
import torch

from cases import fragmented_manager
from engine.config import ModelConfig
from engine.device_tables import DeviceBlockTables
from engine.model import Qwen2Model
from engine.paged_cache import PagedKVCache, build_metadata
from oracle import paged_ref

pytestmark = pytest.mark.gpu


def assert_matches_oracle(dev, m, batch):
    """Every field of the device metadata equals the oracle's for the same tables and batch."""
    ref = paged_ref.metadata({s: m.block_table(s) for s, _, _ in batch}, batch, m.block_size)
    assert dev.query_starts == ref["query_starts"] and dev.context_lens == ref["context_lens"]
    for f in ("positions", "slot_mapping", "slot_blocks", "slot_offsets", "block_tables"):
        assert getattr(dev, f).tolist() == ref[f], f
    assert dev.context_lens_t.tolist() == ref["context_lens"]
    assert dev.last_token_indices.tolist() == ref["last_token_indices"]
    assert list(dev.slots_cpu) == ref["slot_mapping"]


def assert_same(dev, host):
    assert dev.num_tokens == host.num_tokens
    assert dev.query_starts == host.query_starts and dev.context_lens == host.context_lens
    for f in ("positions", "slot_mapping", "slot_blocks", "slot_offsets", "block_tables", "context_lens_t",
              "last_token_indices"):
        a, b = getattr(dev, f), getattr(host, f)
        assert a.dtype == b.dtype and a.shape == b.shape and torch.equal(a, b), f
    assert list(dev.slots_cpu) == list(host.slots_cpu)
    for i in range(dev.num_seqs):
        assert dev.block_ids_cpu[i] == host.block_ids_cpu[i]
        assert torch.equal(dev.block_ids[i], host.block_ids[i])


@pytest.mark.parametrize("seed", range(4))
def test_device_metadata_equals_host_metadata(seed):
    rng = random.Random(seed)
    m = fragmented_manager(3000, 16, torch.Generator().manual_seed(seed))
    dt = DeviceBlockTables(m, "cuda", max_seqs=64, max_blocks=256)
    lens = {s: rng.randint(1, 1500) for s in range(40)}
    for s, n in lens.items():
        m.allocate(s, n)
    for step in range(6):
        print(f"case seed {seed} step {step}", flush=True)
        batch = []
        for s in rng.sample(sorted(lens), rng.randint(1, 40)):
            if rng.random() < 0.3:  # a chunk of new tokens
                n = rng.randint(2, 70)
                m.append_slots(s, n)
                batch.append((s, lens[s], n))
                lens[s] += n
            else:
                m.append_slot(s)
                batch.append((s, lens[s], 1))
                lens[s] += 1
        if step == 3:  # a freed sequence's row goes to a new one
            victim = next(s for s in sorted(lens) if s not in {b[0] for b in batch})
            m.free(victim)
            del lens[victim]
            m.allocate(1000 + step, 33)
            lens[1000 + step] = 33
            batch.append((1000 + step, 0, 33))
        dev = dt.build(batch)
        host = build_metadata(m, batch, "cuda")
        torch.cuda.synchronize()
        assert_matches_oracle(dev, m, batch)
        assert_same(dev, host)
    s0 = min(lens)
    with pytest.raises(ValueError):
        dt.build([(s0, lens[s0], 1)])  # past what the sequence holds


def test_model_forward_on_device_metadata():
    cfg = ModelConfig(vocab_size=256, hidden_size=896, intermediate_size=256, num_layers=2, num_q_heads=14,
                      num_kv_heads=2, head_dim=64)
    m = fragmented_manager(600, 16, torch.Generator().manual_seed(1))
    cache = PagedKVCache(cfg, 600, 16, "cuda", torch.bfloat16, attn_backend="triton")
    g = torch.Generator(device="cuda").manual_seed(1)
    cache.k.normal_(generator=g)
    cache.v.normal_(generator=g)
    model = Qwen2Model(cfg, "cuda", torch.bfloat16, seed=1, max_positions=4096, std=0.05)
    dt = DeviceBlockTables(m, "cuda", max_seqs=16, max_blocks=256)
    lens = [700, 33, 1500, 64]
    for s, n in enumerate(lens):
        m.allocate(s, n)
    m.allocate(9, 0)
    m.append_slots(9, 40)
    for s in range(4):
        m.append_slot(s)
    batch = [(0, 700, 1), (9, 0, 40), (1, 33, 1), (2, 1500, 1), (3, 64, 1)]
    ids = torch.randint(0, cfg.vocab_size, (44,), device="cuda", generator=g)
    outs = []
    for meta in (build_metadata(m, batch, "cuda"), dt.build(batch)):
        outs.append(model.forward(ids, meta.positions, cache, meta, last_only=False))
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])
