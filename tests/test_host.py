"""Host-side logic of the drop-in path on the CPU: block bookkeeping, per-forward metadata, the cache's write /
gather on CPU pools, the INT8 staging plan, and pool budgets. Mirrors the reference's tests/test_block_manager.py,
tests/test_paged.py:41-76,132-137 and tests/test_quant_cache.py:42-115; known answers come from
tests/golden/reference_known_answers.json.
"""

import json
import random
from pathlib import Path

import pytest
import torch

from engine.block_manager import BlockManager, OutOfBlocks
from engine.config import QWEN2_5_0_5B, ModelConfig
from engine.paged_cache import PagedKVCache, build_metadata
from engine.quant_cache import QuantPagedKVCache, blocks_for_budget, kv_bytes_per_token

GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_known_answers.json").read_text())
TINY = ModelConfig(vocab_size=97, hidden_size=32, intermediate_size=64, num_layers=2, num_q_heads=4,
                   num_kv_heads=2, head_dim=16)


# ---- block manager ------------------------------------------------------------------------------------------------

def test_allocate_append_known_answer():
    ka = GOLDEN["block_manager_allocate_append"]
    m = BlockManager(ka["num_blocks"], ka["block_size"])
    for op, seq, arg, *want in ka["ops"]:
        if op == "allocate":
            assert m.allocate(seq, arg) == want[0]
            assert m.block_table(seq) == ka["table_after_first_allocate"]
        elif op == "append_slot":
            assert m.append_slot(seq) == arg
        else:
            assert m.block_table(seq) == ka["table_before_last_append"] and m.seq_len(seq) == 9
            assert m.append_slots(seq, arg) == want[0]
    m.check_invariants()


def test_lifo_reuse_known_answer():
    ka = GOLDEN["block_manager_lifo"]
    m = BlockManager(ka["num_blocks"], ka["block_size"])
    for s in range(4):
        m.allocate(s, 8)
    assert [m.block_table(s)[0] // 2 for s in range(4)] == ka["allocate_each_8_tokens"]
    for s in ka["free"]:
        m.free(s)
    m.allocate(9, 16)
    t = m.block_table(9)
    assert sorted(t) == ka["then_allocate_16_tokens_table_sorted"] and t != sorted(t)
    assert t == [6, 7, 2, 3]  # sequence 3's blocks first (freed last), each sequence's in its old table order


def test_zero_length_and_errors():
    m = BlockManager(num_blocks=2, block_size=4)
    assert m.allocate(0, 0) == [] and m.block_table(0) == []
    assert m.append_slots(0, 8) == list(range(8))
    with pytest.raises(OutOfBlocks):
        m.append_slot(0)
    with pytest.raises(OutOfBlocks):
        m.allocate(1, 1)
    with pytest.raises(ValueError):
        m.allocate(0, 1)
    assert m.seq_len(0) == 8 and m.num_free_blocks() == 0
    assert not m.can_allocate(1) and not m.can_append(0)
    m.free(0)
    assert m.can_allocate(8) and not m.can_allocate(8, watermark_blocks=1)
    m.check_invariants()


def test_check_invariants_catches_corruption():
    m = BlockManager(num_blocks=4, block_size=4)
    m.allocate(0, 4)
    m._free.append(m.block_table(0)[0])
    with pytest.raises(AssertionError):
        m.check_invariants()
    m = BlockManager(num_blocks=4, block_size=4)
    m._free.pop()
    with pytest.raises(AssertionError):
        m.check_invariants()


@pytest.mark.parametrize("seed", range(20))
def test_randomized_no_leaks(seed):
    """Random allocate / append / free, some failing: bookkeeping stays consistent, live slots are disjoint and
    match a shadow model, and freeing everything returns every block exactly once."""
    rng = random.Random(seed)
    B = rng.choice([1, 4, 16])
    m = BlockManager(num_blocks=rng.randint(4, 64), block_size=B)
    shadow: dict[int, list[int]] = {}
    next_id = 0
    for _ in range(400):
        op = rng.random()
        if op < 0.3 or not shadow:
            n = rng.randint(0, 3 * B)
            if m.can_allocate(n):
                shadow[next_id] = m.allocate(next_id, n)
            else:
                with pytest.raises(OutOfBlocks):
                    m.allocate(next_id, n)
            next_id += 1
        elif op < 0.8:
            s, n = rng.choice(list(shadow)), rng.choice([1, 1, 1, rng.randint(1, 2 * B)])
            if m.can_append(s, n):
                shadow[s] += m.append_slots(s, n)
            else:
                before = (m.block_table(s), m.num_free_blocks())
                with pytest.raises(OutOfBlocks):
                    m.append_slots(s, n)
                assert (m.block_table(s), m.num_free_blocks()) == before
        else:
            s = rng.choice(list(shadow))
            m.free(s)
            del shadow[s]
        m.check_invariants()
        live = [x for slots in shadow.values() for x in slots]
        assert len(live) == len(set(live))
        for s, slots in shadow.items():
            assert m.slots(s, 0, m.seq_len(s)) == slots
    for s in list(shadow):
        m.free(s)
    assert sorted(m._free) == list(range(m.num_blocks))


# ---- metadata -----------------------------------------------------------------------------------------------------

def test_metadata_known_answer():
    ka = GOLDEN["metadata_packed_batch"]
    m = BlockManager(ka["num_blocks"], ka["block_size"])
    for op, seq, n in ka["setup"]:
        getattr(m, op)(seq, n)
    meta = build_metadata(m, [tuple(b) for b in ka["batch"]], "cpu")
    assert meta.num_tokens == ka["num_tokens"] and meta.query_starts == ka["query_starts"]
    assert meta.context_lens == ka["context_lens"] and meta.positions.tolist() == ka["positions"]
    assert meta.slot_mapping.tolist() == ka["slot_mapping"] and meta.slots_cpu == ka["slot_mapping"]
    assert meta.slot_blocks.tolist() == ka["slot_blocks"] and meta.slot_offsets.tolist() == ka["slot_offsets"]
    assert [b.tolist() for b in meta.block_ids] == ka["block_ids"] and meta.block_ids_cpu == ka["block_ids"]
    assert meta.block_tables.tolist() == ka["block_tables"] and meta.block_tables.dtype == torch.int32
    assert meta.context_lens_t.tolist() == ka["context_lens_t"] and meta.context_lens_t.dtype == torch.int32
    assert meta.last_token_indices.tolist() == ka["last_token_indices"]
    with pytest.raises(ValueError):
        build_metadata(m, [(0, 8, 1)], "cpu")  # position 8 has no slot yet


def fragmented(num_blocks, B, seed=0):
    m = BlockManager(num_blocks, B)
    for s in range(num_blocks):
        m.allocate(100 + s, B)
    for s in random.Random(seed).sample(range(num_blocks), num_blocks):
        m.free(100 + s)
    return m


def test_write_then_gather_roundtrip():
    """K/V written at shuffled slots come back from gather() in position order (CPU pool, torch indexing)."""
    m = fragmented(10, 4)
    cache = PagedKVCache(TINY, 10, 4, "cpu", torch.float64)
    m.allocate(7, 11)
    meta = build_metadata(m, [(7, 0, 11)], "cpu")
    cache.begin(11, meta)
    k = torch.randn(11, 2, 16, dtype=torch.float64)
    v = torch.randn_like(k)
    cache.write(1, k, v)
    gk, gv = cache.gather(1, 0)
    assert torch.equal(gk, k.transpose(0, 1)) and torch.equal(gv, v.transpose(0, 1))
    t = m.block_table(7)
    assert any(b != a + 1 for a, b in zip(t, t[1:]))


def test_kernel_backend_refuses_cpu_pool():
    """The HIP backends run only on GPU pools: a CPU pool fails loudly instead of falling back."""
    m = BlockManager(4, 4)
    m.allocate(0, 3)
    for backend in ("hip", "triton"):
        cache = PagedKVCache(TINY, 4, 4, "cpu", torch.float32, attn_backend=backend)
        with pytest.raises(ValueError, match="GPU"):
            cache.begin(3, build_metadata(m, [(0, 0, 3)], "cpu"))
    with pytest.raises(ValueError):
        PagedKVCache(TINY, 4, 4, "cpu", torch.float32, attn_backend="flash")


def test_gather_backend_attend_matches_oracle():
    """attend() on the gather backend for a mixed prefill + decode batch equals causal softmax attention."""
    from oracle import paged_ref

    torch.manual_seed(1)
    m = fragmented(16, 4)
    cache = PagedKVCache(TINY, 16, 4, "cpu", torch.float64)
    m.allocate(0, 9)
    m.allocate(1, 5)
    meta = build_metadata(m, [(0, 0, 9), (1, 0, 5)], "cpu")
    cache.begin(14, meta)
    k, v = torch.randn(14, 2, 16, dtype=torch.float64), torch.randn(14, 2, 16, dtype=torch.float64)
    cache.write(0, k, v)
    m.append_slot(0)
    meta = build_metadata(m, [(0, 9, 1), (1, 3, 2)], "cpu")  # one decode row, one 2-token chunk (rewrite 3, 4)
    cache.begin(3, meta)
    k2, v2 = torch.randn(3, 2, 16, dtype=torch.float64), torch.randn(3, 2, 16, dtype=torch.float64)
    cache.write(0, k2, v2)
    q = torch.randn(3, 4, 16, dtype=torch.float64)
    out = cache.attend(0, q, meta.positions, 0.25).view(3, 4, 16)
    keys0 = torch.cat([k[:9], k2[:1]]).transpose(0, 1).numpy()
    vals0 = torch.cat([v[:9], v2[:1]]).transpose(0, 1).numpy()
    torch.testing.assert_close(out[0], torch.from_numpy(paged_ref.attend_one(q[0].numpy(), keys0, vals0, 0.25)))
    keys1 = torch.cat([k[9:12], k2[1:]]).transpose(0, 1).numpy()
    vals1 = torch.cat([v[9:12], v2[1:]]).transpose(0, 1).numpy()
    for r, n in ((1, 4), (2, 5)):  # causal: row at position p sees keys 0..p
        want = paged_ref.attend_one(q[r].numpy(), keys1[:, :n], vals1[:, :n], 0.25)
        torch.testing.assert_close(out[r], torch.from_numpy(want))


# ---- INT8 caches ----------------------------------------------------------------------------------------------------

def make_quant_cache(fmt, num_blocks=24, B=4):
    m = BlockManager(num_blocks, B)
    return m, QuantPagedKVCache(TINY, num_blocks, B, "cpu", torch.float32, "gather", fmt, m, n_stage=32)


def write_chunks(m, cache, seq, k, v, chunks, layer=0):
    pos = m.seq_len(seq) if seq in m.seq_ids() else 0
    if seq not in m.seq_ids():
        m.allocate(seq, 0)
    i = 0
    for n in chunks:
        m.append_slots(seq, n)
        meta = build_metadata(m, [(seq, pos, n)], "cpu")
        cache.begin(n, meta)
        cache.write(layer, k[i:i + n], v[i:i + n])
        pos, i = pos + n, i + n
    return meta


@pytest.mark.parametrize("fmt", ["int8", "int8-kchannel"])
def test_quant_roundtrip_across_chunks(fmt):
    """Gathered K/V are within half a quantization step of the originals through chunked writes that cross block
    boundaries; format B's partial last block is only bf16-rounded."""
    torch.manual_seed(0)
    n = 23
    k = torch.randn(n, 2, 16) * torch.rand(1, 2, 16) * 4
    v = torch.randn(n, 2, 16)
    m, cache = make_quant_cache(fmt)
    write_chunks(m, cache, 0, k, v, [1, 6, 9, 7])
    gk, gv = cache.gather(0, 0)
    assert gk.shape == (2, n, 16)
    v_step = v.abs().amax(-1).t()[..., None] / 127
    assert ((gv - v.transpose(0, 1)).abs() <= v_step * 0.51 + 1e-6).all()
    kt = k.transpose(0, 1)
    if fmt == "int8":
        k_step = k.abs().amax(-1).t()[..., None] / 127
        assert ((gk - kt).abs() <= k_step * 0.51 + 1e-6).all()
    else:
        blocks = kt[:, :20].reshape(2, 5, 4, 16).to(torch.bfloat16).float()
        step = blocks.abs().amax(2, keepdim=True) / 127
        assert ((gk[:, :20].reshape(2, 5, 4, 16) - blocks).abs() <= step * 0.51 + 1e-6).all()
        assert torch.equal(gk[:, 20:], kt[:, 20:].to(torch.bfloat16).float())


def test_kchannel_blocks_do_not_depend_on_chunking():
    """A block's int8 codes and channel scales are the same whether it was staged token by token or written whole."""
    torch.manual_seed(2)
    k, v = torch.randn(16, 2, 16) * 3, torch.randn(16, 2, 16)
    pools = []
    for chunks in ([16], [1] * 16, [3, 5, 8], [4, 4, 4, 4]):
        m, cache = make_quant_cache("int8-kchannel")
        write_chunks(m, cache, 0, k, v, chunks)
        t = m.block_table(0)
        pools.append((cache.k[0][:, t].clone(), cache.k_scale[0][:, t].clone()))
    for kq, ks in pools[1:]:
        assert torch.equal(kq, pools[0][0]) and torch.equal(ks, pools[0][1])


def test_staging_slots_follow_partial_blocks():
    """Format B keeps a staging slot exactly for each live sequence's partial last block over random appends and
    frees: no leaks, no double assignment."""
    rng = random.Random(0)
    m, cache = make_quant_cache("int8-kchannel", num_blocks=64, B=4)
    live = {}
    for step in range(300):
        if live and rng.random() < 0.2:
            s = rng.choice(list(live))
            m.free(s)
            del live[s]
        else:
            s = rng.choice(list(live)) if live and rng.random() < 0.7 else 1000 + step
            n = rng.randint(1, 9)
            if (s in live and not m.can_append(s, n)) or (s not in live and not m.can_allocate(n)):
                continue
            write_chunks(m, cache, s, torch.randn(n, 2, 16), torch.randn(n, 2, 16), [n])
            live[s] = m.seq_len(s)
        partial = {m.block_table(s)[-1] for s, length in live.items() if length % 4}
        assert set(cache._stage_of) == partial
        assert len(cache._free_stage) + len(cache._stage_of) == cache.n_stage
        assert len(set(cache._free_stage)) == len(cache._free_stage)
    for s in list(live):
        m.free(s)
    assert cache._stage_of == {} and len(cache._free_stage) == cache.n_stage


def test_static_decode_plan_matches_begin():
    """Format B under the graph runner: the host plan of a decode step (plan_static_decode, with padding rows at
    offset 0 of a scratch block that holds its own slot) hands out the staging slots, frees and tail slots that
    begin() plans for the same rows, and the static begin path (every row staged, every row's slot quantized,
    into the scratch block unless the row completes its block) leaves the pools as the per-forward plan does,
    outside the scratch block and its slot."""
    torch.manual_seed(4)
    B, seqs = 4, [0, 1, 2, 3]
    m, cache = make_quant_cache("int8-kchannel", num_blocks=64, B=B)
    m.allocate(-1, 1)
    scratch = m.block_table(-1)[0]
    cache.plan_static_decode([scratch], [0], scratch)  # the runner's first plan: the scratch block's slot
    scratch_slot = cache._stage_of[scratch]
    for s, n in zip(seqs, [3, 6, 8, 1]):
        write_chunks(m, cache, s, torch.randn(n, 2, 16), torch.randn(n, 2, 16), [n])
    names = ("k", "k_scale", "v", "v_scale", "stage")
    completed = 0
    for step in range(7):
        for s in seqs:
            m.append_slot(s)
        lens = [m.seq_len(s) for s in seqs]
        k, v = torch.randn(6, 2, 16), torch.randn(6, 2, 16)
        books = (dict(cache._stage_of), list(cache._free_stage))
        pools = {n: getattr(cache, n).clone() for n in names}
        cache.begin(4, build_metadata(m, [(s, L - 1, 1) for s, L in zip(seqs, lens)], "cpu"))
        cache.write(0, k[:4], v[:4])
        want_books, want_tails = (dict(cache._stage_of), list(cache._free_stage)), cache._tails.tolist()
        want = {n: getattr(cache, n).clone() for n in names}
        cache._stage_of.clear()
        cache._stage_of.update(books[0])
        cache._free_stage[:] = books[1]
        for n in names:
            getattr(cache, n).copy_(pools[n])
        blocks = [m.block_table(s)[(L - 1) // B] for s, L in zip(seqs, lens)] + [scratch] * 2
        offsets = [(L - 1) % B for L in lens] + [0, 0]
        slots, src, dst, tails = cache.plan_static_decode(blocks, offsets, scratch)
        assert (dict(cache._stage_of), list(cache._free_stage)) == want_books
        assert tails == want_tails + [scratch_slot] * 2
        completed += sum(o == B - 1 for o in offsets)
        i64 = lambda xs: torch.tensor(xs, dtype=torch.int64)  # noqa: E731
        cache.use_static_plan((torch.arange(6), i64(slots), i64(src), i64(dst), torch.tensor(tails, dtype=torch.int32)))
        cache.begin(6, build_metadata(m, [(s, L - 1, 1) for s, L in zip(seqs, lens)] + [(-1, 0, 1)] * 2, "cpu"))
        cache.use_static_plan(None)
        cache.write(0, k, v)
        assert cache._tails.tolist() == tails
        keep = torch.ones(64, dtype=torch.bool)
        keep[scratch] = False
        for n in ("k", "k_scale", "v", "v_scale"):
            assert torch.equal(getattr(cache, n)[:, :, keep], want[n][:, :, keep]), (step, n)
        live = torch.ones(cache.n_stage, dtype=torch.bool)
        live[scratch_slot] = False
        assert torch.equal(cache.stage[:, :, live], want["stage"][:, :, live]), step
    assert completed >= 4  # blocks completed (and new ones started) along the way


def test_bytes_and_budget():
    ka = GOLDEN["budgets"]
    cfg = ModelConfig(**ka["qwen2_5_0_5b"])
    assert cfg == QWEN2_5_0_5B
    for fmt, want in ka["kv_bytes_per_token"].items():
        assert kv_bytes_per_token(cfg, fmt) == want
    gib2 = 2 * 2 ** 30
    assert PagedKVCache.blocks_for_budget(cfg, gib2, 16) == ka["blocks_2_gib"]["bf16"]
    assert blocks_for_budget(cfg, "bf16", gib2, 16) == ka["blocks_2_gib"]["bf16"]
    assert blocks_for_budget(cfg, "int8", gib2, 16) == ka["blocks_2_gib"]["int8"]
    assert blocks_for_budget(cfg, "int8-kchannel", gib2, 16, n_stage=128) > \
        ka["blocks_2_gib"]["int8-kchannel_n_stage_128_more_than"]


def test_torch_quantizer_bounds():
    """engine.quant (the CPU-pool quantizer) keeps the reference's bounds: per-channel beats per-token on
    outlier channels (reference tests/test_quant.py:39-51)."""
    from engine.quant import dequantize, quantize_per_channel, quantize_per_token

    def relative_error(x, x_hat):
        return ((x.float() - x_hat.float()).norm() / x.float().norm()).item()

    torch.manual_seed(0)
    x = torch.randn(64, 128)
    x[:, :4] *= 50
    qt, st = quantize_per_token(x)
    qc, sc = quantize_per_channel(x, dim=0)
    e_tok = relative_error(x, dequantize(qt, st[:, None]))
    e_ch = relative_error(x, dequantize(qc, sc[None, :]))
    assert e_ch < e_tok / 3


@pytest.mark.parametrize("seed", range(5))
def test_metadata_matches_oracle_on_random_batches(seed):
    """build_metadata (array mirrors, packed uploads, rows made on access) equals the oracle's restatement of the
    reference's metadata on random mixes of decode rows and multi-token chunks over a fragmented pool."""
    from oracle import paged_ref

    rng = random.Random(seed)
    B = rng.choice([4, 16])
    m = fragmented(4096, B, seed)
    batch, tables = [], {}
    for s in range(rng.randint(1, 40)):
        start = rng.randint(0, 300)
        n = rng.choice([1, 1, 1, rng.randint(1, 70)])
        m.allocate(s, start + n)
        batch.append((s, start, n))
        tables[s] = m.block_table(s)
    meta = build_metadata(m, batch, "cpu")
    ref = paged_ref.metadata(tables, batch, B)
    for key in ("query_starts", "context_lens", "positions", "slot_mapping", "slot_blocks", "slot_offsets",
                "block_tables", "last_token_indices"):
        got = getattr(meta, key)
        got = got.tolist() if isinstance(got, torch.Tensor) else got
        assert got == ref[key], key
    assert meta.slots_cpu == ref["slot_mapping"] and meta.num_tokens == ref["query_starts"][-1]
    want = [tables[s][:-(-(start + n) // B)] for s, start, n in batch]
    assert [b.tolist() for b in meta.block_ids] == want and meta.block_ids_cpu == want
    assert meta.context_lens_t.dtype == meta.block_tables.dtype == torch.int32


def test_metadata_from_a_manager_with_only_the_reference_api():
    """build_metadata also takes a block manager that offers only the reference's API (block_table() lists,
    seq_len(), block_size; engine/block_manager.py:106-113), as when the reference's own manager stays in place:
    same metadata as from this package's manager with its int32 mirrors."""

    class ReferenceApi:
        def __init__(self, m):
            self.block_size = m.block_size
            self.block_table = m.block_table
            self.seq_len = m.seq_len

    m = fragmented(1024, 16, 3)
    batch = [(0, 0, 37), (1, 100, 1), (2, 15, 2), (3, 0, 1)]
    for s, start, n in batch:
        m.allocate(s, start + n)
    ours, ref_api = build_metadata(m, batch, "cpu"), build_metadata(ReferenceApi(m), batch, "cpu")
    assert not hasattr(ReferenceApi(m), "table_array")
    for key in ("query_starts", "context_lens", "positions", "slot_mapping", "slot_blocks", "slot_offsets",
                "block_tables", "context_lens_t", "last_token_indices"):
        a, b = getattr(ours, key), getattr(ref_api, key)
        assert (torch.equal(a, b) if isinstance(a, torch.Tensor) else a == b), key
    assert list(ours.block_ids_cpu) == list(ref_api.block_ids_cpu)


def test_graph_runner_needs_a_gpu_kernel_cache():
    """Graph capture is for the HIP backend on a GPU pool: a CPU or gather cache is refused before any device
    allocation."""
    from engine.graph_runner import DecodeGraphRunner

    cfg = ModelConfig(vocab_size=32, hidden_size=32, intermediate_size=32, num_layers=1, num_q_heads=2,
                      num_kv_heads=1, head_dim=16)
    cache = PagedKVCache(cfg, 8, 4, "cpu", torch.float32)
    with pytest.raises(ValueError):
        DecodeGraphRunner(None, cache, BlockManager(8, 4), max_batch=2, max_context=16)


def test_device_tables_follow_the_manager():
    """DeviceBlockTables (on a CPU tensor here) mirrors every live sequence's table in its row after sync(), through
    allocations, appends across block boundaries, frees and row reuse; sequences allocated before it was made are
    picked up; too many live sequences is an error."""
    from engine.device_tables import DeviceBlockTables

    rng = random.Random(5)
    m = BlockManager(400, 4)
    m.allocate(100, 9)
    dt = DeviceBlockTables(m, "cpu", max_seqs=8, max_blocks=64)
    live = {100}
    for step in range(300):
        op = rng.random()
        if op < 0.25 and len(live) < 8:
            s = rng.randrange(1000)
            if s not in live and m.can_allocate(40):
                m.allocate(s, rng.randrange(0, 40))
                live.add(s)
        elif op < 0.35 and live:
            s = rng.choice(sorted(live))
            m.free(s)
            live.discard(s)
        elif live:
            s = rng.choice(sorted(live))
            if m.can_append(s, 3) and m.seq_len(s) < 200:
                m.append_slots(s, rng.randrange(1, 4))
        if step % 7 == 0:
            dt.sync()
            for s in live:
                t = m.block_table(s)
                assert dt.table[dt.row(s), :len(t)].tolist() == t
    assert len({dt.row(s) for s in live}) == len(live)
    while len(live) < 8:
        s = max(live) + 1
        m.allocate(s, 1)
        live.add(s)
    with pytest.raises(RuntimeError):
        m.allocate(max(live) + 1, 1)


def test_parity_helper_admits_only_output_rounding():
    """assert_decode_close (the GPU parity bar): an element passes within 8e-3 of the fp32 oracle or as one of the
    two bf16 values around it. Planted on the CPU: a result one bf16 unit beyond the bracket at |ref| in [4, 8)
    (1.6e-2 off) fails; the correctly rounded value and the other side of the bracket pass; small values need 8e-3."""
    import numpy as np
    import pytest
    import torch

    from cases import assert_decode_close, bf16_bracket

    rng = np.random.default_rng(0)
    ref = np.concatenate([rng.standard_normal(500), rng.uniform(4, 8, 500) * rng.choice([-1, 1], 500)])
    ref = ref.astype(np.float32).astype(np.float64)
    lo, hi = bf16_bracket(ref)
    rne = torch.from_numpy(ref.astype(np.float32)).bfloat16().double().numpy()
    assert np.all((rne == lo) | (rne == hi)) and np.all(lo <= ref) and np.all(ref <= hi)
    assert np.all(hi - lo <= np.abs(ref) * 2.0 ** -7)
    assert_decode_close(rne, ref, "correctly rounded")
    assert_decode_close(np.where(rne == lo, hi, lo), ref, "other side of the bracket")
    big = np.abs(ref) >= 4
    bad = rne.copy()
    bad[big] = np.where(ref[big] > 0, hi[big] + (hi[big] - lo[big]), lo[big] - (hi[big] - lo[big]))
    with pytest.raises(AssertionError):
        assert_decode_close(bad, ref, "one unit past the bracket")
    ref2, off = ref.copy(), rne.copy()
    ref2[3], off[3] = 0.5, 0.51171875  # three bf16 units (1.2e-2) above a bf16 oracle value of 0.5
    with pytest.raises(AssertionError):
        assert_decode_close(off, ref2, "1.2e-2 off at |ref| = 0.5")


def _plan_per_token(slot_of: dict, free: list, slots_cpu, query_starts, context_lens, B):
    """A plain per-token restatement of the reference's format-B staging plan (engine/quant_cache.py:84-122): group
    the forward's slots by block in order of first token; a block without a slot written whole at offsets 0 .. B-1
    is quantized directly from its rows; every other block takes a slot (from the end of the free list) on first
    use and stages its rows; a block whose last offset is written is done and gives its slot back after the loop;
    each sequence's tail is the slot of its last block when that block is partial. Mutates slot_of and free."""
    by_block = {}
    for row, slot in enumerate(slots_cpu):
        by_block.setdefault(slot // B, []).append((row, slot % B))
    staged, done, whole, whole_rows = [], [], [], []
    for b, items in by_block.items():
        if b not in slot_of and items[0][1] == 0 and len(items) == B:
            whole.append(b)
            whole_rows += [r for r, _ in items]
            continue
        if b not in slot_of:
            slot_of[b] = free.pop()
        staged += [(r, slot_of[b], o) for r, o in items]
        if items[-1][1] == B - 1:
            done.append(b)
    done_slots = [slot_of[b] for b in done]
    for b in done:
        free.append(slot_of.pop(b))
    tails = []
    for i, ctx in enumerate(context_lens):
        last_block = slots_cpu[query_starts[i + 1] - 1] // B
        tails.append(slot_of[last_block] if ctx % B else -1)
    return staged, done, done_slots, whole, whole_rows, tails


def test_plan_staging_equals_the_per_token_plan():
    """engine/quant_cache.plan_staging (vectorised: one pass over held slots, tails by binary search) equals the
    plain per-token plan over 400 random mixed forwards of a live block manager: decode rows, prefill chunks of
    1-40 tokens (whole 16-token blocks among them), sequences that start and finish (freed blocks return their
    slots through the manager's listener, in the same order for both); every plan field and the book's state
    (block -> slot map, free-slot stack order) after each forward."""
    import random

    from engine.block_manager import BlockManager
    from engine.paged_cache import build_metadata
    from engine.quant_cache import StagingBook, plan_staging

    B, rng = 16, random.Random(3)
    m = BlockManager(4096, B)
    book = StagingBook(256)
    ref_slot_of, ref_free = {}, list(book.free)

    def release_both(blocks):
        book.release(blocks)
        for b in blocks:
            s = ref_slot_of.pop(b, None)
            if s is not None:
                ref_free.append(s)

    m.add_free_listener(release_both)
    live, next_id, checked = {}, 0, 0
    for step in range(400):
        for s in [s for s in live if rng.random() < 0.08]:
            m.free(s)
            del live[s]
        while len(live) < 12 and rng.random() < 0.7:
            m.allocate(next_id, 0)
            live[next_id] = 0
            next_id += 1
        batch = []
        for s in sorted(live):
            n = 1 if rng.random() < 0.6 else rng.choice([rng.randint(1, 40), B, 2 * B, B - live[s] % B])
            m.append_slots(s, n)
            batch.append((s, live[s], n))
            live[s] += n
        if not batch:
            continue
        meta = build_metadata(m, batch, "cpu")
        args = (meta.slots_cpu, meta.query_starts, meta.context_lens, B)
        plan = plan_staging(book, *args)
        staged, done, done_slots, whole, whole_rows, tails = _plan_per_token(ref_slot_of, ref_free, *args)
        assert [tuple(x) for x in zip(plan.staged_rows.tolist(), plan.staged_slots.tolist(),
                                      plan.staged_offs.tolist())] == staged, step
        assert plan.done_blocks.tolist() == done and plan.done_slots.tolist() == done_slots, step
        assert plan.whole_blocks.tolist() == whole and plan.whole_rows.tolist() == whole_rows, step
        assert plan.tails.tolist() == tails, step
        assert book.slot_of == ref_slot_of and book.free == ref_free, step
        checked += len(meta.slots_cpu)
    assert checked > 3000 and next_id > 20
