"""The path end to end under a model (engine/model.py drives the cache as the reference's model does), after the
reference's model-level tests (tests/test_paged.py:99-130): a prompt prefilled in chunks gives the logits of the
same prompt prefilled in one forward, a packed batch gives each sequence's logits from its own forwards, decode
steps continue from either, and the HIP backend agrees with the gather backend (the reference's attention).

Tolerances, written here: the schedules differ in split counts and so in the order of fp32 sums, which moves a few
bf16 logits by a few bf16 steps through the layers: max-abs 0.02 x max|logit| with a mean under 2e-3 x max|logit|;
against the gather backend, whose reference attention also rounds scores to bf16 (engine/attention.py:22-27),
0.05 x max|logit| and a mean under 5e-3 x max|logit|.
"""

import pytest
import torch

from cases import fragmented_manager
from engine.config import ModelConfig
from engine.model import Qwen2Model
from engine.paged_cache import PagedKVCache, build_metadata
from engine.quant_cache import QuantPagedKVCache

pytestmark = pytest.mark.gpu

CFG = ModelConfig(vocab_size=512, hidden_size=896, intermediate_size=512, num_layers=2, num_q_heads=14,
                  num_kv_heads=2, head_dim=64)


def close(a, b, frac=0.02, mean_frac=2e-3, what=""):
    a, b = a.float(), b.float()
    scale = b.abs().max().item()
    err = (a - b).abs()
    assert err.max().item() <= frac * scale, f"{what}: max {err.max().item():.3e} of scale {scale:.3e}"
    assert err.mean().item() <= mean_frac * scale, f"{what}: mean {err.mean().item():.3e} of scale {scale:.3e}"


def new_cache(fmt, m, backend="triton"):
    if fmt == "bf16":
        return PagedKVCache(CFG, m.num_blocks, 16, "cuda", torch.bfloat16, attn_backend=backend)
    return QuantPagedKVCache(CFG, m.num_blocks, 16, "cuda", torch.bfloat16, backend, fmt, m, n_stage=32)


def run(model, cache, m, batch, ids):
    """One forward over batch [(seq, start, n)] whose slots were appended; logits of every token."""
    meta = build_metadata(m, batch, "cuda")
    return model.forward(ids, meta.positions, cache, meta, last_only=False)


@pytest.mark.parametrize("fmt", ["bf16", "int8", "int8-kchannel"])
def test_chunked_prefill_then_decode(fmt):
    """300-token prompt in one forward vs in chunks of 100, 117 and 83, then 4 decode steps each."""
    model = Qwen2Model(CFG, "cuda", torch.bfloat16, seed=2, max_positions=1024, std=0.05)
    g = torch.Generator(device="cuda").manual_seed(3)
    prompt = torch.randint(0, CFG.vocab_size, (300,), device="cuda", generator=g)
    caches, logits = [], []
    for chunks in ([300], [100, 117, 83]):
        print(f"case {fmt} chunks {chunks}", flush=True)
        m = fragmented_manager(256, 16, torch.Generator().manual_seed(5))
        cache = new_cache(fmt, m)
        m.allocate(0, 0)
        outs, at = [], 0
        for n in chunks:
            m.append_slots(0, n)
            outs.append(run(model, cache, m, [(0, at, n)], prompt[at:at + n]))
            at += n
        caches.append((m, cache))
        logits.append(torch.cat(outs))
    torch.cuda.synchronize()
    close(logits[1], logits[0], what="chunked vs one-shot prefill")
    tok = logits[0][-1].argmax().view(1)
    for step in range(4):
        steps = []
        for m, cache in caches:
            m.append_slot(0)
            steps.append(run(model, cache, m, [(0, m.seq_len(0) - 1, 1)], tok))
        torch.cuda.synchronize()
        close(steps[1], steps[0], what=f"decode step {step}")
        tok = steps[0][-1].argmax().view(1)


def test_packed_batch_matches_individual_forwards():
    """Three prompts (37, 300, 16 tokens) prefilled each in its own forward vs packed in one, then one packed decode
    step against three single ones; and the packed forward on the gather backend."""
    model = Qwen2Model(CFG, "cuda", torch.bfloat16, seed=4, max_positions=1024, std=0.05)
    g = torch.Generator(device="cuda").manual_seed(6)
    lens = [37, 300, 16]
    prompts = [torch.randint(0, CFG.vocab_size, (n,), device="cuda", generator=g) for n in lens]
    res = {}
    for mode in ("single", "packed", "gather"):
        m = fragmented_manager(256, 16, torch.Generator().manual_seed(7))
        cache = new_cache("bf16", m, "gather" if mode == "gather" else "triton")
        for s, n in enumerate(lens):
            m.allocate(s, n)
        if mode == "single":
            pre = [run(model, cache, m, [(s, 0, n)], prompts[s]) for s, n in enumerate(lens)]
        else:
            pre = list(run(model, cache, m, [(s, 0, n) for s, n in enumerate(lens)], torch.cat(prompts))
                       .split(lens))
        toks = torch.stack([p[-1].argmax() for p in pre]) if mode == "single" else res["single"][2]
        for s in range(3):
            m.append_slot(s)
        batch = [(s, n, 1) for s, n in enumerate(lens)]
        if mode == "single":
            dec = torch.cat([run(model, cache, m, [batch[s]], toks[s:s + 1]) for s in range(3)])
        else:
            dec = run(model, cache, m, batch, toks)
        res[mode] = (torch.cat(pre), dec, toks)
        print(f"case packed mode {mode}", flush=True)
    torch.cuda.synchronize()
    close(res["packed"][0], res["single"][0], what="packed vs single prefill")
    close(res["packed"][1], res["single"][1], what="packed vs single decode")
    close(res["gather"][0], res["packed"][0], 0.05, 5e-3, what="gather backend vs kernels, prefill")
    close(res["gather"][1], res["packed"][1], 0.05, 5e-3, what="gather backend vs kernels, decode")
