"""sipa_decode_noalloc (the allocation-free decode entry point, split workspace in the library's device array)
against sipa_decode with a caller workspace: identical outputs, bit for bit, through the C ABI, on two calls in a
row whose second is smaller (the array keeps the first call's contents), for the split grid, the ragged work list
and an INT8 pool; sizes past the array are refused before any launch."""

import ctypes

import numpy as np
import pytest
import torch

from cases import HEADS, make_case
from engine import _hip
from engine.hip_decode import DecodePlan, QuantKV

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 16 << 20


def both_entries(plan: DecodePlan, q, k, v, quant=None):
    """Outputs of sipa_decode (the plan's own workspace) and of sipa_decode_noalloc for the same parameters."""
    lib, st = _hip.lib(), plan.stream
    out_ws = torch.full(plan.shape, float("nan"), device="cuda", dtype=plan.dtype)
    out_na = torch.full(plan.shape, float("nan"), device="cuda", dtype=plan.dtype)
    plan(q=q, k_cache=k, v_cache=v, quant=quant, out=out_ws)
    p = _hip.DecodeParams.from_buffer_copy(plan.params)
    p.workspace, p.workspace_bytes = None, 0
    p.out, p.out_stride_s, p.out_stride_h = out_na.data_ptr(), out_na.stride(0), out_na.stride(1)
    rc = lib.sipa_decode_noalloc(ctypes.byref(p), st)
    assert rc == _hip.OK, lib.sipa_last_error()
    torch.cuda.synchronize()
    return out_ws, out_na


@pytest.mark.parametrize("path", ["grid", "work list", "int8"])
def test_noalloc_equals_workspace_entry_on_two_calls(path):
    Hq, Hkv, D = HEADS["0.5B"]
    first, second = [8192] * 24, [300, 5000, 17]  # the second call smaller: fewer sequences and splits
    if path == "work list":
        first = [16, 3000, 9000, 40, 700, 12000, 2500, 65] * 3
    for call, lengths in enumerate((first, second)):
        q, k, v, bt, ctx, tables = make_case(lengths, Hq, Hkv, D, 16, torch.bfloat16, seed=50 + call)
        quant = None
        if path == "int8":
            g = torch.Generator(device="cuda").manual_seed(60 + call)
            k = torch.randint(-127, 128, k.shape, device="cuda", dtype=torch.int8, generator=g)
            v = torch.randint(-127, 128, v.shape, device="cuda", dtype=torch.int8, generator=g)
            ks = (torch.rand(k.shape[:3], device="cuda", generator=g) / 64 + 1 / 256).half()
            vs = (torch.rand(v.shape[:3], device="cuda", generator=g) / 64 + 1 / 256).half()
            quant = QuantKV(1, ks, vs)
        plan = DecodePlan(q, k, v, bt, ctx, D ** -0.5, max(lengths), quant=quant, host_context_lens=lengths,
                          work_list="on" if path == "work list" else "off")
        print(f"case noalloc {path} call {call}: {len(lengths)} sequences, {plan.splits} splits", flush=True)
        assert plan.splits > 1  # the split workspace is in use
        out_ws, out_na = both_entries(plan, q, k, v, quant)
        assert not torch.isnan(out_ws).any()
        assert torch.equal(out_ws, out_na), f"call {call}: the allocation-free entry differs"


def test_noalloc_refuses_a_workspace_past_its_array():
    """A split count whose partials exceed the 16 MiB array fails with SIPA_EWORKSPACE and launches nothing (the
    output keeps its contents)."""
    Hq, Hkv, D = HEADS["1.5B"]
    lengths = [512] * 600  # 8 splits of 64 tokens: 600 x 12 heads x 8 splits x (128 + 2) x 4 B > 16 MiB
    q, k, v, bt, ctx, tables = make_case(lengths, Hq, Hkv, D, 16, torch.bfloat16, seed=70, spare=1)
    plan = DecodePlan(q, k, v, bt, ctx, D ** -0.5, 512, num_splits=8)
    assert plan.splits == 8
    need = _hip.lib().sipa_decode_workspace_bytes(600, Hq, Hkv, D, 8)
    assert need > SCRATCH_BYTES
    out = torch.full(plan.shape, 3.0, device="cuda", dtype=plan.dtype)
    p = _hip.DecodeParams.from_buffer_copy(plan.params)
    p.out = out.data_ptr()
    rc = _hip.lib().sipa_decode_noalloc(ctypes.byref(p), plan.stream)
    assert rc == _hip.EWORKSPACE
    assert b"allocation-free" in _hip.lib().sipa_last_error()
    torch.cuda.synchronize()
    assert bool((out == 3.0).all())
