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


_FIRST_CALL_UNDER_CAPTURE = r"""
import ctypes, sys
import torch
sys.path[:0] = [sys.argv[1], sys.argv[2], sys.argv[3]]
from cases import HEADS, make_case
from engine import _hip
from engine.hip_decode import DecodePlan
Hq, Hkv, D = HEADS["0.5B"]
lengths = [8192] * 16 + [300, 5000]
q, k, v, bt, ctx, tables = make_case(lengths, Hq, Hkv, D, 16, torch.bfloat16, seed=80)
plan = DecodePlan(q, k, v, bt, ctx, D ** -0.5, max(lengths))
assert plan.splits > 1
out_ws = torch.empty(plan.shape, device="cuda", dtype=plan.dtype)
plan(q=q, k_cache=k, v_cache=v, out=out_ws)
out_na = torch.full(plan.shape, float("nan"), device="cuda", dtype=plan.dtype)
p = _hip.DecodeParams.from_buffer_copy(plan.params)
p.workspace, p.workspace_bytes = None, 0
p.out, p.out_stride_s, p.out_stride_h = out_na.data_ptr(), out_na.stride(0), out_na.stride(1)
lib = _hip.lib()
torch.cuda.synchronize()
graph = torch.cuda.CUDAGraph()
print("capturing the process's first sipa_decode_noalloc call", flush=True)
with torch.cuda.graph(graph):
    rc = lib.sipa_decode_noalloc(ctypes.byref(p), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
assert rc == _hip.OK, lib.sipa_last_error()
torch.cuda.synchronize()
for i in range(4):
    out_na.fill_(float("nan"))
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(out_na, out_ws), f"replay {i} differs from sipa_decode"
free0 = torch.cuda.mem_get_info()[0]
st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
for _ in range(3):
    assert lib.sipa_decode_noalloc(ctypes.byref(p), st) == _hip.OK, lib.sipa_last_error()
torch.cuda.synchronize()
free1 = torch.cuda.mem_get_info()[0]
assert torch.equal(out_na, out_ws)
assert free1 == free0, (free0, free1)
print("ok: first call captured, 4 replays and 3 eager calls equal sipa_decode; free device memory unchanged", flush=True)
"""


def test_noalloc_first_call_under_graph_capture_in_a_fresh_process():
    """The use case the entry exists for: a process's first sipa_decode_noalloc call made while a HIP graph is
    being captured (the counter-clearing kernel is recorded as a node of the graph), replayed four times with eager
    work between the replays, then three eager calls; every output equals sipa_decode's with a caller workspace,
    and the device's free memory is the same before and after the eager calls. Runs in a child process, so that
    the call is the first of its process."""
    import subprocess
    import sys
    from pathlib import Path

    root = Path(__file__).resolve().parents[1]
    print("case noalloc: first call under capture (child process)", flush=True)
    r = subprocess.run([sys.executable, "-c", _FIRST_CALL_UNDER_CAPTURE, str(root / "tests"), str(root),
                        str(root / "small-inference_amd")], capture_output=True, text=True, timeout=110)
    print(r.stdout[-2000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0 and "ok: first call captured" in r.stdout


def test_noalloc_reset_recovers_after_an_inconsistent_work_list():
    """A work list that states three splits for a pair but lists two leaves that pair's merge counter in the
    library's array at two (forced from the host; every kernel ends normally, the pair is simply never merged).
    After sipa_decode_noalloc_reset, calls merge correctly again: the same call equals sipa_decode's output."""
    Hq, Hkv, D = HEADS["0.5B"]
    lengths = [3000, 2000]
    q, k, v, bt, ctx, tables = make_case(lengths, Hq, Hkv, D, 16, torch.bfloat16, seed=90)
    plan = DecodePlan(q, k, v, bt, ctx, D ** -0.5, max(lengths), host_context_lens=lengths, work_list="on")
    assert plan.splits > 1
    lib, st = _hip.lib(), plan.stream
    # pair (0, 0) claims 3 splits but lists 2; every other pair as the plan made it
    items = np.array([[0, 0, 0, 3, 0, 1024, 0, 0], [0, 0, 1, 3, 1024, 2048, 0, 0],
                      [1, 0, 0, 1, 0, 2000, 0, 0], [0, 1, 0, 1, 0, 3000, 0, 0], [1, 1, 0, 1, 0, 2000, 0, 0]],
                     dtype=np.int32)
    bad = torch.from_numpy(items).cuda()
    p = _hip.DecodeParams.from_buffer_copy(plan.params)
    p.workspace, p.workspace_bytes = None, 0
    p.work_items, p.num_items, p.num_splits = bad.data_ptr(), items.shape[0], 3
    scratch_out = torch.zeros(plan.shape, device="cuda", dtype=plan.dtype)
    p.out = scratch_out.data_ptr()
    print("case noalloc reset: inconsistent work list", flush=True)
    assert lib.sipa_decode_noalloc(ctypes.byref(p), st) == _hip.OK, lib.sipa_last_error()
    torch.cuda.synchronize()
    assert lib.sipa_decode_noalloc_reset(st) == _hip.OK, lib.sipa_last_error()
    out_ws, out_na = both_entries(plan, q, k, v)
    assert torch.equal(out_ws, out_na)
