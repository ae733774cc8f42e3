"""The C-ABI library loads, exports every entry point include/smallinf_hip.h declares, and rejects bad arguments
on the host before launching anything (no GPU needed)."""

import ctypes
import re
from pathlib import Path

import pytest

from engine import _hip

HEADER = Path(__file__).resolve().parents[1] / "include" / "smallinf_hip.h"


def declared_functions() -> list[str]:
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\**(sipa_\w+)\s*\(", text, flags=re.M)))


def test_library_exports_every_declared_symbol():
    lib = _hip.lib()
    names = declared_functions()
    assert len(names) >= 10, names
    for name in names:
        assert hasattr(lib, name), f"{name} declared in the header but not exported"
    assert set(names) == set(_hip.SIGNATURES), "the ctypes binding and the header disagree"


def test_abi_and_struct_layout():
    assert _hip.lib().sipa_abi_version() == _hip.ABI_VERSION == 8
    # 13 int32 + 1 float, then pointers/strides: the binding's layout is what the header's struct gives; the
    # work-list fields, then the table width and staging count come last.
    assert _hip.DecodeParams.work_items.offset == _hip.DecodeParams.workspace_bytes.offset + 8
    assert _hip.DecodeParams.bt_width.offset == _hip.DecodeParams.num_items.offset + 4
    pad8 = lambda n: -(-n // 8) * 8  # noqa: E731  (the structs hold 8-byte members: their size rounds up to 8)
    assert ctypes.sizeof(_hip.DecodeParams) == pad8(_hip.DecodeParams.num_stage.offset + 4)
    assert _hip.PrefillParams.merge_path.offset == _hip.PrefillParams.bt_width.offset + 4
    assert _hip.PrefillParams.wg_layout.offset == _hip.PrefillParams.merge_path.offset + 4
    assert ctypes.sizeof(_hip.PrefillParams) == pad8(_hip.PrefillParams.wg_layout.offset + 4)


def bad_params(**over):
    p = _hip.DecodeParams()
    p.struct_size = ctypes.sizeof(_hip.DecodeParams)
    p.num_seqs, p.num_q_heads, p.num_kv_heads, p.head_dim, p.block_size = 1, 14, 2, 64, 16
    p.max_context, p.num_blocks, p.q_dtype, p.scale = 16, 64, _hip.BF16, 0.125
    p.bt_width = 1024  # covers 16384 tokens
    for ptr in ("q", "k_cache", "v_cache", "block_tables", "context_lens", "out"):
        setattr(p, ptr, 4096)
    for k, v in over.items():
        setattr(p, k, v)
    return p


@pytest.mark.parametrize("over,code", [
    ({"struct_size": 8}, _hip.EINVAL),
    ({"num_q_heads": 13}, _hip.EINVAL),
    ({"num_q_heads": 34}, _hip.EUNSUPPORTED),          # group 17 > 16
    ({"head_dim": 96}, _hip.EUNSUPPORTED),
    ({"block_size": 12}, _hip.EINVAL),                  # must divide 64
    ({"max_context": 0}, _hip.EINVAL),
    ({"num_blocks": 0}, _hip.EINVAL),
    ({"q_dtype": _hip.F16}, _hip.EUNSUPPORTED),
    ({"scale": 0.0}, _hip.EINVAL),                      # the kernels take maxima of the unscaled scores
    ({"scale": -0.125}, _hip.EINVAL),
    ({"scale": float("inf")}, _hip.EINVAL),
    ({"kv_mode": 1}, _hip.EINVAL),                      # INT8 without scales
    ({"k_cache": 4100}, _hip.EINVAL),                   # unaligned pool
    ({"out": None}, _hip.EINVAL),
    ({"max_context": 8192, "num_splits": 16}, _hip.EWORKSPACE),
    ({"bt_width": 0}, _hip.EINVAL),
    ({"max_context": 16385}, _hip.EINVAL),              # a table row of 1024 entries covers 16384 tokens
    ({"bt_width": 511, "max_context": 8192}, _hip.EINVAL),
    ({"kv_mode": 2, "k_scale": 4096, "v_scale": 4096, "k_scale_dtype": _hip.F16, "v_scale_dtype": _hip.F16,
      "stage": 4096, "tail_slots": 4096, "num_stage": 0}, _hip.EINVAL),  # per-channel K without staging slots
])
def test_decode_rejects_bad_arguments_before_launch(over, code):
    lib = _hip.lib()
    rc = lib.sipa_decode(ctypes.byref(bad_params(**over)), None)
    assert rc == code, lib.sipa_last_error()
    assert lib.sipa_last_error()


def test_zero_sequences_is_a_no_op():
    assert _hip.lib().sipa_decode(ctypes.byref(bad_params(num_seqs=0)), None) == _hip.OK


def test_store_entry_points_reject_bad_arguments():
    lib = _hip.lib()
    assert lib.sipa_quantize_store_tokens(4096, _hip.BF16, 128, 64, 4, 2, 48, 4096, 4096, 4096, 1, 1, 16, 4096,
                                          1, 1, None) == _hip.EUNSUPPORTED
    assert lib.sipa_quantize_store_tokens(None, _hip.BF16, 128, 64, 0, 2, 64, None, None, None, 1, 1, 16, None, 1,
                                          1, None) == _hip.OK  # T = 0
    assert lib.sipa_quantize_store_blocks(4096, _hip.I8, 1, 1, 1, 4096, 4096, 1, 2, 16, 64, 4096, 1, 1, 4096, 1, 1,
                                          None) == _hip.EUNSUPPORTED
    assert lib.sipa_store_tokens(4096, 4096, _hip.BF16, 1, 1, 1, 1, None, 3, 2, 64, 4096, 4096, 4096, None,
                                 _hip.BF16, 1, 1, 1, None) == _hip.EINVAL  # x2 without pool2


def test_split_policy_host_side():
    """CU-count split policy: at most one workgroup per CU; splits of at most 2048 tokens (64-token multiples) and,
    past 8 splits, at least 512 (short contexts: up to 8 splits of at least 128); a grid that is already full is
    not split unless a sequence is longer than 2048 tokens. The INT8 policy sizes for two workgroups per CU,
    splits of at least 256 tokens past 8 splits and at most 4096."""
    lib = _hip.lib()
    for S, Hkv, ctx in [(1, 2, 8192), (32, 2, 8192), (256, 2, 8192), (64, 2, 4096), (1, 2, 1024), (512, 2, 300),
                        (1, 2, 16384), (8, 2, 4096)]:
        req = lib.sipa_choose_splits(S, Hkv, ctx, 256)
        chunk = lib.sipa_split_chunk(ctx, req)
        launched = -(-ctx // chunk)
        assert chunk % 64 == 0 and chunk <= 2048
        assert S * Hkv * launched <= max(256, S * Hkv * -(-ctx // 2048)), (S, Hkv, ctx, req, chunk)
        assert launched <= 8 or chunk >= 512, (S, Hkv, ctx, req, chunk)
        assert lib.sipa_choose_splits_for(S, Hkv, ctx, 256, 0) == req
    # the measured optima of the policy's comment (bf16, 2 KV heads)
    for S, ctx, want in [(1, 1024, 8), (1, 8192, 16), (1, 16384, 32), (4, 8192, 16), (8, 4096, 8), (16, 2048, 8),
                         (32, 8192, 4), (256, 8192, 4), (512, 300, 1)]:
        assert lib.sipa_choose_splits(S, 2, ctx, 256) == want, (S, ctx)
    assert lib.sipa_split_chunk(8192, 4) == 2048
    # INT8: twice the CUs, 256-token floor, 4096-token ceiling
    assert lib.sipa_choose_splits_for(1, 2, 4096, 256, 1) == 16
    assert lib.sipa_choose_splits_for(1, 2, 1024, 256, 1) == 8      # short context: 8 splits of 128
    assert lib.sipa_choose_splits_for(64, 2, 4096, 256, 1) == 4
    assert lib.sipa_choose_splits_for(128, 2, 9000, 256, 2) == 5    # a full grid: splits of at most 2048 tokens
    assert lib.sipa_choose_splits_for(1, 2, 9000, 256, 2) == 36     # 256-token splits (2 x 256 CUs / 2 programs)
    assert lib.sipa_decode_workspace_bytes(32, 14, 2, 64, 1) == 0


def work_list(lengths, Hkv, cu=256, per_cu=2, max_piece=0):
    lib = _hip.lib()
    ctx = (ctypes.c_int32 * len(lengths))(*lengths)
    n = lib.sipa_build_work_list(ctx, len(lengths), Hkv, cu, per_cu, max_piece, None, 0, None)
    assert n > 0
    items = (ctypes.c_int32 * (8 * n))()
    maxs = ctypes.c_int32(0)
    assert lib.sipa_build_work_list(ctx, len(lengths), Hkv, cu, per_cu, max_piece, items, n, ctypes.byref(maxs)) == n
    return [tuple(items[8 * i:8 * i + 8]) for i in range(n)], maxs.value


@pytest.mark.parametrize("seed", range(5))
def test_work_list_partitions_every_pair(seed):
    """Each (sequence, KV head) pair is cut into pieces that tile [0, ctx) exactly, start on 64-token boundaries
    and are numbered 0 .. n-1 with n recorded in every item; items are ordered longest first."""
    import random

    rng = random.Random(seed)
    lengths = [max(1, min(40000, int(rng.lognormvariate(6.4, 1.2)))) for _ in range(rng.randint(1, 300))]
    Hkv = rng.choice([1, 2, 4])
    items, maxs = work_list(lengths, Hkv)
    sizes = [e - b for (_, _, _, _, b, e, _, _) in items]
    assert sizes == sorted(sizes, reverse=True)
    pieces = {}
    for s, h, sp, n, b, e, z0, z1 in items:
        assert z0 == z1 == 0 and 0 <= b < e <= lengths[s] and b % 64 == 0 and 1 <= n <= maxs
        pieces.setdefault((s, h), []).append((sp, n, b, e))
    assert set(pieces) == {(s, h) for s in range(len(lengths)) for h in range(Hkv)}
    for (s, h), ps in pieces.items():
        ps.sort()
        assert [p[0] for p in ps] == list(range(len(ps))) and all(p[1] == len(ps) for p in ps)
        assert ps[0][2] == 0 and ps[-1][3] == lengths[s]
        assert all(a[3] == b[2] for a, b in zip(ps, ps[1:]))
        assert all(p[3] - p[2] <= 32768 for p in ps)
    assert maxs == max(len(ps) for ps in pieces.values())


def test_work_list_piece_size_and_errors():
    """Pieces are about total / (cu * items_per_cu) tokens, at least 256; bad lengths and short buffers fail."""
    items, maxs = work_list([8192] * 32, 2, cu=256, per_cu=2)  # 524288 token-heads / 512 -> 1024-token pieces
    assert len(items) == 512 and maxs == 8 and {e - b for *_, b, e, _, _ in items} == {1024}
    items, maxs = work_list([100, 50], 2)
    assert len(items) == 4 and maxs == 1
    lib = _hip.lib()
    bad = (ctypes.c_int32 * 2)(5, 0)
    assert lib.sipa_build_work_list(bad, 2, 2, 256, 2, 0, None, 0, None) == _hip.EINVAL
    ok = (ctypes.c_int32 * 2)(5000, 7)
    small = (ctypes.c_int32 * 8)()
    assert lib.sipa_build_work_list(ok, 2, 2, 256, 2, 0, small, 1, None) == _hip.EINVAL
    assert lib.sipa_build_work_list(ok, 2, 2, 256, 2, 100, None, 0, None) == _hip.EINVAL  # max_piece < 256
    items, maxs = work_list([40000, 300], 2, cu=4, per_cu=1, max_piece=4096)  # huge total: pieces capped
    assert max(e - b for *_, b, e, _, _ in items) <= 4096 and maxs == 10


def check_list(items, S, Hkv, max_ctx, splits):
    flat = (ctypes.c_int32 * (8 * max(1, len(items))))(*[x for it in items for x in it])
    return _hip.lib().sipa_check_work_list(flat, len(items), S, Hkv, max_ctx, splits)


@pytest.mark.parametrize("seed", range(3))
def test_work_list_check_accepts_built_lists_and_rejects_broken_ones(seed):
    """Lists from sipa_build_work_list pass the checker; a dropped, duplicated, renumbered, overlapping or
    out-of-range item is refused with SIPA_EINVAL (such a list would leave a merge counter non-zero)."""
    import random

    rng = random.Random(seed)
    lengths = [rng.randint(1, 20000) for _ in range(rng.randint(2, 40))]
    items, maxs = work_list(lengths, 2)
    S, mx = len(lengths), max(lengths)
    assert check_list(items, S, 2, mx, maxs) == _hip.OK
    multi = [i for i, it in enumerate(items) if it[3] > 1]
    assert multi, "the case needs a pair with several splits"
    k = multi[0]
    bad = {
        "dropped": items[:k] + items[k + 1:],
        "duplicated": items + [items[k]],
        "renumbered": items[:k] + [items[k][:2] + (items[k][3],) + items[k][3:]] + items[k + 1:],
        "overlap": items[:k] + [items[k][:4] + (max(0, items[k][4] - 64) if items[k][2] else items[k][4],
                                              items[k][5] + 64) + items[k][6:]] + items[k + 1:],
        "sequence": items[:k] + [(S,) + items[k][1:]] + items[k + 1:],
        "past max_context": items[:k] + [items[k][:5] + (mx + 1,) + items[k][6:]] + items[k + 1:],
    }
    for name, lst in bad.items():
        assert check_list(lst, S, 2, mx, maxs) == _hip.EINVAL, name
    assert check_list(items, S, 2, mx, maxs - 1) == _hip.EINVAL  # num_splits below a pair's split count


def prefill_params(**over):
    p = _hip.PrefillParams()
    p.struct_size = ctypes.sizeof(_hip.PrefillParams)
    p.num_seqs, p.num_tokens, p.num_q_heads, p.num_kv_heads, p.head_dim, p.block_size = 2, 40, 14, 2, 64, 16
    p.num_blocks, p.max_context, p.max_query_len, p.scale = 8, 64, 32, 0.125
    p.q_stride_t, p.q_stride_h, p.out_stride_t, p.out_stride_h = 14 * 64, 64, 14 * 64, 64
    p.kv_stride_h, p.kv_stride_n, p.bt_stride_s, p.bt_width = 8 * 16 * 64, 16 * 64, 4, 2048
    for ptr in ("q", "k_cache", "v_cache", "block_tables", "context_lens", "query_starts", "query_lens", "out"):
        setattr(p, ptr, 4096)
    for k, v in over.items():
        setattr(p, k, v)
    return p


@pytest.mark.parametrize("over,code", [
    ({"struct_size": 8}, _hip.EINVAL),
    ({"num_q_heads": 13}, _hip.EINVAL),
    ({"num_q_heads": 18}, _hip.EUNSUPPORTED),           # group 9 > 8
    ({"head_dim": 96}, _hip.EUNSUPPORTED),
    ({"block_size": 32}, _hip.EUNSUPPORTED),
    ({"max_context": 32784}, _hip.EUNSUPPORTED),
    ({"num_tokens": 0}, _hip.EINVAL),
    ({"scale": -0.125}, _hip.EINVAL),
    ({"scale": float("nan")}, _hip.EINVAL),
    ({"query_lens": None}, _hip.EINVAL),
    ({"q": 4100}, _hip.EINVAL),                         # unaligned rows
    ({"out_stride_h": 66}, _hip.EINVAL),
    ({"kv_stride_n": 1020}, _hip.EINVAL),
    ({"bt_width": 3}, _hip.EINVAL),                     # 3 x 16 tokens < max_context 64
    ({"bt_width": 0}, _hip.EINVAL),
])
def test_prefill_rejects_bad_arguments_before_launch(over, code):
    lib = _hip.lib()
    rc = lib.sipa_prefill(ctypes.byref(prefill_params(**over)), None)
    assert rc == code, lib.sipa_last_error()
    assert lib.sipa_last_error()


def test_prefill_layout_and_empty_calls():
    """The binding's struct size is the library's (a mismatch is rejected), and empty batches launch nothing."""
    lib = _hip.lib()
    assert lib.sipa_prefill(ctypes.byref(prefill_params(num_seqs=0)), None) == _hip.OK
    assert lib.sipa_prefill(ctypes.byref(prefill_params(max_query_len=0)), None) == _hip.OK


def test_prefill_split_policy_and_workspace():
    """About two workgroups per CU over (KV head, 16-token query tile) units, no split under 256 keys, at most
    32; the workspace holds (m, l) fp32 (the row's exponent in l's low mantissa bits) and O / l fp16 for 8 heads
    x 16 tokens per unit and split, and nothing for one split."""
    lib = _hip.lib()
    assert lib.sipa_prefill_splits(12, 2, 128, 32, 8192, 256) == 8    # 1.5B, 512-token chunk at 8K: 64 units
    assert lib.sipa_prefill_splits(14, 2, 64, 32, 8192, 256) == 8     # 0.5B likewise
    assert lib.sipa_prefill_splits(14, 2, 64, 512, 2048, 256) == 1    # 4 prompts of 2048: 1024 units
    assert lib.sipa_prefill_splits(8, 2, 128, 32, 8192, 256) == 16    # G = 4: 32-token units, 32 of them
    assert lib.sipa_prefill_splits(14, 2, 64, 1, 100, 256) == 1       # never under 256 keys per split
    assert lib.sipa_prefill_splits(7, 1, 128, 1, 32768, 256) == 32    # capped
    assert lib.sipa_prefill_workspace_bytes(1, 12, 2, 128, 512, 8192, 1) == 0
    rows = 2 * 32 * 8 * 128           # units x splits x 8 columns x 16 tokens, after the 256 KiB of counters
    got = lib.sipa_prefill_workspace_bytes(1, 12, 2, 128, 512, 8192, 8)
    assert (1 << 18) + rows * (2 * 128 + 8) <= got <= (1 << 18) + rows * (2 * 128 + 8) + 3 * 256
    d64 = lib.sipa_prefill_workspace_bytes(1, 14, 2, 64, 512, 8192, 8)
    assert (1 << 18) + rows * (2 * 64 + 8) <= d64 <= (1 << 18) + rows * (2 * 64 + 8) + 3 * 256
    assert lib.sipa_prefill_workspace_bytes(1, 4, 2, 64, 512, 8192, 8) < d64  # G = 2: 64-token units
    rc = lib.sipa_prefill(ctypes.byref(prefill_params(max_context=8192, num_splits=8)), None)
    assert rc == _hip.EWORKSPACE, lib.sipa_last_error()


def test_kchan_write_rows_checks_arguments():
    """The format-B decode write refuses bad shapes and missing pools before any launch; no rows is a no-op."""
    lib = _hip.lib()

    def params(**over):
        p = _hip.KchanWriteParams()
        p.T, p.H, p.D, p.B, p.x_dtype = 4, 2, 64, 16, _hip.BF16
        for name in ("k", "v", "blocks", "offsets", "stage_slots", "v_pool", "v_scale", "k_pool", "k_scale", "stage"):
            setattr(p, name, 4096)
        for key, val in over.items():
            setattr(p, key, val)
        return p

    assert lib.sipa_kchan_write_rows(ctypes.byref(params(T=0)), None) == _hip.OK
    assert lib.sipa_kchan_write_rows(None, None) == _hip.EINVAL
    assert lib.sipa_kchan_write_rows(ctypes.byref(params(D=24)), None) == _hip.EUNSUPPORTED
    assert lib.sipa_kchan_write_rows(ctypes.byref(params(B=65)), None) == _hip.EUNSUPPORTED
    assert lib.sipa_kchan_write_rows(ctypes.byref(params(x_dtype=99)), None) == _hip.EUNSUPPORTED
    assert lib.sipa_kchan_write_rows(ctypes.byref(params(stage=None)), None) == _hip.EINVAL
    assert lib.sipa_kchan_write_rows(ctypes.byref(params(H=0)), None) == _hip.EINVAL
