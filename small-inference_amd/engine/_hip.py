"""ctypes binding of libsmallinf_hip.so, the C ABI declared in include/smallinf_hip.h.

The decode and store paths run only through this library. If it is missing or fails to load, every kernel entry
point raises: there is no CPU or torch fallback behind the HIP backends.

torch is imported first on purpose: its bundled libamdhip64 (SONAME libamdhip64.so.7) is then the HIP runtime
the library binds to, so torch's device pointers and streams are valid in our launches.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch  # noqa: F401  (load torch's HIP runtime before the library; see the module docstring)

# SIPA_LIB overrides the location (for copies of these modules placed inside another package).
LIB_PATH = Path(os.environ.get("SIPA_LIB") or Path(__file__).resolve().parent.parent / "build" / "libsmallinf_hip.so")
ABI_VERSION = 8

# element types (SIPA_F32 ...)
F32, BF16, F16, I8 = 0, 1, 2, 3
# return codes
OK, EINVAL, EUNSUPPORTED, EHIP, EWORKSPACE = 0, -1, -2, -3, -4
# kv modes, implementations, combine strategies
KV_PLAIN, KV_INT8_TOKEN, KV_INT8_KCHAN = 0, 1, 2
IMPL = {"auto": 0, "valu": 1, "mfma": 2, "valu_stream": 3, "valu_dot2": 4, "mfma_pbf16": 5}
COMBINE = {"fused": 0, "kernel": 1}

_c = ctypes
i32, i64, f32, vp = _c.c_int32, _c.c_int64, _c.c_float, _c.c_void_p


class DecodeParams(ctypes.Structure):
    """Mirror of struct sipa_decode_params (field order and types must match the header)."""
    _fields_ = [
        ("struct_size", i32), ("num_seqs", i32), ("num_q_heads", i32), ("num_kv_heads", i32), ("head_dim", i32),
        ("block_size", i32), ("num_blocks", i32), ("max_context", i32), ("num_splits", i32), ("q_dtype", i32),
        ("kv_mode", i32), ("impl", i32), ("combine", i32), ("scale", f32),
        ("q", vp), ("q_stride_s", i64), ("q_stride_h", i64),
        ("k_cache", vp), ("v_cache", vp), ("kv_stride_h", i64), ("kv_stride_n", i64),
        ("block_tables", vp), ("bt_stride_s", i64), ("context_lens", vp),
        ("out", vp), ("out_stride_s", i64), ("out_stride_h", i64),
        ("k_scale", vp), ("k_scale_dtype", i32), ("ks_stride_h", i64), ("ks_stride_n", i64),
        ("v_scale", vp), ("v_scale_dtype", i32), ("vs_stride_h", i64), ("vs_stride_n", i64),
        ("stage", vp), ("st_stride_h", i64), ("st_stride_n", i64), ("st_stride_b", i64),
        ("tail_slots", vp), ("workspace", vp), ("workspace_bytes", i64),
        ("work_items", vp), ("num_items", i32), ("bt_width", i32), ("num_stage", i32),
    ]


class PrefillParams(ctypes.Structure):
    """Mirror of struct sipa_prefill_params."""
    _fields_ = [
        ("struct_size", i32), ("num_seqs", i32), ("num_tokens", i32), ("num_q_heads", i32), ("num_kv_heads", i32),
        ("head_dim", i32), ("block_size", i32), ("num_blocks", i32), ("max_context", i32), ("max_query_len", i32),
        ("scale", f32),
        ("q", vp), ("q_stride_t", i64), ("q_stride_h", i64),
        ("k_cache", vp), ("v_cache", vp), ("kv_stride_h", i64), ("kv_stride_n", i64),
        ("block_tables", vp), ("bt_stride_s", i64), ("context_lens", vp), ("query_starts", vp), ("query_lens", vp),
        ("out", vp), ("out_stride_t", i64), ("out_stride_h", i64),
        ("kv_mode", i32), ("k_scale", vp), ("k_scale_dtype", i32), ("ks_stride_h", i64), ("ks_stride_n", i64),
        ("v_scale", vp), ("v_scale_dtype", i32), ("vs_stride_h", i64), ("vs_stride_n", i64),
        ("stage", vp), ("st_stride_h", i64), ("st_stride_n", i64), ("st_stride_b", i64), ("num_stage", i32),
        ("tail_slots", vp), ("num_splits", i32), ("workspace", vp), ("workspace_bytes", i64), ("bt_width", i32),
        ("merge_path", i32), ("wg_layout", i32),
    ]


class KchanWriteParams(ctypes.Structure):
    """Mirror of struct sipa_kchan_write_params."""
    _fields_ = [
        ("k", vp), ("v", vp), ("x_dtype", i32),
        ("k_stride_t", i64), ("k_stride_h", i64), ("v_stride_t", i64), ("v_stride_h", i64),
        ("T", i32), ("H", i32), ("D", i32), ("B", i32),
        ("blocks", vp), ("offsets", vp), ("stage_slots", vp), ("quant_dst", vp),
        ("v_pool", vp), ("v_scale", vp), ("k_pool", vp), ("k_scale", vp),
        ("q_stride_h", i64), ("q_stride_n", i64), ("vs_stride_h", i64), ("vs_stride_n", i64),
        ("ks_stride_h", i64), ("ks_stride_n", i64),
        ("stage", vp), ("st_stride_h", i64), ("st_stride_n", i64), ("st_stride_b", i64),
    ]


# name -> (restype, argtypes); every symbol the header declares
SIGNATURES = {
    "sipa_abi_version": (i32, []),
    "sipa_last_error": (_c.c_char_p, []),
    "sipa_device_cu_count": (i32, [i32]),
    "sipa_choose_splits": (i32, [i32, i32, i32, i32]),
    "sipa_choose_splits_for": (i32, [i32, i32, i32, i32, i32]),
    "sipa_split_chunk": (i32, [i32, i32]),
    "sipa_decode_workspace_bytes": (i64, [i32, i32, i32, i32, i32]),
    "sipa_decode_split_grid": (i32, [i32, i32, i32, i32, i32, vp, vp, vp]),
    "sipa_decode": (i32, [_c.POINTER(DecodeParams), vp]),
    "sipa_decode_noalloc": (i32, [_c.POINTER(DecodeParams), vp]),
    "sipa_decode_noalloc_reset": (i32, [vp]),
    "sipa_build_work_list": (i32, [vp, i32, i32, i32, i32, i32, vp, i32, vp]),
    "sipa_check_work_list": (i32, [vp, i32, i32, i32, i32, i32]),
    "sipa_prefill": (i32, [_c.POINTER(PrefillParams), vp]),
    "sipa_paged_metadata": (i32, [vp, i64, i32, i32, vp, i32, i32, i32, i32, vp, vp, vp, vp, vp, vp, vp, vp]),
    "sipa_prefill_splits": (i32, [i32, i32, i32, i64, i32, i32]),
    "sipa_prefill_workspace_bytes": (i64, [i32, i32, i32, i32, i32, i32, i32]),
    "sipa_quantize_store_tokens": (i32, [vp, i32, i64, i64, i32, i32, i32, vp, vp, vp, i64, i64, i32, vp, i64, i64,
                                         vp]),
    "sipa_quantize_store_tokens_kv": (i32, [vp, vp, i32, i64, i64, i64, i64, i32, i32, i32, vp, vp, vp, vp, i64, i64,
                                            i32, vp, vp, i64, i64, vp]),
    "sipa_quantize_store_blocks": (i32, [vp, i32, i64, i64, i64, vp, vp, i32, i32, i32, i32, vp, i64, i64, vp, i64,
                                         i64, vp]),
    "sipa_quantize_store_block_rows": (i32, [vp, i32, i64, i64, vp, vp, i32, i32, i32, i32, vp, i64, i64, vp, i64,
                                             i64, vp]),
    "sipa_store_tokens": (i32, [vp, vp, i32, i64, i64, i64, i64, vp, i32, i32, i32, vp, vp, vp, vp, i32, i64, i64,
                                i64, vp]),
    "sipa_kchan_write_rows": (i32, [_c.POINTER(KchanWriteParams), vp]),
}

_lib = None


class HipLibraryError(RuntimeError):
    """libsmallinf_hip.so is missing, stale, or failed at run time."""


def lib() -> ctypes.CDLL:
    """The loaded library (loaded on first use). Raises HipLibraryError if it is not built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise HipLibraryError(f"{LIB_PATH} is not built; run `python small-inference_amd/build.py` "
                                  "(or __graft_entry__.build())")
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype, fn.argtypes = res, args
        if handle.sipa_abi_version() != ABI_VERSION:
            raise HipLibraryError(f"{LIB_PATH} has ABI {handle.sipa_abi_version()}, this binding {ABI_VERSION}")
        _lib = handle
    return _lib


def check(rc: int, what: str) -> None:
    """Raise for a negative return code: ValueError for bad arguments, HipLibraryError otherwise."""
    if rc == OK:
        return
    msg = lib().sipa_last_error().decode(errors="replace")
    if rc in (EINVAL, EUNSUPPORTED, EWORKSPACE):
        raise ValueError(f"{what}: {msg}")
    raise HipLibraryError(f"{what} failed ({rc}): {msg}")


_DTYPES = {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16, torch.int8: I8}


def dtype_code(dt: torch.dtype) -> int:
    """SIPA_* code of a torch dtype."""
    try:
        return _DTYPES[dt]
    except KeyError:
        raise ValueError(f"dtype {dt} is not supported by the HIP kernels") from None


def ptr(t: torch.Tensor | None) -> int | None:
    """Device address of a tensor's first element (None for None)."""
    return None if t is None else t.data_ptr()


def stream_of(t: torch.Tensor) -> int:
    """The current torch stream of t's device, as a hipStream_t value."""
    return torch.cuda.current_stream(t.device).cuda_stream


def require_gpu(*tensors: torch.Tensor) -> None:
    """The kernels read device memory: every tensor must live on one GPU."""
    devs = {t.device for t in tensors if t is not None}
    if len(devs) != 1 or next(iter(devs)).type != "cuda":
        raise ValueError(f"HIP kernels need all tensors on one GPU, got {sorted(map(str, devs))}")
