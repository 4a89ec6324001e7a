"""ctypes binding of `libbpt_amd.so` (declared in include/bpt_amd.h).

The structures below mirror the C structs field for field; `struct_size` lets the library refuse a binding
that went stale. Loading fails loudly when the library has not been built: there is no fallback path.
"""

from __future__ import annotations

import ctypes
import functools
import hashlib
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libbpt_amd.so"
CSRC = Path(__file__).resolve().parent.parent / "csrc"
INCLUDE = Path(__file__).resolve().parent.parent.parent / "include"


def source_files() -> list[Path]:
    """Every file the library is compiled from: csrc/*.hip, csrc/*.h and include/*.h."""
    return sorted([*CSRC.glob("*.hip"), *CSRC.glob("*.h"), *INCLUDE.glob("*.h")])


def source_hash() -> str:
    """SHA-256 (first 16 hex digits) over the names and contents of the library's sources. The build embeds it
    in the library (bpt_source_hash), so a library built from other sources is refused at load time."""
    h = hashlib.sha256()
    for f in source_files():
        h.update(f.name.encode() + b"\0" + f.read_bytes() + b"\0")
    return h.hexdigest()[:16]

BPT_OK = 0
BPT_ERR_INVALID_ARGUMENT = 1
BPT_ERR_HIP = 2

KV_BF16, KV_FP8_E4M3FN, KV_INT8 = 0, 1, 2
SCALE_NONE, SCALE_PER_HEAD, SCALE_PER_TOKEN_HEAD = 0, 1, 2
F_BF16, F_F16, F_F32 = 0, 1, 2
IDX_I32, IDX_I64 = 0, 1

_vp = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64


class DecodeArgs(ctypes.Structure):
    _fields_ = [
        ("struct_size", ctypes.c_uint32),
        ("kv_dtype", _i32),
        ("scale_kind", _i32),
        ("q_dtype", _i32),
        ("out_dtype", _i32),
        ("table_dtype", _i32),
        ("batch", _i32),
        ("num_queries", _i32),
        ("num_q_heads", _i32),
        ("num_kv_heads", _i32),
        ("head_dim", _i32),
        ("page_size", _i32),
        ("num_blocks", _i32),
        ("max_blocks_per_seq", _i32),
        ("max_context", _i32),
        ("num_splits", _i32),
        ("chunk_tokens", _i32),
        ("grid_groups", _i32),
        ("rows_per_group", _i32),
        ("sm_scale", ctypes.c_float),
        ("q", _vp),
        ("q_stride_b", _i64),
        ("q_stride_q", _i64),
        ("q_stride_h", _i64),
        ("k_cache", _vp),
        ("v_cache", _vp),
        ("kv_stride_block", _i64),
        ("kv_stride_token", _i64),
        ("kv_stride_head", _i64),
        ("k_scale", _vp),
        ("v_scale", _vp),
        ("scale_stride_block", _i64),
        ("scale_stride_token", _i64),
        ("scale_stride_head", _i64),
        ("block_table", _vp),
        ("table_stride_b", _i64),
        ("context_lens", _vp),
        ("out", _vp),
        ("out_stride_b", _i64),
        ("out_stride_q", _i64),
        ("out_stride_h", _i64),
        ("workspace", _vp),
        ("workspace_bytes", ctypes.c_size_t),
        ("counters", _vp),
        ("counters_bytes", ctypes.c_size_t),
        ("flags", _i32),
        ("len_offset", _i32),
        ("lse_out", _vp),
        ("merge_out", _vp),
        ("merge_lse", _vp),
    ]


DECODE_NONCAUSAL = 1


class AppendArgs(ctypes.Structure):
    _fields_ = [
        ("struct_size", ctypes.c_uint32),
        ("kv_dtype", _i32),
        ("scale_kind", _i32),
        ("src_dtype", _i32),
        ("slot_dtype", _i32),
        ("batch", _i32),
        ("num_queries", _i32),
        ("num_kv_heads", _i32),
        ("head_dim", _i32),
        ("page_size", _i32),
        ("num_blocks", _i32),
        ("k", _vp),
        ("v", _vp),
        ("new_stride_b", _i64),
        ("new_stride_q", _i64),
        ("new_stride_h", _i64),
        ("write_blocks", _vp),
        ("write_offsets", _vp),
        ("slot_stride_b", _i64),
        ("slot_stride_q", _i64),
        ("k_cache", _vp),
        ("v_cache", _vp),
        ("kv_stride_block", _i64),
        ("kv_stride_token", _i64),
        ("kv_stride_head", _i64),
        ("k_scale", _vp),
        ("v_scale", _vp),
        ("scale_stride_block", _i64),
        ("scale_stride_token", _i64),
        ("scale_stride_head", _i64),
    ]


KIVI_INT4, KIVI_INT8, KIVI_F16, KIVI_BF16, KIVI_F32 = 0, 1, 2, 3, 4


class KiviArgs(ctypes.Structure):
    _fields_ = [
        ("struct_size", ctypes.c_uint32),
        ("format", _i32),
        ("q_dtype", _i32),
        ("batch", _i32),
        ("num_q_heads", _i32),
        ("num_kv_heads", _i32),
        ("head_dim", _i32),
        ("tokens", _i32),
        ("group", _i32),
        ("num_groups", _i32),
        ("split", _i32),
        ("num_splits", _i32),
        ("grid_groups", _i32),
        ("sm_scale", ctypes.c_float),
        ("q", _vp),
        ("q_stride_b", _i64),
        ("q_stride_h", _i64),
        ("k_codes", _vp),
        ("v_codes", _vp),
        ("code_stride_b", _i64),
        ("code_stride_h", _i64),
        ("code_stride_t", _i64),
        ("k_scale", _vp),
        ("k_zero", _vp),
        ("kgrid_stride_b", _i64),
        ("kgrid_stride_h", _i64),
        ("kgrid_stride_g", _i64),
        ("v_scale", _vp),
        ("v_zero", _vp),
        ("vgrid_stride_b", _i64),
        ("vgrid_stride_h", _i64),
        ("lengths", _vp),
        ("out", _vp),
        ("out_stride_b", _i64),
        ("out_stride_h", _i64),
        ("out_stride_s", _i64),
        ("lse", _vp),
        ("lse_stride_b", _i64),
        ("lse_stride_h", _i64),
        ("lse_stride_s", _i64),
        ("workspace", _vp),
        ("workspace_bytes", ctypes.c_size_t),
        ("counters", _vp),
        ("counters_bytes", ctypes.c_size_t),
        ("tail_k", _vp),
        ("tail_v", _vp),
        ("tail_stride_b", _i64),
        ("tail_stride_h", _i64),
        ("tail_stride_t", _i64),
        ("tail_dtype", _i32),
        ("tail_len", _i32),
    ]


class PrepareArgs(ctypes.Structure):
    _fields_ = [
        ("struct_size", ctypes.c_uint32),
        ("batch", _i32),
        ("num_queries", _i32),
        ("n_blocks", _i32),
        ("num_slots", _i32),
        ("max_blocks", _i32),
        ("page_size", _i32),
        ("positions_dtype", _i32),
        ("table", _vp),
        ("table_stride", _i64),
        ("reserved", _vp),
        ("slots", _vp),
        ("positions", _vp),
        ("pos_stride_b", _i64),
        ("pos_stride_q", _i64),
        ("block_table", _vp),
        ("write_blocks", _vp),
        ("write_offsets", _vp),
        ("context_lens", _vp),
    ]


class Tuning(ctypes.Structure):
    """bpt_tuning: plan constants for sweeps (a field at 0, or -1 for piece_cost, keeps the built-in choice)."""

    _fields_ = [
        ("struct_size", ctypes.c_uint32),
        ("groups_per_cu", _i32),
        ("piece_cost", _i32),
        ("min_chunks", _i32),
    ]


class KiviQuantArgs(ctypes.Structure):
    _fields_ = [
        ("struct_size", ctypes.c_uint32),
        ("bits", _i32),
        ("src_dtype", _i32),
        ("batch", _i32),
        ("num_kv_heads", _i32),
        ("tokens", _i32),
        ("head_dim", _i32),
        ("group", _i32),
        ("k", _vp),
        ("v", _vp),
        ("src_stride_b", _i64),
        ("src_stride_h", _i64),
        ("src_stride_t", _i64),
        ("k_codes", _vp),
        ("v_codes", _vp),
        ("code_stride_b", _i64),
        ("code_stride_h", _i64),
        ("code_stride_t", _i64),
        ("k_scale", _vp),
        ("k_zero", _vp),
        ("kgrid_stride_b", _i64),
        ("kgrid_stride_h", _i64),
        ("kgrid_stride_g", _i64),
        ("v_scale", _vp),
        ("v_zero", _vp),
        ("vgrid_stride_b", _i64),
        ("vgrid_stride_h", _i64),
    ]


class NormQuantArgs(ctypes.Structure):
    _fields_ = [
        ("struct_size", ctypes.c_uint32),
        ("x_dtype", _i32),
        ("weight_dtype", _i32),
        ("rows", _i32),
        ("d", _i32),
        ("eps", ctypes.c_float),
        ("x", _vp),
        ("x_stride_row", _i64),
        ("weight", _vp),
        ("codes", _vp),
        ("codes_stride_row", _i64),
        ("scale", _vp),
    ]


# Every symbol include/bpt_amd.h declares, with its ctypes signature.
SIGNATURES = {
    "bpt_decode_plan": (
        _i32,
        [ctypes.POINTER(DecodeArgs), ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_size_t)],
    ),
    "bpt_paged_decode": (_i32, [ctypes.POINTER(DecodeArgs), _vp]),
    "bpt_set_tuning": (_i32, [ctypes.POINTER(Tuning)]),
    "bpt_paged_decode_noalloc": (_i32, [ctypes.POINTER(DecodeArgs), _vp]),
    "bpt_paged_decode_timed": (_i32, [ctypes.POINTER(DecodeArgs), _vp, _vp, _vp]),
    "bpt_quant_append": (_i32, [ctypes.POINTER(AppendArgs), _vp]),
    "bpt_paged_append_decode": (_i32, [ctypes.POINTER(AppendArgs), ctypes.POINTER(DecodeArgs), _vp]),
    "bpt_kivi_plan": (
        _i32,
        [ctypes.POINTER(KiviArgs), ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_size_t)],
    ),
    "bpt_kivi_decode": (_i32, [ctypes.POINTER(KiviArgs), _vp]),
    "bpt_rms_norm_int8": (_i32, [ctypes.POINTER(NormQuantArgs), _vp]),
    "bpt_kivi_quantize": (_i32, [ctypes.POINTER(KiviQuantArgs), _vp]),
    "bpt_paged_prepare": (_i32, [ctypes.POINTER(PrepareArgs), _vp]),
    "bpt_last_error": (ctypes.c_char_p, []),
    "bpt_abi_version": (_i32, []),
    "bpt_source_hash": (ctypes.c_char_p, []),
    "bpt_fp8_decode_table": (_i32, [_vp, _vp]),
    "bpt_fp8_encode": (_i32, [_vp, ctypes.c_float, _vp, _i64, _vp]),
    "bpt_read_probe": (_i32, [_vp, ctypes.c_uint64, _vp, ctypes.POINTER(_i64), _vp]),
    "bpt_read_probe_timed": (_i32, [_vp, ctypes.c_uint64, _vp, _vp, _vp, _vp]),
    "bpt_page_read_probe": (_i32, [ctypes.POINTER(DecodeArgs), _vp, ctypes.POINTER(_i64), _vp, _vp, _vp]),
    "bpt_copy_probe": (_i32, [_vp, _vp, ctypes.c_uint64, _vp]),
}

ABI_VERSION = 13


class BptError(RuntimeError):
    """A HIP runtime error reported by the library."""


class StaleLibraryError(RuntimeError):
    """The built library was compiled from other sources than the ones in the tree."""


@functools.cache
def lib() -> ctypes.CDLL:
    """The loaded library. Raises if it was never built (the kernels have no fallback), or if it was built
    from sources other than the tree's (a stale build)."""
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"{LIB_PATH} is not built: run `python __graft_entry__.py` (build()) or "
            "`python bytes-per-token_amd/bpt_amd/_build.py` first"
        )
    handle = ctypes.CDLL(str(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = res
        fn.argtypes = args
    if handle.bpt_abi_version() != ABI_VERSION:
        raise RuntimeError(f"libbpt_amd.so ABI {handle.bpt_abi_version()} != binding {ABI_VERSION}: rebuild")
    built, tree = handle.bpt_source_hash().decode(), source_hash()
    if source_files() and built != tree:
        raise StaleLibraryError(f"{LIB_PATH} was built from sources {built}, the tree holds {tree}: rebuild it "
                                "(python bytes-per-token_amd/bpt_amd/_build.py)")
    return handle


def check(rc: int) -> None:
    """Turn a return code into the exception the reference's callers expect (ValueError for bad args)."""
    if rc == BPT_OK:
        return
    msg = lib().bpt_last_error().decode()
    if rc == BPT_ERR_INVALID_ARGUMENT:
        raise ValueError(msg)
    raise BptError(msg)


def set_tuning(groups_per_cu: int = 0, piece_cost: int = -1, min_chunks: int = 0) -> None:
    """Override the decode plan's constants process-wide (bpt_set_tuning), for tuning sweeps; no arguments
    restores the built-in ones."""
    t = Tuning(ctypes.sizeof(Tuning), groups_per_cu, piece_cost, min_chunks)
    check(lib().bpt_set_tuning(ctypes.byref(t)))
