"""Paged decode attention and quantize-on-write over a BF16 / FP8 (e4m3fn) / INT8 KV cache, on HIP.

The Python surface of the path. Tensors stay on the GPU, nothing here synchronizes with the host, and the
work is done by the gfx950 kernels in `libbpt_amd.so` (there is no other implementation to fall back to).

Conventions, as in fastserve (paths relative to its src/fastserve/):

* Pools are `[num_blocks, page_size, Hkv, D]` per layer (engine/kv_cache.py:108). Any strided view with
  those four dimensions works, e.g. a head-major pool `[num_blocks, Hkv, page_size, D]` passed as
  `pool.transpose(1, 2)`.
* Block tables are `[B, max_blocks]`, int64 like engine/kv_cache.py:149 or int32; entries past a
  sequence's length are never read (engine/kv_cache.py:148 pads them with block 0).
* `context_lens[b]` counts the tokens the cache holds for sequence b, this step's new tokens included
  (they are stored before attention, integration/kv_cache.py:160-168). Query i of Q sits at position
  `context_lens[b] - Q + i` and sees every slot up to it (engine/attention.py:12-20).
* GQA: KV head h serves query heads h*G ... h*G + G - 1 (engine/attention.py:23-31).
* Bad arguments raise ValueError (kernels/kv_attention.py:216-217 style); HIP failures raise BptError.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from ._lib import (
    F_BF16,
    F_F16,
    F_F32,
    IDX_I32,
    IDX_I64,
    KV_BF16,
    KV_FP8_E4M3FN,
    KV_INT8,
    SCALE_NONE,
    SCALE_PER_HEAD,
    SCALE_PER_TOKEN_HEAD,
)

_FLOAT_CODES = {torch.bfloat16: F_BF16, torch.float16: F_F16, torch.float32: F_F32}
_INDEX_CODES = {torch.int32: IDX_I32, torch.int64: IDX_I64}


def kv_dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.bfloat16:
        return KV_BF16
    if dtype == torch.float8_e4m3fn:
        return KV_FP8_E4M3FN
    if dtype == torch.int8:
        return KV_INT8
    raise ValueError(f"KV cache dtype must be bfloat16, float8_e4m3fn or int8, got {dtype}")


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


def _scale_layout(k_scale, v_scale, kv_code: int, pool_shape) -> tuple[int, tuple[int, int, int]]:
    """Scale kind and the (block, token, head) strides of per-token-head scale pools."""
    if kv_code == KV_BF16:
        _require(k_scale is None and v_scale is None, "a bfloat16 cache takes no scales")
        return SCALE_NONE, (0, 0, 0)
    _require(k_scale is not None and v_scale is not None, "k_scale and v_scale are required for a quantized cache")
    for s in (k_scale, v_scale):
        _require(s.dtype == torch.float32, f"scales must be float32, got {s.dtype}")
    nb, p, hkv, _ = pool_shape
    if k_scale.dim() == 1:
        _require(tuple(k_scale.shape) == (hkv,) and tuple(v_scale.shape) == (hkv,), f"per-head scales must be [{hkv}]")
        _require(k_scale.is_contiguous() and v_scale.is_contiguous(), "per-head scales must be contiguous")
        return SCALE_PER_HEAD, (0, 0, 0)
    _require(
        tuple(k_scale.shape) == (nb, p, hkv) and tuple(v_scale.shape) == (nb, p, hkv),
        f"per-token-head scales must be [{nb}, {p}, {hkv}] like the pools",
    )
    _require(k_scale.stride() == v_scale.stride(), "k_scale and v_scale must share strides")
    return SCALE_PER_TOKEN_HEAD, tuple(k_scale.stride())


def _decode_args(
    q, k_cache, v_cache, block_table, context_lens, k_scale, v_scale, scale, max_context, num_splits, out_dtype
) -> tuple[_lib.DecodeArgs, tuple[int, int, int, int]]:
    _require(q.dim() == 4, f"q must be [B, Q, Hq, D], got {tuple(q.shape)}")
    b, nq, hq, d = q.shape
    _require(q.dtype in _FLOAT_CODES, f"q must be bf16, f16 or f32, got {q.dtype}")
    _require(q.stride(-1) == 1, "q's channel dimension must be contiguous")
    _require(k_cache.dim() == 4 and k_cache.shape == v_cache.shape, "k_cache and v_cache must be [NB, P, Hkv, D]")
    _require(k_cache.dtype == v_cache.dtype, "k_cache and v_cache must share a dtype")
    _require(k_cache.stride() == v_cache.stride(), "k_cache and v_cache must share strides")
    _require(k_cache.stride(-1) == 1, "the caches' channel dimension must be contiguous")
    kv_code = kv_dtype_code(k_cache.dtype)
    nb, page, hkv, dk = k_cache.shape
    _require(dk == d, f"q head_dim {d} != cache head_dim {dk}")
    _require(block_table.dim() == 2 and block_table.shape[0] == b, f"block_table must be [{b}, max_blocks]")
    _require(block_table.dtype in _INDEX_CODES, "block_table must be int32 or int64")
    _require(block_table.stride(1) == 1, "block_table rows must be contiguous")
    if context_lens is not None:
        _require(context_lens.dim() == 1 and context_lens.shape[0] == b, f"context_lens must be [{b}]")
        _require(context_lens.dtype == torch.int32 and context_lens.is_contiguous(), "context_lens must be contiguous int32")
    _require(out_dtype in _FLOAT_CODES, f"out dtype must be bf16, f16 or f32, got {out_dtype}")
    scale_kind, sc_strides = _scale_layout(k_scale, v_scale, kv_code, k_cache.shape)

    a = _lib.DecodeArgs()
    a.struct_size = ctypes.sizeof(_lib.DecodeArgs)
    a.kv_dtype = kv_code
    a.scale_kind = scale_kind
    a.q_dtype = _FLOAT_CODES[q.dtype]
    a.out_dtype = _FLOAT_CODES[out_dtype]
    a.table_dtype = _INDEX_CODES[block_table.dtype]
    a.batch, a.num_queries, a.num_q_heads, a.num_kv_heads, a.head_dim, a.page_size = b, nq, hq, hkv, d, page
    a.num_blocks = nb
    a.max_blocks_per_seq = block_table.shape[1]
    a.max_context = int(max_context)
    a.num_splits = int(num_splits or 0)
    a.sm_scale = float(scale)
    a.q = q.data_ptr()
    a.q_stride_b, a.q_stride_q, a.q_stride_h = q.stride(0), q.stride(1), q.stride(2)
    a.k_cache, a.v_cache = k_cache.data_ptr(), v_cache.data_ptr()
    a.kv_stride_block, a.kv_stride_token, a.kv_stride_head = k_cache.stride(0), k_cache.stride(1), k_cache.stride(2)
    a.k_scale, a.v_scale = _ptr(k_scale), _ptr(v_scale)
    a.scale_stride_block, a.scale_stride_token, a.scale_stride_head = sc_strides
    a.block_table = block_table.data_ptr()
    a.table_stride_b = block_table.stride(0)
    a.context_lens = _ptr(context_lens)
    return a, (b, nq, hq, d)


def _plan(q, k_cache, v_cache, block_table, context_lens, k_scale, v_scale, scale, max_context, num_splits):
    q4 = q if q.dim() == 4 else q[:, None]
    a, _ = _decode_args(
        q4, k_cache, v_cache, block_table, context_lens, k_scale, v_scale, scale, max_context, num_splits,
        torch.bfloat16,
    )
    ws, cnt = ctypes.c_size_t(0), ctypes.c_size_t(0)
    _lib.check(_lib.lib().bpt_decode_plan(ctypes.byref(a), ctypes.byref(ws), ctypes.byref(cnt)))
    return a, ws.value, cnt.value


def decode_plan(
    q, k_cache, v_cache, block_table, context_lens, k_scale=None, v_scale=None, *, scale, max_context, num_splits=None
) -> tuple[int, int, int, int]:
    """(workgroups, tokens per chunk, workspace bytes, counter bytes) the call would use. Host only."""
    a, ws, cnt = _plan(q, k_cache, v_cache, block_table, context_lens, k_scale, v_scale, scale, max_context,
                       num_splits)
    return a.grid_groups, a.chunk_tokens, ws, cnt


def decode_kernel_name(
    q, k_cache, v_cache, block_table, context_lens, k_scale=None, v_scale=None, *, scale, max_context, num_splits=None
) -> str:
    """The kernel the call launches: "decode_mfma_kernel" (matrix cores) or "decode_kernel" (vector)."""
    a, _, _ = _plan(q, k_cache, v_cache, block_table, context_lens, k_scale, v_scale, scale, max_context,
                    num_splits)
    return "decode_mfma_kernel" if a.rows_per_group == 16 else "decode_kernel"


# Per (device, stream): one partials workspace and one zero-filled counter buffer. The kernel leaves the
# counters at zero, so calls issued in order on one stream share them; other streams get their own.
_BUFFERS: dict[tuple[str, int, int], torch.Tensor] = {}
_GRAIN = 1 << 20


def cached_buffer(kind: str, device: torch.device, stream: int, nbytes: int) -> torch.Tensor:
    """The cached zero-initialized uint8 buffer `kind` for (device, stream), grown to at least `nbytes`."""
    key = (kind, device.index if device.index is not None else torch.cuda.current_device(), stream)
    buf = _BUFFERS.get(key)
    if buf is None or buf.numel() < nbytes:
        size = max((nbytes + _GRAIN - 1) // _GRAIN * _GRAIN, _GRAIN)
        buf = torch.zeros(size, dtype=torch.uint8, device=device)
        _BUFFERS[key] = buf
    return buf


def paged_decode_attention(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_table: torch.Tensor,
    context_lens: torch.Tensor,
    k_scale: torch.Tensor | None = None,
    v_scale: torch.Tensor | None = None,
    *,
    scale: float,
    max_context: int,
    num_splits: int | None = None,
    out: torch.Tensor | None = None,
    out_dtype: torch.dtype = torch.bfloat16,
    workspace: torch.Tensor | None = None,
    counters: torch.Tensor | None = None,
    lse: torch.Tensor | None = None,
    _cascade: dict | None = None,
    _events: tuple | None = None,
    _append: object | None = None,
) -> torch.Tensor:
    """softmax(q kᵀ · scale) v over each sequence's paged cache, dequantized in registers.

    q             [B, Q, Hq, D] (or [B, Hq, D] for one query per sequence), bf16 / f16 / f32
    k/v_cache     [num_blocks, page_size, Hkv, D] views, bfloat16 / float8_e4m3fn / int8
    block_table   [B, max_blocks] int32 or int64
    context_lens  [B] int32, at most `max_context`
    k/v_scale     FP8 or INT8 only: [Hkv] per head, or [num_blocks, page_size, Hkv] per token and head (fp32)
    max_context   upper bound on context_lens, known on the host (no device read); sizes the launch
    num_splits    split-K partitions of a max_context-long sequence (None: balanced over the whole batch)
    out           optional [B, Q, Hq, D] output buffer; returned
    workspace     optional device buffer of at least decode_plan(...)[2] bytes for the split-K partials
    counters      optional device buffer of at least decode_plan(...)[3] bytes, zero-filled before its first
                  use (every call leaves it zeroed); default for both: cached per (device, stream)
    lse           optional contiguous float32 [B, Q, Hq] (or [B, Hq]) receiving each row's log-sum-exp of
                  scale * q.k over the tokens it saw (natural log, -inf for none): with `out` in float32 it is
                  the partial that kernels/reference.py:205-211 merges

    Returns out [B, Q, Hq, D] (or [B, Hq, D]) in `out_dtype` (bf16 by default). One kernel launch.
    """
    squeeze = q.dim() == 3
    q4 = q[:, None] if squeeze else q
    a, (b, nq, hq, d) = _decode_args(
        q4, k_cache, v_cache, block_table, context_lens, k_scale, v_scale, scale, max_context, num_splits,
        out.dtype if out is not None else out_dtype,
    )
    dev = q.device
    _require(dev.type == "cuda", "paged_decode_attention runs on a GPU: q must be a cuda tensor")
    for name, t in (("k_cache", k_cache), ("v_cache", v_cache), ("block_table", block_table),
                    ("context_lens", context_lens), ("k_scale", k_scale), ("v_scale", v_scale)):
        _require(t is None or t.device == dev, f"{name} is on {t.device if t is not None else None}, q on {dev}")
    if out is None:
        out4 = torch.empty((b, nq, hq, d), dtype=out_dtype, device=dev)
    else:
        out4 = out[:, None] if out.dim() == 3 else out
        _require(tuple(out4.shape) == (b, nq, hq, d), f"out must be [{b}, {nq}, {hq}, {d}]")
        _require(out4.stride(-1) == 1 and out4.device == dev, "out must be a cuda tensor with contiguous channels")
    a.out = out4.data_ptr()
    a.out_stride_b, a.out_stride_q, a.out_stride_h = out4.stride(0), out4.stride(1), out4.stride(2)
    if lse is not None:
        _require(lse.dtype == torch.float32 and lse.is_contiguous() and lse.numel() == b * nq * hq and lse.device == dev,
                 f"lse must be a contiguous float32 tensor of {b} x {nq} x {hq} on q's device")
        a.lse_out = lse.data_ptr()
    if _cascade is not None:  # the cascade's two launches (cascade.py): flags, length offset, partial to merge
        a.flags = _cascade.get("flags", 0)
        a.len_offset = _cascade.get("len_offset", 0)
        merge = _cascade.get("merge")
        if merge is not None:
            m_out, m_lse = merge
            _require(m_out.dtype == torch.float32 and m_out.is_contiguous() and tuple(m_out.shape) == (b, nq, hq, d),
                     "the merged partial must be contiguous float32 [B, Q, Hq, D]")
            _require(m_lse.dtype == torch.float32 and m_lse.is_contiguous() and m_lse.numel() == b * nq * hq,
                     "the merged partial's lse must be contiguous float32 [B, Q, Hq]")
            a.merge_out, a.merge_lse = m_out.data_ptr(), m_lse.data_ptr()
    lib = _lib.lib()
    ws_bytes, cnt_bytes = ctypes.c_size_t(0), ctypes.c_size_t(0)
    _lib.check(lib.bpt_decode_plan(ctypes.byref(a), ctypes.byref(ws_bytes), ctypes.byref(cnt_bytes)))
    stream = _stream(dev)
    if workspace is None:
        workspace = cached_buffer("partials", dev, stream, ws_bytes.value)
    if counters is None:
        counters = cached_buffer("counters", dev, stream, cnt_bytes.value)
    for name, t in (("workspace", workspace), ("counters", counters)):
        _require(t.device == dev and t.is_contiguous(), f"{name} must be a contiguous tensor on q's device")
    a.workspace, a.workspace_bytes = workspace.data_ptr(), workspace.numel() * workspace.element_size()
    a.counters, a.counters_bytes = counters.data_ptr(), counters.numel() * counters.element_size()
    if _append is not None:  # paged_append_decode: store the new rows, then attend (one launch where it can)
        _lib.check(lib.bpt_paged_append_decode(ctypes.byref(_append), ctypes.byref(a), ctypes.c_void_p(stream)))
    elif _events is None:
        _lib.check(lib.bpt_paged_decode(ctypes.byref(a), ctypes.c_void_p(stream)))
    else:  # measurement: two raw hipEvent_t handles recorded around the kernel itself
        _lib.check(lib.bpt_paged_decode_timed(ctypes.byref(a), ctypes.c_void_p(stream), ctypes.c_void_p(_events[0]),
                                              ctypes.c_void_p(_events[1])))
    result = out if out is not None else out4
    return result[:, 0] if (squeeze and result.dim() == 4) else result


def quantize_append(
    k: torch.Tensor,
    v: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    k_scale: torch.Tensor | None,
    v_scale: torch.Tensor | None,
    write_blocks: torch.Tensor,
    write_offsets: torch.Tensor,
) -> None:
    """Store new rows k, v [B, Q, Hkv, D] at slot write_offsets[b, i] of page write_blocks[b, i].

    FP8 with [Hkv] scales: code = e4m3fn(clamp(x / scale[h], ±448)) (kv/quant.py:44-45 with a per-head scale).
    INT8 (or FP8) with [num_blocks, page_size, Hkv] scales: a fresh per-token-head scale
    max(amax / 127, 1e-12) (448 for FP8) is computed and stored next to the codes (quant/w8a8.py:55-74).
    BF16: the rows are copied. Rows whose page is negative or outside the pool are skipped.
    """
    a, dev = _append_args(k, v, k_cache, v_cache, k_scale, v_scale, write_blocks, write_offsets)
    _lib.check(_lib.lib().bpt_quant_append(ctypes.byref(a), ctypes.c_void_p(_stream(dev))))


def _append_args(k, v, k_cache, v_cache, k_scale, v_scale, write_blocks, write_offsets):
    """The checked bpt_append_args of quantize_append's arguments, and their device."""
    _require(k.dim() == 4 and k.shape == v.shape, "k and v must be [B, Q, Hkv, D]")
    _require(k.dtype == v.dtype and k.dtype in _FLOAT_CODES, "k and v must share a bf16/f16/f32 dtype")
    _require(k.stride() == v.stride() and k.stride(-1) == 1, "k and v must share strides, channels contiguous")
    b, nq, hkv, d = k.shape
    _require(k_cache.dim() == 4 and k_cache.shape == v_cache.shape, "k_cache and v_cache must be [NB, P, Hkv, D]")
    _require(k_cache.dtype == v_cache.dtype and k_cache.stride() == v_cache.stride(), "caches must match")
    _require(k_cache.shape[2] == hkv and k_cache.shape[3] == d, "cache heads/head_dim must match the rows")
    _require(k_cache.stride(-1) == 1, "the caches' channel dimension must be contiguous")
    kv_code = kv_dtype_code(k_cache.dtype)
    scale_kind, sc_strides = _scale_layout(k_scale, v_scale, kv_code, k_cache.shape)
    _require(write_blocks.shape == (b, nq) and write_offsets.shape == (b, nq), f"write slots must be [{b}, {nq}]")
    _require(write_blocks.dtype == write_offsets.dtype and write_blocks.dtype in _INDEX_CODES, "slots: int32/int64")
    _require(write_blocks.stride() == write_offsets.stride(), "write_blocks and write_offsets must share strides")
    dev = k.device
    _require(dev.type == "cuda", "quantize_append runs on a GPU: k must be a cuda tensor")
    for name, t in (("v", v), ("k_cache", k_cache), ("v_cache", v_cache), ("write_blocks", write_blocks),
                    ("write_offsets", write_offsets), ("k_scale", k_scale), ("v_scale", v_scale)):
        _require(t is None or t.device == dev, f"{name} is not on {dev}")

    a = _lib.AppendArgs()
    a.struct_size = ctypes.sizeof(_lib.AppendArgs)
    a.kv_dtype, a.scale_kind = kv_code, scale_kind
    a.src_dtype = _FLOAT_CODES[k.dtype]
    a.slot_dtype = _INDEX_CODES[write_blocks.dtype]
    a.batch, a.num_queries, a.num_kv_heads, a.head_dim = b, nq, hkv, d
    a.page_size, a.num_blocks = k_cache.shape[1], k_cache.shape[0]
    a.k, a.v = k.data_ptr(), v.data_ptr()
    a.new_stride_b, a.new_stride_q, a.new_stride_h = k.stride(0), k.stride(1), k.stride(2)
    a.write_blocks, a.write_offsets = write_blocks.data_ptr(), write_offsets.data_ptr()
    a.slot_stride_b, a.slot_stride_q = write_blocks.stride(0), write_blocks.stride(1)
    a.k_cache, a.v_cache = k_cache.data_ptr(), v_cache.data_ptr()
    a.kv_stride_block, a.kv_stride_token, a.kv_stride_head = k_cache.stride(0), k_cache.stride(1), k_cache.stride(2)
    a.k_scale, a.v_scale = _ptr(k_scale), _ptr(v_scale)
    a.scale_stride_block, a.scale_stride_token, a.scale_stride_head = sc_strides
    return a, dev


def paged_append_decode(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_table: torch.Tensor,
    context_lens: torch.Tensor,
    k_scale: torch.Tensor | None,
    v_scale: torch.Tensor | None,
    write_blocks: torch.Tensor,
    write_offsets: torch.Tensor,
    *,
    scale: float,
    max_context: int,
    num_splits: int | None = None,
    out: torch.Tensor | None = None,
    out_dtype: torch.dtype = torch.bfloat16,
) -> torch.Tensor:
    """Store the new rows k, v [B, Q, Hkv, D] (as quantize_append), then attend (as paged_decode_attention):
    the cache's store-then-attend (integration/kv_cache.py:160-192).

    The rows are the last Q tokens of each sequence (row i of sequence b is token context_lens[b] - Q + i), and a
    row is stored only where the decode reads that token (its write slot is the block table's page and offset for
    it, as paged_prepare produces them); a row with no slot (-1) or a slot elsewhere is not stored. One launch when
    the decode runs on the matrix-core kernel with per-head scales, Q <= 8, bf16 rows, head dim 128: the kernel
    stores the codes and uses them for those tokens directly. Otherwise the store, then the decode, with the
    same results.
    """
    a, dev = _append_args(k, v, k_cache, v_cache, k_scale, v_scale, write_blocks, write_offsets)
    _require(q.device == dev, f"q is on {q.device}, the new rows on {dev}")
    return paged_decode_attention(q, k_cache, v_cache, block_table, context_lens, k_scale, v_scale, scale=scale,
                                  max_context=max_context, num_splits=num_splits, out=out, out_dtype=out_dtype,
                                  _append=a)


def paged_prepare(
    table: torch.Tensor,
    reserved: torch.Tensor,
    slots: torch.Tensor,
    positions: torch.Tensor,
    page_size: int,
    block_table: torch.Tensor,
    write_blocks: torch.Tensor,
    write_offsets: torch.Tensor,
    context_lens: torch.Tensor,
) -> None:
    """Per-forward paged metadata on the device (bpt_paged_prepare; engine/kv_cache.py:140-156 without the host
    round trip): from each row's slot of the device table [num_slots, max_blocks] (reserved[slot] blocks held)
    and the positions [B, Q], fill block_table [B, n_blocks] (padded with block 0), write_blocks / write_offsets
    [B, Q] and context_lens [B] (the last position + 1, clamped to the reserved tokens). A position gets a write
    block only when it is its row's token context_len - Q + i inside the reserved blocks (-1 otherwise: positions
    past the reservation or out of order store nothing). One launch, no host read."""
    _require(table.dtype == torch.int32 and table.dim() == 2 and table.stride(1) == 1, "table: int32 [slots, blocks]")
    _require(reserved.dtype == torch.int32 and reserved.is_contiguous() and reserved.numel() == table.shape[0],
             "reserved: int32 [slots]")
    _require(positions.dim() == 2 and positions.dtype in _INDEX_CODES, "positions: int32 / int64 [B, Q]")
    b, nq = positions.shape
    _require(slots.dtype == torch.int32 and slots.is_contiguous() and slots.numel() == b, f"slots: int32 [{b}]")
    for name, t, shape in (("block_table", block_table, None), ("write_blocks", write_blocks, (b, nq)),
                           ("write_offsets", write_offsets, (b, nq)), ("context_lens", context_lens, (b,))):
        _require(t.dtype == torch.int32 and t.is_contiguous() and (shape is None or tuple(t.shape) == shape),
                 f"{name}: contiguous int32")
    _require(block_table.dim() == 2 and block_table.shape[0] == b, f"block_table: [{b}, n_blocks]")
    dev = positions.device
    for name, t in (("table", table), ("reserved", reserved), ("slots", slots), ("block_table", block_table)):
        _require(t.device == dev, f"{name} is not on {dev}")
    a = _lib.PrepareArgs()
    a.struct_size = ctypes.sizeof(_lib.PrepareArgs)
    a.batch, a.num_queries, a.n_blocks = b, nq, block_table.shape[1]
    a.num_slots, a.max_blocks, a.page_size = table.shape[0], table.shape[1], page_size
    a.positions_dtype = _INDEX_CODES[positions.dtype]
    a.table, a.table_stride = table.data_ptr(), table.stride(0)
    a.reserved, a.slots = reserved.data_ptr(), slots.data_ptr()
    a.positions, a.pos_stride_b, a.pos_stride_q = positions.data_ptr(), positions.stride(0), positions.stride(1)
    a.block_table, a.write_blocks = block_table.data_ptr(), write_blocks.data_ptr()
    a.write_offsets, a.context_lens = write_offsets.data_ptr(), context_lens.data_ptr()
    _lib.check(_lib.lib().bpt_paged_prepare(ctypes.byref(a), ctypes.c_void_p(_stream(dev))))


def kv_read_bytes(context_lens_host, num_kv_heads: int, head_dim: int, kv_dtype: torch.dtype, per_token_scales: bool,
                  num_queries: int = 1) -> int:
    """Algorithmic KV bytes one call must read: codes for K and V, plus scales (q, out, tables excluded)."""
    elem = 2 if kv_dtype == torch.bfloat16 else 1
    tokens = int(sum(int(t) for t in context_lens_host))
    per_token = num_kv_heads * head_dim * 2 * elem
    if per_token_scales:
        per_token += num_kv_heads * 2 * 4
    total = tokens * per_token
    if kv_dtype != torch.bfloat16 and not per_token_scales:
        total += num_kv_heads * 2 * 4
    return total
