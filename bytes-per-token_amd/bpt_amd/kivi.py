"""Decode attention over a KIVI-quantized KV cache, on HIP: fastserve's kernel-2 call surface.

Mirrors fastserve's kernels/kv_attention.py (paths relative to its src/fastserve/):

* `decode_attention(q, kv, lengths, scale, *, tokens=None, split=None, num_warps=1)` -> (out, lse) is the
  launcher of :190-245: one partial attention per `split` tokens, out float32 [B, Hq, S, D], lse float32
  [B, Hq, S] (natural log), S = max(ceil(tokens / split), 1); `split` defaults to `default_split` (:178-187)
  and must be a multiple of the key group (ValueError otherwise, as :216-217). It is the `DecodeFn` that
  integration/kv_cache.py:39 injects into QuantizedKVCache.
* `attend(q, kv, lengths, scale, **launch)` is :248-252 (merge_partials of the above). Here it is one
  launch that writes the merged result directly (the splits of one row are combined inside the kernel).
* `quantize_kv(k, v, bits, group=32)` is kernels/reference.py:132-160 (the write half: codes and float16
  grids, bit-exact with its formulas), and `quantize_kv_into(k, v, kv, start)` the same written straight into
  a cache at token `start`, which is what integration/kv_cache.py:147-156 QuantizedKVCache._append does with
  each completed key group.
* `kv` is anything with QuantKV's fields (kernels/reference.py:66-100): bits 4 / 8 with uint8 codes
  [B, Hkv, T, D] (bits 4: [B, Hkv, T, D/2], channel d low nibble, d + D/2 high) and float16 grids
  k_scale / k_zero [B, Hkv, T/group, D], v_scale / v_zero [B, Hkv, T]; or bits 16 with float16 / bfloat16 /
  float32 keys and values and no grids. fastserve's own QuantKV objects work unchanged.

`num_warps` is accepted for signature parity and ignored: the launch shape is the library's. Head dim 128
with 4 / 8-bit codes or float16 / bfloat16 caches runs on the matrix-core kernel (key group and split
multiples of 32 tokens); any other even head dim up to 256 (fastserve's tiny test model has 16) and float32
bits-16 caches (a float32 model's QuantizedKVCache) run on a float32 kernel with one workgroup per (sequence,
KV head, split). At most 16 query heads per KV head.
"""

from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass
from typing import Any

import torch

from . import _lib
from ._lib import F_BF16, F_F16, F_F32, KIVI_BF16, KIVI_F16, KIVI_F32, KIVI_INT4, KIVI_INT8
from .paged_attention import cached_buffer

_Q_CODES = {torch.bfloat16: F_BF16, torch.float16: F_F16, torch.float32: F_F32}


@dataclass
class QuantKV:
    """One layer's cached keys and values for B sequences, with the fields of fastserve's QuantKV
    (kernels/reference.py:66-100): bits 4 / 8 uint8 codes [B, Hkv, T, D] ([..., D/2] for 4 bits) with float16
    grids k_scale / k_zero [B, Hkv, T/group, D] and v_scale / v_zero [B, Hkv, T]; bits 16 the keys and values."""

    bits: int
    group: int
    k_codes: torch.Tensor
    v_codes: torch.Tensor
    k_scale: torch.Tensor | None = None
    k_zero: torch.Tensor | None = None
    v_scale: torch.Tensor | None = None
    v_zero: torch.Tensor | None = None

    @property
    def tokens(self) -> int:
        return self.k_codes.shape[2]

    @property
    def head_dim(self) -> int:
        return self.k_codes.shape[3] * (2 if self.bits == 4 else 1)

    def bytes_per_token(self) -> float:
        """Bytes one token occupies across this layer's KV heads, grids included."""
        ts = [self.k_codes, self.v_codes, self.k_scale, self.k_zero, self.v_scale, self.v_zero]
        return sum(t.numel() * t.element_size() for t in ts if t is not None) / (self.k_codes.shape[0] * self.tokens)


def quantize_kv(k: torch.Tensor, v: torch.Tensor, bits: int, group: int = 32) -> QuantKV:
    """k, v [B, Hkv, T, D] stored in `bits` bits (kernels/reference.py:132-160); T a whole number of groups.

    bits 4 / 8: one launch of the quantize-on-write kernel into freshly allocated codes and grids. bits 16:
    the keys and values themselves (contiguous), as the reference stores them."""
    if bits == 16:
        return QuantKV(16, group, k.contiguous(), v.contiguous())
    if bits not in (4, 8):
        raise ValueError(f"bits must be 4, 8 or 16, got {bits}")
    b, h, t, d = k.shape
    if t % group:
        raise ValueError(f"{t} tokens are not a whole number of groups of {group}")
    dev = k.device
    width = d // 2 if bits == 4 else d
    kv = QuantKV(
        bits, group,
        torch.empty((b, h, t, width), dtype=torch.uint8, device=dev),
        torch.empty((b, h, t, width), dtype=torch.uint8, device=dev),
        torch.empty((b, h, t // group, d), dtype=torch.float16, device=dev),
        torch.empty((b, h, t // group, d), dtype=torch.float16, device=dev),
        torch.empty((b, h, t), dtype=torch.float16, device=dev),
        torch.empty((b, h, t), dtype=torch.float16, device=dev),
    )
    quantize_kv_into(k, v, kv, 0)
    return kv


def quantize_kv_into(k: torch.Tensor, v: torch.Tensor, kv: Any, start: int) -> None:
    """Quantize k, v [B, Hkv, n, D] (n a whole number of kv.group tokens) into cache `kv` (QuantKV's fields) at
    tokens start .. start + n: the codes, key grids start/group .. and value grids, in one launch. Bits 16
    caches get the values copied. Integration/kv_cache.py:147-156 does this with reference.quantize_kv and
    slice assignments."""
    b, h, n, d = k.shape
    _require(tuple(v.shape) == (b, h, n, d) and v.dtype == k.dtype and v.stride() == k.stride(),
             "k and v must be [B, Hkv, n, D] with one dtype and layout")
    _require(kv.k_codes.shape[0] == b and kv.k_codes.shape[1] == h, "the cache's batch and KV heads must match")
    _require(start >= 0 and start % kv.group == 0 and start + n <= kv.k_codes.shape[2],
             f"tokens {start} .. {start + n} must start on a key group and fit the cache")
    if kv.bits == 16:
        kv.k_codes[:, :, start:start + n].copy_(k)
        kv.v_codes[:, :, start:start + n].copy_(v)
        return
    a = quantize_args(k, v, kv, start)
    stream = torch.cuda.current_stream(k.device).cuda_stream
    _lib.check(_lib.lib().bpt_kivi_quantize(ctypes.byref(a), ctypes.c_void_p(stream)))


def quantize_args(k: torch.Tensor, v: torch.Tensor, kv: Any, start: int) -> Any:
    """The checked bpt_kivi_quantize arguments that quantize_kv_into launches with (bits 4 / 8 caches), for a
    caller that launches the same write again without the Python checks (a timing loop, a captured graph).
    The struct holds raw pointers: the tensors must stay alive and in place while it is used."""
    b, h, n, d = k.shape
    _require(tuple(v.shape) == (b, h, n, d) and v.dtype == k.dtype and v.stride() == k.stride(),
             "k and v must be [B, Hkv, n, D] with one dtype and layout")
    _require(kv.k_codes.shape[0] == b and kv.k_codes.shape[1] == h, "the cache's batch and KV heads must match")
    _require(start >= 0 and start % kv.group == 0 and start + n <= kv.k_codes.shape[2],
             f"tokens {start} .. {start + n} must start on a key group and fit the cache")
    _require(kv.bits in (4, 8), f"bits must be 4, 8 or 16, got {kv.bits}")
    _require(n % kv.group == 0, f"{n} tokens are not a whole number of groups of {kv.group}")
    _require(k.dtype in _Q_CODES and k.stride(-1) == 1, "k and v must be bf16, f16 or f32 with contiguous channels")
    dev = k.device
    _require(dev.type == "cuda", "quantize_kv runs on a GPU: k must be a cuda tensor")
    kc = kv.k_codes[:, :, start:start + n]
    vc = kv.v_codes[:, :, start:start + n]
    g0, g1 = start // kv.group, (start + n) // kv.group
    ks, kz = kv.k_scale[:, :, g0:g1], kv.k_zero[:, :, g0:g1]
    vs, vz = kv.v_scale[:, :, start:start + n], kv.v_zero[:, :, start:start + n]
    _require(kc.dtype == torch.uint8 and kc.stride() == vc.stride() and kc.stride(-1) == 1, "codes: uint8, shared layout")
    _require(kc.shape[3] * (2 if kv.bits == 4 else 1) == d, f"codes hold {kc.shape[3]} bytes per token, k has D={d}")
    _require(all(t.dtype == torch.float16 for t in (ks, kz, vs, vz)), "grids must be float16")
    _require(ks.stride() == kz.stride() and ks.stride(-1) == 1, "key grids: shared layout, contiguous channels")
    _require(vs.stride() == vz.stride() and vs.stride(-1) == 1, "value grids: shared layout, unit token stride")
    for t in (v, kc, vc, ks, kz, vs, vz):
        _require(t.device == dev, f"every tensor must be on {dev}")
    a = _lib.KiviQuantArgs()
    a.struct_size = ctypes.sizeof(_lib.KiviQuantArgs)
    a.bits, a.src_dtype = kv.bits, _Q_CODES[k.dtype]
    a.batch, a.num_kv_heads, a.tokens, a.head_dim, a.group = b, h, n, d, kv.group
    a.k, a.v = k.data_ptr(), v.data_ptr()
    a.src_stride_b, a.src_stride_h, a.src_stride_t = k.stride(0), k.stride(1), k.stride(2)
    a.k_codes, a.v_codes = kc.data_ptr(), vc.data_ptr()
    a.code_stride_b, a.code_stride_h, a.code_stride_t = kc.stride(0), kc.stride(1), kc.stride(2)
    a.k_scale, a.k_zero = ks.data_ptr(), kz.data_ptr()
    a.kgrid_stride_b, a.kgrid_stride_h, a.kgrid_stride_g = ks.stride(0), ks.stride(1), ks.stride(2)
    a.v_scale, a.v_zero = vs.data_ptr(), vz.data_ptr()
    a.vgrid_stride_b, a.vgrid_stride_h = vs.stride(0), vs.stride(1)
    return a


def default_split(batch: int, kv_heads: int, tokens: int, group: int = 32, max_programs: int = 16384) -> int:
    """kernels/kv_attention.py:178-187: tokens per split, 4 key groups or more once that passes
    `max_programs` (sequence, KV head, split) units; a power of two."""
    per_program = max(tokens * batch * kv_heads // max_programs, 4 * group)
    return max(group, 1 << (per_program.bit_length() - 1))


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


def _format(kv: Any) -> int:
    if kv.bits == 4:
        return KIVI_INT4
    if kv.bits == 8:
        return KIVI_INT8
    if kv.bits == 16:
        if kv.k_codes.dtype == torch.float16:
            return KIVI_F16
        if kv.k_codes.dtype == torch.bfloat16:
            return KIVI_BF16
        if kv.k_codes.dtype == torch.float32:
            return KIVI_F32
        raise ValueError(f"a bits-16 cache must hold float16, bfloat16 or float32 keys and values, got "
                         f"{kv.k_codes.dtype}")
    raise ValueError(f"bits must be 4, 8 or 16, got {kv.bits}")


def _launch(q, kv, lengths, scale, split, n_splits, out, lse, tail=None) -> None:
    fmt = _format(kv)
    b, hq, d = q.shape
    kc, vc = kv.k_codes, kv.v_codes
    _require(kc.dim() == 4 and kc.shape == vc.shape, "k_codes and v_codes must be [B, Hkv, T, E] of one shape")
    _require(kc.shape[0] == b, f"the cache holds {kc.shape[0]} sequences, q {b}")
    hkv, t_max = kc.shape[1], kc.shape[2]
    quant = fmt in (KIVI_INT4, KIVI_INT8)
    if quant:
        _require(kc.dtype == torch.uint8 and vc.dtype == torch.uint8, "4- and 8-bit codes must be uint8")
        _require(kc.shape[3] * (2 if fmt == KIVI_INT4 else 1) == d, f"codes hold {kc.shape[3]} bytes per token, q has D={d}")
    else:
        _require(vc.dtype == kc.dtype and kc.shape[3] == d, "bits-16 keys and values must share q's head dim and a dtype")
    _require(q.dtype in _Q_CODES, f"q must be bfloat16, float16 or float32, got {q.dtype}")
    _require(q.stride(-1) == 1 and kc.stride(-1) == 1 and vc.stride() == kc.stride(), "channels must be contiguous")
    _require(lengths.dtype == torch.int32 and tuple(lengths.shape) == (b,) and lengths.is_contiguous(),
             f"lengths must be int32 [{b}]")
    dev = q.device
    _require(dev.type == "cuda", "decode_attention runs on a GPU: q must be a cuda tensor")
    grids = (kv.k_scale, kv.k_zero, kv.v_scale, kv.v_zero) if quant else ()
    for t in (kc, vc, lengths, *grids):
        _require(t.device == dev, f"every tensor must be on {dev}")

    a = _lib.KiviArgs()
    a.struct_size = ctypes.sizeof(_lib.KiviArgs)
    a.format, a.q_dtype = fmt, _Q_CODES[q.dtype]
    a.batch, a.num_q_heads, a.num_kv_heads, a.head_dim = b, hq, hkv, d
    a.tokens, a.group = t_max, kv.group
    a.split, a.num_splits = split, n_splits
    a.sm_scale = float(scale)
    a.q, a.q_stride_b, a.q_stride_h = q.data_ptr(), q.stride(0), q.stride(1)
    a.k_codes, a.v_codes = kc.data_ptr(), vc.data_ptr()
    a.code_stride_b, a.code_stride_h, a.code_stride_t = kc.stride(0), kc.stride(1), kc.stride(2)
    if quant:
        ks, kz, vs, vz = grids
        for name, g in (("k_scale", ks), ("k_zero", kz), ("v_scale", vs), ("v_zero", vz)):
            _require(g.dtype == torch.float16, f"{name} must be float16, got {g.dtype}")
        _require(ks.dim() == 4 and ks.shape == kz.shape and tuple(ks.shape[:2]) == (b, hkv) and ks.shape[3] == d,
                 f"k_scale / k_zero must be [{b}, {hkv}, groups, {d}]")
        _require(ks.stride() == kz.stride() and ks.stride(-1) == 1, "k_scale and k_zero must share contiguous channels")
        _require(tuple(vs.shape) == (b, hkv, t_max) and vs.shape == vz.shape and vs.stride() == vz.stride()
                 and vs.stride(-1) == 1, f"v_scale / v_zero must be [{b}, {hkv}, {t_max}] with unit token stride")
        a.num_groups = ks.shape[2]
        a.k_scale, a.k_zero = ks.data_ptr(), kz.data_ptr()
        a.kgrid_stride_b, a.kgrid_stride_h, a.kgrid_stride_g = ks.stride(0), ks.stride(1), ks.stride(2)
        a.v_scale, a.v_zero = vs.data_ptr(), vz.data_ptr()
        a.vgrid_stride_b, a.vgrid_stride_h = vs.stride(0), vs.stride(1)
    a.lengths = lengths.data_ptr()
    a.out = out.data_ptr()
    a.out_stride_b, a.out_stride_h, a.out_stride_s = out.stride(0), out.stride(1), out.stride(2)
    a.lse = lse.data_ptr()
    a.lse_stride_b, a.lse_stride_h, a.lse_stride_s = lse.stride(0), lse.stride(1), lse.stride(2)
    if tail is not None:
        tk, tv = tail
        _require(tk.dim() == 4 and tk.shape == tv.shape and tuple(tk.shape[:2]) == (b, hkv) and tk.shape[3] == d,
                 f"tail keys and values must be [{b}, {hkv}, tail_len, {d}]")
        _require(tk.dtype == tv.dtype and tk.dtype in _Q_CODES, "tail keys and values must share a bf16/f16/f32 dtype")
        _require(tk.stride() == tv.stride() and tk.stride(-1) == 1, "tail keys and values must share strides, channels contiguous")
        _require(tk.device == dev and tv.device == dev, f"the tail must be on {dev}")
        a.tail_k, a.tail_v = tk.data_ptr(), tv.data_ptr()
        a.tail_stride_b, a.tail_stride_h, a.tail_stride_t = tk.stride(0), tk.stride(1), tk.stride(2)
        a.tail_dtype, a.tail_len = _Q_CODES[tk.dtype], tk.shape[2]
    lib = _lib.lib()
    ws_bytes, cnt_bytes = ctypes.c_size_t(0), ctypes.c_size_t(0)
    _lib.check(lib.bpt_kivi_plan(ctypes.byref(a), ctypes.byref(ws_bytes), ctypes.byref(cnt_bytes)))
    stream = torch.cuda.current_stream(dev).cuda_stream
    workspace = cached_buffer("partials", dev, stream, ws_bytes.value)
    counters = cached_buffer("counters", dev, stream, cnt_bytes.value)
    a.workspace, a.workspace_bytes = workspace.data_ptr(), workspace.numel()
    a.counters, a.counters_bytes = counters.data_ptr(), counters.numel()
    _lib.check(lib.bpt_kivi_decode(ctypes.byref(a), ctypes.c_void_p(stream)))


def decode_attention(
    q: torch.Tensor,
    kv: Any,
    lengths: torch.Tensor,
    scale: float,
    *,
    tokens: int | None = None,
    split: int | None = None,
    num_warps: int = 1,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Partial attentions of one query per head over a KIVI cache, one per split (kv_attention.py:190-245).

    q [B, Hq, D] (bf16 / f16 / f32); lengths [B] int32 on q's device. `tokens` (the longest row's length,
    when the caller knows it) sizes the splits without a device read. Returns (out float32 [B, Hq, S, D],
    lse float32 [B, Hq, S]); `merge_partials` of the two is the attention.
    """
    del num_warps  # launch shape is the library's
    b, hq, d = q.shape
    hkv, t_max = kv.k_codes.shape[1], kv.k_codes.shape[2]
    tokens = t_max if tokens is None else tokens
    if split is None:
        split = default_split(b, hkv, tokens, kv.group)
    if split % kv.group:
        raise ValueError(f"split {split} must be a multiple of the key group {kv.group}")
    n_splits = max(-(-tokens // split), 1)
    out = torch.empty((b, hq, n_splits, d), dtype=torch.float32, device=q.device)
    lse = torch.empty((b, hq, n_splits), dtype=torch.float32, device=q.device)
    _launch(q, kv, lengths, scale, split, n_splits, out, lse)
    return out, lse


def attend(q: torch.Tensor, kv: Any, lengths: torch.Tensor, scale: float, *,
           tail: tuple[torch.Tensor, torch.Tensor] | None = None, **launch: int | None) -> torch.Tensor:
    """Decode attention over a KIVI cache: [B, Hq, D] float32 (kv_attention.py:248-252).

    The result does not depend on the split; a given `split` is still checked against the key group. The
    tokens past `tokens` (when given) are not read, as in decode_attention.

    tail: the cache's full-precision tail (tail_k, tail_v) [B, Hkv, n, D], n <= 64 tokens every row sees in
    full (the tokens whose key group is not complete yet). Its attention is merged into the result in the same
    launch: what QuantizedKVCache.attend's decode branch computes with three (integration/kv_cache.py:172-185:
    decode over the codes, partial_attention over the tail, merge_partials). A row with no codes gets the
    tail's attention alone.
    """
    b, hq, d = q.shape
    t_max = kv.k_codes.shape[2]
    tokens = launch.get("tokens")
    tokens = t_max if tokens is None else tokens
    split = launch.get("split")
    if split is None:
        split = default_split(b, kv.k_codes.shape[1], tokens, kv.group)
    if split % kv.group:
        raise ValueError(f"split {split} must be a multiple of the key group {kv.group}")
    reach = max(-(-tokens // split), 1) * split  # the tokens decode_attention's splits would cover
    step = kv.group * 32 // math.gcd(kv.group, 32)
    whole = max(-(-reach // step), 1) * step  # one split covering all of them
    out = torch.empty((b, hq, 1, d), dtype=torch.float32, device=q.device)
    lse = torch.empty((b, hq, 1), dtype=torch.float32, device=q.device)
    if tail is not None and tail[0].shape[2] == 0:
        tail = None
    _launch(q, kv, lengths, scale, whole, 1, out, lse, tail)
    return out[:, :, 0]
