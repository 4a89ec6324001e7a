"""KIVI asymmetric KV storage and decode attention over it, in float32 numpy (oracle; test infrastructure only).

Restates fastserve's kernel-2 format and read (paths relative to src/fastserve/):
* QuantKV (fields, bytes_per_token)     kernels/reference.py:66-100
* grid / codes                          kernels/reference.py:103-118: per-axis asymmetric grid; the scale
                                        is rounded to float16 *before* the codes are computed
* pack_nibbles / unpack_nibbles         kernels/reference.py:121-129: channel d low nibble, d + D/2 high
* quantize_kv                           kernels/reference.py:132-160: keys per channel per `group` tokens,
                                        values per token; bits 16 stores the inputs unchanged
* dequantize_kv                         kernels/reference.py:163-180
* decode_attention                      kernels/kv_attention.py:190-245 (and the kernel :56-175): one
                                        partial attention per `split` tokens, (out [B, Hq, S, D],
                                        lse [B, Hq, S]) with lse = log sum exp (natural log); a split past
                                        a row's length gives out 0 and lse -inf
* attend                                kernels/kv_attention.py:248-252: merge_partials of the above
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from .attention import default_split, merge_partials, partial_attention


@dataclass
class QuantKV:
    """One layer's cache for B sequences, as stored (kernels/reference.py:66-100).

    bits 4 / 8: uint8 codes plus float16 grids; bits 16: the float16 (or bfloat16-as-float32) keys and
    values themselves and no grids.
      k_codes, v_codes  [B, Hkv, T, D]   (bits 4: [B, Hkv, T, D/2], channel d and d + D/2 share a byte)
      k_scale, k_zero   [B, Hkv, T/group, D] float16
      v_scale, v_zero   [B, Hkv, T] float16
    """

    bits: int
    group: int
    k_codes: np.ndarray
    v_codes: np.ndarray
    k_scale: np.ndarray | None = None
    k_zero: np.ndarray | None = None
    v_scale: np.ndarray | None = None
    v_zero: np.ndarray | None = None

    @property
    def tokens(self) -> int:
        return self.k_codes.shape[2]

    @property
    def head_dim(self) -> int:
        return self.k_codes.shape[3] * (2 if self.bits == 4 else 1)

    def bytes_per_token(self) -> float:
        """Bytes one token occupies across this layer's KV heads, grids included (reference.py:95-100)."""
        arrays = [self.k_codes, self.v_codes, self.k_scale, self.k_zero, self.v_scale, self.v_zero]
        total = sum(a.size * a.itemsize for a in arrays if a is not None)
        return total / (self.k_codes.shape[0] * self.tokens)


def grid(x: np.ndarray, bits: int, axis: int) -> tuple[np.ndarray, np.ndarray]:
    """kernels/reference.py:103-114: (scale, zero) float16 of the values along `axis` (kept as size 1).

    The range always contains 0; scale = f16((hi - lo) / (2^bits - 1)) (1 where that is 0);
    zero = clamp(round_half_even(-lo / scale), 0, 2^bits - 1).
    """
    x = np.asarray(x, dtype=np.float32)
    lo = np.minimum(x.min(axis=axis, keepdims=True), np.float32(0.0))
    hi = np.maximum(x.max(axis=axis, keepdims=True), np.float32(0.0))
    scale = ((hi - lo) / np.float32(2**bits - 1)).astype(np.float16)
    scale = np.where(scale > 0, scale, np.float16(1.0)).astype(np.float16)
    zero = np.clip(np.round(-lo / scale.astype(np.float32)), 0, 2**bits - 1).astype(np.float16)
    return scale, zero


def codes(x: np.ndarray, scale: np.ndarray, zero: np.ndarray, bits: int) -> np.ndarray:
    """kernels/reference.py:117-118: clamp(round_half_even(x / scale) + zero, 0, 2^bits - 1) as uint8."""
    x = np.asarray(x, dtype=np.float32)
    c = np.round(x / scale.astype(np.float32)) + zero.astype(np.float32)
    return np.clip(c, 0, 2**bits - 1).astype(np.uint8)


def pack_nibbles(c: np.ndarray) -> np.ndarray:
    """kernels/reference.py:121-124: 4-bit codes [..., D] -> bytes [..., D/2], channel d low, d + D/2 high."""
    half = c.shape[-1] // 2
    return (c[..., :half] | (c[..., half:] << 4)).astype(np.uint8)


def unpack_nibbles(packed: np.ndarray) -> np.ndarray:
    """kernels/reference.py:127-129: bytes [..., D/2] -> 4-bit codes [..., D]."""
    return np.concatenate([packed & 0xF, packed >> 4], axis=-1).astype(np.uint8)


def quantize_kv(k: np.ndarray, v: np.ndarray, bits: int, group: int = 32) -> QuantKV:
    """kernels/reference.py:132-160: store k, v [B, Hkv, T, D] in `bits` bits (T a whole number of groups)."""
    if bits == 16:
        return QuantKV(16, group, np.ascontiguousarray(k), np.ascontiguousarray(v))
    if bits not in (4, 8):
        raise ValueError(f"bits must be 4, 8 or 16, got {bits}")
    b, h, t, d = k.shape
    if t % group:
        raise ValueError(f"{t} tokens are not a whole number of groups of {group}")
    k32 = np.asarray(k, dtype=np.float32)
    v32 = np.asarray(v, dtype=np.float32)
    blocks = k32.reshape(b, h, t // group, group, d)
    k_scale, k_zero = grid(blocks, bits, axis=3)  # [B, Hkv, G, 1, D]
    k_codes = codes(blocks, k_scale, k_zero, bits).reshape(b, h, t, d)
    v_scale, v_zero = grid(v32, bits, axis=3)  # [B, Hkv, T, 1]
    v_codes = codes(v32, v_scale, v_zero, bits)
    if bits == 4:
        k_codes, v_codes = pack_nibbles(k_codes), pack_nibbles(v_codes)
    return QuantKV(
        bits,
        group,
        np.ascontiguousarray(k_codes),
        np.ascontiguousarray(v_codes),
        np.ascontiguousarray(k_scale[:, :, :, 0]),
        np.ascontiguousarray(k_zero[:, :, :, 0]),
        np.ascontiguousarray(v_scale[..., 0]),
        np.ascontiguousarray(v_zero[..., 0]),
    )


def dequantize_kv(kv: QuantKV, tokens: int | None = None) -> tuple[np.ndarray, np.ndarray]:
    """kernels/reference.py:163-180: the first `tokens` keys and values in float32, [B, Hkv, tokens, D]."""
    t = kv.tokens if tokens is None else tokens
    if kv.bits == 16:
        return kv.k_codes[:, :, :t].astype(np.float32), kv.v_codes[:, :, :t].astype(np.float32)
    kc, vc = kv.k_codes[:, :, :t], kv.v_codes[:, :, :t]
    if kv.bits == 4:
        kc, vc = unpack_nibbles(kc), unpack_nibbles(vc)
    groups = -(-t // kv.group)
    ks = np.repeat(kv.k_scale[:, :, :groups].astype(np.float32), kv.group, axis=2)[:, :, :t]
    kz = np.repeat(kv.k_zero[:, :, :groups].astype(np.float32), kv.group, axis=2)[:, :, :t]
    k = ks * (kc.astype(np.float32) - kz)
    v = kv.v_scale[:, :, :t, None].astype(np.float32) * (vc.astype(np.float32) - kv.v_zero[:, :, :t, None].astype(np.float32))
    return k.astype(np.float32), v.astype(np.float32)


def decode_attention(q, kv: QuantKV, lengths, scale: float, *, tokens: int | None = None, split: int | None = None):
    """kernels/kv_attention.py:190-245: per-split partial attentions of q [B, Hq, D] over the cache.

    Split s covers tokens [s * split, min((s + 1) * split, lengths[b])); there are max(ceil(tokens / split), 1)
    splits (tokens defaults to the cache's T). Returns (out [B, Hq, S, D], lse [B, Hq, S]), float32.
    """
    q = np.asarray(q, dtype=np.float32)
    b, hq, d = q.shape
    hkv, t_max = kv.k_codes.shape[1], kv.tokens
    tokens = t_max if tokens is None else tokens
    if split is None:
        split = default_split(b, hkv, tokens, kv.group)
    if split % kv.group:
        raise ValueError(f"split {split} must be a multiple of the key group {kv.group}")
    n_splits = max(-(-tokens // split), 1)
    k, v = dequantize_kv(kv)
    lengths = np.minimum(np.asarray(lengths, dtype=np.int64), t_max)
    outs, lses = [], []
    for s in range(n_splits):
        start = s * split
        if start >= t_max:  # nothing stored this far: an empty split
            outs.append(np.zeros((b, hq, d), np.float32))
            lses.append(np.full((b, hq), -np.inf, np.float32))
            continue
        seen = np.clip(lengths - start, 0, split)
        out, lse = partial_attention(q, k[:, :, start : start + split], v[:, :, start : start + split], seen, scale)
        outs.append(out)
        lses.append(lse)
    return np.stack(outs, axis=2).astype(np.float32), np.stack(lses, axis=2).astype(np.float32)


def attend(q, kv: QuantKV, lengths, scale: float, **launch) -> np.ndarray:
    """kernels/kv_attention.py:248-252: the merged attention [B, Hq, D]."""
    return merge_partials(*decode_attention(q, kv, lengths, scale, **launch))
