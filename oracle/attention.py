"""Decode attention in float32 numpy (oracle; test infrastructure only).

Restates fastserve's reference math:
* partial_attention / merge_partials  kernels/reference.py:186-211
* repeat_kv, causal_mask, attention   engine/attention.py:12-47
* default_split                       kernels/kv_attention.py:178-187
and composes them into `paged_decode`, the computation of the HIP decode kernel: gather each sequence's
pages (engine/kv_cache.py:165-169), dequantize (oracle.quant.dequantize), then causal multi-query attention
with query i of Q at position context_len - Q + i (store-before-attend, integration/kv_cache.py:160-168).
"""

from __future__ import annotations

import numpy as np

from . import paged, quant


def repeat_kv(x: np.ndarray, n_rep: int) -> np.ndarray:
    """engine/attention.py:23-31: [B, Hkv, T, D] -> [B, Hkv * n_rep, T, D]; KV head h serves h*n_rep + j."""
    return np.repeat(x, n_rep, axis=1) if n_rep > 1 else x


def _softmax_lse(scores: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Row softmax over the last axis with -inf masking; fully masked rows give 0 weights and lse -inf."""
    m = np.max(scores, axis=-1, keepdims=True)
    m_safe = np.where(np.isfinite(m), m, np.float32(0.0))
    e = np.exp(scores - m_safe)
    total = np.sum(e, axis=-1, keepdims=True)
    with np.errstate(divide="ignore", invalid="ignore"):
        probs = np.where(total > 0, e / total, np.float32(0.0))
        lse = np.where(total[..., 0] > 0, m_safe[..., 0] + np.log(total[..., 0]), -np.inf)
    return probs.astype(np.float32), lse.astype(np.float32)


def partial_attention(q, k, v, lengths, scale):
    """kernels/reference.py:186-202: q [B, Hq, D]; k, v [B, Hkv, T, D]; row b sees its first lengths[b] tokens.

    Returns (out [B, Hq, D], lse [B, Hq]); a row with no visible token gets out 0 and lse -inf.
    """
    q = np.asarray(q, dtype=np.float32)
    group = q.shape[1] // k.shape[1]
    k = repeat_kv(np.asarray(k, dtype=np.float32), group)
    v = repeat_kv(np.asarray(v, dtype=np.float32), group)
    scores = np.einsum("bhd,bhtd->bht", q, k) * np.float32(scale)
    visible = np.arange(k.shape[2])[None, :] < np.asarray(lengths)[:, None]
    scores = np.where(visible[:, None], scores, -np.inf).astype(np.float32)
    probs, lse = _softmax_lse(scores)
    return np.einsum("bht,bhtd->bhd", probs, v).astype(np.float32), lse


def merge_partials(outs, lses):
    """kernels/reference.py:205-211: softmax over the parts' lse (NaN -> 0), weighted sum of outs."""
    lses = np.asarray(lses, dtype=np.float32)
    share, _ = _softmax_lse(lses)
    return np.sum(share[..., None] * np.asarray(outs, dtype=np.float32), axis=-2)


def causal_mask(positions, kv_len):
    """engine/attention.py:12-20: slot j visible to a query at position p iff j <= p; [B, 1, Q, T]."""
    slots = np.arange(kv_len)
    return (slots[None, None, :] <= np.asarray(positions)[:, :, None])[:, None]


def attention(q, k, v, mask, scale):
    """engine/attention.py:34-47: softmax(q kᵀ · scale, masked) v; q [B, Hq, Q, D], k, v [B, Hkv, T, D]."""
    q = np.asarray(q, dtype=np.float32)
    group = q.shape[1] // k.shape[1]
    k = repeat_kv(np.asarray(k, dtype=np.float32), group)
    v = repeat_kv(np.asarray(v, dtype=np.float32), group)
    scores = (q @ np.swapaxes(k, -1, -2)) * np.float32(scale)
    scores = np.where(mask, scores, -np.inf).astype(np.float32)
    probs, _ = _softmax_lse(scores)
    return (probs @ v).astype(np.float32)


def default_split(batch: int, kv_heads: int, tokens: int, group: int = 32, max_programs: int = 16384) -> int:
    """kernels/kv_attention.py:178-187: max(tokens*B*Hkv // max_programs, 4*group), rounded down to a power of
    two, at least one group."""
    per_program = max(tokens * batch * kv_heads // max_programs, 4 * group)
    return max(group, 1 << (per_program.bit_length() - 1))


def dequantized_sequence(pool, scales, table_row, length, kv_format):
    """One sequence's [length, Hkv, D] float32 keys (or values) read through its block table."""
    codes = paged.gather_sequence(pool, table_row, length)
    if kv_format == "bf16":
        return np.asarray(codes, dtype=np.float32)
    s = np.asarray(scales, dtype=np.float32)
    if s.ndim == 1:  # per head: [Hkv] broadcast over tokens and channels
        scale = s[None, :, None]
    else:  # per token and head: [NB, P, Hkv] paged like the codes
        scale = paged.gather_sequence(s, table_row, length)[..., None]
    return quant.dequantize(codes, kv_format, scale)


def paged_decode(q, k_pool, v_pool, block_table, context_lens, k_scale, v_scale, kv_format, scale):
    """The paged decode-attention result: q [B, Q, Hq, D] -> (out [B, Q, Hq, D], lse [B, Q, Hq]) float32.

    kv_format 'bf16' (pools hold float values), 'fp8' (uint8 e4m3fn codes) or 'int8' (int8 codes); scales
    per head [Hkv] or per token and head [NB, P, Hkv]. Query i of sequence b sees slots
    0 .. context_lens[b] - Q + i (causal by absolute position); lse is the natural-log normalizer.
    """
    q = np.asarray(q, dtype=np.float32)
    b_sz, nq, hq, d = q.shape
    hkv = k_pool.shape[2]
    g = hq // hkv
    out = np.zeros((b_sz, nq, hq, d), dtype=np.float32)
    lse = np.full((b_sz, nq, hq), -np.inf, dtype=np.float32)
    for b in range(b_sz):
        t = int(context_lens[b])
        if t <= 0:
            continue
        k = dequantized_sequence(k_pool, k_scale, block_table[b], t, kv_format)  # [T, Hkv, D]
        v = dequantized_sequence(v_pool, v_scale, block_table[b], t, kv_format)
        kt = np.ascontiguousarray(np.transpose(k, (1, 2, 0)))  # [Hkv, D, T]
        vt = np.ascontiguousarray(np.transpose(v, (1, 0, 2)))  # [Hkv, T, D]
        qb = q[b].reshape(nq, hkv, g, d).transpose(1, 0, 2, 3).reshape(hkv, nq * g, d)  # rows (i, j)
        scores = (qb @ kt) * np.float32(scale)  # [Hkv, Q*G, T]
        visible = t - nq + np.repeat(np.arange(nq), g) + 1  # per row
        mask = np.arange(t)[None, :] < visible[:, None]
        scores = np.where(mask[None], scores, -np.inf).astype(np.float32)
        probs, l = _softmax_lse(scores)
        o = probs @ vt  # [Hkv, Q*G, D]
        out[b] = o.reshape(hkv, nq, g, d).transpose(1, 0, 2, 3).reshape(nq, hq, d)
        lse[b] = l.reshape(hkv, nq, g).transpose(1, 0, 2).reshape(nq, hq)
    return out, lse
