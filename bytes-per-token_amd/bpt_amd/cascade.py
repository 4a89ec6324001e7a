"""Shared-prefix cascade decode: a prefix that several sequences share is attended once, then merged.

When sequences start with the same pages (a system prompt, or the branches of a speculative verify step;
fastserve's prefix cache decides the sharing, kv/prefix_cache.py:42-140), plain paged decode reads the
shared pages once per sequence. The cascade reads them once per 16 query rows of the whole group:

1. Prefix pass. All queries of a group (members x Q queries x G heads per KV head) attend the group's
   `prefix_pages` shared pages, 16 rows at a time, non-causally (every query sits after the prefix), and
   leave float32 partials: each row's normalized output and log-sum-exp.
2. Suffix pass. Every sequence attends its own pages after the prefix with the usual causal rule; each row's
   result is merged with its prefix partial as kernels/reference.py:205-211 merges split partials, so the
   output is the attention over the whole context.

Both passes are the library's paged decode kernels (two launches in all, plus one per extra group); the
merge happens in the suffix pass's final write. The result equals `paged_decode_attention` on the same
inputs up to float32 rounding.

Requirements: every sequence of a group holds the group's prefix in its first `prefix_pages` block-table
entries (the same physical pages), all groups share one prefix length, and every query sits at or after
the prefix's last token (context_len >= prefix_pages * page_size + Q - 1). `context_lens_host`, when given,
is checked against the last rule.
"""

from __future__ import annotations

import torch

from ._lib import DECODE_NONCAUSAL
from .paged_attention import _require, paged_decode_attention


def _rows_per_pass(total_queries: int, heads_per_kv: int) -> int:
    """Queries per prefix-pass sequence: the largest divisor of the group's query count whose rows (times the
    query heads per KV head) fit one 16-row matrix-core group."""
    best = 1
    for qv in range(1, max(1, 16 // heads_per_kv) + 1):
        if total_queries % qv == 0:
            best = qv
    return best


def cascade_decode_attention(
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
    prefix_pages: int,
    groups: list[tuple[int, int]] | None = None,
    num_splits: int | None = None,
    out: torch.Tensor | None = None,
    out_dtype: torch.dtype = torch.bfloat16,
    context_lens_host: list[int] | None = None,
) -> torch.Tensor:
    """Paged decode attention with a shared prefix read once per group (see the module docstring).

    Arguments as `paged_decode_attention` (`num_splits` applies to the suffix pass), plus `prefix_pages`
    (leading block-table entries shared within a group) and `groups`: contiguous batch ranges [start, end)
    sharing them (default: the whole batch).
    """
    squeeze = q.dim() == 3
    q4 = q[:, None] if squeeze else q
    b, nq, hq, d = q4.shape
    hkv, page = k_cache.shape[2], k_cache.shape[1]
    _require(hq % hkv == 0, f"{hq} query heads are not a multiple of {hkv} KV heads")
    heads_per_kv = hq // hkv
    _require(prefix_pages >= 1, "prefix_pages must be at least 1 (use paged_decode_attention without a prefix)")
    _require(block_table.dim() == 2 and block_table.shape[1] >= prefix_pages,
             f"block_table must hold at least the {prefix_pages} prefix pages")
    prefix = prefix_pages * page
    _require(max_context >= prefix, f"max_context {max_context} is shorter than the {prefix}-token prefix")
    groups = [(0, b)] if groups is None else [(int(s), int(e)) for s, e in groups]
    at = 0
    for s, e in groups:
        _require(s == at and e > s, "groups must be consecutive, non-empty [start, end) ranges covering the batch")
        at = e
    _require(at == b, "groups must cover the whole batch")
    if context_lens_host is not None:
        short = [i for i, n in enumerate(context_lens_host) if n < prefix + nq - 1]
        _require(not short, f"sequences {short[:8]} end inside the shared prefix: their queries would see all of it")
    dev = q4.device
    q4c = q4 if q4.stride(0) == nq * q4.stride(1) and q4.stride(1) == hq * q4.stride(2) and q4.stride(2) == d else q4.contiguous()

    # 1. The prefix pass: per group, its queries as sequences of qv queries over the shared pages.
    part = torch.empty((b, nq, hq, d), dtype=torch.float32, device=dev)
    part_lse = torch.empty((b, nq, hq), dtype=torch.float32, device=dev)
    for s, e in groups:
        total = (e - s) * nq
        qv = _rows_per_pass(total, heads_per_kv)
        nv = total // qv
        table = block_table[s, :prefix_pages].expand(nv, prefix_pages)
        paged_decode_attention(
            q4c[s:e].reshape(nv, qv, hq, d), k_cache, v_cache, table, None, k_scale, v_scale,
            scale=scale, max_context=prefix, out=part[s:e].view(nv, qv, hq, d), lse=part_lse[s:e],
            _cascade={"flags": DECODE_NONCAUSAL},
        )

    # 2. The suffix pass: each sequence's own pages, merged with its rows' prefix partials on the way out.
    rest = block_table[:, prefix_pages:] if block_table.shape[1] > prefix_pages else block_table[:, -1:]
    return paged_decode_attention(
        q, k_cache, v_cache, rest, context_lens, k_scale, v_scale, scale=scale, max_context=max_context - prefix,
        num_splits=num_splits, out=out, out_dtype=out_dtype, _cascade={"len_offset": prefix, "merge": (part, part_lse)},
    )
