"""Paged KV-cache metadata and layout in numpy (oracle; test infrastructure only).

Restates fastserve engine/kv_cache.py:90-169 (PagedMeta, PagedKVCache.prepare / update / _gather):
pools are [num_blocks, block_size, Hkv, D]; a sequence's block table lists its physical blocks in logical
order and is padded with block 0 up to the batch's longest; token at position p is written to slot
p % block_size of block table[p // block_size].
"""

from __future__ import annotations

import math

import numpy as np


def blocks_needed(num_tokens: int, block_size: int) -> int:
    """engine/kv_cache.py:119-120."""
    return math.ceil(num_tokens / block_size)


def prepare(tables: list[list[int]], positions: np.ndarray, block_size: int):
    """engine/kv_cache.py:140-156: (write_blocks [B, Q], write_offsets [B, Q], block_table [B, n], kv_len).

    Raises ValueError when a row's table cannot hold its furthest position ("call reserve() first").
    """
    positions = np.asarray(positions, dtype=np.int64)
    kv_len = int(positions.max()) + 1
    n_blocks = blocks_needed(kv_len, block_size)
    rows = []
    for i, table in enumerate(tables):
        if len(table) * block_size < int(positions[i].max()) + 1:
            raise ValueError(f"sequence {i} has too few blocks: call reserve() first")
        rows.append(list(table[:n_blocks]) + [0] * (n_blocks - len(table)))
    block_table = np.asarray(rows, dtype=np.int64)
    logical = positions // block_size
    write_blocks = np.take_along_axis(block_table, logical, axis=1)
    return write_blocks, positions % block_size, block_table, kv_len


def scatter(pool: np.ndarray, write_blocks: np.ndarray, write_offsets: np.ndarray, rows: np.ndarray) -> None:
    """engine/kv_cache.py:160-161: pool[write_blocks[b, i], write_offsets[b, i]] = rows[b, i] ([Hkv, D])."""
    pool[write_blocks, write_offsets] = rows


def gather(pool: np.ndarray, block_table: np.ndarray, kv_len: int) -> np.ndarray:
    """engine/kv_cache.py:165-169: [B, n] table -> the first kv_len tokens as [B, Hkv, kv_len, ...]."""
    b, n = block_table.shape
    blocks = pool[block_table]  # [B, n, P, Hkv, ...]
    flat = blocks.reshape(b, n * pool.shape[1], *pool.shape[2:])[:, :kv_len]
    return np.swapaxes(flat, 1, 2)


def gather_sequence(pool: np.ndarray, table_row: np.ndarray, length: int) -> np.ndarray:
    """One sequence's first `length` tokens from its table row: [length, Hkv, ...] (token-major)."""
    p = pool.shape[1]
    pages = np.asarray(table_row[: blocks_needed(length, p)], dtype=np.int64)
    return pool[pages].reshape(len(pages) * p, *pool.shape[2:])[:length]
