"""A paged KV cache that stores FP8 / INT8 / BF16 codes and attends over them with the HIP kernels.

The drop-in for fastserve's engine (paths relative to its src/fastserve/):

* Memory management is PagedKVCache's (engine/kv_cache.py:98-138): one pool of fixed-size blocks per layer,
  a block table per sequence, `reserve` / `can_reserve` / `free`, block 0 handed out first, freed blocks
  reused, `OutOfBlocksError` when the pool is empty.
* `prepare(rows, positions)` builds the per-forward metadata once for all layers (engine/kv_cache.py:140-156:
  write blocks and offsets by position, block tables padded with block 0) plus each row's context length, on
  the device: every sequence's block table lives in a row ("slot") of a device table written by `reserve`, and
  one kernel (bpt_paged_prepare) gathers the rows' tables and derives the write slots and lengths from the
  positions. With device positions nothing is read back to the host, so a whole decode step (prepare plus every
  layer's attend) can be captured in a HIP graph; host positions are checked on the host first, as fastserve's
  prepare does.
* `attend(layer, q, k, v, meta, scale)` is the cache-owned attention hook the model calls when a cache has
  one (engine/model.py:72-74, contract of integration/kv_cache.py:160-168): the step's keys and values are
  quantized into their slots first (store before attend), then one fused paged decode attention reads the
  codes; a query at position p sees the slots 0..p of its row (engine/attention.py:12-20), so decode steps
  (Q = 1), speculative verify steps (Q = k + 1) and prefill chunks all go through the same kernel.
* `update` raises, as QuantizedKVCache.update does (integration/kv_cache.py:136-137): the cache never hands
  out float keys and values.

Formats: FP8 e4m3fn with static per-(layer, KV head) scales (default 1.0, fastserve kv/quant.py:16 stores
FP8 unscaled), INT8 with dynamic per-(token, head) scales amax/127 paged like the codes, or plain BF16.
"""

from __future__ import annotations

import heapq
from dataclasses import dataclass
from typing import Any

import torch

from .paged_attention import paged_append_decode, paged_prepare

_FORMATS = {torch.float8_e4m3fn: "fp8", torch.int8: "int8", torch.bfloat16: "bf16"}
HEAD_DIM = 128  # the one head size the paged decode kernels are built for


class OutOfBlocksError(RuntimeError):
    """A reservation asked for more blocks (or sequence slots) than are free right now."""


@dataclass(frozen=True)
class PagedMeta:
    write_blocks: torch.Tensor  # [batch, q_len] int32: physical block receiving each new token (-1: none)
    write_offsets: torch.Tensor  # [batch, q_len] int32: slot inside that block
    block_table: torch.Tensor  # [batch, n_blocks] int32: physical blocks of logical blocks 0 .. n_blocks - 1
    context_lens: torch.Tensor  # [batch] int32: tokens in the cache once this step is written
    kv_len: int  # a bound on the longest row's context length, known on the host (its reserved tokens)


class PagedQuantKVCache:
    """Paged, quantized KV cache with fused attention (see the module docstring).

    `cfg` is any object with num_layers, num_kv_heads and head_dim (fastserve's ModelConfig); the three can
    also be given directly. `k_scale` / `v_scale` (FP8 only): float32 [num_layers, num_kv_heads].
    """

    def __init__(
        self,
        cfg: Any = None,
        *,
        num_blocks: int,
        block_size: int,
        kv_dtype: torch.dtype = torch.float8_e4m3fn,
        device: torch.device | str,
        num_layers: int | None = None,
        num_kv_heads: int | None = None,
        head_dim: int | None = None,
        k_scale: torch.Tensor | None = None,
        v_scale: torch.Tensor | None = None,
        max_seqs: int = 256,
        max_blocks_per_seq: int | None = None,
    ):
        if kv_dtype not in _FORMATS:
            raise ValueError(f"kv_dtype must be float8_e4m3fn, int8 or bfloat16, got {kv_dtype}")
        self.num_layers = num_layers if cfg is None else cfg.num_layers
        self.num_kv_heads = num_kv_heads if cfg is None else cfg.num_kv_heads
        self.head_dim = head_dim if cfg is None else cfg.head_dim
        if None in (self.num_layers, self.num_kv_heads, self.head_dim):
            raise ValueError("give cfg, or num_layers, num_kv_heads and head_dim")
        if self.head_dim != HEAD_DIM:  # refuse here, before any attend() could write into the pools
            raise ValueError(f"head_dim {self.head_dim} not supported: the paged decode kernels take {HEAD_DIM}")
        if block_size < 1 or block_size & (block_size - 1):
            raise ValueError(f"block_size {block_size} must be a power of two")
        self.kv_dtype = kv_dtype
        self.format = _FORMATS[kv_dtype]
        self.block_size = block_size
        self.num_blocks = num_blocks
        self.device = torch.device(device)
        shape = (num_blocks, block_size, self.num_kv_heads, self.head_dim)  # [block, slot, kv_heads, head_dim]
        self.k = [torch.zeros(shape, dtype=kv_dtype, device=self.device) for _ in range(self.num_layers)]
        self.v = [torch.zeros(shape, dtype=kv_dtype, device=self.device) for _ in range(self.num_layers)]
        if self.format == "fp8":
            hs = (self.num_layers, self.num_kv_heads)
            ks = torch.ones(hs) if k_scale is None else k_scale
            vs = torch.ones(hs) if v_scale is None else v_scale
            for s in (ks, vs):
                if tuple(s.shape) != hs:
                    raise ValueError(f"FP8 scales must be [{hs[0]}, {hs[1]}], got {tuple(s.shape)}")
            self.k_scale = [ks[i].to(self.device, torch.float32).contiguous() for i in range(self.num_layers)]
            self.v_scale = [vs[i].to(self.device, torch.float32).contiguous() for i in range(self.num_layers)]
        elif self.format == "int8":
            if k_scale is not None or v_scale is not None:
                raise ValueError("INT8 scales are per token and computed on write: pass none")
            ss = (num_blocks, block_size, self.num_kv_heads)
            self.k_scale = [torch.zeros(ss, dtype=torch.float32, device=self.device) for _ in range(self.num_layers)]
            self.v_scale = [torch.zeros(ss, dtype=torch.float32, device=self.device) for _ in range(self.num_layers)]
        else:
            if k_scale is not None or v_scale is not None:
                raise ValueError("a bfloat16 cache takes no scales")
            self.k_scale = self.v_scale = [None] * self.num_layers
        # Allocation state. Free block ids live in a min-heap: the lowest free id is granted first (block 0 on a
        # fresh pool) and a released block is granted again before any higher one. `tables` maps each live
        # sequence to the physical blocks of its logical blocks 0, 1, ...; `free_blocks` is the heap itself
        # (only its length means anything to a scheduler).
        self.free_blocks: list[int] = list(range(num_blocks))
        self.tables: dict[Any, list[int]] = {}
        # The device mirror of `tables`: row `slot_of[seq]` of table_dev holds the sequence's block ids and
        # reserved_dev[slot] how many of them are valid. Slots are granted lowest first as well.
        self.max_seqs = max_seqs
        self.max_blocks_per_seq = min(num_blocks, 4096) if max_blocks_per_seq is None else max_blocks_per_seq
        self.table_dev = torch.zeros((max_seqs, self.max_blocks_per_seq), dtype=torch.int32, device=self.device)
        self.reserved_dev = torch.zeros(max_seqs, dtype=torch.int32, device=self.device)
        self.slot_of: dict[Any, int] = {}
        self.free_slots: list[int] = list(range(max_seqs))
        self._rows_key: tuple | None = None  # the rows of the last prepare and their device slots
        self._rows_slots: torch.Tensor | None = None

    # -- block allocation ---------------------------------------------------------------------------------------

    def blocks_needed(self, num_tokens: int) -> int:
        """Blocks that hold positions [0, num_tokens)."""
        return -(-num_tokens // self.block_size)

    def _shortfall(self, seq_id: Any, num_tokens: int) -> int:
        """Blocks `seq_id` lacks for num_tokens positions (negative or zero: it has enough)."""
        return self.blocks_needed(num_tokens) - len(self.tables.get(seq_id, ()))

    def can_reserve(self, seq_id: Any, num_tokens: int) -> bool:
        return self._shortfall(seq_id, num_tokens) <= len(self.free_blocks)

    def reserve(self, seq_id: Any, num_tokens: int) -> None:
        """Grow `seq_id`'s block table until it covers positions [0, num_tokens), granting the lowest free blocks,
        and mirror the new entries into the sequence's device row (a host-to-device copy: call it outside graph
        capture). Raises OutOfBlocksError, changing nothing, when the pool or the slots run out."""
        grow = self._shortfall(seq_id, num_tokens)
        if grow > len(self.free_blocks):
            raise OutOfBlocksError(f"sequence {seq_id!r} needs {grow} more blocks, the pool has {len(self.free_blocks)}")
        owned = self.tables.get(seq_id)
        if owned is None and not self.free_slots:
            raise OutOfBlocksError(f"no sequence slot left (all {self.max_seqs} are live)")
        have = 0 if owned is None else len(owned)
        if have + max(grow, 0) > self.max_blocks_per_seq:
            raise ValueError(f"sequence {seq_id!r} would need more than {self.max_blocks_per_seq} blocks")
        if owned is None:
            owned = self.tables[seq_id] = []
            self.slot_of[seq_id] = heapq.heappop(self.free_slots)
        slot = self.slot_of[seq_id]
        if grow > 0:
            granted = [heapq.heappop(self.free_blocks) for _ in range(grow)]
            owned += granted
            self.table_dev[slot, have : have + grow] = torch.tensor(granted, dtype=torch.int32)
        self.reserved_dev[slot] = len(owned)

    def free(self, seq_id: Any) -> None:
        """Release a finished sequence: its blocks and its device slot become grantable again."""
        for block in self.tables.pop(seq_id, ()):
            heapq.heappush(self.free_blocks, block)
        slot = self.slot_of.pop(seq_id, None)
        if slot is not None:
            heapq.heappush(self.free_slots, slot)

    def bytes_per_token(self) -> int:
        """Bytes one token occupies across all layers and KV heads (codes, plus INT8's per-token scales)."""
        elem = 2 if self.format == "bf16" else 1
        per_head = 2 * (self.head_dim * elem + (4 if self.format == "int8" else 0))
        return self.num_layers * self.num_kv_heads * per_head

    # -- the per-forward metadata and the attention hook ------------------------------------------------------

    def prepare(self, rows: list[Any], positions: torch.Tensor) -> PagedMeta:
        """Metadata for one forward pass. positions: [batch, q_len], consecutive within each row.

        Host positions are checked on the host first, as engine/kv_cache.py:140-146 does (consecutive,
        non-negative, reserved), and give the reference's exact kv_len and table width. Device positions are
        never read back: kv_len is then the rows' reserved tokens (a bound the launch is sized by), lengths are
        clamped to the reserved tokens, and a row whose positions run past its reserved blocks (or are out of
        order) gets no write slots: such a step stores nothing for it and attends its reserved tokens.
        On a GPU cache the tables come from one kernel (bpt_paged_prepare); a CPU cache (allocator tests) builds
        the same tables with torch index operations."""
        if positions.dim() != 2 or positions.shape[0] != len(rows):
            raise ValueError(f"positions must be [{len(rows)}, q_len], got {tuple(positions.shape)}")
        missing = [s for s in rows if s not in self.tables]
        if missing:
            raise ValueError(f"sequence {missing[0]!r} has too few blocks: call reserve() first")
        if positions.device.type == "cpu":
            pos = positions.to(torch.int64)
            if pos.shape[1] > 1 and not bool((pos[:, 1:] - pos[:, :-1] == 1).all()):
                raise ValueError("the positions of a row must be consecutive (one new token after another)")
            if bool((pos < 0).any()):
                raise ValueError("positions must be non-negative")
            for i, seq_id in enumerate(rows):
                if len(self.tables[seq_id]) * self.block_size < int(pos[i].max()) + 1:
                    raise ValueError(f"sequence {seq_id!r} has too few blocks: call reserve() first")
            kv_len = int(pos.max()) + 1 if pos.numel() else 0
            n_blocks = self.blocks_needed(kv_len)
        elif self.device.type == "cpu":
            raise ValueError("a CPU cache takes host positions")
        else:
            pos = positions
            n_blocks = max((len(self.tables[s]) for s in rows), default=0)  # the reserved blocks: a host bound
            kv_len = n_blocks * self.block_size
        b, nq = pos.shape
        if self.device.type == "cpu":
            tables = [self.tables[s][:n_blocks] + [0] * (n_blocks - len(self.tables[s][:n_blocks])) for s in rows]
            block_table = torch.tensor(tables, dtype=torch.int32).reshape(b, n_blocks)
            write_blocks = torch.gather(block_table.long(), 1, pos // self.block_size).to(torch.int32)
            return PagedMeta(write_blocks=write_blocks, write_offsets=(pos % self.block_size).to(torch.int32),
                             block_table=block_table, context_lens=(pos[:, -1] + 1).to(torch.int32), kv_len=kv_len)
        key = tuple(rows)
        if key != self._rows_key:  # rows change between steps only when the batch does
            self._rows_slots = torch.tensor([self.slot_of[s] for s in rows], dtype=torch.int32, device=self.device)
            self._rows_key = key
        dev = self.device
        block_table = torch.empty((b, max(n_blocks, 1)), dtype=torch.int32, device=dev)
        write_blocks = torch.empty((b, nq), dtype=torch.int32, device=dev)
        write_offsets = torch.empty((b, nq), dtype=torch.int32, device=dev)
        context_lens = torch.empty(b, dtype=torch.int32, device=dev)
        paged_prepare(self.table_dev, self.reserved_dev, self._rows_slots, pos.to(dev), self.block_size, block_table,
                      write_blocks, write_offsets, context_lens)
        return PagedMeta(write_blocks=write_blocks, write_offsets=write_offsets, block_table=block_table,
                         context_lens=context_lens, kv_len=kv_len)

    def update(self, layer: int, k: torch.Tensor, v: torch.Tensor, meta: PagedMeta):
        raise NotImplementedError("a quantized cache never returns float keys and values: use attend()")

    def attend(
        self, layer: int, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, meta: PagedMeta, scale: float
    ) -> torch.Tensor:
        """Store this step's k, v [B, Hkv, Q, D] in their slots, then attend: q [B, Hq, Q, D] -> [B, Hq, Q, D]."""
        b, hq, nq, d = q.shape
        if tuple(k.shape) != (b, self.num_kv_heads, nq, d) or k.shape != v.shape:
            raise ValueError(f"k and v must be [{b}, {self.num_kv_heads}, {nq}, {d}]")
        if tuple(meta.write_blocks.shape) != (b, nq):
            raise ValueError(f"meta was prepared for {tuple(meta.write_blocks.shape)} tokens, not {(b, nq)}")
        # Store, then attend; one launch where the decode kernel can store the rows itself (paged_append_decode).
        out = paged_append_decode(
            q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), self.k[layer], self.v[layer], meta.block_table,
            meta.context_lens, self.k_scale[layer], self.v_scale[layer], meta.write_blocks, meta.write_offsets,
            scale=scale, max_context=meta.kv_len, out_dtype=q.dtype,
        )  # [B, Q, Hq, D] in q's dtype: the kernel rounds once, from float32 (integration/kv_cache.py:177-181)
        return out.transpose(1, 2)
