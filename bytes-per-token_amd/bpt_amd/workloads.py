"""Seeded synthetic decode workloads at the five measured shapes (one attention layer each).

Every workload is built on the target device with torch: random keys and values, quantized with plain torch
ops (not the library's write kernel, which is tested against them separately), scattered into a page pool
through a seeded random block table. Shapes (Hq query heads / Hkv KV heads, head_dim 128, page size 16):

  qwen3-0.6b-bf16     1 sequence x 512 tokens, 16/8 heads, BF16 cache, pool = exactly its 32 pages, permuted
  qwen3-1.7b-fp8      32 sequences, lengths ~ U[256, 4096], FP8 e4m3fn with per-KV-head scales amax/448;
                      K ~ N(0,1) with 4 of 128 channels x8, V ~ N(0,1); pages scattered over a 2x pool
  qwen3-1.7b-int8     64 sequences x 8192 tokens, INT8 with per-token-per-head scales amax/127; the
                      newest token of every sequence (position 8191, slot 15 of its last page) is the
                      step's quantize-on-write row
  qwen3-8b-fp8-long   4 sequences x 32768 tokens, 32/8 heads, FP8 as above, 32 split-K partitions
  qwen3-1.7b-verify   16 sequences, 5 causal queries each, lengths ~ U[1024, 3072], FP8; the first 64 pages
                      (1024 tokens) of every block table are the same physical pages (a shared prefix)
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

PAGE = 16
HEAD_DIM = 128


@dataclass
class Shape:
    name: str
    batch: int
    q_heads: int
    kv_heads: int
    kv_format: str  # bf16 | fp8 | int8
    scales: str  # none | head | token
    lengths: tuple[int, int] | int  # fixed, or (lo, hi) inclusive uniform
    queries: int = 1
    num_splits: int | None = None
    pool_factor: float = 1.0
    shared_prefix_pages: int = 0
    outliers: bool = False


SHAPES = {
    "qwen3-0.6b-bf16": Shape("qwen3-0.6b-bf16", 1, 16, 8, "bf16", "none", 512),
    "qwen3-1.7b-fp8": Shape("qwen3-1.7b-fp8", 32, 16, 8, "fp8", "head", (256, 4096), pool_factor=2.0, outliers=True),
    "qwen3-1.7b-int8": Shape("qwen3-1.7b-int8", 64, 16, 8, "int8", "token", 8192),
    "qwen3-8b-fp8-long": Shape("qwen3-8b-fp8-long", 4, 32, 8, "fp8", "head", 32768, num_splits=32, outliers=True),
    "qwen3-1.7b-verify": Shape(
        "qwen3-1.7b-verify", 16, 16, 8, "fp8", "head", (1024, 3072), queries=5, shared_prefix_pages=64, outliers=True
    ),
}
DEFAULT = "qwen3-1.7b-fp8"


@dataclass
class Workload:
    shape: Shape
    q: torch.Tensor  # [B, Q, Hq, D] bf16
    k_cache: torch.Tensor  # [NB, P, Hkv, D]
    v_cache: torch.Tensor
    k_scale: torch.Tensor | None
    v_scale: torch.Tensor | None
    block_table: torch.Tensor  # [B, max_blocks] int32
    context_lens: torch.Tensor  # [B] int32
    lengths: list[int]
    max_context: int
    sm_scale: float
    unique_tokens: int
    extra: dict = field(default_factory=dict)

    def kwargs(self) -> dict:
        return dict(
            scale=self.sm_scale, max_context=self.max_context, num_splits=self.shape.num_splits
        )

    def args(self) -> tuple:
        return (self.q, self.k_cache, self.v_cache, self.block_table, self.context_lens, self.k_scale, self.v_scale)

    def kv_bytes(self, unique: bool = False) -> int:
        """Algorithmic KV bytes one call reads (codes + scales); `unique` counts shared pages once."""
        tokens = self.unique_tokens if unique else sum(self.lengths)
        hkv, elem = self.shape.kv_heads, (2 if self.shape.kv_format == "bf16" else 1)
        per_token = hkv * HEAD_DIM * 2 * elem + (hkv * 2 * 4 if self.shape.scales == "token" else 0)
        return tokens * per_token + (hkv * 2 * 4 if self.shape.scales == "head" else 0)


def _lengths(shape: Shape, gen: torch.Generator, batch: int) -> list[int]:
    if isinstance(shape.lengths, int):
        return [shape.lengths] * batch
    lo, hi = shape.lengths
    return torch.randint(lo, hi + 1, (batch,), generator=gen).tolist()


def quantize_per_head_fp8(x: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """[..., Hkv, D] float32 -> float8_e4m3fn codes with static per-head scales (clamp to ±448, then cast)."""
    return (x / scale[:, None]).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)


def quantize_per_token_int8(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """[..., D] float32 -> (int8 codes, float32 scale [...]): s = max(amax/127, 1e-12), round half to even."""
    scale = (x.abs().amax(-1, keepdim=True) / 127.0).clamp(min=1e-12)
    return torch.clamp(torch.round(x / scale), -128, 127).to(torch.int8), scale[..., 0]


def make(name: str = DEFAULT, device="cuda", seed: int = 0, batch: int | None = None,
         length_cap: int | None = None, shape: Shape | None = None) -> Workload:
    """Build workload `name` (or the given `shape`) on `device`. `batch` / `length_cap` shrink it (tests)."""
    shape = SHAPES[name] if shape is None else shape
    gen = torch.Generator().manual_seed(seed)
    b = batch if batch is not None else shape.batch
    lengths = _lengths(shape, gen, b)
    if length_cap is not None:
        lengths = [min(t, length_cap) for t in lengths]
    hq, hkv, d, nq = shape.q_heads, shape.kv_heads, HEAD_DIM, shape.queries
    shared = shape.shared_prefix_pages
    shared_tokens = shared * PAGE

    # Logical pages of each sequence: the shared prefix pages first (same physical pages for all).
    own_pages = [math.ceil(max(t - shared_tokens, 0) / PAGE) if shared else math.ceil(t / PAGE) for t in lengths]
    needed = shared + sum(own_pages)
    num_blocks = max(int(math.ceil(needed * shape.pool_factor)), 1)
    perm = torch.randperm(num_blocks, generator=gen)
    shared_phys = perm[:shared].tolist()
    cursor = shared
    tables = []
    for n in own_pages:
        tables.append(shared_phys + perm[cursor : cursor + n].tolist())
        cursor += n
    max_blocks = max(max((len(t) for t in tables), default=1), 1)
    table = torch.zeros((b, max_blocks), dtype=torch.int32)
    for i, row in enumerate(tables):
        table[i, : len(row)] = torch.tensor(row, dtype=torch.int32)

    # Token values: one stream per sequence (the shared prefix once), float32 on the device.
    gdev = torch.Generator(device=device).manual_seed(seed + 1)
    outlier_channels = torch.randperm(d, generator=gen)[:4] if shape.outliers else None

    def rand_tokens(n: int) -> tuple[torch.Tensor, torch.Tensor]:
        k = torch.randn((n, hkv, d), generator=gdev, device=device)
        if outlier_channels is not None:
            k[..., outlier_channels.to(device)] *= 8.0
        v = torch.randn((n, hkv, d), generator=gdev, device=device)
        return k, v

    prefix_k, prefix_v = rand_tokens(shared_tokens) if shared else (None, None)
    seq_k, seq_v = [], []
    for t in lengths:
        n = t - shared_tokens if shared else t
        k, v = rand_tokens(max(n, 0))
        seq_k.append(k)
        seq_v.append(v)

    # Physical placement: slot index of every token in the flattened pool [NB * P].
    def slots_of(row: list[int], n_tok: int, start_tok: int = 0) -> torch.Tensor:
        pos = torch.arange(start_tok, start_tok + n_tok)
        pages = torch.tensor(row, dtype=torch.int64)[pos // PAGE] if n_tok else torch.zeros(0, dtype=torch.int64)
        return (pages * PAGE + pos % PAGE).to(device)

    all_k = [prefix_k] if shared else []
    all_v = [prefix_v] if shared else []
    all_slots = [slots_of(shared_phys, shared_tokens)] if shared else []
    for i, t in enumerate(lengths):
        start = shared_tokens if shared else 0
        all_k.append(seq_k[i])
        all_v.append(seq_v[i])
        all_slots.append(slots_of(tables[i], max(t - start, 0), start))
    k_all = torch.cat(all_k) if all_k else torch.zeros((0, hkv, d), device=device)
    v_all = torch.cat(all_v) if all_v else torch.zeros((0, hkv, d), device=device)
    slots = torch.cat(all_slots) if all_slots else torch.zeros(0, dtype=torch.int64, device=device)

    k_scale = v_scale = None
    if shape.kv_format == "bf16":
        dtype = torch.bfloat16
        k_codes, v_codes = k_all.to(dtype), v_all.to(dtype)
    elif shape.kv_format == "fp8":
        dtype = torch.float8_e4m3fn
        k_scale = (k_all.abs().amax(dim=(0, 2)) / 448.0).clamp(min=1e-12).float()
        v_scale = (v_all.abs().amax(dim=(0, 2)) / 448.0).clamp(min=1e-12).float()
        k_codes, v_codes = quantize_per_head_fp8(k_all, k_scale), quantize_per_head_fp8(v_all, v_scale)
    else:
        dtype = torch.int8
        k_codes, ks = quantize_per_token_int8(k_all)
        v_codes, vs = quantize_per_token_int8(v_all)
        k_scale = torch.zeros((num_blocks * PAGE, hkv), dtype=torch.float32, device=device)
        v_scale = torch.zeros_like(k_scale)
        k_scale[slots] = ks
        v_scale[slots] = vs
        k_scale = k_scale.view(num_blocks, PAGE, hkv)
        v_scale = v_scale.view(num_blocks, PAGE, hkv)

    k_cache = torch.zeros((num_blocks * PAGE, hkv, d), dtype=dtype, device=device)
    v_cache = torch.zeros_like(k_cache)
    if dtype == torch.bfloat16:
        k_cache[slots] = k_codes
        v_cache[slots] = v_codes
    else:  # one-byte codes are scattered through a uint8 view (index_put has no float8 kernel)
        k_cache.view(torch.uint8)[slots] = k_codes.view(torch.uint8)
        v_cache.view(torch.uint8)[slots] = v_codes.view(torch.uint8)
    k_cache = k_cache.view(num_blocks, PAGE, hkv, d)
    v_cache = v_cache.view(num_blocks, PAGE, hkv, d)
    del k_all, v_all, k_codes, v_codes

    q = torch.randn((b, nq, hq, d), generator=gdev, device=device).to(torch.bfloat16)
    unique = shared_tokens + sum(max(t - shared_tokens, 0) for t in lengths) if shared else sum(lengths)
    return Workload(
        shape=shape,
        q=q,
        k_cache=k_cache,
        v_cache=v_cache,
        k_scale=k_scale,
        v_scale=v_scale,
        block_table=table.to(device),
        context_lens=torch.tensor(lengths, dtype=torch.int32, device=device),
        lengths=lengths,
        max_context=max(lengths) if lengths else 0,
        sm_scale=d**-0.5,
        unique_tokens=unique,
        extra={"num_blocks": num_blocks, "tables": tables},
    )


def to_oracle(w: Workload) -> dict:
    """The workload as numpy arrays in the oracle's conventions (codes as stored, scales as float32)."""
    fmt = w.shape.kv_format

    def codes(t: torch.Tensor):
        if fmt == "fp8":
            return t.view(torch.uint8).cpu().numpy()
        if fmt == "int8":
            return t.cpu().numpy()
        return t.float().cpu().numpy()

    return dict(
        q=w.q.float().cpu().numpy(),
        k_pool=codes(w.k_cache),
        v_pool=codes(w.v_cache),
        block_table=w.block_table.cpu().numpy(),
        context_lens=w.context_lens.cpu().numpy(),
        k_scale=None if w.k_scale is None else w.k_scale.cpu().numpy(),
        v_scale=None if w.v_scale is None else w.v_scale.cpu().numpy(),
        kv_format=fmt,
        scale=w.sm_scale,
    )


# ---- KIVI caches (contiguous, fastserve's kernel-2 format) ------------------------------------------------

# The shapes of fastserve's kernel-2 benchmark (experiments/m7.py:210-290, one Qwen3-1.7B attention layer:
# 16 query / 8 KV heads, head dim 128), as (batch, context): every batch of 1, 4, 16, 64 with every context
# of 512 .. 32768 tokens up to 524288 tokens in all (benchmarks/configs/m7_kernels.yaml:26-31).
KIVI_SHAPES = tuple((b, t) for b in (1, 4, 16, 64) for t in (512, 2048, 8192, 32768) if b * t <= 524288)
KIVI_BITS = (4, 8, 16)


@dataclass
class KiviWorkload:
    """A KIVI cache with QuantKV's fields (kernels/reference.py:66-100) plus the decode call's inputs."""

    bits: int
    group: int
    k_codes: torch.Tensor
    v_codes: torch.Tensor
    k_scale: torch.Tensor | None
    k_zero: torch.Tensor | None
    v_scale: torch.Tensor | None
    v_zero: torch.Tensor | None
    q: torch.Tensor  # [B, Hq, D] bf16
    lengths: torch.Tensor  # [B] int32, every row full
    context: int

    def cache_bytes(self) -> int:
        """Bytes the cache occupies for `context` tokens per row, grids included: what one call reads
        (experiments/m7.py:207-208 cache_bytes)."""
        ts = [self.k_codes, self.v_codes, self.k_scale, self.k_zero, self.v_scale, self.v_zero]
        return sum(t.numel() * t.element_size() for t in ts if t is not None)


def kivi_name(batch: int, context: int, bits: int) -> str:
    return f"kivi-{'int4' if bits == 4 else 'int8' if bits == 8 else 'bf16'}-{batch}x{context}"


def make_kivi(batch: int, context: int, bits: int, device="cuda", seed: int = 0, q_heads: int = 16,
              kv_heads: int = 8, group: int = 32) -> KiviWorkload:
    """Random codes and grids of the right format (timing input; parity is tested on quantized data).

    bits 4 / 8: uniform codes, key scales U[0.01, 0.1] per channel per group with integer zero points, value
    scales likewise per token; bits 16: bfloat16 N(0, 1) keys and values.
    """
    gen = torch.Generator(device=device).manual_seed(seed)
    d = HEAD_DIM
    shape = (batch, kv_heads, context, d)
    q = torch.randn((batch, q_heads, d), generator=gen, device=device).to(torch.bfloat16)
    lengths = torch.full((batch,), context, dtype=torch.int32, device=device)
    if bits == 16:
        k = torch.randn(shape, generator=gen, device=device).to(torch.bfloat16)
        v = torch.randn(shape, generator=gen, device=device).to(torch.bfloat16)
        return KiviWorkload(16, group, k, v, None, None, None, None, q, lengths, context)
    levels = 2**bits
    width = d // 2 if bits == 4 else d
    codes = lambda: torch.randint(0, 256, (batch, kv_heads, context, width), generator=gen, device=device,  # noqa: E731
                                  dtype=torch.uint8)
    groups = context // group

    def scale(*s):
        return (torch.rand(s, generator=gen, device=device) * 0.09 + 0.01).to(torch.float16)

    def zero(*s):
        return torch.randint(0, levels, s, generator=gen, device=device).to(torch.float16)

    return KiviWorkload(
        bits, group, codes(), codes(),
        scale(batch, kv_heads, groups, d), zero(batch, kv_heads, groups, d),
        scale(batch, kv_heads, context), zero(batch, kv_heads, context),
        q, lengths, context,
    )
