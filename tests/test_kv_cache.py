"""The paged quantized KV cache on the CPU: allocator, per-forward metadata and sizing, against fastserve's own
known answers (tests/engine/test_kv_cache.py:36-60, tests/kv/test_sizing.py:18-24) and the paging oracle."""

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from bpt_amd.kv_cache import OutOfBlocksError, PagedQuantKVCache
from oracle import paged

GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_known_answers.json").read_text())


def make(fmt="fp8", num_blocks=4, block_size=2, layers=2, heads=2, d=128):
    dtype = {"fp8": torch.float8_e4m3fn, "int8": torch.int8, "bf16": torch.bfloat16}[fmt]
    return PagedQuantKVCache(num_layers=layers, num_kv_heads=heads, head_dim=d, num_blocks=num_blocks,
                             block_size=block_size, kv_dtype=dtype, device="cpu")


def test_allocator_hands_out_and_reuses_blocks():
    g = GOLDEN["paged_allocator"]
    cache = make(num_blocks=g["num_blocks"], block_size=g["block_size"])
    cache.reserve("a", 3)  # 3 tokens -> 2 blocks
    cache.reserve("b", 4)  # 4 tokens -> 2 blocks
    assert cache.tables["a"] == [0, 1] and len(cache.free_blocks) == 0  # block 0 first
    assert not cache.can_reserve("c", 1)
    with pytest.raises(OutOfBlocksError):
        cache.reserve("c", 1)
    freed = set(cache.tables["a"])
    cache.free("a")
    cache.reserve("c", 4)
    assert set(cache.tables["c"]) == freed


def test_prepare_refuses_unreserved_positions():
    g = GOLDEN["paged_allocator"]
    cache = make(num_blocks=g["num_blocks"], block_size=g["block_size"])
    cache.reserve("a", g["refuse"]["reserved_tokens"])
    with pytest.raises(ValueError, match=g["refuse"]["message"]):
        cache.prepare(["a"], torch.tensor([[g["refuse"]["position"]]]))


def test_prepare_matches_the_paging_oracle():
    rng = np.random.default_rng(0)
    cache = make(num_blocks=64, block_size=4)
    lengths = {"x": 9, "y": 1, "z": 17}
    for s, n in lengths.items():
        cache.reserve(s, n + 3)
    rows = ["z", "x", "y"]
    starts = [lengths[s] for s in rows]
    positions = torch.tensor([[p + i for i in range(3)] for p in starts])
    meta = cache.prepare(rows, positions)
    wb, wo, bt, kv_len = paged.prepare([cache.tables[s] for s in rows], positions.numpy(), 4)
    assert meta.kv_len == kv_len == max(starts) + 3
    assert np.array_equal(meta.write_blocks.numpy(), wb) and np.array_equal(meta.write_offsets.numpy(), wo)
    assert np.array_equal(meta.block_table.numpy(), bt)
    assert meta.context_lens.tolist() == [s + 3 for s in starts]
    assert meta.block_table.dtype == torch.int32 and rng is not None


def test_prepare_needs_consecutive_positions_and_update_is_refused():
    cache = make(num_blocks=8, block_size=4)
    cache.reserve("a", 8)
    with pytest.raises(ValueError, match="consecutive"):
        cache.prepare(["a"], torch.tensor([[3, 5]]))
    meta = cache.prepare(["a"], torch.tensor([[3, 4]]))
    with pytest.raises(NotImplementedError, match="attend"):
        cache.update(0, None, None, meta)


def test_attend_needs_a_gpu():
    cache = make(num_blocks=8, block_size=4)
    cache.reserve("a", 4)
    meta = cache.prepare(["a"], torch.tensor([[0]]))
    q = torch.zeros((1, 4, 1, 128), dtype=torch.bfloat16)
    k = torch.zeros((1, 2, 1, 128), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU"):
        cache.attend(0, q, k, k, meta, scale=0.1)


@pytest.mark.parametrize("fmt", ["bf16", "fp8", "int8"])
def test_bytes_per_token_known_answers(fmt):
    g = GOLDEN["kv_bytes_per_token"]
    cache = make(fmt, layers=g["layers"], heads=g["kv_heads"], d=g["head_dim"], num_blocks=1, block_size=1)
    expect = {"bf16": g["bf16"], "fp8": g["fp8"], "int8": g["fp8"] + g["layers"] * g["kv_heads"] * 2 * 4}[fmt]
    assert cache.bytes_per_token() == expect


def test_constructor_checks():
    with pytest.raises(ValueError, match="kv_dtype"):
        PagedQuantKVCache(num_layers=1, num_kv_heads=1, head_dim=128, num_blocks=1, block_size=1,
                          kv_dtype=torch.float16, device="cpu")
    with pytest.raises(ValueError, match="power of two"):
        make(block_size=3)
    with pytest.raises(ValueError, match="FP8 scales"):
        PagedQuantKVCache(num_layers=2, num_kv_heads=2, head_dim=128, num_blocks=1, block_size=1,
                          device="cpu", k_scale=torch.ones(3))
