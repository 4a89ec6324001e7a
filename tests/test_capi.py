"""The C-ABI library on the CPU: it loads, exports every symbol include/bpt_amd.h declares, plans splits, and
refuses bad arguments with ValueError before touching a GPU (no compute calls here)."""

import ctypes
import re
from pathlib import Path

import pytest
import torch

from bpt_amd import _lib, decode_plan, paged_decode_attention, quantize_append

HEADER = Path(__file__).resolve().parent.parent / "include" / "bpt_amd.h"


def declared_symbols() -> list[str]:
    text = HEADER.read_text()
    return re.findall(r"^\s*(?:int|const char\*)\s+(bpt_\w+)\s*\(", text, flags=re.M)


def test_every_declared_symbol_is_exported(built_lib):
    names = declared_symbols()
    assert len(names) >= 9
    for name in names:
        assert hasattr(built_lib, name), name
    assert set(names) == set(_lib.SIGNATURES)
    assert built_lib.bpt_abi_version() == _lib.ABI_VERSION


def cpu_case(fmt="fp8", b=2, nq=1, hq=16, hkv=8, d=128, nb=64, page=16, max_blocks=8):
    dtype = {"fp8": torch.float8_e4m3fn, "int8": torch.int8, "bf16": torch.bfloat16}[fmt]
    q = torch.zeros((b, nq, hq, d), dtype=torch.bfloat16)
    k = torch.zeros((nb, page, hkv, d), dtype=dtype)
    v = torch.zeros_like(k)
    table = torch.zeros((b, max_blocks), dtype=torch.int32)
    lens = torch.zeros(b, dtype=torch.int32)
    if fmt == "fp8":
        ks, vs = torch.ones(hkv), torch.ones(hkv)
    elif fmt == "int8":
        ks, vs = torch.ones(nb, page, hkv), torch.ones(nb, page, hkv)
    else:
        ks = vs = None
    return q, k, v, table, lens, ks, vs


def test_plan_honours_requested_splits(built_lib):
    q, k, v, table, lens, ks, vs = cpu_case(b=4, hq=32, max_blocks=2048, nb=8192)
    splits, split_tokens, ws = decode_plan(q, k, v, table, lens, ks, vs, scale=0.1, max_context=32768, num_splits=32)
    assert (splits, split_tokens) == (32, 1024)
    assert ws == 4 * 1 * 32 * 32 * (128 + 1) * 4  # out partials + lse, float32


def test_plan_auto_single_split_needs_no_workspace(built_lib):
    q, k, v, table, lens, ks, vs = cpu_case("bf16", b=1)
    splits, split_tokens, ws = decode_plan(q, k, v, table, lens, ks, vs, scale=0.1, max_context=64, num_splits=1)
    assert splits == 1 and ws == 0 and split_tokens % 16 == 0 and split_tokens >= 64


@pytest.mark.parametrize("max_context", [1, 100, 4096, 32768])
def test_auto_plan_covers_the_context_in_whole_chunks(built_lib, max_context):
    q, k, v, table, lens, ks, vs = cpu_case(b=32, max_blocks=4096, nb=8192)
    splits, split_tokens, _ = decode_plan(q, k, v, table, lens, ks, vs, scale=0.1, max_context=max_context)
    assert split_tokens % 32 == 0 and splits * split_tokens >= max_context
    assert (splits - 1) * split_tokens < max(max_context, 1)
    assert split_tokens // 16 + 1 <= 512  # the split's pages fit the LDS page table


def test_stale_binding_is_refused(built_lib):
    a = _lib.DecodeArgs()
    a.struct_size = 12
    with pytest.raises(ValueError, match="stale binding"):
        _lib.check(built_lib.bpt_decode_plan(ctypes.byref(a), None))


@pytest.mark.parametrize(
    "change,match",
    [
        (dict(hq=12), "not a multiple"),
        (dict(d=64), "head_dim"),
        (dict(page=12), "power of two"),
    ],
)
def test_plan_rejects_bad_shapes(built_lib, change, match):
    q, k, v, table, lens, ks, vs = cpu_case(**change)
    with pytest.raises(ValueError, match=match):
        decode_plan(q, k, v, table, lens, ks, vs, scale=0.1, max_context=16)


def test_python_layer_rejects_bad_tensors_before_any_gpu_call(built_lib):
    q, k, v, table, lens, ks, vs = cpu_case()
    with pytest.raises(ValueError, match="k_scale and v_scale are required"):
        decode_plan(q, k, v, table, lens, None, None, scale=0.1, max_context=16)
    with pytest.raises(ValueError, match="int32"):
        decode_plan(q, k, v, table, lens.long(), ks, vs, scale=0.1, max_context=16)
    with pytest.raises(ValueError, match="dtype"):
        decode_plan(q, k.view(torch.uint8), v.view(torch.uint8), table, lens, ks, vs, scale=0.1, max_context=16)
    with pytest.raises(ValueError, match="on a GPU"):
        paged_decode_attention(q, k, v, table, lens, ks, vs, scale=0.1, max_context=16)
    with pytest.raises(ValueError, match="takes no scales"):
        qb, kb, vb, tb, lb, _, _ = cpu_case("bf16")
        decode_plan(qb, kb, vb, tb, lb, ks, vs, scale=0.1, max_context=16)


def test_quantize_append_rejects_bad_tensors(built_lib):
    _, k_cache, v_cache, _, _, ks, vs = cpu_case("int8")
    rows = torch.zeros((2, 1, 8, 128), dtype=torch.bfloat16)
    slots = torch.zeros((2, 1), dtype=torch.int32)
    with pytest.raises(ValueError, match="must be \\[2, 1\\]"):
        quantize_append(rows, rows, k_cache, v_cache, ks, vs, slots[:1], slots[:1])
    with pytest.raises(ValueError, match="on a GPU"):
        quantize_append(rows, rows, k_cache, v_cache, ks, vs, slots, slots)
    with pytest.raises(ValueError, match="per-token-head scales"):
        quantize_append(rows, rows, k_cache, v_cache, ks[:3], vs[:3], slots, slots)
