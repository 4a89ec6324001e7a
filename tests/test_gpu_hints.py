"""GPU: launch hints (paged_decode_hints / bpt_decode_hints) change when the decode's first loads go out, never
what it computes. Every call with a hint must equal the same call without one bit for bit, whether the hint
matches the call, was built from other lengths, another block table or another launch shape, or holds random
bytes; and the call without a hint is itself checked against the oracle in test_gpu_decode.py.
"""

import pytest
import torch

from bpt_amd import paged_append_decode, paged_decode_attention, paged_decode_hints, workloads

pytestmark = pytest.mark.gpu

DEV = "cuda"


def run(w, hints=None, out_dtype=torch.bfloat16):
    out = paged_decode_attention(*w.args(), **w.kwargs(), out_dtype=out_dtype, hints=hints)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize(
    "name,batch,cap",
    [("qwen3-1.7b-fp8", 32, None), ("qwen3-1.7b-fp8", 5, 700), ("qwen3-1.7b-verify", 16, None),
     ("qwen3-8b-fp8-long", 4, None), ("qwen3-1.7b-fp8", 1, 3000)],
)
def test_hinted_decode_equals_unhinted(name, batch, cap):
    print(f"hinted decode {name} batch {batch} cap {cap}", flush=True)
    w = workloads.make(name, device=DEV, seed=3, batch=batch, length_cap=cap)
    hints = paged_decode_hints(*w.args(), **w.kwargs())
    assert hints is not None and hints.numel() > 0
    want = run(w)
    assert torch.equal(run(w, hints), want)
    assert torch.equal(run(w, hints, torch.float32), run(w, None, torch.float32))


def test_hints_from_other_lengths_table_or_shape_change_nothing():
    w = workloads.make("qwen3-1.7b-fp8", device=DEV, seed=4, batch=12, length_cap=2500)
    want = run(w)
    # Other lengths: every hint names a different range start.
    lens0 = w.context_lens.clone()
    w.context_lens.copy_(torch.clamp(lens0 - 37, min=0))
    stale = paged_decode_hints(*w.args(), **w.kwargs())
    w.context_lens.copy_(lens0)
    assert torch.equal(run(w, stale), want)
    # Another block table: the ranges match, the hinted pages do not.
    table0 = w.block_table.clone()
    w.block_table.copy_(torch.roll(table0, 1, dims=1))
    other_pages = paged_decode_hints(*w.args(), **w.kwargs())
    w.block_table.copy_(table0)
    assert torch.equal(run(w, other_pages), want)
    # Another launch shape (a fixed split count: other ranges, another grid), padded to this call's size.
    kw = w.kwargs()
    kw["num_splits"] = 4
    foreign = paged_decode_hints(*w.args(), **kw)
    need = paged_decode_hints(*w.args(), **w.kwargs()).numel()
    buf = torch.zeros(max(need, foreign.numel()), dtype=torch.uint8, device=DEV)
    buf[: foreign.numel()] = foreign
    assert torch.equal(run(w, buf), want)
    # Random bytes.
    gen = torch.Generator(device=DEV).manual_seed(9)
    noise = torch.randint(0, 256, (need,), generator=gen, device=DEV, dtype=torch.int32).to(torch.uint8)
    assert torch.equal(run(w, noise), want)
    # Flags set, fields random: every hinted load is clamped into the pools, then re-issued.
    rec = torch.randint(-(1 << 30), 1 << 30, (need // 4,), generator=gen, device=DEV, dtype=torch.int32)
    rec.view(-1, 32)[:, 0] = 1
    assert torch.equal(run(w, rec.view(torch.uint8)), want)


def test_hints_with_empty_and_truncated_lengths():
    w = workloads.make("qwen3-1.7b-fp8", device=DEV, seed=5, batch=9, length_cap=1200)
    w.context_lens[2] = 0
    w.context_lens[5] = 1
    w.context_lens[7] = w.max_context + 500  # truncated to max_context by the launch
    hints = paged_decode_hints(*w.args(), **w.kwargs())
    assert torch.equal(run(w, hints), run(w))


def test_hinted_store_then_attend_equals_unhinted():
    """The fused store-then-attend launch with hints stores the same codes and returns the same rows."""
    outs = []
    for use_hints in (False, True):
        w = workloads.make("qwen3-1.7b-fp8", device=DEV, seed=6, batch=10, length_cap=1800)
        b, hkv, page = w.q.shape[0], w.shape.kv_heads, w.k_cache.shape[1]
        gen = torch.Generator(device=DEV).manual_seed(2)
        kn = torch.randn((b, 1, hkv, 128), generator=gen, device=DEV).to(torch.bfloat16)
        vn = torch.randn((b, 1, hkv, 128), generator=gen, device=DEV).to(torch.bfloat16)
        pos = w.context_lens.long()[:, None] - 1
        wb = torch.gather(w.block_table.long(), 1, pos // page).to(torch.int32)
        wo = (pos % page).to(torch.int32)
        hints = paged_decode_hints(*w.args(), **w.kwargs()) if use_hints else None
        out = paged_append_decode(w.q, kn, vn, *w.args()[1:], wb, wo, **w.kwargs(), hints=hints)
        torch.cuda.synchronize()
        outs.append((out, w.k_cache.clone(), w.v_cache.clone()))
    for a, c in zip(outs[0], outs[1]):
        assert torch.equal(a.view(torch.uint8) if a.dtype == torch.float8_e4m3fn else a,
                           c.view(torch.uint8) if c.dtype == torch.float8_e4m3fn else c)


def test_too_small_hint_buffer_is_refused():
    w = workloads.make("qwen3-1.7b-fp8", device=DEV, seed=7, batch=4, length_cap=600)
    hints = paged_decode_hints(*w.args(), **w.kwargs())
    with pytest.raises(ValueError, match="hints"):
        run(w, hints[:-16])
