"""GPU: store-then-attend in one call (bpt_amd.paged_append_decode -> bpt_paged_append_decode) against the two
calls it replaces, quantize_append then paged_decode_attention, on copies of the same pools.

Where the matrix-core kernel stores the new rows itself (per-head scales, bf16 rows of the last Q <= 8 tokens),
the pools must come out byte for byte the same and the outputs bit for bit the same (the same codes go through
the same kernel arithmetic). The other layouts (per-token scales, BF16 caches, the vector kernel) take the two
launches inside the call and must match too. The codes themselves are pinned to the oracle's quantizers by
test_gpu_quant.py, and the attention by test_gpu_decode.py.
"""

import pytest
import torch

from test_gpu_decode import DEV, make_case

pytestmark = pytest.mark.gpu


def new_rows(c, nq, seed):
    """New bf16 rows [B, Q, Hkv, D] and their slots: the table's pages for the last Q positions of each length."""
    b = len(c["lens"])
    hkv, d = c["k"].shape[2], c["k"].shape[3]
    page = c["k"].shape[1]
    g = torch.Generator(device=DEV).manual_seed(seed)
    k = (torch.randn((b, nq, hkv, d), generator=g, device=DEV) * 2).to(torch.bfloat16)
    v = (torch.randn((b, nq, hkv, d), generator=g, device=DEV) * 2).to(torch.bfloat16)
    lens = c["lens"].long()
    pos = (lens[:, None] - nq + torch.arange(nq, device=DEV)[None]).clamp(min=0)
    blocks = torch.gather(c["table"].long(), 1, pos // page).to(torch.int32)
    offsets = (pos % page).to(torch.int32)
    return k, v, blocks, offsets


def both_ways(c, k, v, blocks, offsets, max_context, scale=0.09, num_splits=None):
    from bpt_amd import paged_append_decode, paged_decode_attention, quantize_append

    pools = []
    outs = []
    for fused in (False, True):
        kc, vc = c["k"].clone(), c["v"].clone()
        ks = None if c["ks"] is None else c["ks"].clone()
        vs = None if c["vs"] is None else c["vs"].clone()
        if fused:
            out = paged_append_decode(c["q"], k, v, kc, vc, c["table"], c["lens"], ks, vs, blocks, offsets,
                                      scale=scale, max_context=max_context, num_splits=num_splits)
        else:
            quantize_append(k, v, kc, vc, ks, vs, blocks, offsets)
            out = paged_decode_attention(c["q"], kc, vc, c["table"], c["lens"], ks, vs, scale=scale,
                                         max_context=max_context, num_splits=num_splits)
        torch.cuda.synchronize()
        pools.append([t.view(torch.uint8) if t.dtype != torch.float32 else t for t in (kc, vc, ks, vs) if t is not None])
        outs.append(out)
    for a, b in zip(*pools):
        assert torch.equal(a, b), "the pools differ after the store"
    assert torch.equal(outs[0], outs[1]), f"outputs differ: max {(outs[0].float() - outs[1].float()).abs().max()}"


@pytest.mark.parametrize("fmt,nq,hq,hkv", [("fp8", 1, 16, 8), ("fp8", 5, 16, 8), ("fp8", 1, 32, 8), ("fp8", 8, 16, 8),
                                           ("int8", 3, 16, 8), ("int8", 5, 16, 8)])
@pytest.mark.parametrize("page", [8, 16, 32])
def test_fused_store_matches_store_then_decode(fmt, nq, hq, hkv, page):
    """Matrix-core cases (2 .. 16 rows per KV head): the kernel stores the rows and uses them in place."""
    lengths = [max(t, nq) for t in (1 + nq, 47, 300, 1024, 33, 2000, 64, 95)]
    c = make_case(fmt, lengths, hq=hq, hkv=hkv, nq=nq, page=page, scales="head", seed=nq + page)
    k, v, blocks, offsets = new_rows(c, nq, seed=7)
    both_ways(c, k, v, blocks, offsets, max_context=max(lengths))
    both_ways(c, k, v, blocks, offsets, max_context=max(lengths) + 700)


@pytest.mark.parametrize("fmt,nq", [("fp8", 1), ("fp8", 2), ("int8", 3)])
def test_fused_store_over_many_segments(fmt, nq):
    """24 sequences x 8 KV heads = 192 segments: the plan's 2-wave workgroups, four to a CU (the shape of the
    decode step's launches), storing and using the rows as the 4-wave ones do."""
    lengths = [max(t, nq) for t in (1, 2, 31, 32, 33, 64, 95, 300, 513, 700, 1024, 1500, 2000, 2047, 2048, 2049,
                                    2900, 3000, 47, 129, 255, 256, 257, 4000)]
    c = make_case(fmt, lengths, nq=nq, scales="head", seed=40 + nq)
    k, v, blocks, offsets = new_rows(c, nq, seed=9)
    both_ways(c, k, v, blocks, offsets, max_context=max(lengths))


@pytest.mark.parametrize("num_splits", [1, 7, 64])
def test_fused_store_with_fixed_split_counts(num_splits):
    """A caller's split count (the partitions that hold a sequence's last chunk change with it)."""
    lengths = [1500, 2, 700, 4096, 31, 333]
    c = make_case("fp8", lengths, nq=2, scales="head", seed=12)
    k, v, blocks, offsets = new_rows(c, 2, seed=13)
    both_ways(c, k, v, blocks, offsets, max_context=4096, num_splits=num_splits)


def test_fused_store_with_lengths_beyond_max_context():
    """Sequences longer than max_context: their new rows are stored but not attended, as the two calls do."""
    lengths = [900, 300, 1500, 64]
    c = make_case("fp8", lengths, nq=1, scales="head", seed=3)
    k, v, blocks, offsets = new_rows(c, 1, seed=8)
    both_ways(c, k, v, blocks, offsets, max_context=512)


def test_fused_store_of_single_token_sequences():
    lengths = [1, 1, 2, 1]
    c = make_case("fp8", lengths, nq=1, scales="head", seed=4)
    k, v, blocks, offsets = new_rows(c, 1, seed=9)
    both_ways(c, k, v, blocks, offsets, max_context=2)


@pytest.mark.parametrize("fmt,scales,nq,hq", [("int8", "token", 1, 16), ("fp8", "token", 2, 16), ("bf16", None, 1, 16),
                                              ("fp8", "head", 1, 8), ("int8", "head", 1, 16)])
def test_other_layouts_take_the_two_launches(fmt, scales, nq, hq):
    """Per-token scales, BF16 caches and vector-kernel shapes (one FP8 row per KV head, INT8 with 2 rows):
    the call stores, then attends, with the same results."""
    lengths = [max(t, nq) for t in (70, 1, 513, 256)]  # every new row has a slot of its own
    c = make_case(fmt, lengths, hq=hq, nq=nq, scales=scales or "head", seed=5)
    k, v, blocks, offsets = new_rows(c, nq, seed=10)
    both_ways(c, k, v, blocks, offsets, max_context=600)


def test_f32_rows_take_the_two_launches():
    """Rows in f32 do not fuse (the kernel reads bf16 rows); the call still stores them and attends."""
    lengths = [200, 40]
    c = make_case("fp8", lengths, nq=1, scales="head", seed=6)
    k, v, blocks, offsets = new_rows(c, 1, seed=11)
    both_ways(c, k.float(), v.float(), blocks, offsets, max_context=200)


def expected_with_rows_in_place(c, k, v, blocks, offsets, in_place, max_context, scale=0.09):
    """Pools and output when only the rows marked in_place [B, Q] are stored: quantize_append of those rows
    (the others' slots set to -1), then paged_decode_attention."""
    from bpt_amd import paged_decode_attention, quantize_append

    kc, vc = c["k"].clone(), c["v"].clone()
    ks = None if c["ks"] is None else c["ks"].clone()
    vs = None if c["vs"] is None else c["vs"].clone()
    quantize_append(k, v, kc, vc, ks, vs, torch.where(in_place, blocks, torch.full_like(blocks, -1)), offsets)
    out = paged_decode_attention(c["q"], kc, vc, c["table"], c["lens"], ks, vs, scale=scale, max_context=max_context)
    return [t for t in (kc, vc, ks, vs) if t is not None], out


@pytest.mark.parametrize("fmt,scales,nq", [("fp8", "head", 1), ("fp8", "head", 3), ("int8", "token", 1),
                                           ("int8", "head", 5), ("bf16", "head", 2)])
def test_rows_aimed_elsewhere_are_neither_stored_nor_attended(fmt, scales, nq):
    """bpt_paged_append_decode stores a new row only where the decode reads token len - Q + qi. A row whose
    slot is another token of its sequence, and a row with no slot (-1), change nothing, in the one-launch path
    (FP8 and INT8 with per-head scales) and in the two-launch one (per-token scales, BF16) alike."""
    from bpt_amd import paged_append_decode

    lengths = [max(t, nq + 2) for t in (70, 40, 513, 256, 33)]
    c = make_case(fmt, lengths, nq=nq, scales=scales, seed=21 + nq)
    k, v, blocks, offsets = new_rows(c, nq, seed=22)
    page = c["k"].shape[1]
    in_place = torch.ones_like(blocks, dtype=torch.bool)
    # Sequence 0, row 0: the slot of the token two places earlier (a slot the decode reads as another token).
    pos = int(c["lens"][0]) - nq - 2
    blocks[0, 0] = c["table"][0, pos // page].to(torch.int32)
    offsets[0, 0] = pos % page
    in_place[0, 0] = False
    # Sequence 2, last row: no slot.
    blocks[2, nq - 1] = -1
    in_place[2, nq - 1] = False
    # Sequence 3, row 0: the right page, the wrong offset.
    offsets[3, 0] = (offsets[3, 0] + 1) % page
    in_place[3, 0] = False
    want_pools, want = expected_with_rows_in_place(c, k, v, blocks, offsets, in_place, max_context=600)
    kc, vc = c["k"].clone(), c["v"].clone()
    ks = None if c["ks"] is None else c["ks"].clone()
    vs = None if c["vs"] is None else c["vs"].clone()
    got = paged_append_decode(c["q"], k, v, kc, vc, c["table"], c["lens"], ks, vs, blocks, offsets, scale=0.09,
                              max_context=600)
    torch.cuda.synchronize()
    for a, b in zip(want_pools, [t for t in (kc, vc, ks, vs) if t is not None]):
        assert torch.equal(a.view(torch.uint8) if a.dtype != torch.float32 else a,
                           b.view(torch.uint8) if b.dtype != torch.float32 else b), "the pools differ"
    assert torch.equal(got, want), f"outputs differ: max {(got.float() - want.float()).abs().max()}"


def every_bf16_row_block(b, hkv, seed):
    """Every bf16 bit pattern but the NaNs (65536 - 254 values, the rest zeros), shuffled into [b, 1, hkv, 128]."""
    bits = torch.arange(65536, dtype=torch.int32)
    exp_all_ones = (bits & 0x7F80) == 0x7F80
    nan = exp_all_ones & ((bits & 0x007F) != 0)
    bits = torch.where(nan, torch.zeros_like(bits), bits)
    bits = bits[torch.randperm(65536, generator=torch.Generator().manual_seed(seed))]
    u16 = (bits & 0xFFFF).to(torch.int16)[: b * hkv * 128].reshape(b, 1, hkv, 128)
    return u16.view(torch.bfloat16).to(DEV)


@pytest.mark.parametrize("fmt", ["fp8", "int8"])
@pytest.mark.parametrize("length", [1, 2])
def test_fused_codes_of_every_bf16_value_at_adversarial_scales(fmt, length):
    """The fused call quantizes each new row twice, in registers for its own chunk and in its store task;
    quantize_append quantizes it once. Every non-NaN bf16 value as a new K and V channel, at per-head scales
    that put values exactly on e4m3 / integer rounding midpoints (1.0), just off them (1 +- 2^-20 ...), tiny
    and large: the pools and the outputs must match the two calls bit for bit. With one token per sequence
    the output is the new V row itself; with two it depends on the new K row's scores."""
    b, hkv = 64, 8
    nq = 1 if fmt == "fp8" else 5  # INT8 goes through the matrix-core store from 5 rows per KV head
    hq = 16 if fmt == "fp8" else 8
    c = make_case(fmt, [nq + length - 1] * b, hq=hq, hkv=hkv, nq=nq, scales="head", seed=30 + length)
    scales = torch.tensor([1.0, 1.0 + 2**-20, 1.0 - 2**-21, 3.0, 0.1, 448.0 / 7, 2.0**-10, 1.5 + 2**-18],
                          dtype=torch.float32, device=DEV)
    c["ks"] = scales.clone()
    c["vs"] = scales.flip(0).contiguous()
    rows = every_bf16_row_block(b, hkv, seed=length)
    k_rows = rows.expand(b, nq, hkv, 128).contiguous()
    v_rows = rows.roll(1, dims=0).expand(b, nq, hkv, 128).contiguous()
    _, _, blocks, offsets = new_rows(c, nq, seed=3)
    both_ways(c, k_rows, v_rows, blocks, offsets, max_context=nq + length - 1)
