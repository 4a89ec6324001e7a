"""GPU: FP8 conversions and quantize-on-write, bit-exact against the oracle.

The write path restates fastserve engine/kv_cache.py:158-161 (scatter by write_blocks / write_offsets) with
kv/quant.py:44-45 (FP8 cast) and quant/w8a8.py:55-74 / kernels/reference.py:44-55 (per-token INT8).
"""

import numpy as np
import pytest
import torch

from oracle import fp8, quant

pytestmark = pytest.mark.gpu

DEV = "cuda"


def test_fp8_decoder_matches_torch_on_all_256_codes():
    from bpt_amd.measure import fp8_decode_table

    got = fp8_decode_table().cpu().numpy()
    want = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    assert np.array_equal(np.isnan(got), np.isnan(want)), np.nonzero(np.isnan(got) != np.isnan(want))
    ok = ~np.isnan(want)
    assert np.array_equal(got[ok].view(np.uint32), want[ok].view(np.uint32)), np.nonzero(got[ok] != want[ok])


@pytest.mark.parametrize("scale", [1.0, 0.37, 3.0e-3])
def test_fp8_encoder_is_bit_exact(scale):
    from bpt_amd.measure import fp8_encode

    g = np.random.default_rng(0)
    vals = fp8.representable_values().astype(np.float64)
    ties = (vals[1:] + vals[:-1]) / 2
    x = np.concatenate(
        [
            g.standard_normal(20000) * 10.0 ** g.integers(-6, 4, 20000),
            vals,
            ties,
            np.nextafter(ties, 0),
            np.nextafter(ties, 1e9),
            [0.0, -0.0, 447.9, 448.0, 449.0, 464.0, 500.0, -1e9, 1e-45, 2.0**-10, np.nan],
        ]
    ).astype(np.float32) * np.float32(scale)
    got = fp8_encode(torch.from_numpy(x).to(DEV), scale).cpu().numpy()
    want = fp8.encode(np.clip(x / np.float32(scale), -448, 448))
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, (x[bad[:8]], got[bad[:8]], want[bad[:8]])


def paged_pool(nb, page, hkv, d, dtype, seed=0):
    g = torch.Generator(device=DEV).manual_seed(seed)
    if dtype == torch.bfloat16:
        return torch.randn((nb, page, hkv, d), generator=g, device=DEV).to(dtype)
    raw = torch.randint(0, 256, (nb, page, hkv, d), generator=g, device=DEV, dtype=torch.uint8)
    return raw.view(dtype)


def run_append(fmt, b=8, nq=3, hkv=8, d=128, page=16, nb=40, src=torch.bfloat16, seed=0, i64=False):
    from bpt_amd import quantize_append

    g = torch.Generator(device=DEV).manual_seed(seed)
    k = torch.randn((b, nq, hkv, d), generator=g, device=DEV) * 3
    k[..., 5] *= 8.0
    v = torch.randn((b, nq, hkv, d), generator=g, device=DEV)
    k[0, 0, 1] = 0.0  # an all-zero row
    k, v = k.to(src), v.to(src)
    dtype = {"fp8": torch.float8_e4m3fn, "int8": torch.int8, "bf16": torch.bfloat16}[fmt]
    k_cache, v_cache = paged_pool(nb, page, hkv, d, dtype, seed), paged_pool(nb, page, hkv, d, dtype, seed + 1)
    k_before, v_before = k_cache.clone(), v_cache.clone()
    # distinct slots: every offset 0..page-1 appears; one row is skipped (negative block)
    perm = torch.randperm(nb * page, generator=torch.Generator().manual_seed(seed))[: b * nq]
    blocks = (perm // page).view(b, nq)
    offsets = (perm % page).view(b, nq)
    blocks[1, 0] = -1
    idx = torch.int64 if i64 else torch.int32
    if fmt == "fp8":
        ks = torch.tensor(np.linspace(0.01, 0.2, hkv), dtype=torch.float32, device=DEV)
        vs = torch.tensor(np.linspace(0.005, 0.05, hkv), dtype=torch.float32, device=DEV)
    elif fmt == "int8":
        ks = torch.full((nb, page, hkv), -1.0, device=DEV)
        vs = torch.full((nb, page, hkv), -1.0, device=DEV)
    else:
        ks = vs = None
    ks_before = None if ks is None else ks.clone()
    quantize_append(k, v, k_cache, v_cache, ks, vs, blocks.to(DEV, idx), offsets.to(DEV, idx))
    torch.cuda.synchronize()
    return dict(k=k, v=v, k_cache=k_cache, v_cache=v_cache, k_before=k_before, v_before=v_before, ks=ks, vs=vs,
                ks_before=ks_before, blocks=blocks, offsets=offsets)


def as_bytes(t):
    return t.view(torch.uint8).cpu().numpy() if t.dtype != torch.bfloat16 else t.view(torch.int16).cpu().numpy()


@pytest.mark.parametrize("fmt", ["fp8", "int8", "bf16"])
@pytest.mark.parametrize("src", [torch.bfloat16, torch.float32])
def test_quantize_append_is_bit_exact(fmt, src):
    check_append(run_append(fmt, src=src), fmt, src)


def check_append(r, fmt, src):
    """Written slots bit-exact against the oracle's quantizers; every other slot (and FP8's scales) untouched."""
    blocks, offsets = r["blocks"].numpy(), r["offsets"].numpy()
    written = blocks >= 0
    for name, rows in (("k", r["k"]), ("v", r["v"])):
        x = rows.float().cpu().numpy()[written]  # [R, Hkv, D]
        cache = as_bytes(r[f"{name}_cache"])
        before = as_bytes(r[f"{name}_before"])
        got = cache[blocks[written], offsets[written]]
        if fmt == "fp8":
            want = quant.fp8_per_head(x, r[f"{name}s"].cpu().numpy())
        elif fmt == "int8":
            codes, scale = quant.per_token(x, "int8")
            want = codes.view(np.uint8)
            got_scale = r[f"{name}s"].cpu().numpy()[blocks[written], offsets[written]]
            assert np.array_equal(got_scale.view(np.uint32), scale[..., 0].view(np.uint32))
        else:
            want = rows.cpu().view(torch.int16).numpy()[written] if src == torch.bfloat16 else \
                torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy()
        assert np.array_equal(got, want), (name, np.argwhere(got != want)[:5])
        # nothing else in the pool changed
        mask = np.ones(cache.shape[:2], dtype=bool)
        mask[blocks[written], offsets[written]] = False
        assert np.array_equal(cache[mask], before[mask])
    if fmt == "fp8":
        assert torch.equal(r["ks"], r["ks_before"])


def test_quantize_append_int64_slots_and_every_offset():
    r = run_append("int8", b=16, nq=1, nb=16, i64=True, seed=3)
    blocks, offsets = r["blocks"].numpy(), r["offsets"].numpy()
    written = blocks >= 0
    x = r["k"].float().cpu().numpy()[written]
    codes, _ = quant.per_token(x, "int8")
    got = as_bytes(r["k_cache"])[blocks[written], offsets[written]]
    assert np.array_equal(got, codes.view(np.uint8))


def test_int8_write_of_one_token_per_sequence_into_partial_last_pages():
    """64 sequences x 8 KV heads, the new token at slot 15 of each sequence's last page (then all offsets)."""
    from bpt_amd import quantize_append

    b, hkv, d, page, nb = 64, 8, 128, 16, 64 * 4
    g = torch.Generator(device=DEV).manual_seed(7)
    k_cache = paged_pool(nb, page, hkv, d, torch.int8, 1)
    v_cache = paged_pool(nb, page, hkv, d, torch.int8, 2)
    ks = torch.zeros((nb, page, hkv), device=DEV)
    vs = torch.zeros_like(ks)
    last_page = torch.randperm(nb, generator=torch.Generator().manual_seed(1))[:b].view(b, 1).to(DEV, torch.int32)
    for offset in range(page):
        k = torch.randn((b, 1, hkv, d), generator=g, device=DEV).to(torch.bfloat16)
        v = torch.randn((b, 1, hkv, d), generator=g, device=DEV).to(torch.bfloat16)
        offs = torch.full((b, 1), offset, dtype=torch.int32, device=DEV)
        quantize_append(k, v, k_cache, v_cache, ks, vs, last_page, offs)
        torch.cuda.synchronize()
        lp = last_page.cpu().numpy()[:, 0]
        for rows, cache, sc in ((k, k_cache, ks), (v, v_cache, vs)):
            codes, scale = quant.per_token(rows.float().cpu().numpy()[:, 0], "int8")
            assert np.array_equal(cache.cpu().numpy()[lp, offset], codes)
            assert np.array_equal(sc.cpu().numpy()[lp, offset].view(np.uint32), scale[..., 0].view(np.uint32))
