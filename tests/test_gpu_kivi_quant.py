"""GPU: KIVI quantize-on-write (bpt_amd.kivi.quantize_kv / quantize_kv_into -> bpt_kivi_quantize) against the
oracle's quantize_kv (oracle/kivi.py, itself pinned by hand-derived known answers in test_oracle_kivi.py):
codes and float16 grids bit-exact (grids compared as raw float16 bits, so a zero point of -0.0, which the
reference formulas give a channel with no negative value, must come out as -0.0 too).

Covers 4 and 8 bits, head dims 16 .. 256, bf16 / f16 / f32 inputs, outlier and all-positive channels, an
all-zero token, values far from one, key groups of 32 and 64, and the cache-append pattern of fastserve's
QuantizedKVCache._append (integration/kv_cache.py:139-158): completed groups quantized straight into a larger
cache at a token offset, leaving the rest of it untouched; then decode attention over codes written this way."""

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from oracle import kivi as okivi

pytestmark = pytest.mark.gpu


def inputs(batch, heads, tokens, d, seed, dtype=torch.float32, scale=1.0):
    g = np.random.default_rng(seed)
    k = g.standard_normal((batch, heads, tokens, d)).astype(np.float32) * scale
    k[..., 3 % d] += 20.0 * scale  # an outlier channel with no negative value: its zero points are -0.0
    v = g.standard_normal((batch, heads, tokens, d)).astype(np.float32) * scale
    v[0, 0, 1] = 0.0  # an all-zero token: scale 1, zero point -0.0, codes 0
    kt, vt = torch.from_numpy(k).to(dtype).cuda(), torch.from_numpy(v).to(dtype).cuda()
    return kt, vt, kt.float().cpu().numpy(), vt.float().cpu().numpy()


def same_bits(got, want, what):
    got = got.detach().cpu().numpy()
    assert got.dtype == want.dtype and got.shape == want.shape, what
    view = np.uint16 if want.dtype == np.float16 else want.dtype
    bad = got.view(view) != want.view(view)
    assert not bad.any(), f"{what}: {bad.sum()} of {bad.size} differ"


def check_quant(kv, ref, what):
    for f in ("k_codes", "v_codes", "k_scale", "k_zero", "v_scale", "v_zero"):
        same_bits(getattr(kv, f), getattr(ref, f), f"{what} {f}")


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("d", [16, 32, 64, 128, 256])
def test_codes_and_grids_bit_exact(bits, d):
    from bpt_amd import kivi

    for dtype in (torch.float32, torch.bfloat16, torch.float16):
        k, v, kn, vn = inputs(2, 3, 96, d, seed=d + bits, dtype=dtype)
        check_quant(kivi.quantize_kv(k, v, bits), okivi.quantize_kv(kn, vn, bits), f"{bits} bits D={d} {dtype}")


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("scale", [1e-3, 1e3])
def test_values_far_from_one_and_larger_groups(bits, scale):
    from bpt_amd import kivi

    k, v, kn, vn = inputs(2, 8, 128, 128, seed=7, scale=scale)
    for group in (32, 64):
        check_quant(kivi.quantize_kv(k, v, bits, group), okivi.quantize_kv(kn, vn, bits, group),
                    f"{bits} bits x{scale:g} group {group}")


@pytest.mark.parametrize("bits", [4, 8, 16])
def test_append_into_a_cache_then_decode(bits):
    """Groups quantized into a 256-token cache at tokens 64 .. 160 (QuantizedKVCache._append's pattern) land
    exactly there, the rest of the cache keeps its contents, and decode attention reads them."""
    from bpt_amd import kivi

    b, h, d, total = 2, 8, 128, 256
    k, v, kn, vn = inputs(b, h, 96, d, seed=3)
    width = d // 2 if bits == 4 else d
    if bits == 16:
        cache = kivi.QuantKV(16, 32, torch.full((b, h, total, d), 7.0, device="cuda"),
                             torch.full((b, h, total, d), 7.0, device="cuda"))
    else:
        sentinel = lambda *s, dt: torch.full(s, 7, dtype=dt, device="cuda")  # noqa: E731
        cache = kivi.QuantKV(bits, 32, sentinel(b, h, total, width, dt=torch.uint8),
                             sentinel(b, h, total, width, dt=torch.uint8), sentinel(b, h, total // 32, d, dt=torch.float16),
                             sentinel(b, h, total // 32, d, dt=torch.float16), sentinel(b, h, total, dt=torch.float16),
                             sentinel(b, h, total, dt=torch.float16))
    kivi.quantize_kv_into(k, v, cache, 64)
    torch.cuda.synchronize()
    ref = okivi.quantize_kv(kn, vn, bits)
    if bits == 16:
        assert torch.equal(cache.k_codes[:, :, 64:160].cpu(), torch.from_numpy(kn))
        untouched = torch.cat([cache.k_codes[:, :, :64], cache.k_codes[:, :, 160:]], 2)
        assert bool((untouched == 7.0).all())
    else:
        part = SimpleNamespace(k_codes=cache.k_codes[:, :, 64:160], v_codes=cache.v_codes[:, :, 64:160],
                               k_scale=cache.k_scale[:, :, 2:5], k_zero=cache.k_zero[:, :, 2:5],
                               v_scale=cache.v_scale[:, :, 64:160], v_zero=cache.v_zero[:, :, 64:160])
        check_quant(part, ref, f"{bits} bits appended")
        assert bool((cache.k_codes[:, :, :64] == 7).all()) and bool((cache.k_codes[:, :, 160:] == 7).all())
        assert bool((cache.k_scale[:, :, :2] == 7).all()) and bool((cache.v_scale[:, :, 160:] == 7).all())
    # Decode over the first 160 tokens of a cache whose first 64 are quantized the same way.
    k0, v0, kn0, vn0 = inputs(b, h, 64, d, seed=4)
    kivi.quantize_kv_into(k0, v0, cache, 0)
    full_ref = okivi.quantize_kv(np.concatenate([kn0, kn], 2), np.concatenate([vn0, vn], 2), bits)
    q = torch.randn((b, 16, d), device="cuda")
    lens = torch.tensor([160, 101], dtype=torch.int32, device="cuda")
    got = kivi.attend(q, cache, lens, 0.1, tokens=160)
    want = okivi.attend(q.cpu().numpy(), full_ref, np.array([160, 101]), 0.1, tokens=160)
    np.testing.assert_allclose(got.cpu().numpy(), want, rtol=2e-4, atol=2e-4 * float(np.abs(want).max()))


@pytest.mark.parametrize("bits", [4, 8])
def test_half_way_quotients_round_to_even(bits):
    """Every x / scale is exactly n + 1/2: ranges [0, qmax / 16] give scale 1/16 and zero point 0, and each
    other value is (n + 1/2) / 16 (n < 127, so bf16 holds it exactly). Codes must be n rounded half to even,
    the closed form torch.round gives, for keys (per channel) and values (per token)."""
    from bpt_amd import kivi

    qmax = (1 << bits) - 1
    n = (np.arange(32)[:, None] * 3 + np.arange(128)[None, :]) % min(qmax, 127)  # [token, channel]
    x = (n + 0.5) / 16.0
    k, v = x.copy(), x.copy()
    k[5] = qmax / 16.0  # each key channel's range reaches qmax / 16 at token 5
    v[:, 7] = qmax / 16.0  # each token's value range reaches it at channel 7
    want = np.where(n % 2 == 0, n, n + 1)
    for dtype in (torch.float32, torch.bfloat16):
        kt = torch.from_numpy(np.stack([k, k[::-1]])[None].astype(np.float32)).to(dtype).cuda()
        vt = torch.from_numpy(np.stack([v, v[::-1]])[None].astype(np.float32)).to(dtype).cuda()
        got = kivi.quantize_kv(kt, vt, bits)
        ref = okivi.quantize_kv(kt.float().cpu().numpy(), vt.float().cpu().numpy(), bits)
        check_quant(got, ref, f"{bits} bits {dtype} half-way")
        kc, vc = got.k_codes[0, 0].cpu().numpy().astype(np.int64), got.v_codes[0, 0].cpu().numpy().astype(np.int64)
        if bits == 4:  # byte c = channel c | channel c + 64 << 4
            kc = np.concatenate([kc & 15, kc >> 4], 1)
            vc = np.concatenate([vc & 15, vc >> 4], 1)
        rows = np.arange(32) != 5
        assert np.array_equal(kc[rows], want[rows]) and (kc[5] == qmax).all()
        cols = np.arange(128) != 7
        assert np.array_equal(vc[:, cols], want[:, cols]) and (vc[:, 7] == qmax).all()


@pytest.mark.parametrize("bits", [4, 8])
def test_quotients_within_ulps_of_half_way(bits):
    """float32 values 0 .. 3 ulps either side of (n + 1/2) * s for a scale s = 41/64 (not a power of two):
    x / s then rounds to n + 1/2 or to a neighbour depending on the last bits, and x times the correctly
    rounded 1 / s rounds hundreds of these codes the wrong way. Keys and values, bit-exact with the oracle."""
    from bpt_amd import kivi

    qmax = (1 << bits) - 1
    s = 41 / 64
    t, c = np.meshgrid(np.arange(64), np.arange(128), indexing="ij")
    n = (t * 7 + c) % qmax
    x0 = ((n + 0.5) * s).astype(np.float32)
    x = (x0.view(np.int32) + ((t + 3 * c) % 7 - 3).astype(np.int32)).view(np.float32)
    k, v = x.copy(), x.copy()
    k[[5, 40]] = np.float32(qmax * s)  # every key channel's range: [0, qmax s], so its scale is s
    v[:, 9] = np.float32(qmax * s)  # every token's value range too
    q = x / np.float32(s)
    assert (np.abs(q - np.floor(q) - 0.5) < np.abs(q) * 2.0**-20).mean() > 0.5  # most sit in the fallback band
    assert (np.rint(x * (np.float32(1) / np.float32(s))) != np.rint(q)).sum() > 300
    kt = torch.from_numpy(np.stack([k, k[::-1]])[None].copy()).cuda()
    vt = torch.from_numpy(np.stack([v, v[::-1]])[None].copy()).cuda()
    got = kivi.quantize_kv(kt, vt, bits)
    ref = okivi.quantize_kv(kt.cpu().numpy(), vt.cpu().numpy(), bits)
    assert (ref.k_scale == np.float16(s)).all() and (ref.v_scale == np.float16(s)).all()
    check_quant(got, ref, f"{bits} bits near half-way")


@pytest.mark.parametrize("bits", [4, 8])
def test_unaligned_rows_take_the_general_kernel(bits):
    """Sources that do not start on 16 bytes (a channel offset of one element, rows of D + 1 elements) and
    codes at an odd byte offset go through the row-at-a-time kernel; same bit-exact result."""
    from bpt_amd import kivi

    b, h, n, d = 2, 4, 64, 128
    for dtype in (torch.bfloat16, torch.float32):
        k, v, kn, vn = inputs(b, h, n, d + 1, seed=11, dtype=dtype)
        k, v = k[..., 1:], v[..., 1:]
        ks = torch.full((b, h, 2, d), 7, dtype=torch.float16, device="cuda")
        width = d // 2 if bits == 4 else d
        raw = torch.zeros((2, b, h, n, width + 1), dtype=torch.uint8, device="cuda")
        cache = kivi.QuantKV(bits, 32, raw[0, ..., 1:], raw[1, ..., 1:], ks, ks.clone(),
                             torch.zeros((b, h, n), dtype=torch.float16, device="cuda"),
                             torch.zeros((b, h, n), dtype=torch.float16, device="cuda"))
        kivi.quantize_kv_into(k, v, cache, 0)
        check_quant(cache, okivi.quantize_kv(kn[..., 1:], vn[..., 1:], bits), f"{bits} bits {dtype} unaligned")


def test_bad_arguments_raise_value_error():
    from bpt_amd import kivi

    k, v, _, _ = inputs(1, 2, 40, 128, seed=1)
    with pytest.raises(ValueError, match="whole number of groups"):
        kivi.quantize_kv(k, v, 8)
    with pytest.raises(ValueError, match="bits"):
        kivi.quantize_kv(k[:, :, :32], v[:, :, :32], 3)
    cache = kivi.quantize_kv(k[:, :, :32], v[:, :, :32], 8)
    with pytest.raises(ValueError, match="start on a key group"):
        kivi.quantize_kv_into(k[:, :, :32], v[:, :, :32], cache, 16)
    k2, v2, _, _ = inputs(1, 2, 32, 96, seed=2)
    with pytest.raises(ValueError, match="power of two"):
        kivi.quantize_kv(k2, v2, 8)
