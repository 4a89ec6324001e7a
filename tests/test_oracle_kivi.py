"""Pins the KIVI oracle (oracle/kivi.py): the reference tests' known answers and properties
(tests/kernels/test_reference.py:59-131, :152-175), hand-derived grids in which a dropped float16 rounding, a
wrong zero point or round-half-up would each change a code, and a float64 brute force of the attention
written the way the reference kernel computes it (grids folded into q and p, kernels/kv_attention.py:9-19)."""

import numpy as np
import pytest

from oracle import attention, kivi


def random_kv(batch=2, heads=2, tokens=64, dim=16, seed=0):
    """Keys with an outlier channel (as Qwen3's have) and ordinary values (the reference tests' inputs)."""
    g = np.random.default_rng(seed)
    k = g.standard_normal((batch, heads, tokens, dim)).astype(np.float32)
    k[..., 3] += 20.0
    return k, g.standard_normal((batch, heads, tokens, dim)).astype(np.float32)


# ---- storage -------------------------------------------------------------------------------------------


def test_nibbles_pair_channel_d_with_d_plus_half():
    c = np.array([[1, 2, 3, 4]], dtype=np.uint8)
    packed = kivi.pack_nibbles(c)
    assert packed.tolist() == [[0x31, 0x42]]  # known answer of test_reference.py:59-65
    assert np.array_equal(kivi.unpack_nibbles(packed), c)
    every = np.tile(np.arange(16, dtype=np.uint8), (3, 2))
    assert np.array_equal(kivi.unpack_nibbles(kivi.pack_nibbles(every)), every)


def test_grid_known_answer_rounds_the_scale_to_float16_first():
    # [-1, 0, 2, 0.5] in 4 bits: scale = f16(3 / 15) = 0.199951171875 (not 0.2), zero = round(5.0012) = 5.
    # 0.5 / 0.19995 = 2.5006 -> 3 -> code 8. With an unrounded scale 0.5 / 0.2 = 2.5 would round (half to
    # even) to 2 -> code 7: this code pins the float16 rounding.
    x = np.array([[-1.0, 0.0, 2.0, 0.5]], dtype=np.float32)
    s, z = kivi.grid(x, 4, axis=1)
    assert s.dtype == np.float16 and z.dtype == np.float16
    assert float(s[0, 0]) == 0.199951171875 and float(z[0, 0]) == 5.0
    assert kivi.codes(x, s, z, 4).tolist() == [[0, 5, 15, 8]]


def test_grid_known_answer_ties_round_to_even_and_zero_is_exact():
    # [0, 15, 2.5, 3.5]: scale 1, zero 0; the ties 2.5 and 3.5 round to 2 and 4 (torch.round's half to even).
    x = np.array([[0.0, 15.0, 2.5, 3.5]], dtype=np.float32)
    s, z = kivi.grid(x, 4, axis=1)
    assert float(s[0, 0]) == 1.0 and float(z[0, 0]) == 0.0
    assert kivi.codes(x, s, z, 4).tolist() == [[0, 15, 2, 4]]
    # All-positive values: the range is widened to include 0 (lo = 0), so zero stays 0 and 8-bit 255 = max.
    x = np.array([[2.0, 4.0, 6.0]], dtype=np.float32)
    s, z = kivi.grid(x, 8, axis=1)
    assert float(z[0, 0]) == 0.0 and kivi.codes(x, s, z, 8)[0, 2] == 255
    # All-zero values: scale 1, zero 0, codes 0 (any step represents them).
    s, z = kivi.grid(np.zeros((1, 5), np.float32), 8, axis=1)
    assert float(s[0, 0]) == 1.0 and float(z[0, 0]) == 0.0


def test_a_real_zero_reads_back_as_exactly_zero():
    k, v = random_kv(seed=3)
    k[:, :, 5, :] = 0.0
    v[:, :, :, 7] = 0.0
    for bits in (4, 8):
        kh, vh = kivi.dequantize_kv(kivi.quantize_kv(k, v, bits))
        assert (kh[:, :, 5, :] == 0).all() and (vh[:, :, :, 7] == 0).all()


@pytest.mark.parametrize("bits", [4, 8])
def test_quantized_kv_is_within_half_a_step(bits):
    # test_reference.py:68-82: shapes, dtypes and the error bound (0.51 + 2^bits * 2^-11 steps).
    k, v = random_kv()
    kv = kivi.quantize_kv(k, v, bits, group=32)
    assert kv.k_codes.dtype == np.uint8 and kv.k_scale.dtype == np.float16
    assert kv.k_codes.shape == (2, 2, 64, 8 if bits == 4 else 16)
    assert kv.k_scale.shape == (2, 2, 2, 16) and kv.v_scale.shape == (2, 2, 64)
    kh, vh = kivi.dequantize_kv(kv)
    k_step = np.repeat(kv.k_scale.astype(np.float32), 32, axis=2)
    v_step = kv.v_scale.astype(np.float32)[..., None]
    bound = 0.51 + 2**bits * 2**-11
    assert (np.abs(kh - k) <= k_step * bound).all()
    assert (np.abs(vh - v) <= v_step * bound).all()


def test_codes_are_the_nearest_grid_point_by_brute_force():
    # Every code minimises |scale * (c - zero) - x| over all 2^bits codes (ties aside), in float64.
    k, v = random_kv(batch=1, heads=1, tokens=32, dim=16, seed=4)
    for bits in (4, 8):
        kv = kivi.quantize_kv(k, v, bits)
        vc = kivi.unpack_nibbles(kv.v_codes) if bits == 4 else kv.v_codes
        s = kv.v_scale.astype(np.float64)[..., None, None]
        z = kv.v_zero.astype(np.float64)[..., None, None]
        grid_pts = s * (np.arange(2**bits, dtype=np.float64) - z)  # [1, 1, T, 1, 2^bits]
        err = np.abs(grid_pts - v.astype(np.float64)[..., None])
        best = err.min(-1)
        chosen = np.take_along_axis(err, vc[..., None].astype(np.int64), -1)[..., 0]
        assert (chosen <= best + 1e-6 * s[..., 0]).all()


def test_key_grids_are_per_channel_and_per_group():
    k, v = random_kv(batch=1, heads=1, tokens=64, dim=8, seed=5)
    a = kivi.quantize_kv(k, v, 8)
    k2 = k.copy()
    k2[0, 0, 40, 2] = 100.0  # group 1, channel 2
    b = kivi.quantize_kv(k2, v, 8)
    changed = a.k_scale != b.k_scale
    assert changed[0, 0, 1, 2] and changed.sum() == 1
    assert np.array_equal(a.k_codes[:, :, :32], b.k_codes[:, :, :32])  # group 0 untouched


def test_more_bits_less_error_and_16_bits_is_exact():
    k, v = random_kv()
    errors = {}
    for bits in (4, 8, 16):
        kh, vh = kivi.dequantize_kv(kivi.quantize_kv(k, v, bits))
        errors[bits] = float(np.mean((kh - k) ** 2) + np.mean((vh - v) ** 2))
    assert errors[16] == 0.0 and errors[8] < errors[4] / 100


def test_partial_groups_are_refused_and_partial_reads_work():
    k, v = random_kv(tokens=70)
    with pytest.raises(ValueError, match="whole number of groups"):
        kivi.quantize_kv(k, v, 4, group=32)
    kv = kivi.quantize_kv(k[:, :, :64], v[:, :, :64], 4, group=32)
    k_all, _ = kivi.dequantize_kv(kv)
    k_some, _ = kivi.dequantize_kv(kv, tokens=40)
    assert k_some.shape == (2, 2, 40, 16) and np.array_equal(k_some, k_all[:, :, :40])


def test_bytes_per_token_match_the_sizing_model():
    # test_reference.py:120-131: one layer of Qwen3 (8 KV heads x 128). The sizing model's bits per element:
    # keys b + 32 / 32 (two f16 per channel per 32 tokens), values b + 32 / 128 (two f16 per token).
    k = np.zeros((1, 8, 64, 128), np.float32)
    for bits in (4, 8):
        per_elem = ((bits + 1.0) + (bits + 0.25)) / 2
        assert kivi.quantize_kv(k, k, bits).bytes_per_token() == 2 * 8 * 128 * per_elem / 8
    assert kivi.quantize_kv(k, k, 4).bytes_per_token() == 8 * 148
    assert kivi.quantize_kv(k.astype(np.float16), k.astype(np.float16), 16).bytes_per_token() == 2 * 8 * 128 * 2


# ---- attention over the codes ---------------------------------------------------------------------------


def folded_attention_f64(q, kv, lengths, scale):
    """float64 loops in the reference kernel's own arrangement: per group, s_t = sum_d (q_d s_d) code_td -
    sum_d q_d s_d z_d; out = (sum_t p_t vs_t code_t - sum_t p_t vs_t vz_t) / sum_t p_t. No dequantized
    tensor is formed."""
    b_, hq, d = q.shape
    hkv = kv.k_codes.shape[1]
    rep = hq // hkv
    kc = kivi.unpack_nibbles(kv.k_codes) if kv.bits == 4 else kv.k_codes
    vc = kivi.unpack_nibbles(kv.v_codes) if kv.bits == 4 else kv.v_codes
    out = np.zeros((b_, hq, d))
    for b in range(b_):
        n = min(int(lengths[b]), kv.tokens)
        for h in range(hq):
            kh = h // rep
            if n == 0:
                continue
            scores = []
            for t in range(n):
                g = t // kv.group
                qs = q[b, h].astype(np.float64) * scale * kv.k_scale[b, kh, g].astype(np.float64)
                bias = -np.dot(qs, kv.k_zero[b, kh, g].astype(np.float64))
                scores.append(np.dot(qs, kc[b, kh, t].astype(np.float64)) + bias)
            scores = np.array(scores)
            p = np.exp(scores - scores.max())
            w = p * kv.v_scale[b, kh, :n].astype(np.float64)
            shift = np.dot(w, kv.v_zero[b, kh, :n].astype(np.float64))
            out[b, h] = (w @ vc[b, kh, :n].astype(np.float64) - shift) / p.sum()
    return out


@pytest.mark.parametrize("bits", [4, 8, 16])
def test_attention_matches_the_folded_float64_brute_force(bits):
    k, v = random_kv(batch=3, heads=2, tokens=96, dim=16, seed=6)
    if bits == 16:
        k, v = k.astype(np.float16), v.astype(np.float16)
    kv = kivi.quantize_kv(k, v, bits)
    q = np.random.default_rng(7).standard_normal((3, 4, 16)).astype(np.float32)
    lengths = np.array([96, 1, 45])
    got = kivi.attend(q, kv, lengths, 0.25, split=32)
    if bits == 16:
        kh, vh = kivi.dequantize_kv(kv)
        want = attention.merge_partials(*(x[:, :, None] for x in attention.partial_attention(q, kh, vh, lengths, 0.25)))
    else:
        want = folded_attention_f64(q, kv, lengths, 0.25)
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)


def test_splits_partition_the_tokens_and_merge_exactly():
    k, v = random_kv(batch=3, heads=2, tokens=96, dim=16, seed=8)
    kv = kivi.quantize_kv(k, v, 8)
    q = np.random.default_rng(9).standard_normal((3, 4, 16)).astype(np.float32)
    lengths = np.array([96, 40, 5])
    out, lse = kivi.decode_attention(q, kv, lengths, 0.25, split=32)
    assert out.shape == (3, 4, 3, 16) and lse.shape == (3, 4, 3)
    # Row 1 sees nothing in split 2, row 2 only in split 0: out 0 and lse -inf there.
    assert np.isneginf(lse[1, :, 2]).all() and (out[1, :, 2] == 0).all()
    assert np.isneginf(lse[2, :, 1:]).all() and (out[2, :, 1:] == 0).all()
    whole = kivi.attend(q, kv, lengths, 0.25, split=96)
    np.testing.assert_allclose(attention.merge_partials(out, lse), whole, rtol=1e-5, atol=1e-6)
    # lse is the natural log of the split's summed weights: one token -> its own score.
    kh, _ = kivi.dequantize_kv(kv)
    s0 = 0.25 * np.einsum("hd,hd->h", q[1], np.repeat(kh[1, :, 0], 2, axis=0))
    o1, l1 = kivi.decode_attention(q, kv, np.array([96, 1, 5]), 0.25, split=32)
    np.testing.assert_allclose(l1[1, :, 0], s0, rtol=1e-5, atol=1e-5)


def test_split_rules_and_the_default():
    k, v = random_kv(batch=1, heads=2, tokens=64, dim=16)
    kv = kivi.quantize_kv(k, v, 4)
    q = np.zeros((1, 4, 16), np.float32)
    with pytest.raises(ValueError, match="multiple of the key group"):
        kivi.decode_attention(q, kv, np.array([64]), 0.1, split=48)
    out, lse = kivi.decode_attention(q, kv, np.array([64]), 0.1)  # default_split(1, 2, 64) = 128: one split
    assert out.shape == (1, 4, 1, 16)
    out, _ = kivi.decode_attention(q, kv, np.array([64]), 0.1, tokens=32, split=32)  # `tokens` sizes the splits
    assert out.shape == (1, 4, 1, 16)
    # A row with no tokens: zeros, not NaN (test_reference.py:169-175).
    got = kivi.attend(q, kv, np.array([0]), 0.1)
    assert np.isfinite(got).all() and (got == 0).all()
