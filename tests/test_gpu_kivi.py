"""KIVI decode attention on the GPU through the C ABI (bpt_amd.kivi -> bpt_kivi_decode) against the oracle
(oracle/kivi.py), on the cases fastserve's own kernel tests use (tests/kernels/test_kernels_gpu.py:69-142:
Qwen3's 16/8 heads, an outlier key channel, 1..4096 tokens, forced splits, ragged and empty rows, the
32768-token maximum, float16 q and caches, a caller-known token count) plus GQA ratios 1..16, bfloat16
caches and value grids far from 1.

Tolerance: the reference tests' own, rtol 2e-4 and atol 2e-4 * max|want| (test_kernels_gpu.py:78-84), for
the merged attention and for every split's partial output; lse (natural log) within 2e-4 absolute + 1e-5
relative."""

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from oracle import kivi as okivi

pytestmark = pytest.mark.gpu

D = 128


def make_cache(batch, kv_heads, tokens, bits, seed=0, half=torch.float16, v_mul=1.0, group=32, d=D):
    """(device cache with QuantKV's fields, oracle QuantKV) holding the same codes."""
    g = np.random.default_rng(seed)
    k = g.standard_normal((batch, kv_heads, tokens, d)).astype(np.float32)
    k[..., 3 % d] += 20.0  # an outlier channel, as Qwen3's keys have
    v = (g.standard_normal((batch, kv_heads, tokens, d)) * v_mul).astype(np.float32)
    if bits == 16:
        kt = torch.from_numpy(k).to(half)
        vt = torch.from_numpy(v).to(half)
        ref = okivi.QuantKV(16, group, kt.float().numpy(), vt.float().numpy())
        dev = SimpleNamespace(bits=16, group=group, k_codes=kt.cuda(), v_codes=vt.cuda(),
                              k_scale=None, k_zero=None, v_scale=None, v_zero=None)
        return dev, ref
    ref = okivi.quantize_kv(k, v, bits, group)
    dev = SimpleNamespace(
        bits=bits, group=group,
        k_codes=torch.from_numpy(ref.k_codes).cuda(), v_codes=torch.from_numpy(ref.v_codes).cuda(),
        k_scale=torch.from_numpy(ref.k_scale).cuda(), k_zero=torch.from_numpy(ref.k_zero).cuda(),
        v_scale=torch.from_numpy(ref.v_scale).cuda(), v_zero=torch.from_numpy(ref.v_zero).cuda(),
    )
    return dev, ref


def make_q(batch, q_heads, seed, dtype=torch.bfloat16, d=D):
    g = np.random.default_rng(seed)
    q = torch.from_numpy(g.standard_normal((batch, q_heads, d)).astype(np.float32)).to(dtype)
    return q.cuda(), q.float().numpy()


def close(got, want, what):
    got = got.detach().cpu().numpy() if isinstance(got, torch.Tensor) else got
    assert np.isfinite(got).all(), what
    tol = 2e-4 * max(float(np.abs(want).max()), 1e-30)
    np.testing.assert_allclose(got, want, rtol=2e-4, atol=tol, err_msg=what)


def check(q, qn, dev, ref, lengths, scale=0.1, **launch):
    from bpt_amd import kivi

    lens = torch.tensor(lengths, dtype=torch.int32, device="cuda")
    got = kivi.attend(q, dev, lens, scale, **launch)
    want = okivi.attend(qn, ref, np.array(lengths), scale, **launch)
    close(got, want, f"attend {launch}")
    out, lse = kivi.decode_attention(q, dev, lens, scale, **launch)
    w_out, w_lse = okivi.decode_attention(qn, ref, np.array(lengths), scale, **launch)
    assert tuple(out.shape) == w_out.shape and tuple(lse.shape) == w_lse.shape
    close(out, w_out, f"partials {launch}")
    lse = lse.cpu().numpy()
    assert np.array_equal(np.isneginf(lse), np.isneginf(w_lse)), f"empty splits {launch}"
    fin = np.isfinite(w_lse)
    np.testing.assert_allclose(lse[fin], w_lse[fin], rtol=1e-5, atol=2e-4, err_msg=f"lse {launch}")


@pytest.mark.parametrize("bits", [4, 8, 16])
@pytest.mark.parametrize(
    "batch,q_heads,kv_heads,tokens",
    [
        (1, 16, 8, 32),  # Qwen3's heads, a single key group
        (2, 16, 8, 96),
        (2, 8, 8, 64),  # no GQA: one query head per KV head
        (1, 16, 8, 4096),
    ],
)
def test_attention_matches_the_oracle(batch, q_heads, kv_heads, tokens, bits):
    for seed in range(2):
        dev, ref = make_cache(batch, kv_heads, tokens, bits, seed=seed)
        q, qn = make_q(batch, q_heads, seed + 7)
        full = [tokens] * batch
        check(q, qn, dev, ref, full)
        for split in sorted({32, 64, tokens}):  # one group per split ... one split per KV head
            check(q, qn, dev, ref, full, split=split)


@pytest.mark.parametrize("bits", [4, 8, 16])
def test_each_rows_length(bits):
    dev, ref = make_cache(4, 8, 160, bits)
    q, qn = make_q(4, 16, 3)
    lengths = [160, 1, 70, 0]  # full, one token, odd, none
    check(q, qn, dev, ref, lengths, split=64)
    check(q, qn, dev, ref, lengths, tokens=160)
    from bpt_amd import kivi

    got = kivi.attend(q, dev, torch.tensor(lengths, dtype=torch.int32, device="cuda"), 0.1, split=32)
    assert got[3].abs().sum().item() == 0  # no tokens: zeros, not NaN


@pytest.mark.parametrize("q_heads", [8, 16])
def test_four_bit_chunk_pairs(q_heads):
    """The 4-bit kernel at 1 or 2 query heads per KV head keeps two chunks in flight per wave, walks them in
    pairs plus an odd last one and reloads a chunk past a piece's end. Ragged rows over ~11 chunks per
    workgroup give waves 0 .. 3 chunks per piece; the splits of 1, 3, 5 and 32 chunks end pieces between
    a pair's two steps."""
    lengths = [4096, 4000, 3100, 2049, 1500, 999, 513, 64, 33, 1, 0, 2047]
    dev, ref = make_cache(len(lengths), 8, 4096, 4, seed=21)
    q, qn = make_q(len(lengths), q_heads, 22)
    check(q, qn, dev, ref, lengths)
    for split in (32, 96, 160, 1024):
        check(q, qn, dev, ref, lengths, split=split)


@pytest.mark.parametrize("q_heads,kv_heads", [(32, 8), (24, 8), (40, 8), (64, 4)])
@pytest.mark.parametrize("bits", [4, 8])
def test_query_heads_per_kv_head(q_heads, kv_heads, bits):
    # 4 (Qwen3-8B), 3 (a padded row group), 5 and 16 query heads per KV head.
    dev, ref = make_cache(2, kv_heads, 256, bits, seed=11)
    q, qn = make_q(2, q_heads, 12)
    check(q, qn, dev, ref, [256, 131])
    check(q, qn, dev, ref, [256, 131], split=64)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("v_mul", [1e3, 1e-3])
def test_value_grids_far_from_one(bits, v_mul):
    # Value scales of ~100 and ~1e-4: the weights fold them in without leaving float16.
    dev, ref = make_cache(2, 8, 192, bits, seed=13, v_mul=v_mul)
    q, qn = make_q(2, 16, 14)
    check(q, qn, dev, ref, [192, 77], split=64)


@pytest.mark.parametrize("q_dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_query_dtypes_and_bfloat16_caches(q_dtype):
    for bits, half in ((8, torch.float16), (16, torch.float16), (16, torch.bfloat16)):
        dev, ref = make_cache(2, 8, 128, bits, seed=5, half=half)
        q, qn = make_q(2, 16, 6, dtype=q_dtype)
        check(q, qn, dev, ref, [64, 64])
        check(q, qn, dev, ref, [64, 64], tokens=64)  # the caller knows only 64 tokens are in use


def test_larger_key_groups():
    dev, ref = make_cache(2, 8, 256, 4, seed=15, group=64)
    q, qn = make_q(2, 16, 16)
    check(q, qn, dev, ref, [256, 200])
    check(q, qn, dev, ref, [256, 200], split=128)


@pytest.mark.parametrize("bits", [4, 8, 16])
def test_max_context(bits):
    """One sequence of 32768 tokens: 8 segments of 1024 chunks, the plan's one-workgroup-per-CU case, each
    segment split over 32 workgroups and combined by the last; and 32001 tokens over a caller's split."""
    dev, ref = make_cache(1, 8, 32768, bits, seed=9)
    q, qn = make_q(1, 16, 9)
    check(q, qn, dev, ref, [32768])
    check(q, qn, dev, ref, [32001], split=2048)


def test_repeat_calls_are_deterministic_and_reuse_the_counters():
    from bpt_amd import kivi

    dev, ref = make_cache(3, 8, 1024, 8, seed=21)
    q, _ = make_q(3, 16, 22)
    lens = torch.tensor([1024, 500, 999], dtype=torch.int32, device="cuda")
    first = kivi.decode_attention(q, dev, lens, 0.1, split=256)
    small, sref = make_cache(1, 8, 64, 4, seed=23)
    kivi.attend(make_q(1, 16, 24)[0], small, torch.tensor([64], dtype=torch.int32, device="cuda"), 0.1)
    again = kivi.decode_attention(q, dev, lens, 0.1, split=256)
    assert torch.equal(first[0], again[0]) and torch.equal(first[1], again[1])


def test_bad_arguments_raise_value_error():
    from bpt_amd import kivi

    dev, _ = make_cache(1, 8, 64, 8)
    q, _ = make_q(1, 16, 1)
    lens = torch.tensor([64], dtype=torch.int32, device="cuda")
    with pytest.raises(ValueError, match="multiple of the key group"):
        kivi.decode_attention(q, dev, lens, 0.1, split=48)
    with pytest.raises(ValueError, match="int32"):
        kivi.decode_attention(q, dev, lens.long(), 0.1)
    f64 = SimpleNamespace(**{**dev.__dict__, "bits": 16, "k_codes": dev.k_codes.double(), "v_codes": dev.v_codes.double()})
    with pytest.raises(ValueError, match="float16, bfloat16 or float32"):
        kivi.attend(q, f64, lens, 0.1)
    odd, _ = make_cache(1, 8, 64, 16, d=258)
    with pytest.raises(ValueError, match="head_dim"):
        kivi.attend(make_q(1, 16, 1, d=258)[0], odd, lens, 0.1)


@pytest.mark.parametrize("bits", [4, 8, 16])
@pytest.mark.parametrize("batch,q_heads,kv_heads,tokens,d", [
    (3, 4, 2, 160, 16),  # a tiny head (fastserve tests/kernels/test_kernels_gpu.py:87-106)
    (2, 4, 4, 64, 32),   # no GQA
    (2, 16, 8, 96, 64),
])
def test_small_head_dims(batch, q_heads, kv_heads, tokens, d, bits):
    """Head dims other than 128 take the float32 kernel; the reference tests' small shapes, two seeds, their
    splits (one group per split ... one split per KV head)."""
    for seed in range(2):
        dev, ref = make_cache(batch, kv_heads, tokens, bits, seed=seed, d=d)
        q, qn = make_q(batch, q_heads, seed + 7, d=d)
        full = [tokens] * batch
        check(q, qn, dev, ref, full)
        for split in sorted({32, 64, tokens}):
            check(q, qn, dev, ref, full, split=split)
        check(q, qn, dev, ref, [tokens, 1, 37][:batch], split=32)  # ragged rows, one of a single token


@pytest.mark.parametrize("d", [16, 128])
def test_float32_caches(d):
    """Bits-16 caches in float32 (a float32 model's QuantizedKVCache, fastserve integration/kv_cache.py:84-92)
    take the float32 kernel, at the tiny model's head dim and at 128."""
    for q_dtype in (torch.float32, torch.bfloat16):
        dev, ref = make_cache(2, 2, 128, 16, seed=31, half=torch.float32, d=d)
        q, qn = make_q(2, 4, 32, dtype=q_dtype, d=d)
        check(q, qn, dev, ref, [128, 90])
        check(q, qn, dev, ref, [128, 90], split=32)
        check(q, qn, dev, ref, [96, 96], tokens=96)


@pytest.mark.parametrize("bits", [4, 8, 16])
def test_tiny_model_decode_steps(bits):
    """fastserve's in-model kernel test (tests/kernels/test_kernels_gpu.py:148-167) in miniature: the tiny
    Qwen3's cache (2 KV heads, head dim 16, float32, 2 sequences, room for 128 tokens) as its decode steps
    see it while the stored tokens grow through whole key groups; float32 q, tokens = the stored count."""
    dev, ref = make_cache(2, 2, 128, bits, seed=41, half=torch.float32, d=16)
    for stored in (32, 64, 96, 128):
        q, qn = make_q(2, 4, 42 + stored, dtype=torch.float32, d=16)
        check(q, qn, dev, ref, [stored, stored], tokens=stored)
