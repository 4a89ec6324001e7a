"""Pins the oracle's attention and paging: float64 brute force on tiny inputs, closed forms, split-merge
exactness, empty rows, the GQA head mapping, causal visibility by position, paged == contiguous, and the
reference tests' known answers (fastserve tests/kernels/test_reference.py:143-190,
tests/engine/test_kv_cache.py:22-54, tests/kernels/test_kernels_gpu.py:136-142)."""

import json
import math
from pathlib import Path

import numpy as np
import pytest

from oracle import attention, fp8, paged, quant

GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_known_answers.json").read_text())


def rand(*shape, seed=0):
    return np.random.default_rng(seed).standard_normal(shape).astype(np.float32)


def brute_force(q, k, v, lengths, scale):
    """softmax(q·k·scale)·v with Python loops in float64, GQA by h // G."""
    b_sz, hq, d = q.shape
    hkv = k.shape[1]
    g = hq // hkv
    out = np.zeros((b_sz, hq, d))
    lse = np.full((b_sz, hq), -math.inf)
    for b in range(b_sz):
        for h in range(hq):
            n = int(lengths[b])
            if n == 0:
                continue
            s = [sum(float(q[b, h, c]) * float(k[b, h // g, t, c]) for c in range(d)) * scale for t in range(n)]
            m = max(s)
            w = [math.exp(x - m) for x in s]
            z = sum(w)
            lse[b, h] = m + math.log(z)
            for c in range(d):
                out[b, h, c] = sum(w[t] * float(v[b, h // g, t, c]) for t in range(n)) / z
    return out, lse


def test_partial_attention_equals_float64_brute_force():
    q, k, v = rand(3, 4, 8, seed=1), rand(3, 2, 11, 8, seed=2), rand(3, 2, 11, 8, seed=3)
    k[..., 3] += 5.0
    lengths = np.array([11, 1, 6])
    out, lse = attention.partial_attention(q, k, v, lengths, 0.3)
    ref_out, ref_lse = brute_force(q, k, v, lengths, 0.3)
    np.testing.assert_allclose(out, ref_out, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(lse, ref_lse, rtol=1e-5, atol=1e-5)


def test_closed_forms_uniform_scores_and_single_token():
    v = rand(1, 1, 7, 4, seed=4)
    k = np.ones((1, 1, 7, 4), dtype=np.float32)
    q = rand(1, 2, 4, seed=5)
    out, lse = attention.partial_attention(q, k, v, np.array([5]), 0.5)
    np.testing.assert_allclose(out[0, 0], v[0, 0, :5].mean(0), rtol=1e-6)  # equal scores: the mean
    np.testing.assert_allclose(lse[0, 0], 0.5 * q[0, 0].sum() + math.log(5), rtol=1e-6)
    out1, _ = attention.partial_attention(q, k, v, np.array([1]), 0.5)
    np.testing.assert_array_equal(out1[0, 1], v[0, 0, 0])  # one visible token: its value


def test_split_merge_is_exact_and_empty_split_has_no_weight():
    gold = GOLDEN["merge_partials"]
    t, s = gold["tokens"], gold["split"]
    q, k, v = rand(3, 4, 16, seed=6), rand(3, 2, t, 16, seed=7), rand(3, 2, t, 16, seed=8)
    lengths = np.array(gold["lengths"])
    outs, lses = [], []
    for start in range(0, t, s):
        seen = np.clip(lengths - start, 0, s)
        o, l = attention.partial_attention(q, k[:, :, start : start + s], v[:, :, start : start + s], seen, 0.25)
        outs.append(o)
        lses.append(l)
    e = gold["empty_split"]
    assert np.isinf(lses[e["split_index"]][e["row"]]).all() and not outs[e["split_index"]][e["row"]].any()
    merged = attention.merge_partials(np.stack(outs, 2), np.stack(lses, 2))
    whole, _ = attention.partial_attention(q, k, v, lengths, 0.25)
    np.testing.assert_allclose(merged, whole, rtol=1e-5, atol=1e-6)


def test_zero_length_row_gives_zeros_not_nan():
    q, k, v = rand(2, 4, 16), rand(2, 2, 64, 16, seed=1), rand(2, 2, 64, 16, seed=2)
    out, lse = attention.partial_attention(q, k, v, np.array(GOLDEN["zero_length_row"]["lengths"]), 0.25)
    assert not out[0].any() and np.isinf(lse[0]).all()
    merged = attention.merge_partials(out[:, :, None], lse[:, :, None])
    assert np.isfinite(merged).all() and not merged[0].any()


def test_gqa_kv_head_h_serves_query_heads_h_times_g_onwards():
    hkv, g, d, t = 4, 3, 8, 5
    v = np.zeros((1, hkv, t, d), dtype=np.float32)
    for h in range(hkv):
        v[0, h] = h  # every value of KV head h is h
    out, _ = attention.partial_attention(rand(1, hkv * g, d), rand(1, hkv, t, d, seed=3), v, np.array([t]), 1.0)
    np.testing.assert_allclose(out[0, :, 0], np.repeat(np.arange(hkv), g), atol=1e-6)


def paged_inputs(lengths, hkv=2, d=16, page=4, seed=0, fmt="bf16"):
    """A random paged cache (pages shuffled) and the same tokens laid out contiguously."""
    g = np.random.default_rng(seed)
    t_max = max(lengths)
    k = g.standard_normal((len(lengths), t_max, hkv, d)).astype(np.float32)
    v = g.standard_normal((len(lengths), t_max, hkv, d)).astype(np.float32)
    n_pages = [math.ceil(t / page) for t in lengths]
    nb = sum(n_pages) + 3
    perm = g.permutation(nb)
    k_pool = np.zeros((nb, page, hkv, d), np.float32)
    v_pool = np.zeros_like(k_pool)
    table = np.zeros((len(lengths), max(n_pages)), np.int64)
    c = 0
    for b, t in enumerate(lengths):
        for j in range(n_pages[b]):
            table[b, j] = perm[c]
            c += 1
        pos = np.arange(t)
        k_pool[table[b, pos // page], pos % page] = k[b, :t]
        v_pool[table[b, pos // page], pos % page] = v[b, :t]
    return k, v, k_pool, v_pool, table


def test_paged_decode_equals_contiguous_attention():
    lengths = [13, 1, 8, 0]
    k, v, k_pool, v_pool, table = paged_inputs(lengths)
    q = rand(4, 1, 6, 16, seed=9)
    out, lse = attention.paged_decode(q, k_pool, v_pool, table, np.array(lengths), None, None, "bf16", 0.2)
    ref, ref_lse = attention.partial_attention(q[:, 0], k.transpose(0, 2, 1, 3), v.transpose(0, 2, 1, 3),
                                               np.array(lengths), 0.2)
    np.testing.assert_allclose(out[:, 0], ref, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(lse[:, 0], ref_lse, rtol=1e-5, atol=1e-6)


def test_multi_query_is_causal_by_position():
    lengths = [11, 6]
    nq = 3
    k, v, k_pool, v_pool, table = paged_inputs(lengths, seed=2)
    q = rand(2, nq, 4, 16, seed=10)
    out, _ = attention.paged_decode(q, k_pool, v_pool, table, np.array(lengths), None, None, "bf16", 0.3)
    kc, vc = k.transpose(0, 2, 1, 3), v.transpose(0, 2, 1, 3)
    positions = np.array([[t - nq + i for i in range(nq)] for t in lengths])
    mask = attention.causal_mask(positions, kc.shape[2])
    ref = attention.attention(q.transpose(0, 2, 1, 3), kc, vc, mask, 0.3).transpose(0, 2, 1, 3)
    np.testing.assert_allclose(out, ref, rtol=1e-5, atol=1e-6)
    for i in range(nq):  # query i alone, as a single decode over its visible prefix
        single, _ = attention.partial_attention(q[:, i], kc, vc, np.array(lengths) - nq + i + 1, 0.3)
        np.testing.assert_allclose(out[:, i], single, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("fmt", ["fp8", "int8"])
def test_quantized_paged_decode_reads_the_cache_as_stored(fmt):
    lengths = [9, 16, 3]
    k, v, k_pool_f, v_pool_f, table = paged_inputs(lengths, seed=4)
    if fmt == "fp8":
        ks = quant.per_head_scale(k_pool_f, 448.0)
        vs = quant.per_head_scale(v_pool_f, 448.0)
        k_pool, v_pool = quant.fp8_per_head(k_pool_f, ks), quant.fp8_per_head(v_pool_f, vs)
        k_hat, v_hat = fp8.decode(k_pool) * ks[:, None], fp8.decode(v_pool) * vs[:, None]
    else:
        k_pool, ks = quant.per_token(k_pool_f, "int8")
        v_pool, vs = quant.per_token(v_pool_f, "int8")
        k_hat, v_hat = k_pool * ks, v_pool * vs
        ks, vs = ks[..., 0], vs[..., 0]
    q = rand(3, 1, 4, 16, seed=11)
    out, _ = attention.paged_decode(q, k_pool, v_pool, table, np.array(lengths), ks, vs, fmt, 0.25)
    want, _ = attention.paged_decode(q, k_hat, v_hat, table, np.array(lengths), None, None, "bf16", 0.25)
    np.testing.assert_allclose(out, want, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("fmt,scales", [("bf16", None), ("fp8", "head"), ("fp8", "token"), ("int8", "token"),
                                         ("int8", "head")])
def test_torch_restatement_equals_the_numpy_oracle(fmt, scales):
    """oracle.torch_paged (the CPU baseline's PyTorch path, padded batch like fastserve's engine) gives the
    numpy oracle's result on ragged lengths (one of them empty), several queries and every cache format."""
    import torch

    from oracle import torch_paged

    lengths = [13, 1, 8, 0, 22]
    nq = 2
    k, v, k_pool_f, v_pool_f, table = paged_inputs(lengths, hkv=2, d=16, page=4, seed=6)
    lens = np.array([max(t, 0) for t in lengths])
    if fmt == "bf16":
        k_pool = torch.from_numpy(k_pool_f).bfloat16()
        v_pool = torch.from_numpy(v_pool_f).bfloat16()
        kn, vn = k_pool.float().numpy(), v_pool.float().numpy()
        ks = vs = None
    elif scales == "head":
        ks = quant.per_head_scale(k_pool_f, 448.0 if fmt == "fp8" else 127.0)
        vs = quant.per_head_scale(v_pool_f, 448.0 if fmt == "fp8" else 127.0)
        enc = quant.fp8_per_head if fmt == "fp8" else quant.int8_per_head
        kn, vn = enc(k_pool_f, ks), enc(v_pool_f, vs)
    else:
        kn, ks = quant.per_token(k_pool_f, fmt)
        vn, vs = quant.per_token(v_pool_f, fmt)
        ks, vs = ks[..., 0], vs[..., 0]
    if fmt != "bf16":
        as_torch = (lambda c: torch.from_numpy(c).view(torch.float8_e4m3fn)) if fmt == "fp8" else torch.from_numpy
        k_pool, v_pool = as_torch(kn), as_torch(vn)
    q = rand(len(lengths), nq, 4, 16, seed=12)
    want, want_lse = attention.paged_decode(q, kn, vn, table, lens, ks, vs, fmt, 0.3)
    got, got_lse = torch_paged.paged_decode(
        torch.from_numpy(q), k_pool, v_pool, torch.from_numpy(table), torch.from_numpy(lens).int(),
        None if ks is None else torch.from_numpy(ks), None if vs is None else torch.from_numpy(vs), fmt, 0.3)
    np.testing.assert_allclose(got.numpy(), want, rtol=1e-5, atol=1e-6)
    np.testing.assert_array_equal(np.isneginf(got_lse.numpy()), np.isneginf(want_lse))
    fin = np.isfinite(want_lse)
    np.testing.assert_allclose(got_lse.numpy()[fin], want_lse[fin], rtol=1e-5, atol=1e-6)


def test_default_split_known_answers():
    gold = GOLDEN["default_split"]
    for c in gold["cases"]:
        assert attention.default_split(c["batch"], c["kv_heads"], c["tokens"]) == c["split"]
    assert all(attention.default_split(b, 8, t) % gold["multiple_of"] == 0 for b in gold["batches"] for t in gold["tokens"])


def test_prepare_write_slots_and_padding():
    tables = [[5, 2, 7], [1]]
    positions = np.array([[9], [2]])
    wb, wo, bt, kv_len = paged.prepare(tables, positions, 4)
    assert kv_len == 10 and bt.tolist() == [[5, 2, 7], [1, 0, 0]]  # padded with block 0
    assert wb.tolist() == [[7], [1]] and wo.tolist() == [[1], [2]]
    with pytest.raises(ValueError, match=GOLDEN["paged_allocator"]["refuse"]["message"]):
        paged.prepare([[3]], np.array([[4]]), 4)


def test_scatter_then_gather_round_trips():
    pool = np.zeros((6, 4, 2, 3), np.float32)
    rows = rand(2, 3, 2, 3, seed=12)
    tables = [[4, 1], [0, 5]]
    positions = np.array([[0, 1, 5], [2, 3, 4]])
    wb, wo, bt, kv_len = paged.prepare(tables, positions, 4)
    paged.scatter(pool, wb, wo, rows)
    got = paged.gather(pool, bt, kv_len)  # [B, Hkv, kv_len, D]
    for b in range(2):
        for i, p in enumerate(positions[b]):
            np.testing.assert_array_equal(got[b, :, p], rows[b, i])


def test_bytes_per_token_known_answer():
    gold = GOLDEN["kv_bytes_per_token"]
    elements = 2 * gold["layers"] * gold["kv_heads"] * gold["head_dim"]
    assert elements * 2 == gold["bf16"] and elements * 1 == gold["fp8"]
