"""Shared-prefix cascade decode (bpt_amd.cascade_decode_attention: a prefix pass and a merging suffix pass,
both through bpt_paged_decode) against the oracle's paged decode, and the log-sum-exp output the cascade is
built on. Same tolerance as every attention test here: max-abs 2e-3 + rel 1e-2 against float32."""

import numpy as np
import pytest
import torch

from oracle import attention

pytestmark = pytest.mark.gpu


def oracle_of(w, q=None):
    from bpt_amd import workloads

    o = workloads.to_oracle(w)
    if q is not None:
        o["q"] = q.float().cpu().numpy()
    return attention.paged_decode(o["q"], o["k_pool"], o["v_pool"], o["block_table"], o["context_lens"],
                                  o["k_scale"], o["v_scale"], o["kv_format"], o["scale"])


def close(got, want, what=""):
    got = got.float().cpu().numpy()
    err = np.abs(got - want)
    assert np.isfinite(got).all() and (err <= 2e-3 + 1e-2 * np.abs(want)).all(), f"{what}: max err {err.max():.3e}"


def test_verify_workload_cascade_matches_plain_decode():
    from bpt_amd import cascade_decode_attention, paged_decode_attention, workloads

    w = workloads.make("qwen3-1.7b-verify", device="cuda", seed=0, batch=8, length_cap=2000)
    want, _ = oracle_of(w)
    kw = w.kwargs()
    got = cascade_decode_attention(*w.args(), **kw, prefix_pages=w.shape.shared_prefix_pages,
                                   context_lens_host=w.lengths)
    close(got, want, "cascade")
    plain = paged_decode_attention(*w.args(), **kw)
    close(plain, want, "plain")


@pytest.mark.parametrize("fmt,scales,q_heads,queries", [("fp8", "head", 16, 1), ("int8", "token", 32, 3), ("bf16", "none", 16, 2)])
def test_two_groups_with_their_own_prefix_pages(fmt, scales, q_heads, queries):
    from bpt_amd import cascade_decode_attention, workloads

    shape = workloads.Shape("t", 6, q_heads, 8, fmt, scales, (100, 300), queries=queries, shared_prefix_pages=4,
                            pool_factor=2.0)
    w = workloads.make(shape=shape, device="cuda", seed=3)
    # Rows 2..5 get their own copy of the prefix pages, with the tokens inside each page rotated: another
    # group, another prefix (an oracle reading row 0's pages for them would disagree).
    tables = w.block_table.clone()
    nb = w.k_cache.shape[0]
    free = [p for p in range(nb) if p not in set(tables.flatten().tolist())]
    assert len(free) >= 4
    for j in range(4):
        src, dst = int(tables[0, j]), free[j]
        for pool in (w.k_cache, w.v_cache) + ((w.k_scale, w.v_scale) if scales == "token" else ()):
            raw = pool.view(torch.uint8) if pool.dtype == torch.float8_e4m3fn else pool
            raw[dst] = torch.roll(raw[src], shifts=5, dims=0)
        tables[2:, j] = dst
    w.block_table = tables
    want, _ = oracle_of(w)
    got = cascade_decode_attention(*w.args(), **w.kwargs(), prefix_pages=4, groups=[(0, 2), (2, 6)],
                                   context_lens_host=w.lengths)
    close(got, want, f"{fmt} groups")


def test_empty_suffixes_give_the_prefix_alone():
    from bpt_amd import cascade_decode_attention, workloads

    shape = workloads.Shape("t", 4, 16, 8, "fp8", "head", 64, queries=1, shared_prefix_pages=4)
    w = workloads.make(shape=shape, device="cuda", seed=5)  # 64 tokens = exactly the prefix
    want, _ = oracle_of(w)
    got = cascade_decode_attention(*w.args(), **w.kwargs(), prefix_pages=4)
    close(got, want, "prefix only")


def test_lse_output_matches_the_oracle():
    from bpt_amd import paged_decode_attention, workloads

    w = workloads.make("qwen3-1.7b-verify", device="cuda", seed=1, batch=4, length_cap=1500)
    want_out, want_lse = oracle_of(w)
    b, nq, hq, _ = w.q.shape
    lse = torch.empty((b, nq, hq), dtype=torch.float32, device="cuda")
    out = paged_decode_attention(*w.args(), **w.kwargs(), lse=lse, out_dtype=torch.float32)
    close(out, want_out, "out")
    np.testing.assert_allclose(lse.cpu().numpy(), want_lse, rtol=1e-4, atol=2e-3)


def test_queries_inside_the_prefix_are_refused():
    from bpt_amd import cascade_decode_attention, workloads

    shape = workloads.Shape("t", 2, 16, 8, "fp8", "head", 66, queries=5, shared_prefix_pages=4)
    w = workloads.make(shape=shape, device="cuda", seed=6)  # queries at positions 61..65, prefix 0..63
    with pytest.raises(ValueError, match="end inside the shared prefix"):
        cascade_decode_attention(*w.args(), **w.kwargs(), prefix_pages=4, context_lens_host=w.lengths)
