"""GPU: a seeded sweep of shared-prefix cascade calls against the oracle's paged decode, at the attention
tolerance (|got - want| <= 2e-3 + 1e-2 * |want|).

Each case draws the format and scales, batch, query and KV heads, queries per sequence, the shared prefix
(1..8 pages), ragged lengths from the prefix's end (the shortest rows' first query exactly there) and a
split count for the suffix pass from one seed; the workload generator makes every row's first pages the
same physical pages.
"""

import numpy as np
import pytest

from test_gpu_cascade import close, oracle_of

pytestmark = pytest.mark.gpu

FORMATS = [("fp8", "head"), ("fp8", "token"), ("int8", "token"), ("int8", "head"), ("bf16", "none")]
HEADS = [(16, 8), (32, 8), (8, 8), (12, 4)]


@pytest.mark.parametrize("seed", range(128))
def test_random_cascade(seed):
    from bpt_amd import cascade_decode_attention, workloads

    g = np.random.default_rng(3000 + seed)
    fmt, scales = FORMATS[g.integers(len(FORMATS))]
    hq, hkv = HEADS[g.integers(len(HEADS))]
    prefix = int(g.choice([1, 2, 4, 8]))
    nq = int(g.choice([1, 1, 2, 5]))
    lo = prefix * 16 + nq - 1 + int(g.choice([0, 0, 1, 30]))  # the first query at or after the prefix's end
    shape = workloads.Shape("sweep", int(g.integers(1, 12)), hq, hkv, fmt, scales, (lo, lo + int(g.integers(1, 600))),
                            queries=nq, shared_prefix_pages=prefix, pool_factor=1.5)
    w = workloads.make(shape=shape, device="cuda", seed=seed)
    kw = {**w.kwargs(), "num_splits": [None, None, 3][int(g.integers(3))]}
    got = cascade_decode_attention(*w.args(), **kw, prefix_pages=prefix, context_lens_host=w.lengths)
    want, _ = oracle_of(w)
    close(got, want, f"seed {seed}: {shape}")
