"""GPU: a seeded sweep of paged decode configurations against the oracle, at the decode tolerance
(|got - want| <= 2e-3 + 1e-2 * |want|).

Each case draws the batch size, ragged lengths (zeros and one-token rows included), query and KV head
counts, queries per sequence, page size, cache format and scale granularity, q dtype and split count from
one seed, so both kernels, the stream-K line walk (pieces, split segments, ranges that hold no chunk) and
the split-K combine meet many combinations that the targeted tests in test_gpu_decode.py do not spell out.
Sizes stay small enough for the oracle to finish in well under a second per case.
A second sweep keeps every sequence of a call at one length, the case the vector kernel cuts into equal
partitions. A third draws only matrix-core calls of 2..7 rows over 128 or more segments with an automatic
split, which run on 2-wave workgroups, four to a CU.
"""

import numpy as np
import pytest
import torch

from test_gpu_decode import check, make_case, run_case

pytestmark = pytest.mark.gpu

FORMATS = [("fp8", "head"), ("fp8", "token"), ("int8", "token"), ("int8", "head"), ("bf16", None)]
HEADS = [(8, 8), (16, 8), (32, 8), (12, 4), (40, 8), (64, 4)]


def draw(seed: int) -> dict:
    g = np.random.default_rng(1000 + seed)
    fmt, scales = FORMATS[g.integers(len(FORMATS))]
    hq, hkv = HEADS[g.integers(len(HEADS))]
    nq = int(g.choice([1, 1, 2, 3, 5]))
    while nq * hq // hkv > 16 and nq > 1:  # keep Q * G within one 16-row group now and then
        nq -= 1
    b = int(g.integers(1, 24))
    cap = int(g.choice([40, 300, 1200, 2500]))
    lengths = [int(x) for x in g.integers(0, cap + 1, b)]
    lengths[int(g.integers(b))] = int(g.choice([0, 1, cap]))
    return dict(
        fmt=fmt, scales=scales, hq=hq, hkv=hkv, nq=nq, lengths=lengths,
        page=int(g.choice([8, 16, 16, 32, 64])),
        q_dtype=[torch.bfloat16, torch.float16, torch.float32][int(g.integers(3))],
        num_splits=[None, None, 1, 3, 17][int(g.integers(5))],
    )


@pytest.mark.parametrize("seed", range(256))
def test_random_configuration(seed):
    cfg = draw(seed)
    c = make_case(cfg["fmt"], cfg["lengths"], hq=cfg["hq"], hkv=cfg["hkv"], nq=cfg["nq"], page=cfg["page"],
                  scales=cfg["scales"] or "head", seed=seed)
    got, want = run_case(c, q=c["q"].to(cfg["q_dtype"]), num_splits=cfg["num_splits"])
    check(got, want, f"seed {seed}: {cfg}")
    for i, t in enumerate(cfg["lengths"]):
        if t == 0:
            assert got[i].float().abs().sum().item() == 0, f"seed {seed}: row {i} has no tokens"


def draw_equal(seed: int) -> dict:
    """Vector-kernel calls (BF16, or INT8 with 1..4 rows per KV head) whose sequences share one length: the
    equal power-of-two partitions, with max_context at or above that length and a batch of one now and then."""
    g = np.random.default_rng(5000 + seed)
    fmt, scales = [("bf16", None), ("int8", "token"), ("int8", "head")][int(g.integers(3))]
    hq, hkv = [(8, 8), (16, 8), (32, 8), (12, 4)][int(g.integers(4))]
    b = int(g.choice([1, 1, 2, 3, 7, 16]))
    t = int(g.choice([1, 15, 16, 17, 100, 513, 1024, 2047, 3000]))
    return dict(fmt=fmt, scales=scales, hq=hq, hkv=hkv, lengths=[t] * b, page=int(g.choice([8, 16, 32])),
                max_context=t + int(g.choice([0, 0, 1, 500])),
                q_dtype=[torch.bfloat16, torch.float16, torch.float32][int(g.integers(3))])


@pytest.mark.parametrize("seed", range(48))
def test_random_equal_lengths(seed):
    cfg = draw_equal(seed)
    c = make_case(cfg["fmt"], cfg["lengths"], hq=cfg["hq"], hkv=cfg["hkv"], page=cfg["page"],
                  scales=cfg["scales"] or "head", seed=seed)
    got, want = run_case(c, q=c["q"].to(cfg["q_dtype"]), max_context=cfg["max_context"])
    check(got, want, f"seed {seed}: {cfg}")


def draw_many_segments(seed: int) -> dict:
    """Matrix-core calls the plan runs on 2-wave workgroups, four to a CU: 2..7 rows per KV head (FP8, or INT8
    from 5 rows), an automatic split and at least 128 (sequence, KV head) segments."""
    g = np.random.default_rng(9000 + seed)
    fmt, scales = [("fp8", "head"), ("fp8", "head"), ("fp8", "token"), ("int8", "head"), ("int8", "token")][
        int(g.integers(5))]
    lo = 5 if fmt == "int8" else 2
    heads = [(hq, hkv) for hq, hkv in [(16, 8), (32, 8), (8, 8), (24, 8), (16, 4)]
             if any(r % (hq // hkv) == 0 for r in range(lo, 8))]
    hq, hkv = heads[int(g.integers(len(heads)))]
    G = hq // hkv
    rows = [r for r in range(lo, 8) if r % G == 0]
    nq = int(g.choice(rows)) // G
    b_min = -(-128 // hkv)
    b = int(g.integers(b_min, b_min + 24))
    cap = int(g.choice([64, 700, 2000]))
    lengths = [int(x) for x in g.integers(0, cap + 1, b)]
    for i in g.choice(b, size=3, replace=False):
        lengths[int(i)] = int(g.choice([0, 1, nq, cap]))
    return dict(fmt=fmt, scales=scales, hq=hq, hkv=hkv, nq=nq, lengths=lengths,
                page=int(g.choice([8, 16, 32])),
                q_dtype=[torch.bfloat16, torch.float16, torch.float32][int(g.integers(3))])


@pytest.mark.parametrize("seed", range(40))
def test_random_many_segments(seed):
    cfg = draw_many_segments(seed)
    assert 2 <= cfg["nq"] * cfg["hq"] // cfg["hkv"] < 8 and len(cfg["lengths"]) * cfg["hkv"] >= 128
    c = make_case(cfg["fmt"], cfg["lengths"], hq=cfg["hq"], hkv=cfg["hkv"], nq=cfg["nq"], page=cfg["page"],
                  scales=cfg["scales"], seed=seed)
    got, want = run_case(c, q=c["q"].to(cfg["q_dtype"]))
    check(got, want, f"seed {seed}: {cfg}")
    for i, t in enumerate(cfg["lengths"]):
        if t == 0:
            assert got[i].float().abs().sum().item() == 0, f"seed {seed}: row {i} has no tokens"
