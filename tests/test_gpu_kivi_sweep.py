"""GPU: a seeded sweep of KIVI decode configurations against the oracle, at the reference tests' tolerance
(rtol 2e-4 and atol 2e-4 * max|want|, tests/kernels/test_kernels_gpu.py:78-84), through the same checks
as test_gpu_kivi.py: the merged attention and every split's partial output and lse.

Each case draws the format (4 / 8 / 16 bits, float16 or bfloat16 for 16), batch, laid-out tokens (a
multiple of the key group), ragged lengths with empty and one-token rows, query and KV head counts, the
split (one key group up to all tokens) and whether the caller passes its token count, from one seed, so
the stream-K line, the split boundaries and the combine meet combinations the targeted tests do not spell
out. Sizes stay small enough for the oracle to finish in well under a second per case.
"""

import numpy as np
import pytest
import torch

from test_gpu_kivi import check, make_cache, make_q

pytestmark = pytest.mark.gpu

HEADS = [(16, 8), (8, 8), (32, 8), (24, 8), (64, 4), (12, 4)]


def draw(seed: int) -> dict:
    g = np.random.default_rng(2000 + seed)
    bits = int(g.choice([4, 8, 16]))
    half = torch.bfloat16 if bits == 16 and g.integers(2) else torch.float16
    hq, hkv = HEADS[g.integers(len(HEADS))]
    batch = int(g.integers(1, 6))
    tokens = 32 * int(g.integers(1, 40))
    lengths = [int(x) for x in g.integers(0, tokens + 1, batch)]
    lengths[int(g.integers(batch))] = int(g.choice([0, 1, tokens]))
    splits = [s for s in (32, 64, 128, 256, tokens) if s <= tokens]
    launch = {}
    if g.integers(3):
        launch["split"] = int(g.choice(splits))
    if g.integers(2):
        launch["tokens"] = max(lengths + [1])
    return dict(bits=bits, half=half, hq=hq, hkv=hkv, batch=batch, tokens=tokens, lengths=lengths, launch=launch)


@pytest.mark.parametrize("seed", range(256))
def test_random_configuration(seed):
    cfg = draw(seed)
    dev, ref = make_cache(cfg["batch"], cfg["hkv"], cfg["tokens"], cfg["bits"], seed=seed, half=cfg["half"])
    q, qn = make_q(cfg["batch"], cfg["hq"], seed + 1)
    check(q, qn, dev, ref, cfg["lengths"], **cfg["launch"])
