"""GPU: a seeded sweep of quantize-on-write calls, bit-exact against the oracle's quantizers (FP8 static
per-head, INT8 per-token-head amax / 127, BF16 copies), with every unwritten slot unchanged.

Each case draws the format, batch, rows per sequence, KV heads, page size, pool size, source dtype and
slot index dtype from one seed (one row is always skipped through a negative block, and one key row is all
zeros)."""

import numpy as np
import pytest
import torch

from test_gpu_quant import check_append, run_append

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("seed", range(48))
def test_random_append(seed):
    g = np.random.default_rng(4000 + seed)
    fmt = ["fp8", "int8", "bf16"][int(g.integers(3))]
    src = [torch.bfloat16, torch.float16, torch.float32][int(g.integers(3))]
    b, nq = int(g.integers(2, 40)), int(g.choice([1, 1, 2, 5]))
    page = int(g.choice([1, 8, 16, 32, 64]))
    nb = -(-b * nq // page) + int(g.integers(1, 8))
    r = run_append(fmt, b=b, nq=nq, hkv=int(g.choice([2, 4, 8])), page=page, nb=nb, src=src, seed=seed,
                   i64=bool(g.integers(2)))
    check_append(r, fmt, src)
