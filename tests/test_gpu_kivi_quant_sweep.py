"""GPU: a seeded sweep of KIVI quantize-on-write calls (bpt_amd.kivi.quantize_kv_into -> bpt_kivi_quantize)
against the oracle's quantize_kv (oracle/kivi.py), codes and float16 grids compared bit for bit.

Each case draws bits (4 / 8), head dim (16 .. 256), source dtype (bf16 / f16 / f32), key group (32 or 64),
batch, KV heads, groups written, the token offset inside a larger cache, the source layout ([B, Hkv, T, D]
contiguous, a token-major [B, T, Hkv, D] view, or a view one channel into wider rows, which is off its
16-byte alignment) and whether the cache's code rows start one byte in (off their 8-byte alignment), with
values from N(0, 1) times 1e-3 .. 1e3 and an outlier channel. So both kernels (16-byte rows for aligned
32-token groups, the row-at-a-time kernel for the rest) meet layouts and shapes the targeted tests do not
spell out, and the cache outside the written tokens must keep its contents.
"""

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from oracle import kivi as okivi

pytestmark = pytest.mark.gpu

DTYPES = [torch.bfloat16, torch.float16, torch.float32]


def draw(seed: int) -> dict:
    g = np.random.default_rng(7000 + seed)
    return dict(
        bits=int(g.choice([4, 8])),
        d=int(g.choice([16, 32, 64, 128, 256])),
        dtype=DTYPES[int(g.integers(3))],
        group=int(g.choice([32, 32, 32, 64])),
        batch=int(g.integers(1, 4)),
        heads=int(g.choice([1, 2, 4, 8])),
        groups=int(g.integers(1, 4)),
        before=int(g.integers(0, 3)),
        layout=str(g.choice(["contiguous", "token-major", "offset"], p=[0.4, 0.35, 0.25])),
        code_offset=int(g.random() < 0.25),
        mag=float(10.0 ** g.uniform(-3, 3)),
        seed=int(g.integers(1 << 30)),
    )


def source(c: dict, n: int, g: np.random.Generator) -> tuple[torch.Tensor, np.ndarray]:
    """One of k / v: [B, Hkv, n, D] on the GPU in the drawn layout, and its float32 values."""
    b, h, d = c["batch"], c["heads"], c["d"]
    x = g.standard_normal((b, h, n, d)).astype(np.float32) * c["mag"]
    x[..., int(g.integers(d))] += 20.0 * c["mag"]
    t = torch.from_numpy(x).to(c["dtype"])
    if c["layout"] == "token-major":
        t = t.permute(0, 2, 1, 3).contiguous().cuda().permute(0, 2, 1, 3)
    elif c["layout"] == "offset":
        wide = torch.zeros((b, h, n, d + 8), dtype=c["dtype"])
        wide[..., 1:d + 1] = t
        t = wide.cuda()[..., 1:d + 1]
    else:
        t = t.cuda()
    return t, t.float().cpu().numpy()


def cache(c: dict, total: int):
    """A KIVI cache of `total` tokens filled with sentinels (codes 0xA5, grids 7.0)."""
    from bpt_amd import kivi

    b, h, d, bits, group = c["batch"], c["heads"], c["d"], c["bits"], c["group"]
    width = d // 2 if bits == 4 else d
    off = c["code_offset"]
    raw = torch.full((2, b, h, total, width + off), 0xA5, dtype=torch.uint8, device="cuda")
    grid = lambda *s: torch.full(s, 7.0, dtype=torch.float16, device="cuda")  # noqa: E731
    return kivi.QuantKV(bits, group, raw[0, ..., off:], raw[1, ..., off:], grid(b, h, total // group, d),
                        grid(b, h, total // group, d), grid(b, h, total), grid(b, h, total))


def same_bits(got: torch.Tensor, want: np.ndarray, what: str) -> None:
    got = got.detach().cpu().numpy()
    assert got.shape == want.shape, what
    view = np.uint16 if want.dtype == np.float16 else want.dtype
    bad = got.view(view) != np.ascontiguousarray(want).view(view)
    assert not bad.any(), f"{what}: {bad.sum()} of {bad.size} differ"


@pytest.mark.parametrize("seed", range(120))
def test_quantize_sweep(seed):
    from bpt_amd import kivi

    c = draw(seed)
    g = np.random.default_rng(c["seed"])
    group = c["group"]
    n = group * c["groups"]
    start = group * c["before"]
    total = start + n + group
    k, kn = source(c, n, g)
    v, vn = source(c, n, g)
    kv = cache(c, total)
    kivi.quantize_kv_into(k, v, kv, start)
    torch.cuda.synchronize()
    ref = okivi.quantize_kv(kn, vn, c["bits"], group)
    g0, g1 = start // group, (start + n) // group
    part = SimpleNamespace(k_codes=kv.k_codes[:, :, start:start + n], v_codes=kv.v_codes[:, :, start:start + n],
                           k_scale=kv.k_scale[:, :, g0:g1], k_zero=kv.k_zero[:, :, g0:g1],
                           v_scale=kv.v_scale[:, :, start:start + n], v_zero=kv.v_zero[:, :, start:start + n])
    for f in ("k_codes", "v_codes", "k_scale", "k_zero", "v_scale", "v_zero"):
        same_bits(getattr(part, f), getattr(ref, f), f"{c} {f}")
    # Everything outside the written tokens keeps its sentinel.
    for codes in (kv.k_codes, kv.v_codes):
        assert bool((codes[:, :, :start] == 0xA5).all()) and bool((codes[:, :, start + n:] == 0xA5).all()), c
    assert bool((kv.k_scale[:, :, :g0] == 7).all()) and bool((kv.k_scale[:, :, g1:] == 7).all()), c
    assert bool((kv.v_zero[:, :, :start] == 7).all()) and bool((kv.v_zero[:, :, start + n:] == 7).all()), c
