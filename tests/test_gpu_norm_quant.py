"""RMSNorm + per-token INT8 on the GPU (bpt_amd.rms_norm_int8 -> bpt_rms_norm_int8) against the oracle, on
fastserve's own kernel-1 cases (tests/kernels/test_kernels_gpu.py:28-65) plus widths that take the other
launch shapes (8192: the whole row in registers at its widest; 12000 and 20000: streamed; odd widths: one
element per lane).

Tolerance: the reference tests' own (test_kernels_gpu.py:39-44): scale within rtol 1e-5, no code off by more
than one, fewer than 0.1% of codes off at all (a value exactly between two codes may round either way when
the two sums of squares differ in the last bit)."""

import numpy as np
import pytest
import torch

from oracle import norm_quant as onq

pytestmark = pytest.mark.gpu

FLOATS = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}


def rand(*shape, seed=0, dtype=torch.float32):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return torch.randn(*shape, generator=g, device="cuda").to(dtype)


def check(x, weight, eps, codes, scale):
    want_codes, want_scale = onq.rms_norm_int8(x.float().cpu().numpy(), weight.float().cpu().numpy(), eps)
    assert codes.dtype == torch.int8 and tuple(codes.shape) == tuple(x.shape)
    assert tuple(scale.shape) == tuple(x.shape[:-1]) + (1,)
    np.testing.assert_allclose(scale.cpu().numpy(), want_scale, rtol=1e-5, atol=0)
    diff = np.abs(codes.cpu().numpy().astype(np.int32) - want_codes.astype(np.int32))
    assert diff.max() <= 1 and (diff > 0).mean() < 1e-3


@pytest.mark.parametrize("dtype", list(FLOATS))
@pytest.mark.parametrize(
    "rows,d", [(1, 1024), (3, 2048), (257, 1000), (64, 3), (5, 1), (4096, 1024), (7, 8192), (3, 12000), (2, 20000), (9, 777)]
)
def test_norm_quant_matches_the_oracle(rows, d, dtype):
    from bpt_amd import rms_norm_int8

    for seed in range(3):
        x = rand(rows, d, seed=seed, dtype=FLOATS[dtype]) * 3
        weight = (rand(d, seed=seed + 100).abs() + 0.5).to(FLOATS[dtype])
        codes, scale = rms_norm_int8(x, weight, 1e-6)
        check(x, weight, 1e-6, codes, scale)


def test_known_answer_on_the_device():
    from bpt_amd import rms_norm_int8

    x = torch.tensor([[3.0, -4.0, 0.0, 0.0]], device="cuda")
    codes, scale = rms_norm_int8(x, torch.ones(4, device="cuda"), 0.0)
    assert codes.tolist() == [[95, -127, 0, 0]]
    assert scale.item() == pytest.approx(1.6 / 127, rel=1e-6)


def test_shapes_views_zero_rows_and_out_buffers():
    from bpt_amd import rms_norm_int8

    x = rand(2, 5, 64, dtype=torch.bfloat16)
    x[1, 2] = 0.0  # an all-zero token must not divide by zero
    weight = torch.ones(64, device="cuda", dtype=torch.bfloat16)
    codes, scale = rms_norm_int8(x, weight, 1e-6)
    check(x, weight, 1e-6, codes, scale)
    assert codes[1, 2].abs().sum().item() == 0 and torch.isfinite(scale).all()

    wide = rand(8, 128)  # every other column: a non-contiguous view, copied first
    codes, scale = rms_norm_int8(wide[:, ::2], weight.float(), 1e-6)
    check(wide[:, ::2], weight.float(), 1e-6, codes, scale)

    out = (torch.empty((8, 64), dtype=torch.int8, device="cuda"), torch.empty(8, device="cuda"))
    again, _ = rms_norm_int8(wide[:, :64].contiguous(), weight.float(), 1e-6, out=out, num_warps=8)
    assert again.data_ptr() == out[0].data_ptr()  # the caller's buffers were used
    with pytest.raises(ValueError):
        rms_norm_int8(wide[:, :64].contiguous(), weight.float(), 1e-6, out=(out[0].float(), out[1]))
