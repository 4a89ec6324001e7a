"""Pins the RMSNorm + INT8 oracle (oracle/norm_quant.py): the reference tests' known answers
(tests/kernels/test_reference.py:27-31, :45-53), a float64 statement of the norm, and properties of the
quantizer that do not restate its formula (nearest code by brute force, half-a-step error, full range,
invariances of RMSNorm)."""

import json
from pathlib import Path

import numpy as np
import pytest

from oracle import norm_quant

GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_known_answers.json").read_text())


@pytest.mark.parametrize("case", GOLDEN["rms_norm_int8"])
def test_known_answers(case):
    codes, scale = norm_quant.rms_norm_int8(
        np.array([case["x"]], np.float32), np.array(case["weight"], np.float32), case["eps"]
    )
    assert codes[0].tolist() == case["codes"]
    if "scale_approx" in case:
        assert scale[0, 0] == pytest.approx(case["scale_approx"], rel=1e-6)
    else:
        assert scale[0, 0] == np.float32(case["scale_exact_float32"])


def test_norm_matches_float64_and_codes_are_the_nearest():
    g = np.random.default_rng(0)
    x = (g.standard_normal((64, 300)) * 3).astype(np.float32)
    w = (np.abs(g.standard_normal(300)) + 0.5).astype(np.float32)
    codes, scale = norm_quant.rms_norm_int8(x, w, 1e-6)
    x64 = x.astype(np.float64)
    y64 = x64 / np.sqrt(np.mean(x64 * x64, axis=-1, keepdims=True) + 1e-6) * w
    s64 = np.abs(y64).max(-1, keepdims=True) / 127
    np.testing.assert_allclose(scale, s64, rtol=1e-6)
    # brute force: every code minimises |c * scale - y| over all 256 int8 codes (up to float32 ties)
    grid_pts = np.arange(-128, 128, dtype=np.float64)[None, None, :] * scale.astype(np.float64)[..., None]
    err = np.abs(grid_pts - y64[..., None])
    chosen = np.take_along_axis(err, (codes.astype(np.int64) + 128)[..., None], -1)[..., 0]
    assert (chosen <= err.min(-1) + 1e-6 * scale).all()


def test_half_a_step_full_range_and_zero_rows():
    g = np.random.default_rng(1)
    x = (g.standard_normal((9, 100)) * 10.0 ** g.integers(-3, 3, (9, 1))).astype(np.float32)
    x[4] = 0.0
    codes, scale = norm_quant.rms_norm_int8(x, np.ones(100, np.float32), 1e-6)
    x64 = x.astype(np.float64)
    y = x64 / np.sqrt(np.mean(x64 * x64, -1, keepdims=True) + 1e-6)
    assert (np.abs(norm_quant.dequantize_int8(codes, scale) - y) <= scale / 2 * (1 + 1e-5) + 1e-7).all()
    assert (codes[4] == 0).all() and np.isfinite(scale).all()
    assert (np.abs(codes[np.arange(9) != 4]).max(-1) == 127).all()


def test_rmsnorm_invariances():
    # With eps = 0, scaling a token by a power of two changes nothing; doubling the weight doubles the scale
    # and keeps the codes (both follow from y = x / rms(x) * w, not from the code's arithmetic).
    g = np.random.default_rng(2)
    x = g.standard_normal((16, 128)).astype(np.float32)
    w = (np.abs(g.standard_normal(128)) + 0.5).astype(np.float32)
    c1, s1 = norm_quant.rms_norm_int8(x, w, 0.0)
    c2, s2 = norm_quant.rms_norm_int8(x * 8, w, 0.0)
    c3, s3 = norm_quant.rms_norm_int8(x, w * 2, 0.0)
    assert np.array_equal(c1, c2) and np.array_equal(s1, s2)
    assert np.array_equal(c1, c3) and np.array_equal(s3, 2 * s1)
