"""Pins the oracle's quantizers: FP8 e4m3fn against torch's float8_e4m3fn cast (the library routine fastserve
itself trusts, tests/quant/test_formats.py:39-52), INT8 against the reference tests' known answers and
properties that do not restate the formula (half-a-step error, full range, zero rows)."""

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import fp8, quant

GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_known_answers.json").read_text())


def torch_fp8_codes(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.asarray(x, dtype=np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def test_decode_table_matches_torch_for_all_256_codes():
    ref = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    got = fp8.decode_table()
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    assert np.array_equal(got[~np.isnan(got)], ref[~np.isnan(ref)])
    assert np.isnan(got[0x7F]) and np.isnan(got[0xFF]) and got[0x7E] == 448.0 and got[0x01] == 2.0**-9


def test_encode_matches_torch_on_randoms_grid_points_and_every_tie():
    g = np.random.default_rng(0)
    scales = 10.0 ** g.integers(-6, 3, 4000)
    vals = fp8.representable_values().astype(np.float64)
    ties = (vals[1:] + vals[:-1]) / 2
    x = np.concatenate([g.standard_normal(4000) * scales, vals, ties, [0.0, -0.0, 2.0**-10, -(2.0**-10), 2.0**-12]])
    x = np.clip(x, -448, 448).astype(np.float32)
    assert np.array_equal(fp8.encode(x), torch_fp8_codes(x))


def test_encode_beyond_the_range_matches_torch():
    # Not reachable through the clamped write path, but the codec agrees with torch past 448 too.
    x = np.array([449.0, 463.9, 464.0, 464.1, 479.0, 480.0, 1e6, -470.0, np.nan, -np.nan], dtype=np.float32)
    assert np.array_equal(fp8.encode(x), torch_fp8_codes(x))


def test_every_finite_code_round_trips():
    codes = np.arange(256, dtype=np.uint8)
    finite = np.isfinite(fp8.decode(codes))
    assert np.array_equal(fp8.encode(fp8.decode(codes[finite])), codes[finite])


def test_fp8_known_answers():
    gold = GOLDEN["fp8_e4m3fn"]
    assert len(fp8.representable_values()) == gold["finite_values"]
    assert fp8.representable_values().max() == gold["max_finite"]
    sat = gold["saturating_store"]
    codes = quant.fp8_per_head(np.array(sat["x"], dtype=np.float32).reshape(2, 1, 1), np.ones(1, np.float32))
    assert fp8.decode(codes).ravel().tolist() == sat["value"]


def test_fp8_per_head_uses_its_heads_scale():
    x = np.array([[[4.0, -2.0]], [[4.0, 1.0]]], dtype=np.float32).reshape(1, 2, 2)  # [1, Hkv=2, D=2]
    codes = quant.fp8_per_head(x, np.array([2.0, 0.5], dtype=np.float32))
    assert fp8.decode(codes).tolist() == [[[2.0, -1.0], [8.0, 2.0]]]


@pytest.mark.parametrize("case", GOLDEN["int8_per_token"])
def test_int8_known_answers(case):
    x = np.array(case["x"], dtype=np.float32)[None]
    codes, scale = quant.per_token(x, "int8")
    assert codes[0].tolist() == case["codes"]
    if "scale_approx" in case:
        assert scale[0, 0] == pytest.approx(case["scale_approx"], rel=1e-6)
    else:
        assert scale[0, 0] == np.float32(case["scale_exact_float32"]) and np.isfinite(scale).all()


def test_int8_error_is_half_a_step_and_rows_use_their_range():
    g = np.random.default_rng(1)
    x = (g.standard_normal((64, 128)) * 10.0 ** g.integers(-3, 3, (64, 1))).astype(np.float32)
    x[5] = 0.0
    codes, scale = quant.per_token(x, "int8")
    err = np.abs(codes.astype(np.float64) * scale - x)
    assert (err <= scale.astype(np.float64) / 2 * (1 + 1e-6) + 1e-30).all()
    nonzero = np.abs(x).max(-1) > 0
    assert (np.abs(codes[nonzero]).max(-1) == 127).all() and (codes[5] == 0).all()


def test_int8_matches_torch_float32_formula_bit_for_bit():
    # The float32 torch statement of kernels/reference.py:53-54 on torch's own CPU arithmetic.
    g = np.random.default_rng(2)
    x = (g.standard_normal((256, 128)) * 3).astype(np.float32)
    x[:, 7] *= 8.0
    t = torch.from_numpy(x)
    t_scale = (t.abs().amax(-1, keepdim=True) / 127.0).clamp(min=1e-12)
    t_codes = torch.clamp(torch.round(t / t_scale), -128, 127).to(torch.int8)
    codes, scale = quant.per_token(x, "int8")
    assert np.array_equal(codes, t_codes.numpy())
    assert np.array_equal(scale.view(np.uint32), t_scale.numpy().view(np.uint32))


def test_fp8_per_token_matches_the_w8a8_float32_formula():
    g = np.random.default_rng(3)
    x = (g.standard_normal((64, 128)) * 5).astype(np.float32)
    t = torch.from_numpy(x)
    t_scale = (t.abs().amax(-1, keepdim=True) / 448.0).clamp(min=1e-12)
    t_codes = (t / t_scale).clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8)
    codes, scale = quant.per_token(x, "fp8")
    assert np.array_equal(codes, t_codes.numpy()) and np.array_equal(scale, t_scale.numpy())
    # Fixed by the formula itself: each row's largest-magnitude element lands on ±448 (0x7E / 0xFE), and
    # nothing saturates past it.
    top = np.abs(x).argmax(-1)
    rows = np.arange(x.shape[0])
    expect = np.where(x[rows, top] > 0, 0x7E, 0xFE)
    assert np.array_equal(codes[rows, top], expect)
    assert np.all((codes & 0x7F) <= 0x7E)
