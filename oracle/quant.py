"""The write-path quantizers in float32 numpy (oracle; test infrastructure only).

Every operation is a single IEEE float32 operation (division correctly rounded, np.rint ties to even),
matching the float32 torch formulas they restate bit for bit.
"""

from __future__ import annotations

import numpy as np

from . import fp8

INT8_MAX = np.float32(127.0)
FP8_MAX = np.float32(448.0)
MIN_SCALE = np.float32(1e-12)  # torch clamp(min=1e-12) on a float32 tensor uses float32(1e-12)


def fp8_per_head(x: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """x [..., Hkv, D] with static per-head scales [Hkv] -> e4m3fn codes.

    kv/quant.py:44-45: `x.clamp(-448, 448).to(torch.float8_e4m3fn)` applied to x / scale.
    """
    x = np.asarray(x, dtype=np.float32)
    y = x / np.asarray(scale, dtype=np.float32)[:, None]
    return fp8.encode(np.clip(y, -FP8_MAX, FP8_MAX))


def per_token(x: np.ndarray, fmt: str) -> tuple[np.ndarray, np.ndarray]:
    """Per-token (last axis) dynamic quantization: (codes, scale [..., 1] float32).

    quant/w8a8.py:55-74 and kernels/reference.py:53-54:
        scale = clamp(amax / QMAX, min=1e-12)    QMAX = 127 (int8) or 448 (fp8)
        int8: codes = clamp(round(x / scale), -128, 127)      round half to even
        fp8:  codes = e4m3fn(clamp(x / scale, ±448))
    """
    x = np.asarray(x, dtype=np.float32)
    amax = np.max(np.abs(x), axis=-1, keepdims=True)
    if fmt == "int8":
        scale = np.maximum(amax / INT8_MAX, MIN_SCALE).astype(np.float32)
        codes = np.clip(np.rint(x / scale), -128, 127).astype(np.int8)
        return codes, scale
    if fmt == "fp8":
        scale = np.maximum(amax / FP8_MAX, MIN_SCALE).astype(np.float32)
        return fp8.encode(np.clip(x / scale, -FP8_MAX, FP8_MAX)), scale
    raise ValueError(f"fmt must be 'int8' or 'fp8', got {fmt!r}")


def int8_per_head(x: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """x [..., Hkv, D] with static per-head scales [Hkv] -> int8 codes: clamp(round(x / s), -128, 127)."""
    x = np.asarray(x, dtype=np.float32)
    y = x / np.asarray(scale, dtype=np.float32)[:, None]
    return np.clip(np.rint(y), -128, 127).astype(np.int8)


def dequantize(codes: np.ndarray, kv_format: str, scale) -> np.ndarray:
    """Codes -> float32: FP8 decode(code) * scale; INT8 code * scale; bf16/float values pass through."""
    if kv_format == "fp8":
        return fp8.decode(codes) * np.asarray(scale, dtype=np.float32)
    if kv_format == "int8":
        return np.asarray(codes, dtype=np.float32) * np.asarray(scale, dtype=np.float32)
    return np.asarray(codes, dtype=np.float32)


def per_head_scale(x: np.ndarray, qmax: float) -> np.ndarray:
    """Static per-(layer, kv-head) scale amax / qmax over everything of that head: x [..., Hkv, D] -> [Hkv]."""
    x = np.asarray(x, dtype=np.float32)
    amax = np.max(np.abs(x.reshape(-1, x.shape[-2], x.shape[-1])), axis=(0, 2))
    return np.maximum(amax / np.float32(qmax), MIN_SCALE).astype(np.float32)
