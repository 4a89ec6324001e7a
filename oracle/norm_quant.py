"""RMSNorm fused with per-token INT8 quantization, in float32 numpy (oracle; test infrastructure only).

Restates fastserve's kernel-1 definition (paths relative to src/fastserve/):
* rms_norm_int8    kernels/reference.py:44-55 (computed by kernels/norm_quant.py:43-69):
                     y = x * rsqrt(mean(x^2) + eps) * weight          float32 throughout
                     scale = max(max|y| / 127, 1e-12)                 one per token
                     codes = clamp(round_half_even(y / scale), -128, 127)
* dequantize_int8  kernels/reference.py:58-60: codes * scale in float32
"""

from __future__ import annotations

import numpy as np


def rms_norm_int8(x, weight, eps: float) -> tuple[np.ndarray, np.ndarray]:
    """(codes int8 [..., d], scale float32 [..., 1]) of x [..., d] (any float dtype, computed in float32)."""
    x32 = np.asarray(x, dtype=np.float32)
    w32 = np.asarray(weight, dtype=np.float32)
    ms = np.mean(x32 * x32, axis=-1, keepdims=True, dtype=np.float32)
    r = np.float32(1.0) / np.sqrt(ms + np.float32(eps), dtype=np.float32)
    y = (x32 * r) * w32
    scale = np.maximum(np.abs(y).max(axis=-1, keepdims=True) / np.float32(127.0), np.float32(1e-12)).astype(np.float32)
    codes = np.clip(np.round(y / scale), -128, 127).astype(np.int8)
    return codes, scale


def dequantize_int8(codes, scale) -> np.ndarray:
    return np.asarray(codes, dtype=np.float32) * np.asarray(scale, dtype=np.float32)
