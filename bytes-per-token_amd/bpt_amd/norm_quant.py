"""RMSNorm fused with per-token INT8 quantization on HIP: fastserve's kernel-1 call surface.

`rms_norm_int8(x, weight, eps, *, out=None, num_warps=4)` mirrors kernels/norm_quant.py:72-109 (paths
relative to fastserve's src/fastserve/): x [..., d] in bf16 / f16 / f32, weight [d]; returns (codes int8
[..., d], scale float32 [..., 1]) with y = x * rsqrt(mean(x^2) + eps) * weight, scale = max(max|y| / 127,
1e-12), codes = round_half_even(y / scale) (kernels/reference.py:44-55). Rows that are not contiguous are
copied first, as the reference does; `out` = (codes [rows, d], scale [rows]) reuses the caller's buffers.
`num_warps` is accepted for signature parity and ignored (one wave per row).
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from ._lib import F_BF16, F_F16, F_F32

_CODES = {torch.bfloat16: F_BF16, torch.float16: F_F16, torch.float32: F_F32}


def rms_norm_int8(
    x: torch.Tensor,
    weight: torch.Tensor,
    eps: float,
    *,
    out: tuple[torch.Tensor, torch.Tensor] | None = None,
    num_warps: int = 4,
) -> tuple[torch.Tensor, torch.Tensor]:
    del num_warps  # one wave per row
    d = x.shape[-1]
    if x.dtype not in _CODES or weight.dtype not in _CODES:
        raise ValueError(f"x and weight must be bfloat16, float16 or float32, got {x.dtype}, {weight.dtype}")
    if tuple(weight.shape) != (d,):
        raise ValueError(f"weight must be [{d}], got {tuple(weight.shape)}")
    if x.device.type != "cuda" or weight.device != x.device:
        raise ValueError("rms_norm_int8 runs on a GPU: x and weight must be cuda tensors on one device")
    rows = x.reshape(-1, d)
    if not rows.is_contiguous():
        rows = rows.contiguous()
    weight = weight.contiguous()
    n = rows.shape[0]
    if out is None:
        out = (
            torch.empty((n, d), dtype=torch.int8, device=x.device),
            torch.empty(n, dtype=torch.float32, device=x.device),
        )
    codes, scale = out
    if codes.dtype != torch.int8 or tuple(codes.shape) != (n, d) or codes.stride(-1) != 1:
        raise ValueError(f"out[0] must be int8 [{n}, {d}] with contiguous channels")
    if scale.dtype != torch.float32 or scale.numel() != n or not scale.is_contiguous():
        raise ValueError(f"out[1] must be a contiguous float32 tensor of {n} elements")
    a = _lib.NormQuantArgs()
    a.struct_size = ctypes.sizeof(_lib.NormQuantArgs)
    a.x_dtype, a.weight_dtype = _CODES[rows.dtype], _CODES[weight.dtype]
    a.rows, a.d, a.eps = n, d, float(eps)
    a.x, a.x_stride_row = rows.data_ptr(), rows.stride(0)
    a.weight = weight.data_ptr()
    a.codes, a.codes_stride_row = codes.data_ptr(), codes.stride(0)
    a.scale = scale.data_ptr()
    stream = torch.cuda.current_stream(x.device).cuda_stream
    _lib.check(_lib.lib().bpt_rms_norm_int8(ctypes.byref(a), ctypes.c_void_p(stream)))
    return codes.view(x.shape), scale.view(*x.shape[:-1], 1)
