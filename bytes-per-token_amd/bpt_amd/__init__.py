"""bpt_amd — MI355X (gfx950) decode attention over quantized KV caches.

The decode hot path of fastserve (kernels/kv_attention.py, engine/kv_cache.py, integration/kv_cache.py),
re-implemented as hand-written HIP kernels behind a C ABI (include/bpt_amd.h, built into libbpt_amd.so)
with a thin PyTorch-ROCm host layer: paged FP8 / INT8 / BF16 pools (paged_attention, kv_cache) and
contiguous KIVI caches (kivi: fastserve's kernels/kv_attention.py call surface), and the fused RMSNorm +
per-token INT8 quantizer (norm_quant: kernels/norm_quant.py). Importing needs no GPU; the library loads on first use and raises if
it has not been built.
"""

from . import kivi
from .cascade import cascade_decode_attention
from .kv_cache import OutOfBlocksError, PagedMeta, PagedQuantKVCache
from .norm_quant import rms_norm_int8
from .paged_attention import (
    decode_kernel_name,
    decode_plan,
    kv_read_bytes,
    paged_append_decode,
    paged_decode_attention,
    paged_prepare,
    quantize_append,
)

__all__ = [
    "cascade_decode_attention",
    "OutOfBlocksError",
    "PagedMeta",
    "PagedQuantKVCache",
    "decode_kernel_name",
    "decode_plan",
    "kivi",
    "kv_read_bytes",
    "paged_append_decode",
    "paged_decode_attention",
    "paged_prepare",
    "quantize_append",
    "rms_norm_int8",
]
