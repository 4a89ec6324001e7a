"""Paged decode attention in float32 PyTorch on the CPU (oracle; test infrastructure and the timed CPU
baseline only — never the product path).

The same result as oracle.attention.paged_decode, computed the way fastserve's own CPU path computes it, so
that it can be timed as the CPU baseline beside the GPU kernel:
* gather each sequence's pages into a contiguous [B, Hkv, kv_len, D] view, kv_len the batch's longest
  context, short sequences padded with block 0 (engine/kv_cache.py:140-156 prepare, :165-169 _gather);
* dequantize: codes.float() * scale (kernels/reference.py:58-60 dequantize_int8; FP8 codes through torch's
  float8_e4m3fn cast), the scale per head or per (token, head), gathered like the codes;
* causal attention by absolute position over the padded view, GQA by repeating KV heads, softmax in float32
  (engine/attention.py:12-47);
* the log-sum-exp of each row, as kernels/reference.py:186-202 partial_attention returns it.
Pinned by tests/test_oracle_attention.py against oracle.attention.paged_decode on every cache format.
"""

from __future__ import annotations

import torch


def _gather(pool: torch.Tensor, table: torch.Tensor, kv_len: int) -> torch.Tensor:
    """engine/kv_cache.py:165-169: pool [NB, P, ...] through table [B, n] -> [B, kv_len, ...]."""
    b, n = table.shape
    blocks = pool[table]  # [B, n, P, ...]
    return blocks.reshape(b, n * pool.shape[1], *pool.shape[2:])[:, :kv_len]


def _dequantize(pool, scale, table, kv_len, kv_format):
    """[B, Hkv, kv_len, D] float32 keys or values of the batch."""
    codes = _gather(pool, table, kv_len)  # [B, T, Hkv, D]
    x = codes.float()
    if kv_format != "bf16":
        s = scale.float()
        x = x * (s[None, None, :, None] if s.dim() == 1 else _gather(s, table, kv_len)[..., None])
    return x.transpose(1, 2)


def paged_decode(q, k_pool, v_pool, block_table, context_lens, k_scale, v_scale, kv_format, scale):
    """q [B, Q, Hq, D] -> (out [B, Q, Hq, D], lse [B, Q, Hq]) float32 torch tensors on the CPU.

    Pools as stored (bfloat16, float8_e4m3fn or int8 [NB, P, Hkv, D]); scales [Hkv] or [NB, P, Hkv]. Query i of
    sequence b sits at position context_lens[b] - Q + i and sees slots 0 .. that position.
    """
    q = q.float()
    b, nq, hq, d = q.shape
    lens = context_lens.long()
    kv_len = int(lens.max()) if b else 0
    n_blocks = -(-kv_len // k_pool.shape[1])
    table = block_table[:, :n_blocks].long().clamp(0, k_pool.shape[0] - 1)
    k = _dequantize(k_pool, k_scale, table, kv_len, kv_format)
    v = _dequantize(v_pool, v_scale, table, kv_len, kv_format)
    group = hq // k.shape[1]
    k = k.repeat_interleave(group, dim=1)  # engine/attention.py:23-31: KV head h serves h*group .. +group-1
    v = v.repeat_interleave(group, dim=1)
    positions = lens[:, None] - nq + torch.arange(nq)[None, :]  # [B, Q]
    mask = (torch.arange(kv_len)[None, None, :] <= positions[:, :, None])[:, None]  # [B, 1, Q, T]
    scores = (q.transpose(1, 2) @ k.transpose(-2, -1)) * scale  # [B, Hq, Q, T]
    scores = scores.masked_fill(~mask, float("-inf"))
    lse = torch.logsumexp(scores, dim=-1)
    probs = torch.softmax(scores, dim=-1).nan_to_num(0.0)
    out = probs @ v  # [B, Hq, Q, D]
    return out.transpose(1, 2).contiguous(), lse.transpose(1, 2).contiguous()
