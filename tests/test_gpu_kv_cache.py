"""GPU: the paged quantized KV cache through an engine-like sequence of steps (per-sequence prefill, batched
decode, a 5-token speculative verify step), checking after every step, on every layer, that the stored codes
are the oracle's quantization of every row written so far (bit-exact) and that attention over them is the
oracle's (max-abs 2e-3 / rel 1e-2)."""

import numpy as np
import pytest
import torch

from bpt_amd.kv_cache import PagedQuantKVCache
from oracle import attention, paged, quant

pytestmark = pytest.mark.gpu
DEV = "cuda"
HQ, HKV, D, LAYERS = 16, 8, 128, 2
SCALE = D ** -0.5


def codes_np(t, fmt):
    if fmt == "fp8":
        return t.view(torch.uint8).cpu().numpy()
    if fmt == "int8":
        return t.cpu().numpy()
    return t.float().cpu().numpy()


class Shadow:
    """Every row written so far, per layer and sequence, in float32 (what the oracle quantizes)."""

    def __init__(self):
        self.k, self.v = {}, {}

    def write(self, layer, seq, start, k, v):  # k, v: [Hkv, Q, D] float32 numpy
        for store, x in ((self.k, k), (self.v, v)):
            rows = store.setdefault((layer, seq), {})
            for i in range(x.shape[1]):
                rows[start + i] = x[:, i]

    def rows(self, store, layer, seq, n):
        return np.stack([store[(layer, seq)][p] for p in range(n)])  # [n, Hkv, D]


def check_codes(cache, shadow, layer, seq, n, fmt):
    table = np.array(cache.tables[seq])
    for store, pool, sc in ((shadow.k, cache.k[layer], cache.k_scale[layer]), (shadow.v, cache.v[layer], cache.v_scale[layer])):
        x = shadow.rows(store, layer, seq, n)
        got = paged.gather_sequence(codes_np(pool, fmt), table, n)
        if fmt == "fp8":
            want = quant.fp8_per_head(x, sc.cpu().numpy())
            assert np.array_equal(got, want)
        elif fmt == "int8":
            want, s = quant.per_token(x, "int8")
            assert np.array_equal(got, want)
            got_s = paged.gather_sequence(sc.cpu().numpy(), table, n)
            assert np.array_equal(got_s.view(np.uint32), s[..., 0].view(np.uint32))  # oracle scales: [n, Hkv, 1]
        else:
            assert np.array_equal(got, torch.from_numpy(x).to(torch.bfloat16).float().numpy())


def check_attention(cache, layer, q, meta, out, fmt):
    want, _ = attention.paged_decode(
        q.transpose(1, 2).float().cpu().numpy(), codes_np(cache.k[layer], fmt), codes_np(cache.v[layer], fmt),
        meta.block_table.cpu().numpy(), meta.context_lens.cpu().numpy(),
        None if cache.k_scale[layer] is None else cache.k_scale[layer].cpu().numpy(),
        None if cache.v_scale[layer] is None else cache.v_scale[layer].cpu().numpy(), fmt, SCALE,
    )  # [B, Q, Hq, D]
    got = out.transpose(1, 2).float().cpu().numpy()
    err = np.abs(got - want)
    assert np.isfinite(got).all() and (err <= 2e-3 + 1e-2 * np.abs(want)).all(), f"worst {err.max():.3e}"


@pytest.mark.parametrize("fmt", ["fp8", "int8", "bf16"])
def test_prefill_decode_and_verify_steps(fmt):
    dtype = {"fp8": torch.float8_e4m3fn, "int8": torch.int8, "bf16": torch.bfloat16}[fmt]
    scales = {}
    if fmt == "fp8":
        scales = dict(k_scale=torch.full((LAYERS, HKV), 5.0 / 448), v_scale=torch.full((LAYERS, HKV), 4.0 / 448))
    cache = PagedQuantKVCache(num_layers=LAYERS, num_kv_heads=HKV, head_dim=D, num_blocks=64, block_size=16,
                              kv_dtype=dtype, device=DEV, **scales)
    g = torch.Generator(device=DEV).manual_seed(7)
    shadow = Shadow()
    length = {"a": 0, "b": 0, "c": 0}

    def step(rows, q_len):
        positions = torch.tensor([[length[s] + i for i in range(q_len)] for s in rows])
        for s in rows:
            cache.reserve(s, length[s] + q_len)
        meta = cache.prepare(rows, positions)
        for layer in range(LAYERS):
            q = torch.randn((len(rows), HQ, q_len, D), generator=g, device=DEV).to(torch.bfloat16)
            k = torch.randn((len(rows), HKV, q_len, D), generator=g, device=DEV).to(torch.bfloat16)
            v = torch.randn((len(rows), HKV, q_len, D), generator=g, device=DEV).to(torch.bfloat16)
            out = cache.attend(layer, q, k, v, meta, scale=SCALE)
            torch.cuda.synchronize()
            assert out.shape == q.shape and out.dtype == q.dtype
            for i, s in enumerate(rows):
                shadow.write(layer, s, length[s], k[i].float().cpu().numpy(), v[i].float().cpu().numpy())
                check_codes(cache, shadow, layer, s, length[s] + q_len, fmt)
            check_attention(cache, layer, q, meta, out, fmt)
        for s in rows:
            length[s] += q_len

    for s, n in (("a", 37), ("b", 5), ("c", 20)):  # prefill, one sequence at a time
        step([s], n)
    for _ in range(3):  # decode, batched, crossing block boundaries
        step(["c", "a", "b"], 1)
    step(["a", "b", "c"], 5)  # speculative verify: 1 accepted + 4 draft tokens, causal within the step
    cache.free("b")
    cache.reserve("d", 3)
    assert cache.tables["d"][0] in set(range(64))
