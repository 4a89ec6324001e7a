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


def test_device_prepare_matches_the_paging_oracle():
    """bpt_paged_prepare from device positions gives fastserve's metadata (engine/kv_cache.py:140-156, the
    paging oracle): the tables are padded to the reserved blocks (a host-known bound), positions outside the
    reserved blocks get no write slot."""
    cache = PagedQuantKVCache(num_layers=1, num_kv_heads=HKV, head_dim=D, num_blocks=64, block_size=4,
                              kv_dtype=torch.int8, device=DEV)
    lengths = {"x": 9, "y": 1, "z": 17}
    for s, n in lengths.items():
        cache.reserve(s, n + 3)
    rows = ["z", "x", "y"]
    starts = [lengths[s] for s in rows]
    positions = torch.tensor([[p + i for i in range(3)] for p in starts])
    host = cache.prepare(rows, positions)
    dev = cache.prepare(rows, positions.to(DEV))
    wb, wo, bt, kv_len = paged.prepare([cache.tables[s] for s in rows], positions.numpy(), 4)
    assert host.kv_len == kv_len and dev.kv_len == max(len(cache.tables[s]) for s in rows) * 4 >= kv_len
    for meta in (host, dev):
        assert np.array_equal(meta.write_blocks.cpu().numpy(), wb)
        assert np.array_equal(meta.write_offsets.cpu().numpy(), wo)
        assert np.array_equal(meta.block_table.cpu().numpy()[:, : bt.shape[1]], bt)
        assert meta.context_lens.tolist() == [s + 3 for s in starts]
    tables = [cache.tables[s] for s in rows]
    pad = dev.block_table.cpu().numpy()
    for i, t in enumerate(tables):  # past a row's own blocks: block 0, as fastserve pads
        assert list(pad[i, : len(t)]) == t and (pad[i, len(t):] == 0).all()
    # A position past the reserved blocks: no write slot, length clamped to the reserved tokens.
    over = torch.tensor([[11]], device=DEV)  # "x" holds 12 reserved tokens in 3 blocks; 11 is the last slot
    cache.reserve("w", 4)
    meta = cache.prepare(["w"], torch.tensor([[9]], device=DEV))
    assert meta.write_blocks.item() == -1 and meta.context_lens.item() == 4
    meta = cache.prepare(["x"], over)
    assert meta.write_blocks.item() == cache.tables["x"][2] and meta.context_lens.item() == 12


def test_float32_model_gets_float32_attention():
    """q in float32 gets float32 output, rounded once from the kernel's float32 result (fastserve merges in
    float32 and casts once, integration/kv_cache.py:177-181), not a bfloat16 intermediate. On a bf16 cache
    (float32 value sums) the output is within 1e-4 relative of the oracle, far inside bfloat16's rounding."""
    cache = PagedQuantKVCache(num_layers=1, num_kv_heads=HKV, head_dim=D, num_blocks=48, block_size=16,
                              kv_dtype=torch.bfloat16, device=DEV)
    g = torch.Generator(device=DEV).manual_seed(3)
    cache.reserve("a", 300)
    cache.reserve("b", 300)
    pos = torch.tensor([[i for i in range(200)]] * 2)
    k = torch.randn((2, HKV, 200, D), generator=g, device=DEV)
    q = torch.randn((2, HQ, 200, D), generator=g, device=DEV)
    meta = cache.prepare(["a", "b"], pos)
    cache.attend(0, q.to(torch.bfloat16), k.to(torch.bfloat16), k.to(torch.bfloat16), meta, scale=SCALE)
    step = cache.prepare(["a", "b"], torch.tensor([[200], [200]]))
    qd = torch.randn((2, HQ, 1, D), generator=g, device=DEV)
    kd = torch.randn((2, HKV, 1, D), generator=g, device=DEV).to(torch.bfloat16).float()
    out = cache.attend(0, qd, kd, kd, step, scale=SCALE)
    torch.cuda.synchronize()
    assert out.dtype == torch.float32
    want, _ = attention.paged_decode(
        qd.transpose(1, 2).cpu().numpy(), codes_np(cache.k[0], "bf16"), codes_np(cache.v[0], "bf16"),
        step.block_table.cpu().numpy(), step.context_lens.cpu().numpy(), None, None, "bf16", SCALE)
    got = out.transpose(1, 2).cpu().numpy()
    np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-5)
    assert (out.to(torch.bfloat16).float() != out).any()  # not bfloat16 values


@pytest.mark.parametrize("fmt", ["fp8", "int8"])
def test_decode_steps_captured_in_a_hip_graph(fmt):
    """prepare (from device positions) plus attend for 2 layers, captured once in a HIP graph and replayed for
    four decode steps with new positions, queries, keys and values each time, eager work between replays; every
    replay's stored codes are the oracle's and its attention the oracle's."""
    dtype = {"fp8": torch.float8_e4m3fn, "int8": torch.int8}[fmt]
    scales = {}
    if fmt == "fp8":
        scales = dict(k_scale=torch.full((LAYERS, HKV), 5.0 / 448), v_scale=torch.full((LAYERS, HKV), 4.0 / 448))
    cache = PagedQuantKVCache(num_layers=LAYERS, num_kv_heads=HKV, head_dim=D, num_blocks=64, block_size=16,
                              kv_dtype=dtype, device=DEV, **scales)
    rows, prefill = ["a", "b", "c"], [37, 5, 20]
    shadow = Shadow()
    gen = torch.Generator(device=DEV).manual_seed(11)
    for s, n in zip(rows, prefill):
        cache.reserve(s, n + 8)  # room for the captured steps: no reserve() inside the graph
        pos = torch.arange(n)[None]
        meta = cache.prepare([s], pos)
        for layer in range(LAYERS):
            k = torch.randn((1, HKV, n, D), generator=gen, device=DEV).to(torch.bfloat16)
            v = torch.randn((1, HKV, n, D), generator=gen, device=DEV).to(torch.bfloat16)
            q = torch.randn((1, HQ, n, D), generator=gen, device=DEV).to(torch.bfloat16)
            cache.attend(layer, q, k, v, meta, scale=SCALE)
            shadow.write(layer, s, 0, k[0].float().cpu().numpy(), v[0].float().cpu().numpy())
    # Static inputs of the captured step.
    positions = torch.zeros((3, 1), dtype=torch.int64, device=DEV)
    qs = [torch.zeros((3, HQ, 1, D), dtype=torch.bfloat16, device=DEV) for _ in range(LAYERS)]
    ks = [torch.zeros((3, HKV, 1, D), dtype=torch.bfloat16, device=DEV) for _ in range(LAYERS)]
    vs = [torch.zeros((3, HKV, 1, D), dtype=torch.bfloat16, device=DEV) for _ in range(LAYERS)]
    side = torch.cuda.Stream()
    lengths = dict(zip(rows, prefill))

    def step():
        meta = cache.prepare(rows, positions)
        return meta, [cache.attend(layer, qs[layer], ks[layer], vs[layer], meta, scale=SCALE) for layer in range(LAYERS)]

    def set_inputs():
        positions.copy_(torch.tensor([[lengths[s]] for s in rows], device=DEV))
        for layer in range(LAYERS):
            qs[layer].copy_(torch.randn(qs[layer].shape, generator=gen, device=DEV).to(torch.bfloat16))
            ks[layer].copy_(torch.randn(ks[layer].shape, generator=gen, device=DEV).to(torch.bfloat16))
            vs[layer].copy_(torch.randn(vs[layer].shape, generator=gen, device=DEV).to(torch.bfloat16))

    def check_step(meta, outs):
        for layer in range(LAYERS):
            for i, s in enumerate(rows):
                shadow.write(layer, s, lengths[s], ks[layer][i].float().cpu().numpy(), vs[layer][i].float().cpu().numpy())
                check_codes(cache, shadow, layer, s, lengths[s] + 1, fmt)
            check_attention(cache, layer, qs[layer], meta, outs[layer], fmt)
        for s in rows:
            lengths[s] += 1

    # One eager step on the side stream (it also creates the cached workspaces there), then the capture.
    set_inputs()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        meta, outs = step()
    side.synchronize()
    check_step(meta, outs)
    graph = torch.cuda.CUDAGraph()
    set_inputs()  # the capture records the work; nothing runs until the first replay
    with torch.cuda.graph(graph, stream=side):
        meta, outs = step()
    for _ in range(4):
        graph.replay()
        torch.cuda.synchronize()
        check_step(meta, outs)
        torch.zeros(1 << 20, device=DEV).sum().item()  # eager work between replays
        set_inputs()


@pytest.mark.parametrize("nq", [1, 3])
def test_positions_past_the_reservation_store_nothing(nq):
    """Device positions that run past a row's reserved blocks (the host path would refuse them): the row gets no
    write slot and attends its reserved tokens, and the cache's one-launch attend (FP8, per-head scales) gives
    exactly what quantize_append then paged_decode_attention give on the same metadata."""
    from bpt_amd import paged_decode_attention, quantize_append

    cache = PagedQuantKVCache(num_layers=1, num_kv_heads=HKV, head_dim=D, num_blocks=32, block_size=4,
                              kv_dtype=torch.float8_e4m3fn, device=DEV,
                              k_scale=torch.full((1, HKV), 4.0 / 448), v_scale=torch.full((1, HKV), 4.0 / 448))
    g = torch.Generator(device=DEV).manual_seed(31)
    cache.reserve("a", 8)   # 2 blocks
    cache.reserve("b", 12)  # 3 blocks
    for i in range(cache.num_blocks):  # every slot holds codes already
        cache.k[0][i] = (torch.randn((4, HKV, D), generator=g, device=DEV)).to(torch.float8_e4m3fn)
        cache.v[0][i] = (torch.randn((4, HKV, D), generator=g, device=DEV)).to(torch.float8_e4m3fn)
    # "a": positions 7 .. 7 + nq - 1 run past its 8 reserved tokens (for nq > 1); "b": inside its reservation.
    positions = torch.tensor([[7 + i for i in range(nq)], [5 + i for i in range(nq)]], device=DEV)
    meta = cache.prepare(["a", "b"], positions)
    wb = meta.write_blocks.cpu()
    if nq > 1:
        assert (wb[0] == -1).all() and int(meta.context_lens[0]) == 8
    else:
        assert wb[0, 0] == cache.tables["a"][1] and int(meta.context_lens[0]) == 8
    assert (wb[1] >= 0).all() and int(meta.context_lens[1]) == 5 + nq
    q = torch.randn((2, HQ, nq, D), generator=g, device=DEV).to(torch.bfloat16)
    k = torch.randn((2, HKV, nq, D), generator=g, device=DEV).to(torch.bfloat16)
    v = torch.randn((2, HKV, nq, D), generator=g, device=DEV).to(torch.bfloat16)
    kc, vc = cache.k[0].clone(), cache.v[0].clone()
    quantize_append(k.transpose(1, 2), v.transpose(1, 2), kc, vc, cache.k_scale[0], cache.v_scale[0],
                    meta.write_blocks, meta.write_offsets)
    want = paged_decode_attention(q.transpose(1, 2), kc, vc, meta.block_table, meta.context_lens, cache.k_scale[0],
                                  cache.v_scale[0], scale=SCALE, max_context=meta.kv_len)
    got = cache.attend(0, q, k, v, meta, scale=SCALE)
    torch.cuda.synchronize()
    assert torch.equal(cache.k[0].view(torch.uint8), kc.view(torch.uint8))
    assert torch.equal(cache.v[0].view(torch.uint8), vc.view(torch.uint8))
    assert torch.equal(got.transpose(1, 2), want)
