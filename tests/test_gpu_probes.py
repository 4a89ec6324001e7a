"""GPU: the bandwidth probes read exactly the bytes they claim to.

Both probes fold every 16-byte load into a per-workgroup checksum (the XOR of the load's four words, summed
mod 2^32 over the workgroup, stored as float32). The host recomputes those checksums from the same bytes
and the probe's documented assignment of loads to workgroups, so a probe that skipped, repeated or misplaced
a load, or read past a sequence's length, fails here:
* read probe: 16-byte element i belongs to workgroup i // ceil(n / groups) (contiguous ranges);
* page-read probe: the decode's own split. Segments (sequence, row group of a KV head) of `chunk`-token
  chunks lie end to end, sequence-major; the launch's workgroups take equal contiguous ranges of that line,
  workgroup x the range at position line_index(x) (XCD-major numbering). A chunk is its tokens' K and V rows
  through the block table plus their per-token K / V scale words when the cache has them; tokens past a
  sequence's length are not counted.
"""

import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def xor16(words: np.ndarray) -> np.ndarray:
    """[..., 4] uint32 -> [...] XOR of the four words."""
    return words[..., 0] ^ words[..., 1] ^ words[..., 2] ^ words[..., 3]


def test_read_probe_checksums_every_element_once():
    from bpt_amd import measure

    probe = measure.ReadProbe(3 << 20, device="cuda:0")
    g = torch.Generator(device="cpu").manual_seed(5)
    host = torch.randint(0, 2**31 - 1, (probe.nbytes // 4,), generator=g, dtype=torch.int64).to(torch.int32)
    probe.buf.copy_(host.view(torch.float32))
    probe.run()
    torch.cuda.synchronize()
    words = host.numpy().view(np.uint32).reshape(-1, 4)
    x = xor16(words).astype(np.uint64)
    groups = probe.partial.numel()
    owner = np.arange(x.size) // -(-x.size // groups)
    want = np.zeros(groups, dtype=np.uint64)
    np.add.at(want, owner, x)
    want = (want % (1 << 32)).astype(np.uint32).astype(np.float32)
    got = probe.partial.cpu().numpy()
    assert np.array_equal(got, want)

    # The timed variant reads the same bytes.
    probe.partial.zero_()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    stop.record()
    torch.cuda.synchronize()
    probe.run(events=(start.cuda_event, stop.cuda_event))
    torch.cuda.synchronize()
    assert np.array_equal(probe.partial.cpu().numpy(), want)
    assert start.elapsed_time(stop) > 0


def line_index(n, x):
    """The decode's XCD-major numbering of workgroup x of n (decode_common.h line_index)."""
    q, r, k = n >> 3, n & 7, x & 7
    return k * q + min(k, r) + (x >> 3)


def page_checksums(w, groups):
    """Host checksums of the page-read probe over workload `w` ([groups] float32), from the decode's plan."""
    from bpt_amd.paged_attention import _plan

    a, _, _ = _plan(*w.args(), **{k: v for k, v in w.kwargs().items()})
    chunk, rows = a.chunk_tokens, a.num_queries * (a.num_q_heads // a.num_kv_heads)
    n_rg = -(-rows // a.rows_per_group)
    k = w.k_cache.contiguous().view(torch.uint8).cpu().numpy()
    v = w.v_cache.contiguous().view(torch.uint8).cpu().numpy()
    nb, page, hkv = k.shape[:3]
    hr_n = hkv * n_rg
    k = k.reshape(nb, page, hkv, -1, 16).view(np.uint32)  # [NB, P, Hkv, parts, 4]
    v = v.reshape(nb, page, hkv, -1, 16).view(np.uint32)
    table = w.block_table.cpu().numpy()
    cap = min(w.max_context, table.shape[1] * page)
    lens = np.clip(w.context_lens.cpu().numpy().astype(np.int64), 0, cap)
    per_token = w.k_scale is not None and w.k_scale.dim() == 3
    if per_token:
        ks = w.k_scale.cpu().numpy().view(np.uint32)
        vs = w.v_scale.cpu().numpy().view(np.uint32)
    nchunks = -(-lens // chunk)
    prefix = np.concatenate([[0], np.cumsum(nchunks)])
    total = hr_n * int(prefix[-1])
    per = -(-total // groups)
    start_of = {line_index(groups, x): x for x in range(groups)}
    out = np.zeros(groups, dtype=np.uint64)
    for b, n in enumerate(lens):
        t = np.arange(int(n))
        e = np.clip(table[b, t // page], 0, nb - 1)
        o = t % page
        for hr in range(hr_n):
            h = hr // n_rg
            per_tok = (xor16(k[e, o, h]).astype(np.uint64) + xor16(v[e, o, h]).astype(np.uint64)).sum(axis=1)
            if per_token:
                per_tok = per_tok + (ks[e, o, h] ^ vs[e, o, h]).astype(np.uint64)
            c = hr_n * int(prefix[b]) + hr * int(nchunks[b]) + t // chunk  # each token's chunk on the line
            np.add.at(out, np.array([start_of[g] for g in c // per]), per_tok)
    return (out % (1 << 32)).astype(np.uint32).astype(np.float32)


@pytest.mark.parametrize("name", ["qwen3-1.7b-fp8", "qwen3-1.7b-int8", "qwen3-0.6b-bf16"])
def test_page_read_probe_reads_the_calls_pages(name):
    from bpt_amd import measure, workloads

    w = workloads.make(name, device="cuda:0", seed=1, batch=3, length_cap=1500)
    probe = measure.PageReadProbe(*w.args(), **w.kwargs())
    probe.run()
    torch.cuda.synchronize()
    got = probe.partial.cpu().numpy()
    want = page_checksums(w, got.size)
    assert got.shape == want.shape
    assert np.array_equal(got, want)


def test_page_read_probe_query_and_events():
    from bpt_amd import _lib, measure, workloads

    w = workloads.make("qwen3-1.7b-fp8", device="cuda:0", seed=2, batch=2, length_cap=600)
    probe = measure.PageReadProbe(*w.args(), **w.kwargs())
    groups = ctypes.c_int64(0)
    _lib.check(_lib.lib().bpt_page_read_probe(ctypes.byref(probe.args), None, ctypes.byref(groups), None, None, None))
    assert groups.value == probe.partial.numel()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    stop.record()
    torch.cuda.synchronize()
    probe.run(events=(start.cuda_event, stop.cuda_event))
    torch.cuda.synchronize()
    assert np.array_equal(probe.partial.cpu().numpy(), page_checksums(w, groups.value))
    assert start.elapsed_time(stop) > 0
    with pytest.raises(ValueError, match="both events or neither"):
        _lib.check(_lib.lib().bpt_page_read_probe(ctypes.byref(probe.args), probe.partial.data_ptr(), None, None,
                                                  ctypes.c_void_p(start.cuda_event), None))
