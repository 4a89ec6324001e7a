#!/usr/bin/env python
"""FP8-KV paged decode attention on one MI355X: KV-read HBM GB/s (% of peak) and µs/call.

One step = one paged decode-attention call (one kernel launch, split-K combined inside) over the Qwen3-1.7B-shaped
FP8 workload (32 sequences, ragged contexts U[256, 4096], pages scattered over a 2x pool), with inputs
resident in HBM and the L2 / Infinity Cache evicted by a 1 GiB streaming read before every call (outside
the timed events). `value` = algorithmic KV bytes read per call / mean event-timed call duration.

Also reported: the dominant kernel's roofline (HBM-bound; algorithmic bytes / its event-timed duration
against 8 TB/s); two read floors timed the same way after the same flush: a contiguous streaming read of
exactly the call's KV bytes (read_floor_us) and a read of exactly the call's pages through its block table
with no attention math (page_read_floor_us); the CPU baseline, the PyTorch float32 restatement of
fastserve's CPU path (padded gather + attention, torch.set_num_threads) on the host cores over a bounded
sample of every workload; µs/call + GB/s for all five measured shapes; the KIVI (contiguous 4/8/16-bit
cache) decode over fastserve's whole kernel-2 sweep and its quantize-on-write at that benchmark's cache
shapes; one 28-layer decode step through the paged cache object (device prepare, then write + decode per
layer), eager and replayed from a graph; and the fused RMSNorm + INT8 quantizer at the shapes of the
kernel-1 benchmark. Prints ONE JSON line.
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT, ROOT / "bytes-per-token_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

METRIC = "KV-read HBM GB/s (% of peak) + µs/call, FP8-KV paged decode attention"
PEAK_GBPS = 8000.0
PROFILES = ROOT / "profiles"


def profiled_traffic(kernel: str, workload: str) -> dict | None:
    """HBM bytes per launch of `kernel` from the committed rocprofv3 counter summary of this workload, if any.

    The summary holds FETCH_SIZE and WRITE_SIZE per dispatch (two --pmc runs of `bench.py --profile`), each
    already scaled by what the counter reads for a copy kernel of known size, as a line
    `traffic_bytes_per_launch: N`.
    """
    path = PROFILES / f"{kernel}_{workload}.md"
    if not path.exists():
        return None
    import re

    m = re.search(r"^traffic_bytes_per_launch:\s*(\d+)", path.read_text(), flags=re.M)
    return {"bytes": int(m.group(1)), "source": f"profiles/{path.name}"} if m else None


def append_call(w):
    """The decode step's quantize-on-write on workload `w`: one new bf16 K/V row per sequence and KV head,
    written into slot 15 of the sequence's last page. Returns (call, {"read": bytes, "written": bytes})."""
    import torch

    from bpt_amd import quantize_append

    b, hkv = w.shape.batch, w.shape.kv_heads
    g = torch.Generator(device="cuda:0").manual_seed(5)
    k_new = torch.randn((b, 1, hkv, 128), generator=g, device="cuda:0").to(torch.bfloat16)
    v_new = torch.randn((b, 1, hkv, 128), generator=g, device="cuda:0").to(torch.bfloat16)
    last = torch.tensor([row[-1] for row in w.extra["tables"]], dtype=torch.int32, device="cuda:0").view(b, 1)
    offs = torch.full((b, 1), 15, dtype=torch.int32, device="cuda:0")

    def write():
        quantize_append(k_new, v_new, w.k_cache, w.v_cache, w.k_scale, w.v_scale, last, offs)

    scale_bytes = 4 if w.k_scale is not None and w.k_scale.dim() == 3 else 0
    return write, {"read": b * hkv * 128 * 2 * 2, "written": b * hkv * (128 + scale_bytes) * 2}


def fused_call(w, out):
    """The workload's decode call as the cache's store-then-attend (paged_append_decode): new bf16 rows for
    the last token of every sequence, written to its slot and attended in the same launch."""
    import torch

    from bpt_amd import paged_append_decode

    b, hkv, page = w.shape.batch, w.shape.kv_heads, w.k_cache.shape[1]
    g = torch.Generator(device="cuda:0").manual_seed(6)
    k_new = torch.randn((b, 1, hkv, 128), generator=g, device="cuda:0").to(torch.bfloat16)
    v_new = torch.randn((b, 1, hkv, 128), generator=g, device="cuda:0").to(torch.bfloat16)
    pos = w.context_lens.long()[:, None] - 1
    blocks = torch.gather(w.block_table.long(), 1, pos // page).to(torch.int32)
    offsets = (pos % page).to(torch.int32)
    pargs, kw = w.args(), w.kwargs()

    def call():
        paged_append_decode(pargs[0], k_new, v_new, *pargs[1:7], blocks, offsets, out=out, **kw)

    return call


def profile_pass(args) -> int:
    """A short run for rocprofv3: cold decode calls on the workload, then three 256 MiB copies.

    The copies calibrate the FETCH_SIZE / WRITE_SIZE counters (each reads a known number of bytes).
    """
    import torch

    from bpt_amd import measure, paged_decode_attention, workloads

    torch.cuda.set_device(0)
    flush = measure.ReadProbe(args.flush_bytes)
    if args.workload.startswith("norm-int8-"):  # norm-int8-<rows>x<d>
        from bpt_amd import rms_norm_int8

        rows, d = (int(x) for x in args.workload.split("-")[2].split("x"))
        gen = torch.Generator(device="cuda:0").manual_seed(d)
        weight = (torch.randn(d, generator=gen, device="cuda:0").abs() + 0.5).to(torch.bfloat16)
        x = (torch.randn((rows, d), generator=gen, device="cuda:0") * 3).to(torch.bfloat16)
        out = (torch.empty((rows, d), dtype=torch.int8, device="cuda:0"),
               torch.empty(rows, dtype=torch.float32, device="cuda:0"))
        for _ in range(args.warmup + args.steps):
            flush.run()
            rms_norm_int8(x, weight, 1e-6, out=out)
        nbytes = rows * (3 * d + 4)
    elif args.workload.startswith("kivi-quantize-"):  # kivi-quantize-<int4|int8>-<batch>x<tokens>
        from bpt_amd import kivi

        fmt, shape = args.workload.split("-")[2:]
        batch, tokens = (int(x) for x in shape.split("x"))
        bits = {"int4": 4, "int8": 8}[fmt]
        cache = workloads.make_kivi(batch, tokens, bits, device="cuda:0", seed=batch + tokens)
        gen = torch.Generator(device="cuda:0").manual_seed(tokens)
        k = torch.randn((batch, 8, tokens, workloads.HEAD_DIM), generator=gen, device="cuda:0").to(torch.bfloat16)
        v = torch.randn_like(k)
        for _ in range(args.warmup + args.steps):
            flush.run()
            kivi.quantize_kv_into(k, v, cache, 0)
        d = workloads.HEAD_DIM
        nbytes = batch * 8 * tokens * (2 * d * 2 + 2 * d * bits // 8 + 4) + batch * 8 * (tokens // 32) * d * 4
    elif args.workload.startswith("kivi-"):  # kivi-<int4|int8|bf16>-<batch>x<context>
        from bpt_amd import kivi

        fmt, shape = args.workload.split("-")[1:]
        batch, context = (int(x) for x in shape.split("x"))
        w = workloads.make_kivi(batch, context, {"int4": 4, "int8": 8, "bf16": 16}[fmt], device="cuda:0",
                                seed=batch + context)
        for _ in range(args.warmup + args.steps):
            flush.run()
            kivi.attend(w.q, w, w.lengths, workloads.HEAD_DIM**-0.5, tokens=context)
        nbytes = w.cache_bytes()
    else:
        w = workloads.make(args.workload, device="cuda:0", seed=0)
        out = torch.empty(tuple(w.q.shape), dtype=torch.bfloat16, device="cuda:0")
        pargs, kw = w.args(), w.kwargs()
        if args.cascade:
            from bpt_amd import cascade_decode_attention

            kw = {**kw, "prefix_pages": w.shape.shared_prefix_pages}
        write = append_call(w)[0] if args.append else (fused_call(w, out) if args.fused else None)
        for _ in range(args.warmup + args.steps):
            flush.run()
            if write is not None:
                write()
            elif args.cascade:
                cascade_decode_attention(*pargs, **kw, out=out)
            else:
                paged_decode_attention(*pargs, **kw, out=out)
        nbytes = w.kv_bytes()
    torch.cuda.synchronize()
    src = torch.ones(64 << 20, dtype=torch.float32, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(3):
        measure.copy_probe(dst, src, src.numel() * 4)
    torch.cuda.synchronize()
    log(f"profile pass: {args.warmup + args.steps} decode calls ({nbytes} KV bytes each), "
        f"3 copies of {src.numel() * 4} bytes")
    return 0


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def timed_calls(call, flush, steps: int, warmup: int, call_ev=None):
    """Warmup, then `steps` cold calls: (ms per call from HIP events, wall seconds of the timed region).

    Each call is one kernel launch. With `call_ev` (a decode call taking two raw hipEvent_t handles), the
    launch itself records the events around its kernel (bpt_paged_decode_timed), which is the kernel's
    duration as rocprofv3 reports it; otherwise events recorded on the stream bracket the call and add a few
    microseconds of their own.
    """
    import torch

    for _ in range(warmup):
        call()
    torch.cuda.synchronize()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    if call_ev is not None:
        for e in starts + ends:  # torch creates an event on its first record
            e.record()
        if not all(e.cuda_event for e in starts + ends):
            call_ev = None
    torch.cuda.synchronize()  # barrier: one rank, so the synchronize is the barrier
    t0 = time.perf_counter()
    for i in range(steps):
        flush.run()
        if call_ev is not None:
            call_ev(starts[i].cuda_event, ends[i].cuda_event)
        else:
            starts[i].record()
            call()
            ends[i].record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return [s.elapsed_time(e) for s, e in zip(starts, ends)], wall


def read_floors(w, flush, iters: int, warmup: int) -> dict:
    """The two read floors of workload `w`'s decode call, each the median of `iters` cold launches timed by
    events recorded around the kernel (as the decode call is): a streaming read of exactly the call's KV
    bytes, and a read of exactly its pages (K / V rows and per-token scales) through its block table."""
    import torch

    from bpt_amd import measure

    nbytes = w.kv_bytes()
    contiguous = measure.ReadProbe(nbytes, device="cuda:0")
    pages = measure.PageReadProbe(*w.args(), **w.kwargs())
    out = {}
    for key, probe in (("read_floor_us", contiguous), ("page_read_floor_us", pages)):
        total, _ = timed_calls(probe.run, flush, iters, warmup, lambda s, e, p=probe: p.run(events=(s, e)))
        out[key] = round(statistics.median(total) * 1e3, 2)
    del contiguous, pages
    torch.cuda.empty_cache()
    return out


def measure_workload(name: str, flush, iters: int, warmup: int) -> dict:
    import torch

    from bpt_amd import measure, paged_decode_attention, workloads

    w = workloads.make(name, device="cuda:0", seed=0)
    out = torch.empty(tuple(w.q.shape), dtype=torch.bfloat16, device="cuda:0")
    args, kw = w.args(), w.kwargs()

    def call():
        paged_decode_attention(*args, **kw, out=out)

    def call_ev(start, stop):
        paged_decode_attention(*args, **kw, out=out, _events=(start, stop))

    total, _ = timed_calls(call, flush, iters, warmup, call_ev)
    graph = measure.graph_time_ms(call, calls=10, warmup=2, iters=10)
    nbytes = w.kv_bytes()
    med = statistics.median(total)
    row = {
        "us_per_call": round(med * 1e3, 2),
        "graph_warm_us_per_call": round(statistics.median(graph) * 1e3, 2),
        "kv_bytes": nbytes,
        "gbps": round(nbytes / (med * 1e-3) / 1e9, 1),
        "pct_of_peak": round(100 * nbytes / (med * 1e-3) / 1e9 / PEAK_GBPS, 1),
        "batch": w.shape.batch,
        "queries": w.shape.queries,
        "q_heads": w.shape.q_heads,
        "kv_heads": w.shape.kv_heads,
        "kv_format": w.shape.kv_format,
        "scales": w.shape.scales,
        "sum_context": sum(w.lengths),
    }
    row.update(read_floors(w, flush, iters, warmup))
    row["pct_of_read_floor"] = round(100 * row["read_floor_us"] / row["us_per_call"], 1)
    row["pct_of_page_read_floor"] = round(100 * row["page_read_floor_us"] / row["us_per_call"], 1)
    if w.unique_tokens != sum(w.lengths):
        ub = w.kv_bytes(unique=True)
        row["unique_kv_bytes"] = ub
        row["unique_gbps"] = round(ub / (med * 1e-3) / 1e9, 1)
        # The shared-prefix cascade over the same inputs: the prefix read once per 16 query rows of the
        # group, each sequence's own pages once, the two merged (two launches).
        from bpt_amd import cascade_decode_attention

        def cascade():
            cascade_decode_attention(*args, **kw, prefix_pages=w.shape.shared_prefix_pages, out=out)

        ctot, _ = timed_calls(cascade, flush, iters, warmup)
        cmed = statistics.median(ctot)
        row["cascade"] = {
            "us_per_call": round(cmed * 1e3, 2),
            "graph_warm_us_per_call": round(statistics.median(measure.graph_time_ms(cascade, calls=10, warmup=2, iters=10)) * 1e3, 2),
            "unique_gbps": round(ub / (cmed * 1e-3) / 1e9, 1),
            "logical_gbps": round(nbytes / (cmed * 1e-3) / 1e9, 1),
        }
    log(f"{name}: {row['us_per_call']} us/call, {row['gbps']} GB/s ({row['pct_of_peak']}% of 8 TB/s); read floors "
        f"{row['read_floor_us']} us contiguous, {row['page_read_floor_us']} us through its pages"
        + (f"; unique {row['unique_gbps']} GB/s" if "unique_gbps" in row else ""))
    if name == "qwen3-1.7b-int8":
        write, row["append_bytes"] = append_call(w)
        wt, _ = timed_calls(write, flush, iters, warmup)
        wg = measure.graph_time_ms(write, calls=20, warmup=2, iters=10)
        row["append_us_per_call"] = round(statistics.median(wt) * 1e3, 2)
        row["append_graph_us_per_call"] = round(statistics.median(wg) * 1e3, 2)
    del w, out
    torch.cuda.empty_cache()
    return row


def measure_kivi(flush, iters: int, warmup: int) -> dict:
    """µs/call and GB/s of KIVI decode attention (attend: one launch, splits combined inside) at the shapes
    and bit widths of fastserve's kernel-2 benchmark, cold caches, `tokens` known to the caller."""
    import torch

    from bpt_amd import kivi, workloads

    table = {}
    for batch, context in workloads.KIVI_SHAPES:
        for bits in workloads.KIVI_BITS:
            name = workloads.kivi_name(batch, context, bits)
            w = workloads.make_kivi(batch, context, bits, device="cuda:0", seed=batch + context)
            scale = workloads.HEAD_DIM**-0.5

            def call():
                kivi.attend(w.q, w, w.lengths, scale, tokens=context)

            total, _ = timed_calls(call, flush, iters, warmup)
            ms = statistics.fmean(total)
            nbytes = w.cache_bytes()
            table[name] = {
                "us_per_call": round(ms * 1e3, 2),
                "gbps": round(nbytes / (ms * 1e-3) / 1e9, 1),
                "pct_of_peak": round(100 * nbytes / (ms * 1e-3) / 1e9 / PEAK_GBPS, 1),
                "cache_bytes": nbytes,
                "split": kivi.default_split(batch, 8, context),
            }
            log(f"{name}: {table[name]['us_per_call']} us, {table[name]['gbps']} GB/s")
            del w
            torch.cuda.empty_cache()
    return table


def measure_kivi_quantize(flush, iters: int, warmup: int) -> dict:
    """The KIVI write path (kivi.quantize_kv_into -> bpt_kivi_quantize) at the kernel-2 benchmark's cache
    shapes: one 32-token key group of new bf16 keys and values per sequence and KV head quantized into the
    cache (what QuantizedKVCache._append does once every 32 decode steps), and the whole context at once (a
    prefill). GB/s counts the bf16 read plus the codes and grids written."""
    import ctypes

    import torch

    from bpt_amd import _lib, kivi, workloads

    table = {}
    for batch, context in ((1, 32768), (64, 8192)):
        for bits in (4, 8):
            cache = workloads.make_kivi(batch, context, bits, device="cuda:0", seed=batch + context)
            for tokens in (32, context):
                gen = torch.Generator(device="cuda:0").manual_seed(tokens)
                k = torch.randn((batch, 8, tokens, workloads.HEAD_DIM), generator=gen, device="cuda:0").to(torch.bfloat16)
                v = torch.randn_like(k)
                args = kivi.quantize_args(k, v, cache, context - tokens)
                stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

                def call():  # the launch alone: the checks in quantize_kv_into cost tens of microseconds of host time
                    _lib.check(_lib.lib().bpt_kivi_quantize(ctypes.byref(args), stream))

                total, _ = timed_calls(call, flush, iters, warmup)
                ms = statistics.fmean(total)
                d = workloads.HEAD_DIM
                moved = batch * 8 * tokens * (2 * d * 2 + 2 * d * bits // 8) + batch * 8 * (tokens // 32) * d * 4 \
                    + batch * 8 * tokens * 4  # bf16 in; codes; key grids (scale + zero per channel per group); value grids
                name = f"kivi-quantize-int{bits}-{batch}x{tokens}"
                table[name] = {
                    "us_per_call": round(ms * 1e3, 2),
                    "gbps": round(moved / (ms * 1e-3) / 1e9, 1),
                    "bytes_moved": moved,
                }
                log(f"{name}: {table[name]['us_per_call']} us, {table[name]['gbps']} GB/s")
                del k, v
            del cache
            torch.cuda.empty_cache()
    return table


def measure_decode_step(iters: int, warmup: int, layers: int = 28) -> dict:
    """One decode step of a 28-layer Qwen3-1.7B through the paged cache object (engine/kv_cache.py's role):
    `PagedQuantKVCache.prepare` from device positions (block tables, write slots and lengths built on the
    device), then per layer `attend` = the new token's quantize-on-write and the decode call, one launch
    (paged_append_decode: the matrix-core kernel stores the token's codes and uses them in place). FP8 codes with
    per-head scales and the headline workload's 32 ragged lengths; the pools hold random codes (the step reads
    them, not their values). Timed eager (29 launches from Python) and replayed from a HIP graph;
    GB/s counts the KV bytes the step's decode calls read. The step's 4.8 GB exceeds every cache, so no
    flush is needed between steps."""
    import torch

    from bpt_amd import measure, workloads
    from bpt_amd.kv_cache import PagedQuantKVCache

    lens = workloads.make("qwen3-1.7b-fp8", device="cuda:0", seed=0).context_lens.cpu().tolist()
    torch.cuda.empty_cache()
    b, hq, hkv, d, page = len(lens), 16, 8, workloads.HEAD_DIM, 16
    gen = torch.Generator(device="cuda:0").manual_seed(3)
    scales = [torch.rand((layers, hkv), generator=gen, device="cuda:0").cpu() * 4 / 448 + 1 / 448 for _ in range(2)]
    cache = PagedQuantKVCache(num_layers=layers, num_kv_heads=hkv, head_dim=d, block_size=page,
                              num_blocks=sum(-(-n // page) for n in lens) + 8, kv_dtype=torch.float8_e4m3fn,
                              device="cuda:0", k_scale=scales[0], v_scale=scales[1], max_seqs=b)
    rows = list(range(b))
    for r, n in zip(rows, lens):
        cache.reserve(r, n)
    for pool in cache.k + cache.v:  # finite e4m3fn codes: 0x00 .. 0x7e with either sign
        codes = torch.randint(0, 0x7F, pool.shape, generator=gen, device="cuda:0", dtype=torch.uint8)
        codes |= torch.randint(0, 2, pool.shape, generator=gen, device="cuda:0", dtype=torch.uint8) << 7
        pool.view(torch.uint8).copy_(codes)
        del codes
    positions = torch.tensor([[n - 1] for n in lens], dtype=torch.int64, device="cuda:0")
    q = torch.randn((b, hq, 1, d), generator=gen, device="cuda:0").to(torch.bfloat16)
    k = torch.randn((b, hkv, 1, d), generator=gen, device="cuda:0").to(torch.bfloat16)
    v = torch.randn((b, hkv, 1, d), generator=gen, device="cuda:0").to(torch.bfloat16)

    def step():
        meta = cache.prepare(rows, positions)
        for layer in range(layers):
            cache.attend(layer, q, k, v, meta, scale=d**-0.5)

    eager = measure.event_times_ms(step, warmup=warmup, iters=iters)
    graph = measure.graph_time_ms(step, calls=4, warmup=2, iters=iters)
    kv = layers * sum(lens) * hkv * d * 2
    us_eager, us_graph = statistics.median(eager) * 1e3, statistics.median(graph) * 1e3
    row = {
        "layers": layers,
        "batch": b,
        "kv_format": "fp8 e4m3fn, per-head scales",
        "kv_bytes_per_step": kv,
        "us_per_step_eager": round(us_eager, 1),
        "us_per_step_graph": round(us_graph, 1),
        "gbps_graph": round(kv / (us_graph * 1e-6) / 1e9, 1),
        "launches_per_step": 1 + layers,
    }
    log(f"decode-step {layers} layers: {row['us_per_step_eager']} us eager, {row['us_per_step_graph']} us in a graph, "
        f"{row['gbps_graph']} GB/s")
    del cache
    torch.cuda.empty_cache()
    return row


def measure_norm_quant(flush, iters: int, warmup: int) -> dict:
    """RMSNorm + per-token INT8 at the shapes of fastserve's kernel-1 benchmark (bf16, d = 1024 / 2048,
    1 .. 32768 rows): cold µs/call and GB/s of the bytes it must move (2d read + d + 4 written per row),
    and µs/call replayed from a graph (the launch-bound decode sizes)."""
    import torch

    from bpt_amd import measure, rms_norm_int8

    table = {}
    for d in (1024, 2048):
        gen = torch.Generator(device="cuda:0").manual_seed(d)
        weight = (torch.randn(d, generator=gen, device="cuda:0").abs() + 0.5).to(torch.bfloat16)
        for rows in (1, 16, 256, 4096, 32768):
            x = (torch.randn((rows, d), generator=gen, device="cuda:0") * 3).to(torch.bfloat16)
            out = (torch.empty((rows, d), dtype=torch.int8, device="cuda:0"),
                   torch.empty(rows, dtype=torch.float32, device="cuda:0"))

            def call():
                rms_norm_int8(x, weight, 1e-6, out=out)

            total, _ = timed_calls(call, flush, iters, warmup)
            graph = measure.graph_time_ms(call, calls=20, warmup=2, iters=10)
            ms = statistics.fmean(total)
            moved = rows * (2 * d + d + 4)
            name = f"norm-int8-{rows}x{d}"
            table[name] = {
                "us_per_call": round(ms * 1e3, 2),
                "us_per_call_graph": round(statistics.median(graph) * 1e3, 2),
                "gbps": round(moved / (ms * 1e-3) / 1e9, 1),
                "bytes_moved": moved,
            }
            log(f"{name}: {table[name]['us_per_call']} us cold, {table[name]['us_per_call_graph']} us in a graph, "
                f"{table[name]['gbps']} GB/s")
    return table


TUNE_PAGED = {  # workload -> batch / length cap (None: the full workload)
    "qwen3-1.7b-fp8": [(None, None), (1, 2943), (4, None)],
    "qwen3-1.7b-int8": [(None, None), (1, None), (16, 2048)],
    "qwen3-8b-fp8-long": [(None, None)],
    "qwen3-1.7b-verify": [(None, None), (2, None)],
    "qwen3-0.6b-bf16": [(None, None)],
}
TUNE_KIVI_SHAPES = [(1, 32768), (1, 2048), (16, 2048), (64, 8192)]  # fastserve benchmarks/configs/m7_kernels.yaml:33-38
TUNE_KIVI_SPLITS = [32, 64, 128, 256, 512, 1024, 2048, 4096, 8192]


def tune(args) -> int:
    """Sweep the decode plans' knobs (bpt_set_tuning: workgroups per CU, the per-segment charge, the fewest
    chunks per workgroup) on the paged workloads and the KIVI kernel at fastserve's tuning shapes, and the
    KIVI split (fastserve experiments/m7.py:292-335 sweeps split x num_warps for its Triton kernel). Cold calls
    (1 GiB read between calls), event-timed; each shape is warmed up before its first point and its built-in
    point measured again after the last (the lower of the two is reported), since the first calls on a freshly
    built workload run slower. One JSON line with every point, the best of each shape on stderr."""
    import torch

    from bpt_amd import _lib, decode_plan, kivi, measure, paged_decode_attention, workloads

    torch.cuda.set_device(0)
    flush = measure.ReadProbe(args.flush_bytes)
    points = []

    def timed(call, iters=args.tune_iters):
        total, _ = timed_calls(call, flush, iters, 3)
        return round(statistics.median(total) * 1e3, 2)

    for name, cases in TUNE_PAGED.items():
        for batch, cap in cases:
            w = workloads.make(name, device="cuda:0", seed=0, batch=batch, length_cap=cap)
            out = torch.empty(tuple(w.q.shape), dtype=torch.bfloat16, device="cuda:0")
            label = f"{name}" + (f" batch {batch}" if batch else "") + (f" cap {cap}" if cap else "")
            timed(lambda: paged_decode_attention(*w.args(), **w.kwargs(), out=out), iters=30)  # warm-up
            best = None
            for gpc in (0, 1, 2, 3, 4):
                for cost in (-1, 0, 4, 8, 12, 16):
                    for mc in ((0, 1, 2, 4, 8, 16) if batch else (0,)):
                        _lib.set_tuning(groups_per_cu=gpc, piece_cost=cost, min_chunks=mc)
                        grid = decode_plan(*w.args(), **w.kwargs())[0]
                        us = timed(lambda: paged_decode_attention(*w.args(), **w.kwargs(), out=out))
                        pt = {"plan": "paged", "shape": label, "groups_per_cu": gpc, "piece_cost": cost,
                              "min_chunks": mc, "grid": grid, "us": us}
                        points.append(pt)
                        if best is None or us < best["us"]:
                            best = pt
            _lib.set_tuning()
            default = next(p for p in points if p["shape"] == label and p["groups_per_cu"] == 0
                           and p["piece_cost"] == -1 and p["min_chunks"] == 0)
            default["us"] = min(default["us"], timed(lambda: paged_decode_attention(*w.args(), **w.kwargs(), out=out)))
            best = default if default["us"] <= best["us"] else best
            log(f"tune {label}: built-in {default['us']} us (grid {default['grid']}); best {best['us']} us at "
                f"groups/CU {best['groups_per_cu'] or 'built-in'}, piece cost "
                f"{best['piece_cost'] if best['piece_cost'] >= 0 else 'built-in'}, min chunks {best['min_chunks'] or 'built-in'}"
                f" (grid {best['grid']})")
            del w, out
            torch.cuda.empty_cache()

    for batch, context in TUNE_KIVI_SHAPES:
        for bits in (4, 8, 16):
            w = workloads.make_kivi(batch, context, bits, device="cuda:0", seed=batch + context)
            scale = workloads.HEAD_DIM**-0.5
            label = workloads.kivi_name(batch, context, bits)
            timed(lambda: kivi.attend(w.q, w, w.lengths, scale, tokens=context), iters=30)  # warm-up
            best = None
            for gpc in (0, 1, 2, 3, 4):
                for mc in (0, 2, 4, 8, 16):
                    _lib.set_tuning(groups_per_cu=gpc, min_chunks=mc)
                    us = timed(lambda: kivi.attend(w.q, w, w.lengths, scale, tokens=context))
                    pt = {"plan": "kivi", "shape": label, "groups_per_cu": gpc, "min_chunks": mc, "us": us}
                    points.append(pt)
                    if best is None or us < best["us"]:
                        best = pt
            _lib.set_tuning()
            for split in [s for s in TUNE_KIVI_SPLITS if s < context] + [context]:
                us = timed(lambda: kivi.decode_attention(w.q, w, w.lengths, scale, tokens=context, split=split))
                points.append({"plan": "kivi-split", "shape": label, "split": split, "us": us})
            default = next(p for p in points if p["shape"] == label and p["plan"] == "kivi"
                           and p["groups_per_cu"] == 0 and p["min_chunks"] == 0)
            default["us"] = min(default["us"], timed(lambda: kivi.attend(w.q, w, w.lengths, scale, tokens=context)))
            best = default if default["us"] <= best["us"] else best
            splits = [p for p in points if p["shape"] == label and p["plan"] == "kivi-split"]
            bs = min(splits, key=lambda p: p["us"])
            log(f"tune {label}: attend built-in {default['us']} us; best {best['us']} us at groups/CU "
                f"{best['groups_per_cu'] or 'built-in'}, min chunks {best['min_chunks'] or 'built-in'}; "
                f"decode_attention splits {min(p['us'] for p in splits)}-{max(p['us'] for p in splits)} us "
                f"(best split {bs['split']})")
            del w
            torch.cuda.empty_cache()
    print(json.dumps({"tune": points}), flush=True)
    return 0


def cpu_model() -> str:
    """The host CPU as /proc/cpuinfo names it: model name, family / model / stepping, cache size."""
    fields = {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if not line.strip():
                    break  # the first processor's block is enough
                key, _, val = line.partition(":")
                fields[key.strip()] = val.strip()
    except OSError:
        pass
    name = fields.get("model name") or platform.processor() or "unknown"
    ids = ", ".join(f"{k} {fields[k]}" for k in ("cpu family", "model", "stepping", "cache size") if k in fields)
    return f"{name} ({ids})" if ids else name


def cpu_threads() -> int:
    """Host threads for the CPU baseline: the cores this process may run on, at most 16 (one GPU's share of
    the host)."""
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = os.cpu_count() or 1
    return max(1, min(avail, 16))


def cpu_baseline(name: str, budget_s: float) -> dict:
    """fastserve's CPU path restated in PyTorch float32 (oracle.torch_paged: the batch's pages gathered into a
    padded contiguous view, dequantized, causal GQA attention) on the host, over the first sequences of
    workload `name`, sized to about `budget_s` seconds."""
    import torch

    from bpt_amd import workloads
    from oracle import torch_paged

    threads = cpu_threads()
    torch.set_num_threads(threads)
    w = workloads.make(name, device="cuda:0", seed=0)
    fmt = w.shape.kv_format
    cpu = dict(q=w.q.cpu(), k=w.k_cache.cpu(), v=w.v_cache.cpu(), table=w.block_table.cpu(),
               lens=w.context_lens.cpu(), ks=None if w.k_scale is None else w.k_scale.cpu(),
               vs=None if w.v_scale is None else w.v_scale.cpu())
    q4 = cpu["q"] if cpu["q"].dim() == 4 else cpu["q"][:, None]
    lengths = w.lengths
    per_token = w.kv_bytes() / max(sum(lengths), 1)  # algorithmic bytes per cached token

    def run(n):
        t = time.perf_counter()
        torch_paged.paged_decode(q4[:n], cpu["k"], cpu["v"], cpu["table"][:n], cpu["lens"][:n], cpu["ks"],
                                 cpu["vs"], fmt, w.sm_scale)
        return time.perf_counter() - t

    n = 1
    first = run(n)
    while n < len(lengths) and first * 2 < budget_s / 4:  # grow the sample while one run stays short
        n = min(len(lengths), n * 2)
        first = run(n)
    times = [first]
    t_end = time.perf_counter() + budget_s
    while len(times) < 3 or (time.perf_counter() < t_end and len(times) < 10):
        times.append(run(n))
    med = statistics.median(times)
    sample_tokens = sum(lengths[:n])
    nbytes = sample_tokens * per_token
    del w, cpu
    return {
        "value": round(nbytes / med / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"oracle.torch_paged.paged_decode (PyTorch {torch.__version__} float32, torch.set_num_threads("
        f"{threads})) over the first {n} of the {len(lengths)} sequences ({sample_tokens} cached tokens, "
        f"padded to the longest as fastserve's engine does), median of {len(times)} runs: {med * 1e3:.2f} ms "
        "per run",
        "ms_per_run": round(med * 1e3, 3),
        "us_per_call_full_workload_est": round(med * (sum(lengths) / max(sample_tokens, 1)) * 1e6, 1),
        "cpu": f"{cpu_model()}, {os.cpu_count()} logical CPUs visible, {threads} used",
    }


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="qwen3-1.7b-fp8")
    ap.add_argument("--flush-bytes", type=int, default=1 << 30)
    ap.add_argument("--no-configs", action="store_true", help="skip the five-shape table")
    ap.add_argument("--no-kivi", action="store_true", help="skip the KIVI (contiguous 4/8/16-bit cache) table")
    ap.add_argument("--no-norm", action="store_true", help="skip the RMSNorm + INT8 table")
    ap.add_argument("--no-step", action="store_true", help="skip the 28-layer decode step through the paged cache")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--profile", action="store_true", help="short run for rocprofv3 (no JSON line)")
    ap.add_argument("--cascade", action="store_true", help="with --profile: the shared-prefix cascade call")
    ap.add_argument("--append", action="store_true", help="with --profile: the step's quantize-on-write call")
    ap.add_argument("--tune", action="store_true", help="sweep the plan constants (one JSON line of points)")
    ap.add_argument("--tune-iters", type=int, default=10, help="with --tune: timed calls per point")
    ap.add_argument("--fused", action="store_true",
                    help="with --profile: the decode call with the last token's store in the same launch")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(
            "bench.py measures one GPU: the decode path is sharded by sequence or KV head with no exchange, "
            "so each GPU runs this same single-GPU call on its own share; this benchmark takes --gpus 1",
            file=sys.stderr,
        )
        return 2

    if args.profile:
        return profile_pass(args)
    if args.tune:
        return tune(args)

    import torch

    from bpt_amd import measure, paged_decode_attention, workloads

    torch.cuda.set_device(0)
    log(f"workload {args.workload}: building")
    w = workloads.make(args.workload, device="cuda:0", seed=0)
    flush = measure.ReadProbe(args.flush_bytes)
    out = torch.empty(tuple(w.q.shape), dtype=torch.bfloat16, device="cuda:0")
    pargs, kw = w.args(), w.kwargs()

    def call():
        paged_decode_attention(*pargs, **kw, out=out)

    def call_ev(start, stop):
        paged_decode_attention(*pargs, **kw, out=out, _events=(start, stop))

    log(f"timing {args.steps} cold steps after {args.warmup} warmup")
    total, wall = timed_calls(call, flush, args.steps, args.warmup, call_ev)
    nbytes = w.kv_bytes()
    ms_per_step = statistics.fmean(total)
    value = nbytes / (ms_per_step * 1e-3) / 1e9
    log(f"{ms_per_step * 1e3:.1f} us/call ({value:.0f} GB/s)")

    floors = read_floors(w, flush, args.steps, args.warmup)
    log(f"read floors: {floors['read_floor_us']} us contiguous, {floors['page_read_floor_us']} us through the pages")
    read_gbps = measure.measured_read_gbps(4 << 30)
    log(f"read probe: {read_gbps:.0f} GB/s")
    from bpt_amd import decode_plan

    from bpt_amd import decode_kernel_name

    groups, chunk_tokens, _, _ = decode_plan(*pargs, **kw)
    kernel = decode_kernel_name(*pargs, **kw)
    traffic = profiled_traffic(kernel, args.workload)
    result = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8_e4m3 codes; bf16 (QK) and f16 (PV) MFMA with f32 accumulation",
        "data": "synthetic",
        "config": {
            "workload": args.workload,
            "batch": w.shape.batch,
            "queries_per_seq": w.shape.queries,
            "q_heads": w.shape.q_heads,
            "kv_heads": w.shape.kv_heads,
            "head_dim": 128,
            "page_size": 16,
            "kv_dtype": "float8_e4m3fn" if w.shape.kv_format == "fp8" else w.shape.kv_format,
            "scales": w.shape.scales,
            "sum_context": sum(w.lengths),
            "kv_bytes_per_call": nbytes,
            "workgroups": groups,
            "chunk_tokens": chunk_tokens,
            "timing": f"HIP events recorded by each call's kernel launch (hipExtLaunchKernel), {args.flush_bytes >> 20} "
                      "MiB read flush before each (untimed)",
        },
        "us_per_call": round(ms_per_step * 1e3, 2),
        "us_per_call_median": round(statistics.median(total) * 1e3, 2),
        "pct_of_peak": round(100 * value / PEAK_GBPS, 1),
        "pct_of_measured_read": round(100 * value / read_gbps, 1),
        "measured_read_gbps": round(read_gbps, 1),
        "read_floor_us": floors["read_floor_us"],
        "page_read_floor_us": floors["page_read_floor_us"],
        "pct_of_read_floor": round(100 * floors["read_floor_us"] / (ms_per_step * 1e3), 1),
        "pct_of_page_read_floor": round(100 * floors["page_read_floor_us"] / (ms_per_step * 1e3), 1),
        "wall_s_timed_region": round(wall, 4),
        "roofline": {
            "bound": "hbm",
            "kernel": kernel,
            "achieved": round(value, 1),
            "peak": PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(value / PEAK_GBPS, 4),
            "kernel_us": round(ms_per_step * 1e3, 2),
            "traffic": traffic["bytes"] if traffic else None,
            "traffic_source": traffic["source"] if traffic else None,
        },
    }
    del w, out, pargs, kw
    torch.cuda.empty_cache()

    if not args.no_configs:
        table = {}
        for name in workloads.SHAPES:
            log(f"shape {name}")
            table[name] = measure_workload(name, flush, iters=20, warmup=5)
        result["configs"] = table
    if not args.no_kivi:
        result["kivi"] = measure_kivi(flush, iters=20, warmup=5)
        result["kivi_quantize"] = measure_kivi_quantize(flush, iters=20, warmup=5)
    if not args.no_step:
        result["decode_step"] = measure_decode_step(iters=10, warmup=3)
    if not args.no_norm:
        result["norm_quant"] = measure_norm_quant(flush, iters=20, warmup=5)
    if not args.no_cpu_baseline:
        log("cpu baseline")
        result["cpu_baseline"] = cpu_baseline(args.workload, args.cpu_seconds)
        if "configs" in result:
            for name, row in result["configs"].items():
                if name == args.workload:
                    row["cpu_baseline"] = result["cpu_baseline"]
                    continue
                log(f"cpu baseline {name}")
                row["cpu_baseline"] = cpu_baseline(name, args.cpu_seconds / 2)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
