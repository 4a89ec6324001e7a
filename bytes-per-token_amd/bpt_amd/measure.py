"""Measurement on the GPU: HIP-event timing with cold caches, graph replay, the read-bandwidth probe.

Follows fastserve's timing methodology (timing.py:59-123): warmup, then events recorded around every call
and one synchronize at the end; optionally the cache is evicted before each timed call *by reading* a
scratch buffer (timing.py:76-80), outside the timed region. On MI355X the buffer must exceed L2 (4 MB per
XCD) plus the 256 MB Infinity Cache, so the default flush reads 1 GiB with the library's own read probe.
Events are recorded on the current stream, which is the stream the library's kernels are launched on.
"""

from __future__ import annotations

import ctypes
from collections.abc import Callable

import torch

from . import _lib

FLUSH_BYTES = 1 << 30
HBM_PEAK_GBPS = 8000.0  # MI355X published HBM3E bandwidth


def _stream(device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


class ReadProbe:
    """The streaming-read kernel over one buffer: `run()` queues one full read."""

    def __init__(self, nbytes: int, device="cuda"):
        nbytes = nbytes // 16 * 16
        self.nbytes = nbytes
        self.buf = torch.ones(nbytes // 4, dtype=torch.float32, device=device)
        groups = ctypes.c_int64(0)
        _lib.check(_lib.lib().bpt_read_probe(None, nbytes, None, ctypes.byref(groups), None))
        self.partial = torch.empty(groups.value, dtype=torch.float32, device=device)
        self.device = self.buf.device

    def run(self, events: tuple | None = None) -> None:
        """One full read; with `events` (two raw hipEvent_t handles) they are recorded around the kernel."""
        if events is None:
            _lib.check(
                _lib.lib().bpt_read_probe(
                    self.buf.data_ptr(), self.nbytes, self.partial.data_ptr(), None, _stream(self.device)
                )
            )
        else:
            _lib.check(
                _lib.lib().bpt_read_probe_timed(
                    self.buf.data_ptr(), self.nbytes, self.partial.data_ptr(), _stream(self.device),
                    ctypes.c_void_p(events[0]), ctypes.c_void_p(events[1]),
                )
            )


class PageReadProbe:
    """Reads every K / V row (and per-token scale) that paged_decode_attention over the same arguments reads,
    through the same block table and lengths, with no attention math: the read floor of the call's pages."""

    def __init__(self, q, k_cache, v_cache, block_table, context_lens, k_scale=None, v_scale=None, *, scale,
                 max_context, num_splits=None):
        from .paged_attention import _decode_args

        q4 = q[:, None] if q.dim() == 3 else q
        self.args, _ = _decode_args(q4, k_cache, v_cache, block_table, context_lens, k_scale, v_scale, scale,
                                    max_context, num_splits, torch.bfloat16)
        self._keep = (k_cache, v_cache, block_table, context_lens, k_scale, v_scale)
        groups = ctypes.c_int64(0)
        _lib.check(_lib.lib().bpt_page_read_probe(ctypes.byref(self.args), None, ctypes.byref(groups), None, None,
                                                  None))
        self.partial = torch.empty(max(groups.value, 1), dtype=torch.float32, device=q.device)
        self.device = q.device

    def run(self, events: tuple | None = None) -> None:
        ev = (None, None) if events is None else (ctypes.c_void_p(events[0]), ctypes.c_void_p(events[1]))
        _lib.check(_lib.lib().bpt_page_read_probe(ctypes.byref(self.args), self.partial.data_ptr(), None,
                                                  _stream(self.device), *ev))


def copy_probe(dst: torch.Tensor, src: torch.Tensor, nbytes: int) -> None:
    _lib.check(_lib.lib().bpt_copy_probe(dst.data_ptr(), src.data_ptr(), nbytes, _stream(dst.device)))


def fp8_decode_table(device="cuda") -> torch.Tensor:
    """float32 [256]: what the kernels' FP8 decoder gives for every e4m3fn code."""
    out = torch.empty(256, dtype=torch.float32, device=device)
    _lib.check(_lib.lib().bpt_fp8_decode_table(out.data_ptr(), _stream(out.device)))
    return out


def fp8_encode(x: torch.Tensor, scale: float = 1.0) -> torch.Tensor:
    """uint8 codes of the write path's FP8 encoder: e4m3fn(clamp(x / scale, ±448))."""
    x = x.float().contiguous()
    out = torch.empty(x.shape, dtype=torch.uint8, device=x.device)
    _lib.check(_lib.lib().bpt_fp8_encode(x.data_ptr(), float(scale), out.data_ptr(), x.numel(), _stream(x.device)))
    return out


def event_times_ms(fn: Callable[[], object], *, warmup: int, iters: int, flush: ReadProbe | None = None) -> list[float]:
    """Milliseconds per call with events on the current stream; one synchronize at the end.

    With `flush`, the probe reads its buffer before every timed call (not timed).
    """
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(iters)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(iters)]
    for i in range(iters):
        if flush is not None:
            flush.run()
        starts[i].record()
        fn()
        ends[i].record()
    torch.cuda.synchronize()
    return [s.elapsed_time(e) for s, e in zip(starts, ends)]


def kernel_event_times_ms(fn: Callable[[int, int], object], *, warmup: int, iters: int,
                          flush: ReadProbe | None = None) -> list[float]:
    """Milliseconds of the kernel itself per call: `fn(start, stop)` launches with the two raw hipEvent_t
    handles recorded around its kernel (bpt_paged_decode_timed), so the separate event records of
    event_times_ms, which add their own microseconds to a single launch, stay out of the interval. With
    `flush`, the probe reads its buffer before every timed call (not timed)."""
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(iters)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(iters)]
    for e in starts + ends:  # creates the events (torch does so on first record)
        e.record()
    torch.cuda.synchronize()
    for _ in range(warmup):
        fn(starts[0].cuda_event, ends[0].cuda_event)
    torch.cuda.synchronize()
    for i in range(iters):
        if flush is not None:
            flush.run()
        fn(starts[i].cuda_event, ends[i].cuda_event)
    torch.cuda.synchronize()
    return [s.elapsed_time(e) for s, e in zip(starts, ends)]


def graph_time_ms(fn: Callable[[], object], *, calls: int = 20, warmup: int = 3, iters: int = 20) -> list[float]:
    """Per-call milliseconds of `fn` replayed from a HIP graph holding `calls` copies (timing.py:102-123)."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(calls):
            fn()
    return [ms / calls for ms in event_times_ms(graph.replay, warmup=warmup, iters=iters)]


def measured_read_gbps(nbytes: int = 4 << 30, iters: int = 10) -> float:
    """Best sustained read rate of the probe over a buffer far larger than L2 + Infinity Cache."""
    probe = ReadProbe(nbytes)
    times = event_times_ms(probe.run, warmup=3, iters=iters)
    del probe
    return nbytes / (min(times) / 1e3) / 1e9
