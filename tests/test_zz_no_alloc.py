"""GPU: bpt_paged_decode_noalloc (partials and counters in the library's device-resident array) gives exactly
what bpt_paged_decode with a caller workspace gives, on two calls in a row (the second smaller), through the C
ABI; a call too large for the array is refused before anything is launched."""

import ctypes

import pytest
import torch

from bpt_amd import _lib, paged_decode_attention
from bpt_amd.paged_attention import _decode_args, _stream

from test_gpu_decode import DEV, check, make_case, run_case

pytestmark = pytest.mark.gpu


def noalloc(c, max_context=None, num_splits=None, out_dtype=torch.bfloat16):
    """One bpt_paged_decode_noalloc call on case c, through the C ABI (no workspace, no counters)."""
    q = c["q"]
    lengths = c["lens"].cpu().tolist()
    mc = max(lengths + [0]) if max_context is None else max_context
    a, (b, nq, hq, d) = _decode_args(q, c["k"], c["v"], c["table"], c["lens"], c["ks"], c["vs"], 0.0883883, mc,
                                     num_splits, out_dtype)
    out = torch.full((b, nq, hq, d), float("nan"), dtype=out_dtype, device=DEV)
    a.out = out.data_ptr()
    a.out_stride_b, a.out_stride_q, a.out_stride_h = out.stride(0), out.stride(1), out.stride(2)
    rc = _lib.lib().bpt_paged_decode_noalloc(ctypes.byref(a), ctypes.c_void_p(_stream(q.device)))
    _lib.check(rc)
    return out


def reference(c, max_context=None, num_splits=None):
    lengths = c["lens"].cpu().tolist()
    mc = max(lengths + [0]) if max_context is None else max_context
    return paged_decode_attention(c["q"], c["k"], c["v"], c["table"], c["lens"], c["ks"], c["vs"], scale=0.0883883,
                                  max_context=mc, num_splits=num_splits)


@pytest.mark.parametrize("fmt,scales,nq", [("fp8", "head", 1), ("int8", "token", 1), ("bf16", None, 1),
                                           ("fp8", "head", 5)])
def test_noalloc_matches_the_workspace_entry_point_on_two_calls(fmt, scales, nq):
    big = make_case(fmt, [4096, 1000, 33, 1, 2500, 0, 700], scales=scales, nq=nq, seed=3)
    small = make_case(fmt, [300, 17], scales=scales, nq=nq, seed=4)
    for c, splits in ((big, None), (small, None), (big, 7), (small, 2)):
        got = noalloc(c, num_splits=splits)
        want = reference(c, num_splits=splits)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"{fmt} Q={nq} splits={splits}: differs from bpt_paged_decode"
        g2, w2 = run_case(c, num_splits=splits)  # and the oracle, at the decode tolerance
        check(got, w2, f"{fmt} Q={nq} splits={splits} against the oracle")


def test_noalloc_matches_on_two_wave_workgroups():
    # 24 sequences x 8 KV heads = 192 segments: the plan's 2-wave workgroups (1024 of them, so twice the
    # partial slots), then a call of 2 sequences on 4-wave ones, sharing the array.
    lengths = [4096, 1000, 33, 1, 2500, 0, 700, 3000, 2048, 64, 95, 300, 513, 1500, 2, 31, 32, 2049, 129, 4000,
               256, 257, 47, 1024]
    big = make_case("fp8", lengths, seed=13)
    small = make_case("fp8", [300, 17], seed=14)
    for c in (big, small, big):
        got = noalloc(c)
        want = reference(c)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"{len(c['lens'])} sequences: differs from bpt_paged_decode"
    check(got, run_case(big)[1], "192 segments against the oracle")


def test_noalloc_refuses_a_call_larger_than_its_array():
    # 4096 sequences x 8 KV heads on the matrix cores need 16-row partial slots: far over 30 MiB.
    lengths = [40] * 4096
    c = make_case("fp8", lengths, pool_extra=3)
    with pytest.raises(ValueError, match="scratch"):
        noalloc(c)
    out = noalloc(make_case("fp8", [64, 65]))  # and the next call works
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
