"""GPU: paged decode attention against the oracle, at the tolerance max-abs 2e-3 / rel 1e-2
(|got - want| <= 2e-3 + 1e-2 * |want| elementwise, want in float32).

Covers what fastserve's kernel tests cover (tests/kernels/test_kernels_gpu.py:78-142): Qwen3 heads, GQA with
1-8 query heads per KV head, per-row lengths including 0 and 1, lengths that end mid-page and mid-split,
forced split counts from one split to one chunk per split, and the maximum context; plus what the paged,
quantized path adds: FP8 / INT8 / BF16 pools, per-head and per-token scales, int32 and int64 block tables,
head-major pools through strides, several causal queries per sequence, and all five measured shapes at full
size. FP8 heads with 2..16 rows take the matrix-core kernel, the others the vector kernel; both are covered
(FP8 with one row per KV head, BF16 and INT8 exercise the vector kernel).
"""

import numpy as np
import pytest
import torch

from oracle import attention

pytestmark = pytest.mark.gpu

DEV = "cuda"
ATOL, RTOL = 2e-3, 1e-2


def check(got: torch.Tensor, want: np.ndarray, what: str = ""):
    got = got.float().cpu().numpy()
    assert np.isfinite(got).all(), what
    err = np.abs(got - want)
    bound = ATOL + RTOL * np.abs(want)
    bad = err > bound
    assert not bad.any(), f"{what}: {bad.sum()} of {bad.size} outside tolerance, worst {err.max():.3e}"


def oracle_out(w):
    from bpt_amd.workloads import to_oracle

    o = to_oracle(w)
    out, _ = attention.paged_decode(
        o["q"], o["k_pool"], o["v_pool"], o["block_table"], o["context_lens"], o["k_scale"], o["v_scale"],
        o["kv_format"], o["scale"],
    )
    return out


def make_case(fmt, lengths, hq=16, hkv=8, nq=1, page=16, scales="head", seed=0, pool_extra=5, head_major=False,
              table_dtype=torch.int32, outliers=True, v_mag=1.0):
    """A small random paged cache in the given format, quantized with torch ops (values ~ N(0, v_mag^2))."""
    from bpt_amd import workloads

    gen = torch.Generator().manual_seed(seed)
    d = 128
    n_pages = [max((t + page - 1) // page, 0) for t in lengths]
    nb = sum(n_pages) + pool_extra
    perm = torch.randperm(nb, generator=gen)
    max_blocks = max(max(n_pages), 1) + 2
    table = torch.zeros((len(lengths), max_blocks), dtype=torch.int64)
    c = 0
    for i, n in enumerate(n_pages):
        table[i, :n] = perm[c : c + n]
        table[i, n:] = perm[(c + n) % nb]  # padding entries point at real pages
        c += n
    g = torch.Generator(device=DEV).manual_seed(seed + 1)
    kf = torch.randn((nb, page, hkv, d), generator=g, device=DEV)
    if outliers:
        kf[..., torch.randperm(d, generator=gen)[:4].to(DEV)] *= 8.0
    vf = torch.randn((nb, page, hkv, d), generator=g, device=DEV) * v_mag
    ks = vs = None
    if fmt == "bf16":
        kc, vc = kf.to(torch.bfloat16), vf.to(torch.bfloat16)
    elif fmt == "fp8" and scales == "head":
        ks = (kf.abs().amax(dim=(0, 1, 3)) / 448.0).float()
        vs = (vf.abs().amax(dim=(0, 1, 3)) / 448.0).float()
        kc, vc = workloads.quantize_per_head_fp8(kf, ks), workloads.quantize_per_head_fp8(vf, vs)
    elif fmt == "int8" and scales == "token":
        kc, ks = workloads.quantize_per_token_int8(kf)
        vc, vs = workloads.quantize_per_token_int8(vf)
    elif fmt == "int8" and scales == "head":
        ks = (kf.abs().amax(dim=(0, 1, 3)) / 127.0).float()
        vs = (vf.abs().amax(dim=(0, 1, 3)) / 127.0).float()
        kc = torch.clamp(torch.round(kf / ks[:, None]), -128, 127).to(torch.int8)
        vc = torch.clamp(torch.round(vf / vs[:, None]), -128, 127).to(torch.int8)
    elif fmt == "fp8" and scales == "token":
        ks = (kf.abs().amax(-1, keepdim=True) / 448.0).clamp(min=1e-12)
        vs = (vf.abs().amax(-1, keepdim=True) / 448.0).clamp(min=1e-12)
        kc = (kf / ks).clamp(-448, 448).to(torch.float8_e4m3fn)
        vc = (vf / vs).clamp(-448, 448).to(torch.float8_e4m3fn)
        ks, vs = ks[..., 0].contiguous(), vs[..., 0].contiguous()
    else:
        raise ValueError((fmt, scales))
    if head_major:  # store as [NB, Hkv, P, D], pass the [NB, P, Hkv, D] view
        kc = kc.transpose(1, 2).contiguous().transpose(1, 2)
        vc = vc.transpose(1, 2).contiguous().transpose(1, 2)
    q = torch.randn((len(lengths), nq, hq, d), generator=g, device=DEV).to(torch.bfloat16)
    lens = torch.tensor(lengths, dtype=torch.int32, device=DEV)
    return dict(q=q, k=kc, v=vc, table=table.to(DEV, table_dtype), lens=lens, ks=ks, vs=vs, fmt=fmt)


def np_codes(t, fmt):
    if fmt == "fp8":
        return t.contiguous().view(torch.uint8).cpu().numpy()
    if fmt == "int8":
        return t.contiguous().cpu().numpy()
    return t.float().contiguous().cpu().numpy()


def run_case(c, scale=0.0883883, max_context=None, num_splits=None, out_dtype=torch.bfloat16, q=None):
    from bpt_amd import paged_decode_attention

    q = c["q"] if q is None else q
    lengths = c["lens"].cpu().tolist()
    mc = max(lengths + [0]) if max_context is None else max_context
    got = paged_decode_attention(q, c["k"], c["v"], c["table"], c["lens"], c["ks"], c["vs"], scale=scale,
                                 max_context=mc, num_splits=num_splits, out_dtype=out_dtype)
    torch.cuda.synchronize()
    want, _ = attention.paged_decode(
        q.float().cpu().numpy(), np_codes(c["k"], c["fmt"]), np_codes(c["v"], c["fmt"]), c["table"].cpu().numpy(),
        np.array(lengths), None if c["ks"] is None else c["ks"].cpu().numpy(),
        None if c["vs"] is None else c["vs"].cpu().numpy(), c["fmt"], scale,
    )
    return got, want


@pytest.mark.parametrize("fmt,scales", [("fp8", "head"), ("int8", "token"), ("bf16", None), ("int8", "head"),
                                        ("fp8", "token")])
@pytest.mark.parametrize("lengths", [[160, 1, 70, 0], [513, 16, 17, 31, 32, 33, 255, 4096]])
def test_formats_and_ragged_lengths(fmt, scales, lengths):
    c = make_case(fmt, lengths, scales=scales)
    got, want = run_case(c)
    check(got, want, f"{fmt}/{scales} auto splits")
    for i, t in enumerate(lengths):
        if t == 0:  # a sequence with no tokens gets zeros, not NaN
            assert got[i].float().abs().sum().item() == 0


@pytest.mark.parametrize("fmt,scales", [("fp8", "head"), ("int8", "token"), ("bf16", None)])
@pytest.mark.parametrize("num_splits", [1, 2, 7, 64, 1000])
def test_forced_split_counts(num_splits, fmt, scales):
    # 64 and 1000 splits give more partitions than resident workgroups: each workgroup then takes several
    # consecutive partitions whole.
    c = make_case(fmt, [4096, 1000, 33, 1], scales=scales)
    got, want = run_case(c, num_splits=num_splits)
    check(got, want, f"{fmt} num_splits={num_splits}")


@pytest.mark.parametrize("nq", [1, 5])
@pytest.mark.parametrize("length", [5, 31, 33, 512, 2943, 9000])
def test_one_sequence_matrix_core(length, nq):
    # One sequence on the matrix-core kernel (2-row and 10-row segments): the plan charges its equally long
    # segments nothing, so the line's ranges fall anywhere inside them, across KV heads and chunk edges.
    c = make_case("fp8", [length], nq=nq, seed=length)
    got, want = run_case(c)
    check(got, want, f"one sequence of {length}, Q={nq}")


@pytest.mark.parametrize("hq,hkv", [(8, 8), (16, 8), (32, 8), (64, 8), (12, 4), (40, 8)])
def test_gqa_groups(hq, hkv):
    c = make_case("fp8", [300, 77, 1024], hq=hq, hkv=hkv)
    got, want = run_case(c)
    check(got, want, f"Hq={hq} Hkv={hkv}")


@pytest.mark.parametrize("nq", [2, 3, 5])
@pytest.mark.parametrize("fmt", ["fp8", "bf16"])
def test_multi_query_causal(nq, fmt):
    c = make_case(fmt, [1030, 5, 64, 2000], nq=nq)
    got, want = run_case(c)
    check(got, want, f"Q={nq}")
    got1, want1 = run_case(c, num_splits=3)
    check(got1, want1, f"Q={nq}, 3 splits")


@pytest.mark.parametrize("page", [1, 4, 8, 32, 64])
def test_page_sizes(page):
    c = make_case("fp8", [100, 257, 31], page=page)
    got, want = run_case(c)
    check(got, want, f"page {page}")


@pytest.mark.parametrize("fmt,scales", [("int8", "token"), ("int8", "head"), ("fp8", "head"), ("bf16", None)])
def test_vector_path_one_row_per_kv_head(fmt, scales):
    """Hq = Hkv: one row per KV head, the vector kernel for every format."""
    c = make_case(fmt, [700, 3, 128, 2049], hq=8, hkv=8, scales=scales)
    got, want = run_case(c)
    check(got, want, f"{fmt} one row")
    got, want = run_case(c, q=c["q"].float(), num_splits=4)
    check(got, want, f"{fmt} one row, f32 q, 4 splits")


def test_head_major_pool_int64_table_f32_out_and_q_dtypes():
    c = make_case("int8", [700, 3, 128], scales="token", head_major=True, table_dtype=torch.int64)
    got, want = run_case(c)
    check(got, want, "head-major")
    got, want = run_case(c, out_dtype=torch.float32)
    assert got.dtype == torch.float32
    check(got, want, "f32 out")
    got, want = run_case(c, q=c["q"].float())
    check(got, want, "f32 q")


def test_lengths_beyond_max_context_are_truncated_to_it():
    c = make_case("fp8", [600, 300])
    from bpt_amd import paged_decode_attention

    got = paged_decode_attention(c["q"], c["k"], c["v"], c["table"], c["lens"], c["ks"], c["vs"], scale=0.1,
                                 max_context=256)
    c2 = dict(c)
    c2["lens"] = torch.tensor([256, 256], dtype=torch.int32, device=DEV)
    want = paged_decode_attention(c["q"], c["k"], c["v"], c["table"], c2["lens"], c["ks"], c["vs"], scale=0.1,
                                  max_context=256)
    assert torch.equal(got, want)


def test_output_buffer_is_used_and_3d_q_is_one_query():
    from bpt_amd import paged_decode_attention

    c = make_case("fp8", [64, 65])
    out = torch.empty((2, 16, 128), dtype=torch.bfloat16, device=DEV)
    r = paged_decode_attention(c["q"][:, 0], c["k"], c["v"], c["table"], c["lens"], c["ks"], c["vs"], scale=0.1,
                               max_context=65, out=out)
    assert r.data_ptr() == out.data_ptr() and r.shape == (2, 16, 128)
    got, want = run_case(c, scale=0.1)
    check(out, want[:, 0], "out buffer")


def test_max_context_one_sequence():
    c = make_case("fp8", [32768], pool_extra=0)
    got, want = run_case(c)
    check(got, want, "32768 tokens")
    lens = torch.tensor([32001], dtype=torch.int32, device=DEV)
    c["lens"] = lens
    got, want = run_case(c, max_context=32768, num_splits=16)
    check(got, want, "32001 tokens in 16 splits")


@pytest.mark.parametrize("name", ["qwen3-0.6b-bf16", "qwen3-1.7b-fp8", "qwen3-1.7b-int8", "qwen3-8b-fp8-long",
                                  "qwen3-1.7b-verify"])
def test_measured_shapes_at_full_size(name):
    from bpt_amd import paged_decode_attention, workloads

    w = workloads.make(name, device=DEV, seed=0)
    got = paged_decode_attention(*w.args(), **w.kwargs())
    torch.cuda.synchronize()
    check(got, oracle_out(w), name)


@pytest.mark.parametrize("fmt,scales", [("bf16", None), ("int8", "token"), ("int8", "head")])
@pytest.mark.parametrize("lengths,max_context", [([2048], None), ([513] * 3, None), ([17] * 8, None),
                                                 ([1] * 64, None), ([4096] * 2, 8192), ([700] * 5, 3000),
                                                 ([0] * 4, 512), ([300] * 6 + [299], None)])
def test_equal_lengths_take_equal_partitions(fmt, scales, lengths, max_context):
    """Small BF16 / INT8 calls on the vector kernel whose sequences all have one length are cut into equal
    power-of-two partitions by part of the launch (the rest leaves at once), ranges crossing sequence
    boundaries; lengths below max_context use fewer of those workgroups. The last case differs in one
    length and keeps the line cut."""
    c = make_case(fmt, lengths, scales=scales)
    got, want = run_case(c, max_context=max_context)
    check(got, want, f"{fmt}/{scales} {len(lengths)} x {lengths[0]}")
    if lengths[0] == 0:
        assert got.float().abs().sum().item() == 0


def test_equal_lengths_beyond_max_context_are_cut_to_it():
    """Lengths that differ but all exceed max_context are equal once cut to it."""
    c = make_case("bf16", [600, 900, 556])
    from bpt_amd import paged_decode_attention

    got = paged_decode_attention(c["q"], c["k"], c["v"], c["table"], c["lens"], c["ks"], c["vs"], scale=0.1,
                                 max_context=256)
    lens = torch.full((3,), 256, dtype=torch.int32, device=DEV)
    want = paged_decode_attention(c["q"], c["k"], c["v"], c["table"], lens, c["ks"], c["vs"], scale=0.1,
                                  max_context=256)
    assert torch.equal(got, want)
    c["lens"] = lens
    got, want = run_case(c, scale=0.1, max_context=256)
    check(got, want, "three lengths cut to 256")


def test_many_short_sequences_share_workgroups():
    """More segments than workgroups: a workgroup's range walks many (sequence, head) segments, with
    empty sequences at the start, middle and end of the batch."""
    lengths = [0] + [int(x) for x in np.random.default_rng(3).integers(1, 200, 300)] + [0, 5, 0]
    c = make_case("fp8", lengths, pool_extra=3)
    got, want = run_case(c)
    check(got, want, "300 short sequences")
    for i, t in enumerate(lengths):
        if t == 0:
            assert got[i].float().abs().sum().item() == 0


@pytest.mark.parametrize("fmt,scales", [("fp8", "head"), ("int8", "token"), ("bf16", None)])
def test_segments_of_one_chunk_mostly_overhead_units(fmt, scales):
    """1500 sequences of 1..40 tokens: each segment is one or two chunks behind its piece-cost units, so
    many workgroup ranges hold no chunk at all (they return at once) and many start among a segment's
    units (they start at its first chunk)."""
    lengths = [int(x) for x in np.random.default_rng(5).integers(1, 41, 1500)]
    c = make_case(fmt, lengths, scales=scales, pool_extra=3)
    got, want = run_case(c)
    check(got, want, f"{fmt}: 1500 sequences of one or two chunks")


@pytest.mark.parametrize("fmt,scales", [("fp8", "head"), ("int8", "token")])
def test_largest_batch(fmt, scales):
    """The largest batch a call takes (4096 sequences: the per-sequence prefix sum fills the most LDS),
    with lengths of 0..40 tokens."""
    from bpt_amd import paged_decode_attention

    lengths = [int(x) for x in np.random.default_rng(9).integers(0, 41, 4096)]
    c = make_case(fmt, lengths, scales=scales, pool_extra=3)
    got, want = run_case(c)
    check(got, want, f"{fmt}: 4096 sequences")
    with pytest.raises(ValueError, match="batch"):
        q = torch.zeros((4097, 1, 16, 128), dtype=torch.bfloat16, device=DEV)
        table = torch.zeros((4097, c["table"].shape[1]), dtype=torch.int32, device=DEV)
        lens = torch.zeros(4097, dtype=torch.int32, device=DEV)
        paged_decode_attention(q, c["k"], c["v"], table, lens, c["ks"], c["vs"], scale=0.1, max_context=40)


def test_timed_entry_records_the_kernel_and_matches_the_plain_call():
    """bpt_paged_decode_timed: the same output as bpt_paged_decode, and two events around the kernel whose
    interval is positive (and empty for a batch with nothing to launch)."""
    from bpt_amd import paged_decode_attention

    c = make_case("fp8", [300, 77, 1024])
    kw = dict(scale=0.0883883, max_context=1024)
    args = (c["q"], c["k"], c["v"], c["table"], c["lens"], c["ks"], c["vs"])
    want = paged_decode_attention(*args, **kw)
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    stop.record()
    torch.cuda.synchronize()
    got = paged_decode_attention(*args, **kw, _events=(start.cuda_event, stop.cuda_event))
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    assert start.elapsed_time(stop) > 0.0
    empty = (c["q"][:0], c["k"], c["v"], c["table"][:0], c["lens"][:0], c["ks"], c["vs"])
    paged_decode_attention(*empty, **kw, _events=(start.cuda_event, stop.cuda_event))
    torch.cuda.synchronize()
    assert start.elapsed_time(stop) >= 0.0


def test_workspace_counters_reset_between_calls_of_different_shapes():
    """One cached workspace serves calls of different shapes in a row; an explicit zeroed one works too."""
    from bpt_amd import decode_plan, paged_decode_attention

    cases = [make_case("fp8", [3000, 17, 900], seed=s) for s in range(2)] + [make_case("int8", [4096] * 4, scales="token")]
    for rep in range(2):
        for c in cases:
            got, want = run_case(c, num_splits=None if rep else 8)
            check(got, want, f"rep {rep}")
    c = cases[0]
    _, _, ws_bytes, cnt_bytes = decode_plan(c["q"], c["k"], c["v"], c["table"], c["lens"], c["ks"], c["vs"],
                                            scale=0.1, max_context=3000, num_splits=16)
    ws = torch.full((ws_bytes,), 0x7F, dtype=torch.uint8, device=DEV)  # partials need no initialization
    cnt = torch.zeros(cnt_bytes, dtype=torch.uint8, device=DEV)
    a = paged_decode_attention(c["q"], c["k"], c["v"], c["table"], c["lens"], c["ks"], c["vs"], scale=0.1,
                               max_context=3000, num_splits=16, workspace=ws, counters=cnt)
    b = paged_decode_attention(c["q"], c["k"], c["v"], c["table"], c["lens"], c["ks"], c["vs"], scale=0.1,
                               max_context=3000, num_splits=16, workspace=ws, counters=cnt)
    torch.cuda.synchronize()
    assert torch.equal(a, b) and cnt.abs().sum().item() == 0


def test_repeated_calls_are_deterministic():
    from bpt_amd import paged_decode_attention, workloads

    w = workloads.make("qwen3-1.7b-fp8", device=DEV, seed=1, batch=8)
    a = paged_decode_attention(*w.args(), **w.kwargs())
    b = paged_decode_attention(*w.args(), **w.kwargs())
    assert torch.equal(a, b)


@pytest.mark.parametrize("fmt,scales", [("fp8", "head"), ("fp8", "token"), ("int8", "token"), ("int8", "head")])
@pytest.mark.parametrize("nq,hq,hkv", [(1, 16, 8), (5, 16, 8), (8, 16, 8), (1, 48, 8), (4, 32, 8), (3, 20, 4)])
def test_matrix_core_path_rows_2_to_16(fmt, scales, nq, hq, hkv):
    """FP8 heads serving 2..16 rows (Q queries x G heads) and INT8 heads serving 5..16 run on the matrix
    cores, all rows at once (INT8 with 2..4 rows on the vector kernel)."""
    c = make_case(fmt, [1030, 5, 64, 2000, 33], nq=nq, hq=hq, hkv=hkv, scales=scales)
    got, want = run_case(c)
    check(got, want, f"Q={nq} Hq={hq} Hkv={hkv} {scales}")
    got, want = run_case(c, num_splits=5)
    check(got, want, f"Q={nq} Hq={hq} Hkv={hkv} {scales}, 5 splits")


@pytest.mark.parametrize("fmt,scales", [("fp8", "head"), ("int8", "token")])
@pytest.mark.parametrize("page", [1, 8, 16, 64])
def test_matrix_core_path_page_sizes_and_q_dtypes(fmt, scales, page):
    """Pages smaller than a 16-token tile take the per-token page lookup; wider q dtypes the hi + lo split."""
    c = make_case(fmt, [100, 257, 31, 1], nq=5, page=page, scales=scales)
    got, want = run_case(c)
    check(got, want, f"page {page}")
    for dt in (torch.float16, torch.float32):
        got, want = run_case(c, q=c["q"].to(dt))
        check(got, want, f"page {page}, q {dt}")


@pytest.mark.parametrize("v_mag", [1e-5, 1e-3, 1e4])
@pytest.mark.parametrize("fmt,nq,hq,hkv", [("fp8", 1, 16, 8), ("fp8", 1, 8, 8), ("int8", 1, 16, 8), ("int8", 3, 16, 8),
                                           ("int8", 1, 8, 8)])
def test_per_token_value_scales_far_from_one(fmt, nq, hq, hkv, v_mag):
    """Per-token value scales of 1e-5 .. 1e4 times those of unit values, on both kernels (FP8 with 2 rows and
    INT8 with 6 rows on the matrix cores, FP8 with 1 row and INT8 with 1..2 rows on the vector kernel). The
    scales ride in f16 softmax weights there, so they must neither overflow f16 (large values) nor fall into
    its subnormals (small ones). Attention is linear in V, so outputs are compared at unit scale:
    |got - want| / v_mag <= 2e-3 + 1e-2 |want| / v_mag."""
    c = make_case(fmt, [1030, 5, 64, 2000, 33], nq=nq, hq=hq, hkv=hkv, scales="token", v_mag=v_mag)
    got, want = run_case(c, out_dtype=torch.float32)
    check(got / v_mag, want / v_mag, f"{fmt} Q={nq} Hq={hq} Hkv={hkv} values x{v_mag:g}")
    got, want = run_case(c, out_dtype=torch.float32, num_splits=3)
    check(got / v_mag, want / v_mag, f"{fmt} Q={nq} Hq={hq} Hkv={hkv} values x{v_mag:g}, 3 splits")


@pytest.mark.parametrize("fmt,scales,nq,hq,hkv", [
    ("fp8", "head", 1, 16, 8),    # matrix cores, 2 rows
    ("fp8", "token", 5, 16, 8),   # matrix cores, 10 rows, per-token scales
    ("fp8", "head", 1, 8, 8),     # vector kernel, 1 row
    ("fp8", "token", 1, 8, 8),
    ("int8", "token", 1, 16, 8),  # vector kernel
    ("int8", "head", 3, 16, 8),   # matrix cores, 6 rows
    ("bf16", None, 1, 16, 8),
])
def test_float32_output_is_float32_accurate(fmt, scales, nq, hq, hkv):
    """With float32 output the kernels stay within 1e-4 of the largest output (float32 arithmetic, the
    softmax weights of the packed f16 value products carried as f16 plus their f16 rounding remainder), some
    20 times inside the bf16-output tolerance the other tests use."""
    c = make_case(fmt, [1030, 5, 64, 2000, 33], nq=nq, hq=hq, hkv=hkv, scales=scales)
    for splits in (None, 4):
        got, want = run_case(c, out_dtype=torch.float32, num_splits=splits)
        err = np.abs(got.cpu().numpy() - want).max()
        assert err <= 1e-4 * np.abs(want).max(), f"{fmt} {scales} Q={nq} Hq={hq}: {err:.3e} vs max {np.abs(want).max():.3e}"


@pytest.mark.parametrize("fmt,scales", [("fp8", "head"), ("int8", "token")])
@pytest.mark.parametrize("lengths", [[0, 700, 0, 0, 1500, 33, 0], [2048] * 3 + [0], [1, 0, 5, 31, 32, 33, 0]])
def test_many_row_segments_head_major_walk(fmt, scales, lengths):
    """Many-row segments (here 10 and 12 rows) lie head-major on the stream-K line: a workgroup's range runs
    over the sequences of one KV head, then wraps to the next head's first sequence holding tokens. Empty
    sequences at the start, the end and in between, and ranges that wrap, must all be walked exactly."""
    for nq, hq in ((5, 16), (3, 32)):
        c = make_case(fmt, lengths, nq=nq, hq=hq, hkv=8, scales=scales)
        for splits in (None, 3):
            got, want = run_case(c, num_splits=splits)
            check(got, want, f"{fmt} Q={nq} Hq={hq} {lengths} splits={splits}")
            for i, t in enumerate(lengths):
                if t == 0:
                    assert got[i].float().abs().sum().item() == 0
