"""The C-ABI library on the CPU: it loads, exports every symbol include/bpt_amd.h declares, plans splits, and
refuses bad arguments with ValueError before touching a GPU (no compute calls here)."""

import ctypes
import re
from pathlib import Path

import pytest
import torch

from bpt_amd import _lib, decode_plan, paged_decode_attention, quantize_append

HEADER = Path(__file__).resolve().parent.parent / "include" / "bpt_amd.h"


def declared_symbols() -> list[str]:
    text = HEADER.read_text()
    return re.findall(r"^\s*(?:int|const char\*)\s+(bpt_\w+)\s*\(", text, flags=re.M)


def test_every_declared_symbol_is_exported(built_lib):
    names = declared_symbols()
    assert len(names) >= 9
    for name in names:
        assert hasattr(built_lib, name), name
    assert set(names) == set(_lib.SIGNATURES)
    assert built_lib.bpt_abi_version() == _lib.ABI_VERSION


def test_library_matches_the_sources_and_a_stale_one_is_refused(built_lib, monkeypatch):
    """The library carries the hash of the sources it was built from; loading one built from other sources
    raises instead of silently running old kernels."""
    assert built_lib.bpt_source_hash().decode() == _lib.source_hash()
    monkeypatch.setattr(_lib, "source_hash", lambda: "0123456789abcdef")
    with pytest.raises(_lib.StaleLibraryError, match="rebuild"):
        _lib.lib.__wrapped__()


def cpu_case(fmt="fp8", b=2, nq=1, hq=16, hkv=8, d=128, nb=64, page=16, max_blocks=8):
    dtype = {"fp8": torch.float8_e4m3fn, "int8": torch.int8, "bf16": torch.bfloat16}[fmt]
    q = torch.zeros((b, nq, hq, d), dtype=torch.bfloat16)
    k = torch.zeros((nb, page, hkv, d), dtype=dtype)
    v = torch.zeros_like(k)
    table = torch.zeros((b, max_blocks), dtype=torch.int32)
    lens = torch.zeros(b, dtype=torch.int32)
    if fmt == "fp8":
        ks, vs = torch.ones(hkv), torch.ones(hkv)
    elif fmt == "int8":
        ks, vs = torch.ones(nb, page, hkv), torch.ones(nb, page, hkv)
    else:
        ks = vs = None
    return q, k, v, table, lens, ks, vs


def align256(x):
    return (x + 255) // 256 * 256


def expected_workspace(batch, segments_per_seq, rows_per_group, parts):
    slots = batch * segments_per_seq + parts
    return align256(slots * rows_per_group * (128 + 1) * 4)  # normalized outputs + log-sum-exp, float32


def expected_counters(batch, segments_per_seq):
    return align256(batch * segments_per_seq * 4)  # one uint32 per segment


def test_plan_honours_requested_splits(built_lib):
    # 32/8 heads: 4 rows per KV head (one 16-row matrix-core group), 32-token chunks; 32768 tokens in 32
    # partitions of 32 chunks each: 1024 partitions, more than the 512 resident workgroups (two per CU), so
    # each workgroup takes two consecutive partitions whole.
    q, k, v, table, lens, ks, vs = cpu_case(b=4, hq=32, max_blocks=2048, nb=8192)
    grid, chunk, ws, cnt = decode_plan(q, k, v, table, lens, ks, vs, scale=0.1, max_context=32768, num_splits=32)
    assert chunk == 32 and grid == 512
    assert ws == expected_workspace(4, 8, 16, grid) and cnt == expected_counters(4, 8)
    # Fewer partitions than resident workgroups: one workgroup each.
    grid, _, ws, _ = decode_plan(q, k, v, table, lens, ks, vs, scale=0.1, max_context=32768, num_splits=8)
    assert grid == 4 * 8 * 8 and ws == expected_workspace(4, 8, 16, grid)


def test_plan_auto_groups_per_cu(built_lib):
    """Few-row matrix-core calls over at least 128 (sequence, KV head) segments run two-wave workgroups, four to
    a CU (1024); fewer segments, or a fixed split count, four-wave ones, two to a CU (512)."""
    def plan(b, num_splits=None):
        q, k, v, table, lens, ks, vs = cpu_case("fp8", b=b, max_blocks=256, nb=8192)
        return decode_plan(q, k, v, table, lens, ks, vs, scale=0.1, max_context=4096, num_splits=num_splits)

    grid, chunk, ws, cnt = plan(32)  # 256 segments
    assert chunk == 32 and grid == 1024 and ws == expected_workspace(32, 8, 16, 1024) and cnt == expected_counters(32, 8)
    assert plan(16)[0] == 1024  # 128 segments
    grid, _, ws, _ = plan(8)  # 64 segments
    assert grid == 512 and ws == expected_workspace(8, 8, 16, 512)
    # A fixed split count keeps four-wave workgroups: 1024 partitions over 512 of them, two partitions each.
    assert plan(32, num_splits=4)[0] == 512
    qb, kb, vb, tb, lb, _, _ = cpu_case("bf16", b=1)
    grid, chunk_bf16, _, _ = decode_plan(qb, kb, vb, tb, lb, None, None, scale=0.1, max_context=64)
    assert chunk_bf16 == 16  # vector kernel: 4 loads of 4 rows (16 lanes per bf16 row)
    assert grid == 8 * -(-64 // chunk_bf16)  # never more groups than chunks that could exist


def test_plan_gives_int8_vector_segments_three_groups_per_cu(built_lib):
    """INT8 on the vector kernel runs three workgroups per CU where its kernels fit 168 VGPRs (one row per
    group; two rows with whole 8-row loads per page and a bf16 q), two otherwise."""
    def grid_of(nq=1, hq=16, page=16, q_dtype=torch.bfloat16):
        q, k, v, table, lens, ks, vs = cpu_case("int8", b=64, nq=nq, hq=hq, nb=8192, page=page, max_blocks=512)
        return decode_plan(q.to(q_dtype), k, v, table, lens, ks, vs, scale=0.1, max_context=8192)[0]

    assert grid_of() == 768                              # 2 rows, page 16, bf16 q
    assert grid_of(hq=8) == 768                          # 1 row
    assert grid_of(hq=8, q_dtype=torch.float32) == 768   # 1 row, f32 q
    assert grid_of(q_dtype=torch.float32) == 512         # 2 rows, f32 q
    assert grid_of(page=4) == 512                        # 2 rows, pages smaller than a load
    assert grid_of(hq=32) == 512                         # 4 rows
    q, k, v, table, lens, ks, vs = cpu_case("int8", b=1, nb=8192, max_blocks=512)
    assert decode_plan(q, k, v, table, lens, ks, vs, scale=0.1, max_context=8192)[0] == 8 * 256 // 8  # 2 per wave


def test_plan_launches_enough_workgroups_for_equal_partitions(built_lib):
    """BF16 and INT8 calls on the vector kernel up to 32768 / 16384 chunks may be cut into partitions of a
    power-of-two number of chunks, about 4 sqrt(chunks) of them and at most 512 (when the kernel finds
    all lengths equal): the launch is the larger of that count and the line cut's, or that count alone for
    one sequence."""
    def plan(fmt, b, ctx, hq=16):
        nb = max(b * ctx // 16, 64)
        q, k, v, table, lens, ks, vs = cpu_case(fmt, b=b, hq=hq, nb=nb, max_blocks=max(ctx // 16, 1))
        grid, chunk, ws, _ = decode_plan(q, k, v, table, lens, ks, vs, scale=0.1, max_context=ctx)
        return grid, chunk, ws

    grid, chunk, ws = plan("bf16", 1, 512)  # 8 heads x 32 chunks of 16 tokens = 256: 64 partitions of 4
    assert (grid, chunk) == (64, 16) and ws == expected_workspace(1, 8, 2, 64)
    assert plan("bf16", 2, 2048)[0] == 512   # 2048 chunks: 256 partitions of 8, the line cut 512
    assert plan("bf16", 8, 8192)[0] == 512   # 32768 chunks: target 512 (724 capped), partitions of 64
    assert plan("int8", 1, 2048)[0] == 128   # 512 chunks of 32 tokens: 128 partitions of 4
    assert plan("bf16", 1, 8192)[0] == 256   # 4096 chunks: 256 partitions of 16 (line cut: 512)
    assert plan("int8", 4, 8192)[0] == 768   # 8192 chunks: 512 partitions of 16, line cut 3 per CU
    assert plan("int8", 16, 8192)[0] == 768  # 32768 chunks: the line cut only, three workgroups per CU


@pytest.mark.parametrize("max_context", [0, 1, 100, 4096, 32768])
def test_plan_workspace_grows_with_the_launch(built_lib, max_context):
    q, k, v, table, lens, ks, vs = cpu_case(b=32, max_blocks=4096, nb=8192)
    grid, chunk, ws, cnt = decode_plan(q, k, v, table, lens, ks, vs, scale=0.1, max_context=max_context)
    bound = 32 * 8 * -(-min(max_context, 4096 * 16) // chunk)
    assert 1 <= grid <= max(min(1024, bound), 1)  # 256 segments: two-wave workgroups, four to a CU
    assert ws == expected_workspace(32, 8, 16, grid) and cnt == expected_counters(32, 8)


@pytest.mark.parametrize("fmt", ["fp8", "int8"])
def test_plan_puts_2_to_16_quantized_rows_in_one_matrix_core_group(built_lib, fmt):
    # 5 queries x 2 heads per KV head = 10 rows: one 16-row group per KV head, 32-token chunks.
    q, k, v, table, lens, ks, vs = cpu_case(fmt, b=16, nq=5, max_blocks=256, nb=8192)
    grid, chunk, ws, cnt = decode_plan(q, k, v, table, lens, ks, vs, scale=0.1, max_context=3072)
    assert chunk == 32 and ws == expected_workspace(16, 8, 16, grid) and cnt == expected_counters(16, 8)
    # One row per KV head keeps the vector kernel; so do INT8 heads with 2..4 rows.
    q, k, v, table, lens, ks, vs = cpu_case(fmt, b=16, hq=8, max_blocks=256, nb=8192)
    grid, chunk, ws, cnt = decode_plan(q, k, v, table, lens, ks, vs, scale=0.1, max_context=3072)
    assert ws == expected_workspace(16, 8, 1, grid)
    q, k, v, table, lens, ks, vs = cpu_case(fmt, b=16, max_blocks=256, nb=8192)
    grid, chunk, ws, cnt = decode_plan(q, k, v, table, lens, ks, vs, scale=0.1, max_context=3072)
    assert ws == expected_workspace(16, 8, 16 if fmt == "fp8" else 2, grid)


def test_plan_gives_many_row_segments_fuller_workgroups(built_lib):
    # 10 rows per KV head (5 queries x 2 heads) on the matrix cores: a small batch gets no more workgroups
    # than 8 chunks each would fill (2 sequences x 8 KV heads x 96 chunks of 32 tokens -> 192)...
    q, k, v, table, lens, ks, vs = cpu_case("fp8", b=2, nq=5, max_blocks=256, nb=8192)
    grid, chunk, ws, _ = decode_plan(q, k, v, table, lens, ks, vs, scale=0.1, max_context=3072)
    assert chunk == 32 and grid == 2 * 8 * 96 // 8 and ws == expected_workspace(2, 8, 16, grid)
    # ... a full batch fills every CU with one 8-wave workgroup, and 2 rows per KV head over 128 segments run
    # four 2-wave workgroups per CU.
    q, k, v, table, lens, ks, vs = cpu_case("fp8", b=16, nq=5, max_blocks=256, nb=8192)
    assert decode_plan(q, k, v, table, lens, ks, vs, scale=0.1, max_context=3072)[0] == 256
    q, k, v, table, lens, ks, vs = cpu_case("fp8", b=16, max_blocks=256, nb=8192)
    assert decode_plan(q, k, v, table, lens, ks, vs, scale=0.1, max_context=3072)[0] == 1024
    q, k, v, table, lens, ks, vs = cpu_case("fp8", b=1, max_blocks=64, nb=64)
    assert decode_plan(q, k, v, table, lens, ks, vs, scale=0.1, max_context=1024)[0] == 8 * 32 // 4
    # Two chunks per wave (8 per workgroup) once that still launches a workgroup per two CUs: 2 x 8 heads x
    # 128 chunks -> 256 workgroups; one sequence of 2944 tokens (736 chunks) keeps 4 per workgroup (184).
    q, k, v, table, lens, ks, vs = cpu_case("fp8", b=2, max_blocks=256, nb=8192)
    assert decode_plan(q, k, v, table, lens, ks, vs, scale=0.1, max_context=4096)[0] == 2 * 8 * 128 // 8
    q, k, v, table, lens, ks, vs = cpu_case("fp8", b=1, max_blocks=256, nb=8192)
    assert decode_plan(q, k, v, table, lens, ks, vs, scale=0.1, max_context=2944)[0] == 8 * 92 // 4
    q, k, v, table, lens, ks, vs = cpu_case("fp8", b=1, nq=5, max_blocks=64, nb=64)
    assert decode_plan(q, k, v, table, lens, ks, vs, scale=0.1, max_context=1024)[0] == 8 * 32 // 8


def test_plan_keeps_bf16_on_the_vector_kernel(built_lib):
    # BF16: 3 groups of 4 rows per KV head for 10 rows.
    q, k, v, table, lens, _, _ = cpu_case("bf16", b=16, nq=5, max_blocks=256, nb=8192)
    grid, chunk, ws, cnt = decode_plan(q, k, v, table, lens, None, None, scale=0.1, max_context=3072)
    assert ws == expected_workspace(16, 24, 4, grid) and cnt == expected_counters(16, 24)


def test_plan_rejects_oversized_batches(built_lib):
    q, k, v, table, lens, ks, vs = cpu_case(b=4097)
    with pytest.raises(ValueError, match="exceeds 4096"):
        decode_plan(q, k, v, table, lens, ks, vs, scale=0.1, max_context=16)


def test_stale_binding_is_refused(built_lib):
    a = _lib.DecodeArgs()
    a.struct_size = 12
    with pytest.raises(ValueError, match="stale binding"):
        _lib.check(built_lib.bpt_decode_plan(ctypes.byref(a), None, None))


@pytest.mark.parametrize(
    "change,match",
    [
        (dict(hq=12), "not a multiple"),
        (dict(d=64), "head_dim"),
        (dict(page=12), "power of two"),
    ],
)
def test_plan_rejects_bad_shapes(built_lib, change, match):
    q, k, v, table, lens, ks, vs = cpu_case(**change)
    with pytest.raises(ValueError, match=match):
        decode_plan(q, k, v, table, lens, ks, vs, scale=0.1, max_context=16)


def test_python_layer_rejects_bad_tensors_before_any_gpu_call(built_lib):
    q, k, v, table, lens, ks, vs = cpu_case()
    with pytest.raises(ValueError, match="k_scale and v_scale are required"):
        decode_plan(q, k, v, table, lens, None, None, scale=0.1, max_context=16)
    with pytest.raises(ValueError, match="int32"):
        decode_plan(q, k, v, table, lens.long(), ks, vs, scale=0.1, max_context=16)
    with pytest.raises(ValueError, match="dtype"):
        decode_plan(q, k.view(torch.uint8), v.view(torch.uint8), table, lens, ks, vs, scale=0.1, max_context=16)
    with pytest.raises(ValueError, match="on a GPU"):
        paged_decode_attention(q, k, v, table, lens, ks, vs, scale=0.1, max_context=16)
    with pytest.raises(ValueError, match="takes no scales"):
        qb, kb, vb, tb, lb, _, _ = cpu_case("bf16")
        decode_plan(qb, kb, vb, tb, lb, ks, vs, scale=0.1, max_context=16)


def test_quantize_append_rejects_bad_tensors(built_lib):
    _, k_cache, v_cache, _, _, ks, vs = cpu_case("int8")
    rows = torch.zeros((2, 1, 8, 128), dtype=torch.bfloat16)
    slots = torch.zeros((2, 1), dtype=torch.int32)
    with pytest.raises(ValueError, match="must be \\[2, 1\\]"):
        quantize_append(rows, rows, k_cache, v_cache, ks, vs, slots[:1], slots[:1])
    with pytest.raises(ValueError, match="on a GPU"):
        quantize_append(rows, rows, k_cache, v_cache, ks, vs, slots, slots)
    with pytest.raises(ValueError, match="per-token-head scales"):
        quantize_append(rows, rows, k_cache, v_cache, ks[:3], vs[:3], slots, slots)


def test_append_decode_checks_both_argument_blocks_before_any_gpu_call(built_lib):
    """bpt_paged_append_decode refuses a stale or missing argument block on the host."""
    stale = _lib.AppendArgs()
    stale.struct_size = 12
    with pytest.raises(ValueError, match="stale binding"):
        _lib.check(built_lib.bpt_paged_append_decode(ctypes.byref(stale), None, None))
    empty = _lib.AppendArgs()  # no rows to store: only the decode block is left to check
    empty.struct_size = ctypes.sizeof(_lib.AppendArgs)
    empty.kv_dtype, empty.scale_kind, empty.src_dtype, empty.slot_dtype = 1, 1, 0, 0
    empty.num_kv_heads, empty.head_dim, empty.num_blocks, empty.page_size = 8, 128, 4, 16
    with pytest.raises(ValueError, match="decode args is NULL"):
        _lib.check(built_lib.bpt_paged_append_decode(ctypes.byref(empty), None, None))
    from bpt_amd import paged_append_decode

    q, k, v, table, lens, ks, vs = cpu_case()
    rows = torch.zeros((q.shape[0], 1, 8, 128), dtype=torch.bfloat16)
    slots = torch.zeros((q.shape[0], 1), dtype=torch.int32)
    with pytest.raises(ValueError, match="on a GPU"):
        paged_append_decode(q, rows, rows, k, v, table, lens, ks, vs, slots, slots, scale=0.1, max_context=16)


@pytest.mark.parametrize("fmt", ["fp8", "int8"])
def test_append_decode_refuses_a_bad_decode_block_before_storing(built_lib, fmt):
    """A valid, non-empty append block with a decode block whose workspace is too small: the call is refused on
    the host with the decode's own message, before the store is launched (no GPU here, so any launch would
    surface as a HIP error instead). Per-head FP8 fuses; per-token INT8 takes the two-launch path."""
    from bpt_amd import paged_attention

    q, k, v, table, lens, ks, vs = cpu_case(fmt)
    d, _ = paged_attention._decode_args(q, k, v, table, lens, ks, vs, 0.1, 128, None, torch.bfloat16)
    small = torch.zeros(256, dtype=torch.uint8)
    counters = torch.zeros(4096, dtype=torch.uint8)
    d.out = q.data_ptr()
    d.workspace, d.workspace_bytes = small.data_ptr(), small.numel()
    d.counters, d.counters_bytes = counters.data_ptr(), counters.numel()
    rows = torch.zeros((q.shape[0], 1, 8, 128), dtype=torch.bfloat16)
    slots = torch.zeros((q.shape[0], 1), dtype=torch.int32)
    a = _lib.AppendArgs()
    a.struct_size = ctypes.sizeof(_lib.AppendArgs)
    a.kv_dtype, a.scale_kind = d.kv_dtype, d.scale_kind
    a.src_dtype, a.slot_dtype = 0, 0
    a.batch, a.num_queries, a.num_kv_heads, a.head_dim = q.shape[0], 1, 8, 128
    a.page_size, a.num_blocks = k.shape[1], k.shape[0]
    a.k = a.v = rows.data_ptr()
    a.new_stride_b, a.new_stride_q, a.new_stride_h = rows.stride(0), rows.stride(1), rows.stride(2)
    a.write_blocks = a.write_offsets = slots.data_ptr()
    a.slot_stride_b, a.slot_stride_q = slots.stride(0), slots.stride(1)
    a.k_cache, a.v_cache = k.data_ptr(), v.data_ptr()
    a.kv_stride_block, a.kv_stride_token, a.kv_stride_head = k.stride(0), k.stride(1), k.stride(2)
    a.k_scale, a.v_scale = d.k_scale, d.v_scale
    a.scale_stride_block, a.scale_stride_token, a.scale_stride_head = (
        d.scale_stride_block, d.scale_stride_token, d.scale_stride_head)
    with pytest.raises(ValueError, match="workspace"):
        _lib.check(built_lib.bpt_paged_append_decode(ctypes.byref(a), ctypes.byref(d), None))


def test_tuning_overrides_the_plan_and_resets(built_lib):
    """bpt_set_tuning changes what the auto plan launches (the sweep's knobs) and NULL restores the built-in plan;
    out-of-range values are refused."""
    q, k, v, table, lens, ks, vs = cpu_case(b=32, max_blocks=256, nb=4096)
    base = decode_plan(q, k, v, table, lens, ks, vs, scale=0.1, max_context=4096)
    try:
        _lib.set_tuning(groups_per_cu=3)
        grid, _, _, _ = decode_plan(q, k, v, table, lens, ks, vs, scale=0.1, max_context=4096)
        assert grid == 256 * 3
        _lib.set_tuning(min_chunks=64)
        grid, _, _, _ = decode_plan(q, k, v, table, lens, ks, vs, scale=0.1, max_context=4096)
        assert grid == (32 * 128 * 8 + 63) // 64
        with pytest.raises(ValueError, match="out of range"):
            _lib.set_tuning(groups_per_cu=99)
    finally:
        _lib.set_tuning()
    assert decode_plan(q, k, v, table, lens, ks, vs, scale=0.1, max_context=4096) == base
