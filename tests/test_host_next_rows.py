"""Host-side behaviour of the KIVI decode, the RMSNorm + INT8 kernel and the cascade, on the CPU: the plans,
the argument checks (ValueError before anything is launched, as kernels/kv_attention.py:216-217 raises),
fastserve's default_split known answers, and how the cascade cuts a group's queries into 16-row passes.
No compute call is made."""

import ctypes
from types import SimpleNamespace

import pytest
import torch

from bpt_amd import _lib, cascade, kivi


def kivi_args(**over):
    a = _lib.KiviArgs()
    a.struct_size = ctypes.sizeof(_lib.KiviArgs)
    vals = dict(format=_lib.KIVI_INT8, q_dtype=_lib.F_BF16, batch=2, num_q_heads=16, num_kv_heads=8, head_dim=128,
                tokens=4096, group=32, num_groups=128, split=128, num_splits=32, sm_scale=0.088)
    vals.update(over)
    for k, v in vals.items():
        setattr(a, k, v)
    return a


def plan(a):
    ws, cnt = ctypes.c_size_t(0), ctypes.c_size_t(0)
    rc = _lib.lib().bpt_kivi_plan(ctypes.byref(a), ctypes.byref(ws), ctypes.byref(cnt))
    return rc, ws.value, cnt.value


def test_kivi_plan_sizes(built_lib):
    a = kivi_args()
    rc, ws, cnt = plan(a)
    assert rc == 0
    grid = a.grid_groups
    assert grid == 256  # 2 x 8 heads x 128 chunks = 2048 chunks, more than one launch of 512: 8 per workgroup
    assert ws == (2 * grid * 2 * (128 + 1) * 4 + 255) // 256 * 256  # two slots per workgroup, 2 rows each
    assert cnt == (2 * 8 * 32 * 4 + 255) // 256 * 256  # one counter per (sequence, KV head, split)
    big = kivi_args(batch=8, tokens=4096, num_splits=32)
    assert plan(big)[0] == 0 and big.grid_groups == 512  # 8192 chunks: the full launch of 2 groups per CU
    mid = kivi_args(batch=1, tokens=2048, num_groups=64, split=128, num_splits=16)
    assert plan(mid)[0] == 0 and mid.grid_groups == 128  # 512 chunks, no more than one launch: 4 per workgroup
    small = kivi_args(batch=1, tokens=64, num_groups=2, split=64, num_splits=1)
    assert plan(small)[0] == 0 and small.grid_groups == 4  # 16 chunks: one per wave of 4 workgroups


def test_kivi_plan_other_head_dims_and_float32_take_the_float32_kernel(built_lib):
    """Head dims other than 128, and float32 caches, run one workgroup per (sequence, KV head, split) with no
    workspace; the 32-token rules of the matrix-core kernel do not apply to them."""
    for over in (dict(head_dim=16), dict(head_dim=64), dict(format=_lib.KIVI_F32)):
        a = kivi_args(**over)
        rc, ws, cnt = plan(a)
        assert rc == 0 and ws == 0 and cnt == 0 and a.grid_groups == 2 * 8 * 32
    a = kivi_args(head_dim=16, tokens=4090, format=_lib.KIVI_F32, split=10, group=2, num_splits=409)
    assert plan(a)[0] == 0 and a.grid_groups == 2 * 8 * 409


@pytest.mark.parametrize(
    "over,msg",
    [
        (dict(group=48, split=96), "power of two"),
        (dict(group=64, num_groups=64, split=96), "multiple of the key group"),
        (dict(group=64, split=64, num_groups=64, tokens=4064), "whole number of groups"),
        (dict(head_dim=258), "head_dim"),
        (dict(head_dim=63), "head_dim"),
        (dict(num_q_heads=136), "query heads per KV head"),
        (dict(tokens=4090), "multiple of 32"),
        (dict(num_groups=100), "do not cover"),
        (dict(format=7), "unknown format"),
    ],
)
def test_kivi_plan_refusals(built_lib, over, msg):
    rc, _, _ = plan(kivi_args(**over))
    assert rc == _lib.BPT_ERR_INVALID_ARGUMENT and msg in _lib.lib().bpt_last_error().decode()


def test_default_split_known_answers():
    # tests/kernels/test_kernels_gpu.py:136-142
    assert kivi.default_split(1, 8, 32768) == 128
    assert kivi.default_split(64, 8, 8192) == 256
    assert kivi.default_split(1, 8, 100) == 128
    assert all(kivi.default_split(b, 8, t) % 32 == 0 for b in (1, 3, 64) for t in (1, 1000, 30000))


def test_kivi_split_rule_is_checked_before_anything_runs():
    kv = SimpleNamespace(bits=8, group=32, k_codes=torch.zeros((1, 8, 64, 128), dtype=torch.uint8))
    q = torch.zeros((1, 16, 128))
    with pytest.raises(ValueError, match="multiple of the key group 32"):
        kivi.decode_attention(q, kv, torch.zeros(1, dtype=torch.int32), 0.1, split=48)
    with pytest.raises(ValueError, match="multiple of the key group 32"):
        kivi.attend(q, kv, torch.zeros(1, dtype=torch.int32), 0.1, split=40)


def test_norm_quant_needs_gpu_tensors():
    from bpt_amd import rms_norm_int8

    with pytest.raises(ValueError, match="runs on a GPU"):
        rms_norm_int8(torch.zeros(2, 8), torch.ones(8), 1e-6)
    with pytest.raises(ValueError, match="weight must be"):
        rms_norm_int8(torch.zeros(2, 8), torch.ones(4), 1e-6)


def test_cascade_rows_per_pass():
    assert cascade._rows_per_pass(80, 2) == 8  # 16 sequences x 5 queries, 2 heads per KV head: 10 passes of 16 rows
    assert cascade._rows_per_pass(15, 2) == 5
    assert cascade._rows_per_pass(7, 4) == 1
    assert cascade._rows_per_pass(12, 1) == 12


def test_cascade_argument_checks():
    q = torch.zeros((4, 1, 16, 128))
    pool = torch.zeros((32, 16, 8, 128), dtype=torch.bfloat16)
    table = torch.zeros((4, 8), dtype=torch.int32)
    lens = torch.full((4,), 100, dtype=torch.int32)
    kw = dict(scale=0.1, max_context=128, prefix_pages=2)
    with pytest.raises(ValueError, match="groups must"):
        cascade.cascade_decode_attention(q, pool, pool, table, lens, groups=[(0, 2), (3, 4)], **kw)
    with pytest.raises(ValueError, match="cover the whole batch"):
        cascade.cascade_decode_attention(q, pool, pool, table, lens, groups=[(0, 3)], **kw)
    with pytest.raises(ValueError, match="end inside the shared prefix"):
        cascade.cascade_decode_attention(q, pool, pool, table, lens, context_lens_host=[100, 20, 100, 100], **kw)
    with pytest.raises(ValueError, match="prefix_pages"):
        cascade.cascade_decode_attention(q, pool, pool, table, lens, scale=0.1, max_context=128, prefix_pages=0)
