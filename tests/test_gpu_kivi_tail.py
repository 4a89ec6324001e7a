"""GPU: the KIVI cache's decode step in one launch, codes + full-precision tail merged (kivi.attend(..., tail=)),
against the oracle restating fastserve's three steps (integration/kv_cache.py:172-185): partial_attention over
the dequantized codes (each row its own length), partial_attention over the tail (every row all of it), then
merge_partials. Tail lengths 0, 1, 31 (one short of a key group) and 64 (the most a call takes); ragged rows,
including rows with no codes (the tail alone); 4- and 8-bit codes and bits-16 caches; the matrix-core kernel
(head dim 128) and the float32 kernel (head dim 64, float32 caches); bf16 / f16 / f32 tails.

Tolerance: fastserve's kernel tests' own (tests/kernels/test_kernels_gpu.py:78-84): rtol 2e-4,
atol 2e-4 * max|want|.
"""

import numpy as np
import pytest
import torch

from oracle import attention as oatt
from oracle import kivi as okivi

from test_gpu_kivi import close, make_cache, make_q

pytestmark = pytest.mark.gpu


def tail_rows(batch, kv_heads, n, d, dtype, seed):
    g = np.random.default_rng(seed)
    k = g.standard_normal((batch, kv_heads, n, d)).astype(np.float32)
    k[..., 3 % d] += 20.0
    v = g.standard_normal((batch, kv_heads, n, d)).astype(np.float32)
    kt, vt = torch.from_numpy(k).to(dtype), torch.from_numpy(v).to(dtype)
    return kt.cuda(), vt.cuda(), kt.float().numpy(), vt.float().numpy()


def want_step(qn, ref, lengths, tk, tv, scale):
    """fastserve's decode branch: codes partial, tail partial, merged (parts that exist)."""
    k_all, v_all = okivi.dequantize_kv(ref)
    outs, lses = [], []
    out, lse = oatt.partial_attention(qn, k_all, v_all, np.asarray(lengths), scale)
    outs.append(out)
    lses.append(lse)
    if tk.shape[2]:
        out, lse = oatt.partial_attention(qn, tk, tv, np.full(len(lengths), tk.shape[2]), scale)
        outs.append(out)
        lses.append(lse)
    return oatt.merge_partials(np.stack(outs, axis=2), np.stack(lses, axis=2))


@pytest.mark.parametrize("bits", [4, 8, 16])
@pytest.mark.parametrize("tail_len", [0, 1, 31, 64])
def test_codes_and_tail_in_one_launch(bits, tail_len):
    from bpt_amd import kivi

    print(f"kivi tail bits {bits} tail {tail_len}", flush=True)
    lengths = [320, 0, 33, 1, 288, 160]
    batch, hkv, hq = len(lengths), 8, 16
    dev, ref = make_cache(batch, hkv, 320, bits, seed=bits + tail_len)
    q, qn = make_q(batch, hq, 5)
    tk, tv, tkn, tvn = tail_rows(batch, hkv, tail_len, 128, torch.bfloat16, 9)
    lens = torch.tensor(lengths, dtype=torch.int32, device="cuda")
    got = kivi.attend(q, dev, lens, 0.1, tail=(tk, tv))
    torch.cuda.synchronize()
    if tail_len:
        close(got, want_step(qn, ref, lengths, tkn, tvn, 0.1), f"bits {bits} tail {tail_len}")
    else:  # no tail: the plain attend, a row without codes gives zeros
        close(got, okivi.attend(qn, ref, np.array(lengths), 0.1), f"bits {bits} no tail")


@pytest.mark.parametrize("tail_dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("q_heads", [8, 32])
def test_tail_dtypes_and_head_ratios(tail_dtype, q_heads):
    """f16 / f32 tails and q; 1 and 4 query heads per KV head; a long row split over many workgroups."""
    from bpt_amd import kivi

    lengths = [4096, 17, 0, 2048]
    dev, ref = make_cache(len(lengths), 8, 4096, 4, seed=3)
    q, qn = make_q(len(lengths), q_heads, 6, dtype=tail_dtype)
    tk, tv, tkn, tvn = tail_rows(len(lengths), 8, 31, 128, tail_dtype, 10)
    got = kivi.attend(q, dev, torch.tensor(lengths, dtype=torch.int32, device="cuda"), 0.088, tail=(tk, tv))
    torch.cuda.synchronize()
    close(got, want_step(qn, ref, lengths, tkn, tvn, 0.088), f"{tail_dtype} G {q_heads // 8}")


@pytest.mark.parametrize("bits", [4, 16])
def test_tail_on_the_float32_kernel(bits):
    """Head dim 64 (and a float32 bits-16 cache) take the float32 kernel; the tail is one more block there."""
    from bpt_amd import kivi

    lengths = [96, 0, 40]
    half = torch.float32 if bits == 16 else torch.float16
    dev, ref = make_cache(len(lengths), 4, 96, bits, seed=4, half=half, d=64)
    q, qn = make_q(len(lengths), 8, 8, dtype=torch.float32, d=64)
    tk, tv, tkn, tvn = tail_rows(len(lengths), 4, 31, 64, torch.float32, 11)
    got = kivi.attend(q, dev, torch.tensor(lengths, dtype=torch.int32, device="cuda"), 0.125, tail=(tk, tv))
    torch.cuda.synchronize()
    close(got, want_step(qn, ref, lengths, tkn, tvn, 0.125), f"float32 kernel bits {bits}")


def test_tail_argument_checks():
    from bpt_amd import kivi

    dev, _ = make_cache(2, 8, 64, 8, seed=1)
    q, _ = make_q(2, 16, 2)
    lens = torch.tensor([64, 64], dtype=torch.int32, device="cuda")
    tk, tv, _, _ = tail_rows(2, 8, 65, 128, torch.bfloat16, 3)
    with pytest.raises(ValueError, match="tail_len"):
        kivi.attend(q, dev, lens, 0.1, tail=(tk, tv))
    tk, tv, _, _ = tail_rows(2, 4, 8, 128, torch.bfloat16, 3)
    with pytest.raises(ValueError, match="tail keys and values"):
        kivi.attend(q, dev, lens, 0.1, tail=(tk, tv))
