"""The oracle: a CPU restatement (numpy) of fastserve's arithmetic for the paged decode-attention path.

TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg may import
this package, and only to check results (or as the timed CPU baseline), never as part of the product path. The
HIP library has no CPU fallback and never calls into this package.

Each function cites the fastserve file:line (relative to src/fastserve/) whose arithmetic it restates:

* fp8.py        e4m3fn encode (round to nearest even, NaN past the range) and decode
                  - kv/quant.py:44-45 (the FP8 cast), quant/formats.py:39-68 (E4M3 RNE, representable values)
* quant.py      the write-path quantizers
                  - FP8 static per-head: clamp(x / scale, ±448) -> e4m3fn (kv/quant.py:44-45)
                  - per-token dynamic: scale = max(amax / 127 (or 448), 1e-12), codes = clamp(round(x/s))
                    (quant/w8a8.py:55-74, kernels/reference.py:44-55)
* paged.py      PagedKVCache's metadata and layout (engine/kv_cache.py:90-169): block tables padded with
                block 0, write_blocks / write_offsets, gather of a sequence's pages
* attention.py  partial_attention / merge_partials (kernels/reference.py:186-211), causal multi-query
                attention by absolute position (engine/attention.py:12-47), the paged decode the HIP kernel
                computes, and default_split (kernels/kv_attention.py:178-187)
* torch_paged.py the same paged decode in float32 PyTorch, computed as fastserve's CPU path does (padded
                gather engine/kv_cache.py:140-169, attention engine/attention.py:12-47): the timed CPU baseline

How each is pinned (tests/test_oracle_*.py): the FP8 codec against torch's float8_e4m3fn cast on all 256
codes, every tie and multi-scale randoms; the INT8 quantizer against the reference tests' known answers and
a brute-force nearest-code search; attention against float64 brute-force loops, closed forms (uniform
scores give the mean of V, one visible token gives its value), split-merge exactness, empty rows, the GQA
head mapping and causal visibility; default_split against the reference tests' known answers; torch_paged
against attention.paged_decode on every cache format.
"""
