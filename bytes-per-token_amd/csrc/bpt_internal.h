// Kernel parameter blocks and launchers shared between the kernel files and the C-ABI layer.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#ifndef BPT_DECODE_LOADS
#define BPT_DECODE_LOADS 4
#endif
#ifndef BPT_DECODE_LOADS_RG4
#define BPT_DECODE_LOADS_RG4 4
#endif
#ifndef BPT_DECODE_GROUPS_PER_CU
#define BPT_DECODE_GROUPS_PER_CU 2
#endif
#ifndef BPT_DECODE_MIN_CHUNKS_MANY_ROWS
#define BPT_DECODE_MIN_CHUNKS_MANY_ROWS 8
#endif
#ifndef BPT_DECODE_WAVES
#define BPT_DECODE_WAVES 4
#endif
#ifndef BPT_DECODE_MFMA_WAVES_PER_SIMD
#define BPT_DECODE_MFMA_WAVES_PER_SIMD 2
#endif
#ifndef BPT_DECODE_PIECE_COST
#define BPT_DECODE_PIECE_COST 8
#endif
#ifndef BPT_DECODE_MANY_ROW_PIECE_COST
#define BPT_DECODE_MANY_ROW_PIECE_COST 10
#endif
#ifndef BPT_DECODE_MFMA_MIN_ROWS
#define BPT_DECODE_MFMA_MIN_ROWS 2
#endif
#ifndef BPT_DECODE_MFMA_MIN_ROWS_INT8
#define BPT_DECODE_MFMA_MIN_ROWS_INT8 5
#endif

namespace bpt {

constexpr int kHeadDim = 128;
// Largest batch the decode kernel takes: its per-sequence prefix sum lives in LDS.
constexpr int kMaxBatch = 4096;
// Waves per decode workgroup.
constexpr int kDecodeWaves = BPT_DECODE_WAVES;
// Compute units of an MI355X; the auto plan launches kDecodeGroupsPerCu workgroups per CU.
constexpr int kComputeUnits = 256;
constexpr int kDecodeGroupsPerCu = BPT_DECODE_GROUPS_PER_CU;
// Matrix-core segments of kManyRows rows or more run in workgroups of kMfmaManyRowWaves waves, one per CU,
// and the auto plan launches no more of them than a max_context batch fills with kDecodeMinChunksManyRows
// chunks each. Their pieces are dear (the merge, partial and combine of up to 16 rows), so fewer, fuller
// workgroups win.
constexpr int kManyRows = 8;
constexpr int kMfmaManyRowWaves = 8;
constexpr int kDecodeMinChunksManyRows = BPT_DECODE_MIN_CHUNKS_MANY_ROWS;
// Workgroups per CU of the vector kernel. INT8 caches run three (12 waves per CU, three per SIMD; those
// kernels are compiled to fit 168 VGPRs for it) with one row per group, and with two when pages hold whole
// 8-row loads and q is bf16 (the other two-row instances would spill at 168); everything else runs two.
// INT8's per-chunk work leaves two waves per SIMD short of memory-level parallelism: on the INT8 workload
// three took the call from 202 to 192 us.
constexpr int kDecodeGroupsPerCuInt8 = 3;
constexpr int decode_groups_per_cu(bool int8, int rows_per_group, bool page_uniform, bool q_split) {
  return int8 && (rows_per_group == 1 || (rows_per_group == 2 && page_uniform && !q_split)) ? kDecodeGroupsPerCuInt8
                                                                                            : kDecodeGroupsPerCu;
}
// Fewest chunks the auto plan gives a workgroup (it launches fewer workgroups for small batches rather than
// thinner ones): many-row matrix-core segments kDecodeMinChunksManyRows, other matrix-core segments one per
// wave, INT8 on the vector kernel two per wave, everything else one. Measured on one sequence of the
// 1.7B shape: FP8 (2 rows, 2943 tokens) 15.7 -> 13.0 us, INT8 (8192 tokens) 26.2 -> 19.3 us; BF16's
// 16-token chunks are best one per workgroup (the 512-token BF16 call: 10.9 us, 11.4 with four).
constexpr int kDecodeMinChunksMfma = 4;
constexpr int kDecodeMinChunksInt8 = 8;
// Matrix-core segments of fewer than kManyRows rows take two chunks per wave instead while that still
// launches at least one workgroup per two CUs: FP8 (2 rows) batches of 2, 3 and 4 sequences 15.2 -> 13.5,
// 15.4 -> 14.0 and 15.0 -> 14.5 us; one sequence keeps one chunk per wave (12.9 us with 184 workgroups, 13.7
// with 92), and INT8's vector kernel and many-row segments were slower with twice their minimum.
constexpr int kDecodeMinChunksMfmaWide = 8;
constexpr int64_t decode_min_chunks(bool mfma, int rows, bool int8, int64_t chunks) {
  return mfma ? (rows >= kManyRows ? kDecodeMinChunksManyRows
                                   : (chunks / kDecodeMinChunksMfmaWide >= kComputeUnits / 2 ? kDecodeMinChunksMfmaWide
                                                                                             : kDecodeMinChunksMfma))
              : (int8 ? kDecodeMinChunksInt8 : 1);
}
// KIVI calls with a few very long (sequence, KV head) segments launch one workgroup per CU: every segment
// is then split over half as many workgroups, and the last one to finish combines half as many partials.
// Measured (4-bit / 8-bit / bf16): 1 x 32768 tokens, 8 KV heads 26.0 -> 24.1, 28.3 -> 27.6, 41.7 -> 39.8 us;
// with 32 segments (4 x 32768) or short ones (1 x 2048) the halved grid cost up to 10 us instead.
constexpr int kKiviFewSegments = 8;
constexpr int kKiviLongSegmentChunks = 512;
// The KIVI kernel's fewest chunks per workgroup: one per wave while the call's chunks number no more than the
// largest grid, two per wave beyond. Measured on INT8 caches: 1 x 2048 tokens 21.0 -> 14.0 us and 4 x 512
// 16.1 -> 13.2 (4 instead of 1); 1 x 8192 22.8 -> 18.5, 4 x 2048 18.2 -> 16.0 and 16 x 512 16.3 -> 15.5 (8
// instead of 4, which costs 1 us on the 512-chunk shapes); 16 or 32 were no better anywhere.
constexpr int kKiviMinChunksSmall = 4;
constexpr int kKiviMinChunks = 8;
constexpr int64_t kivi_min_chunks(int64_t chunks, int64_t max_grid) {
  return chunks <= max_grid ? kKiviMinChunksSmall : kKiviMinChunks;
}
// Small and mid-size calls on the vector kernel (BF16 caches up to kAlignedMaxChunksBf16 chunks in all, INT8
// up to kAlignedMaxChunksInt8): when every sequence has the same length (the kernel checks, in LDS, while it
// builds the segment line), about 4 sqrt(chunks) workgroups (at most 512; the launch holds at least that
// many) cut equal partitions of a power-of-two number of chunks, the fewest that they cover, as a caller's
// num_splits would: no piece cost, and every KV head of a sequence covers the same tokens at the same time
// (per-token scale lines, which hold all heads, are read once). The rest of the launch leaves at once;
// ragged batches keep the line cut over the whole launch. A single sequence gets its partitions from the
// plan directly (no check in the kernel). Measured on equal lengths against the line cut:
// BF16 1 x 512 tokens 12.9 -> 12.2 us, 1 x 2048 18.0 -> 15.1, 2 x 2048 19.2 -> 17.0; INT8 1 x 2048
// 17.6 -> 16.3, 4 x 8192 29.6 -> 28.1, 16 x 2048 29.3 -> 28.5; ragged batches within 0.3 us. INT8 at
// 16 x 8192 and beyond is faster on the line cut with three workgroups per CU (62.6 against 65.4 us).
constexpr int64_t kAlignedMaxChunksBf16 = 32768;
constexpr int64_t kAlignedMaxChunksInt8 = 16384;
constexpr int64_t kAlignedMaxGrid = 512;

// Matrix-core workgroups per CU for segments of `rows` rows (8-wave workgroups from kManyRows rows on, else
// 4-wave ones; the plan picks 2-wave ones over many segments, kMfmaPairGroupsPerCu to a CU).
constexpr int mfma_groups_per_cu(int rows) { return rows >= kManyRows ? 1 : kDecodeGroupsPerCu; }
// Stream-K line units charged for each segment start, in chunks: the cost of merging one more piece (the
// wave merge, the partial's round trip and, for one workgroup, the combine), so that a workgroup whose
// range starts a segment gets correspondingly fewer chunks.
constexpr int kDecodePieceCost = BPT_DECODE_PIECE_COST;
// The same for matrix-core segments of kManyRows rows or more (8-wave workgroups; dearer merges).
constexpr int kManyRowPieceCost = BPT_DECODE_MANY_ROW_PIECE_COST;
constexpr int kMaxPieceCost = kDecodePieceCost > kManyRowPieceCost ? kDecodePieceCost : kManyRowPieceCost;
// Few-row matrix-core calls over many segments (at least kMfmaPairMinSegments (sequence, KV head) pairs, an
// automatic split) run in workgroups of kMfmaPairWaves waves, kMfmaPairGroupsPerCu to a CU (the same waves
// per SIMD), charged kMfmaPairPieceCost per segment: with two waves dealing a piece's chunks, a range's last
// round leaves at most one wave idle. Measured against four-wave workgroups: 128 to 1024 segments of ragged
// lengths 1-6 % faster, equal lengths within 1 %; 64 or fewer segments, or a fixed split count over long
// sequences, 2-20 % slower (those keep four waves).
constexpr int kMfmaPairWaves = 2;
constexpr int kMfmaPairGroupsPerCu = 4;
constexpr int kMfmaPairPieceCost = 4;
constexpr int kMfmaPairMinSegments = 128;

// 16-byte K loads (and V loads) per lane per chunk: fewer for 4-row groups, whose q and accumulators take
// twice the registers.
constexpr int decode_loads(int rows_per_group) { return rows_per_group >= 4 ? BPT_DECODE_LOADS_RG4 : BPT_DECODE_LOADS; }

// Matrix-core decode: FP8 KV heads with kMfmaMinRows .. kMfmaRows rows per sequence (Q * G), INT8 ones with
// kMfmaMinRowsInt8 .. kMfmaRows, are computed as one 16-row group in 32-token chunks (for FP8 faster than
// the vector kernel from 2 rows up: its per-token VALU work is shared by all rows).
constexpr int kMfmaMinRows = BPT_DECODE_MFMA_MIN_ROWS;
constexpr int kMfmaMinRowsInt8 = BPT_DECODE_MFMA_MIN_ROWS_INT8;
constexpr int kMfmaRows = 16;
constexpr int kMfmaChunk = 32;
// Waves per SIMD the matrix-core decode kernel is compiled for (its register budget: 512 / this).
constexpr int kMfmaWavesPerSimd = BPT_DECODE_MFMA_WAVES_PER_SIMD;

// Launch-ready form of bpt_decode_args (cache strides in bytes).
struct DecodeParams {
  const void* q;
  int64_t q_sb, q_sq, q_sh;
  const uint8_t* k;
  const uint8_t* v;
  int64_t kv_sblk, kv_stok, kv_shead;  // bytes
  const float* ks;
  const float* vs;
  int64_t sc_sblk, sc_stok, sc_shead;  // elements
  const void* table;
  int64_t table_sb;
  const int32_t* lens;
  void* out;
  int64_t o_sb, o_sq, o_sh;
  float* ws_out;       // [slots, RG, D] normalized partial outputs
  float* ws_lse;       // [slots, RG] log2-sum-exp of each partial
  unsigned* counters;  // [B * HR] arrivals per segment; zero between calls
  int B, Q, Hq, Hkv, G, P, logP, num_blocks, max_blocks, len_cap;
  int n_rg, HR;      // row groups per KV head; segments per sequence (Hkv * n_rg)
  int waves;         // matrix-core kernel: waves per workgroup (kMfmaPairWaves, kDecodeWaves or kMfmaManyRowWaves)
  int grid;          // workgroups launched
  int64_t per_forced;  // chunks per workgroup when the caller fixed the split count, else 0
  int piece_cost;      // line units charged per segment start (0 with a fixed split count)
  int equal_grid;      // > 0: if every sequence has the same length, the first equal_grid workgroups cut
                       // equal power-of-two partitions instead and the others leave
  float qscale;      // sm_scale * log2(e)
  int q_dtype, out_dtype, table_i64;
  int noncausal;        // every query sees all of its sequence's tokens
  int len_offset;       // subtracted from every context length
  float* lse_out;       // optional [B, Q, Hq]: each row's log-sum-exp (natural log)
  const float* merge_out;  // optional [B, Q, Hq, D]: another token range's normalized partial, merged into out
  const float* merge_lse;  // its log-sum-exp [B, Q, Hq] (natural log, -inf when empty)
  // Quantize-on-write in the same launch (fuse_q > 0, matrix-core kernel, per-head scales): the bf16 rows
  // [B, fuse_q, Hkv, D] of the last fuse_q tokens of every sequence, stored to their slots and used for
  // those tokens in place of what the pool held.
  int fuse_q;
  const uint16_t* nk;
  const uint16_t* nv;
  int64_t n_sb, n_sq, n_sh;  // elements
  const void* w_blocks;
  const void* w_offsets;
  int64_t w_sb, w_sq;
  int w_i64;
};

struct AppendParams {
  const void* k;
  const void* v;
  int64_t n_sb, n_sq, n_sh;
  const void* blocks;
  const void* offsets;
  int64_t s_sb, s_sq;
  uint8_t* kc;
  uint8_t* vc;
  int64_t kv_sblk, kv_stok, kv_shead;  // bytes
  float* ks;
  float* vs;
  int64_t sc_sblk, sc_stok, sc_shead;  // elements
  int B, Q, Hkv, P, num_blocks;
  int src_dtype, slot_i64;
  // in_place: store only the rows whose slot is where the decode reads the sequence's token lens[b] - Q + qi
  // (slot_is_token), reading the decode's block table and lengths (bpt_paged_append_decode's rule).
  int in_place;
  const void* table;
  int64_t table_sb;
  int table_i64, max_blocks, logP;
  const int32_t* lens;
};

// Launch-ready form of bpt_kivi_args: decode attention over a KIVI cache (asymmetric 4/8-bit codes with
// float16 grids, or float16 / bfloat16 keys and values), one partial result per split.
struct KiviParams {
  const void* q;
  int64_t q_sb, q_sh;  // elements
  const uint8_t* kc;
  const uint8_t* vc;
  int64_t c_sb, c_sh, c_st;  // bytes
  const uint16_t* ks;        // float16 key grid [B, Hkv, groups, D]
  const uint16_t* kz;
  int64_t g_sb, g_sh, g_sg;  // elements
  const uint16_t* vs;        // float16 value grid [B, Hkv, T]
  const uint16_t* vz;
  int64_t t_sb, t_sh;  // elements
  const int32_t* lens;
  float* out;  // [B, Hq, S, D]
  int64_t o_sb, o_sh, o_ss;
  float* lse;  // [B, Hq, S]
  int64_t l_sb, l_sh, l_ss;
  float* ws_out;       // [2 * grid, G, D] normalized partials
  float* ws_lse;       // [2 * grid, G] their log2-sum-exp
  unsigned* counters;  // [B * Hkv * S] arrivals per (sequence, KV head, split); zero between calls
  int B, Hq, Hkv, G, S;
  int cps;      // chunks per split
  int gshift;   // log2(chunks per key group)
  int len_cap;  // lengths are clamped to this (the laid-out tokens, and the splits' reach)
  int len_offset;  // always 0 here (the paged decode's parameter of the same name)
  int grid;
  float qscale;  // sm_scale * log2(e)
  int q_dtype;
  int D, split;       // head dim; tokens per split
  int gshift_tokens;  // log2(tokens per key group)
  // Full-precision tail merged into the (single) split's result: [B, Hkv, tail_len, D], strides in elements.
  const void* tk;
  const void* tv;
  int64_t tk_sb, tk_sh, tk_st;
  int tail_dtype, tail_len;
};

// The most tail tokens a KIVI call takes (a tail is shorter than a key group).
constexpr int kKiviMaxTail = 64;

// Launch-ready form of bpt_kivi_quant_args: KIVI quantize-on-write of keys and values [B, Hkv, T, D].
struct KiviQuantParams {
  const void* k;
  const void* v;
  int64_t x_sb, x_sh, x_st;  // elements (channel stride 1)
  int src_dtype;
  uint8_t* kc;
  uint8_t* vc;
  int64_t c_sb, c_sh, c_st;  // bytes
  uint16_t* ks;              // float16 key grid [B, Hkv, T / group, D]
  uint16_t* kz;
  int64_t g_sb, g_sh, g_sg;  // elements
  uint16_t* vs;              // float16 value grid [B, Hkv, T]
  uint16_t* vz;
  int64_t t_sb, t_sh;  // elements (token stride 1)
  int B, Hkv, T, D, group, bits;
};

// Launch-ready form of bpt_prepare_args: per-forward paged metadata from device positions.
struct PrepareParams {
  const int32_t* table;     // [num_slots, table_stride] block ids of each slot's sequence
  int64_t table_stride;
  const int32_t* reserved;  // [num_slots] blocks reserved per slot
  const int32_t* slots;     // [B] each row's slot
  const void* positions;    // [B, Q] int32 / int64
  int64_t pos_sb, pos_sq;
  int pos_i64;
  int32_t* block_table;     // [B, n_blocks]
  int32_t* write_blocks;    // [B, Q]
  int32_t* write_offsets;   // [B, Q]
  int32_t* context_lens;    // [B]
  int B, Q, n_blocks, num_slots, max_blocks, P, logP;
};

// Launch-ready form of bpt_norm_quant_args.
struct NormQuantParams {
  const void* x;
  int64_t x_rs;  // elements between rows (channel stride 1)
  const void* w;
  int8_t* codes;
  int64_t c_rs;
  float* scale;
  int rows, d;
  float eps;
  int x_dtype, w_dtype;
};

// KIVI storage formats of bpt_kivi_args.bits / kv_dtype.
constexpr int kKivi4 = 0;
constexpr int kKivi8 = 1;
constexpr int kKiviF16 = 2;
constexpr int kKiviBf16 = 3;
constexpr int kKiviF32 = 4;

int decode_rows_per_load(int kv_dtype);
int decode_chunk_tokens(int kv_dtype, int rows_per_group);
// Optional events recorded around a kernel's own execution (hipExtLaunchKernel) when `start` is set.
struct LaunchEvents {
  hipEvent_t start = nullptr, stop = nullptr;
};

template <typename K, typename... A>
inline void launch_kernel(K kernel, dim3 grid, dim3 block, size_t lds, hipStream_t stream, const LaunchEvents& ev,
                          const A&... args) {
  if (ev.start) hipExtLaunchKernelGGL(kernel, grid, block, (uint32_t)lds, stream, ev.start, ev.stop, 0u, args...);
  else hipLaunchKernelGGL(kernel, grid, block, lds, stream, args...);
}

hipError_t launch_decode(const DecodeParams& p, int kv_dtype, int scale_kind, int rows_per_group, hipStream_t stream,
                         const LaunchEvents& ev = {});
hipError_t launch_decode_mfma(const DecodeParams& p, int kv_dtype, int scale_kind, hipStream_t stream,
                              const LaunchEvents& ev = {});
hipError_t launch_kivi(const KiviParams& p, int fmt, hipStream_t stream);
// Any even head dim up to 256 and float32 bits-16 caches: one workgroup per (sequence, KV head, split).
hipError_t launch_kivi_any(const KiviParams& p, int fmt, hipStream_t stream);
hipError_t launch_norm_quant(const NormQuantParams& p, bool vec8, hipStream_t stream);
hipError_t launch_kivi_quantize(const KiviQuantParams& p, hipStream_t stream);
hipError_t launch_paged_prepare(const PrepareParams& p, hipStream_t stream);
hipError_t launch_append(const AppendParams& p, int kv_dtype, int scale_kind, int head_dim, hipStream_t stream);
hipError_t launch_fp8_table(float* out, hipStream_t stream);
hipError_t launch_fp8_encode(const float* x, float scale, uint8_t* out, int64_t n, hipStream_t stream);
int64_t read_probe_groups(uint64_t bytes);
hipError_t launch_read_probe(const void* buf, uint64_t bytes, float* partial, hipStream_t stream,
                             const LaunchEvents& ev = {});
// The decode's ranges read only (p.grid workgroups, p.HR segments per sequence, `chunk`-token chunks).
hipError_t launch_page_read_probe(const DecodeParams& p, int row_bytes, int chunk, bool with_scales, float* partial,
                                  hipStream_t stream, const LaunchEvents& ev = {});
hipError_t launch_copy_probe(void* dst, const void* src, uint64_t bytes, hipStream_t stream);

}  // namespace bpt
