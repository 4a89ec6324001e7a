/*
 * bpt_amd.h — C ABI of the MI355X (gfx950) paged decode-attention path.
 *
 * Everything here takes plain device pointers, element strides and sizes; no framework types cross the
 * boundary. Every entry point returns 0 on success, BPT_ERR_INVALID_ARGUMENT for a caller mistake found
 * on the host (nothing launched), or BPT_ERR_HIP for a HIP runtime error; bpt_last_error() then holds a
 * thread-local message. Launches go on the caller's stream; nothing synchronizes with the host, so every
 * call can be captured in a HIP graph. The caller owns caches, block tables, lengths and outputs; the
 * library writes only outputs and the caller-provided workspace.
 *
 * Reference interfaces replaced (paths relative to the fastserve source tree, src/fastserve/):
 *   bpt_paged_decode     kernels/kv_attention.py:190-245 decode_attention (launcher) and :56-175 (the
 *                        kernel), kernels/reference.py:205-211 merge_partials (the split-K combine), read
 *                        through engine/kv_cache.py:165-169 PagedKVCache._gather's block-table layout,
 *                        with engine/attention.py:12-20 causal_mask for several queries per sequence.
 *   bpt_quant_append     engine/kv_cache.py:158-161 PagedKVCache.update (scatter write by write_blocks /
 *                        write_offsets) fused with the quantizers kv/quant.py:44-45 (FP8 cast) and
 *                        quant/w8a8.py:55-74 / kernels/reference.py:44-55 (per-token INT8, amax/127).
 *   bpt_paged_prepare    engine/kv_cache.py:140-156 PagedKVCache.prepare (the per-forward PagedMeta), built on
 *                        the device from device positions.
 *   bpt_decode_plan      kernels/kv_attention.py:178-187 default_split (tokens per program) and the
 *                        out/lse allocation of :218-220, as a host-only planning call.
 *   bpt_kivi_decode      kernels/kv_attention.py:190-245 decode_attention (launcher) and :56-175 (the
 *                        kernel) over kernels/reference.py:66-160's QuantKV (KIVI asymmetric 4/8-bit codes
 *                        with float16 grids, or float16 / bfloat16 keys and values): one partial
 *                        (out, lse) per split, as that launcher returns them.
 *   bpt_kivi_plan        the workspace / counter sizing for bpt_kivi_decode (host only).
 *   bpt_kivi_quantize    kernels/reference.py:103-160 quantize_kv (KIVI codes and float16 grids), where
 *                        integration/kv_cache.py:139-158 QuantizedKVCache._append quantizes completed groups.
 *   bpt_rms_norm_int8    kernels/norm_quant.py:43-109 rms_norm_int8 (kernel 1), defined by
 *                        kernels/reference.py:44-55: RMSNorm fused with per-token INT8 quantization.
 */
#ifndef BPT_AMD_H
#define BPT_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define BPT_ABI_VERSION 13

/* return codes */
#define BPT_OK 0
#define BPT_ERR_INVALID_ARGUMENT 1
#define BPT_ERR_HIP 2

/* element type of the KV cache pools */
typedef enum {
  BPT_KV_BF16 = 0,        /* no quantization: bfloat16 keys and values                         */
  BPT_KV_FP8_E4M3FN = 1,  /* OCP e4m3fn codes (0x7F/0xFF NaN, max 448), static per-head scale  */
  BPT_KV_INT8 = 2         /* symmetric int8 codes, dynamic per-(token, head) scale amax/127     */
} bpt_kv_dtype;

/* how the fp32 scales are laid out */
typedef enum {
  BPT_SCALE_NONE = 0,            /* BF16 cache                                      */
  BPT_SCALE_PER_HEAD = 1,        /* k_scale[Hkv], v_scale[Hkv]                       */
  BPT_SCALE_PER_TOKEN_HEAD = 2   /* [num_blocks, page_size, Hkv], same paging as codes */
} bpt_scale_kind;

/* element type of q / new k, v rows and of the output */
typedef enum { BPT_F_BF16 = 0, BPT_F_F16 = 1, BPT_F_F32 = 2 } bpt_float_dtype;

/* element type of block tables and write-slot tensors */
typedef enum { BPT_IDX_I32 = 0, BPT_IDX_I64 = 1 } bpt_index_dtype;

/*
 * Paged decode attention, Q >= 1 queries per sequence, causal within the query block.
 *
 *   q            [B, Q, Hq, D]   strides q_stride_{b,q,h} (elements; channel stride 1)
 *   k/v_cache    [num_blocks, page_size, Hkv, D] by default; any layout expressible by
 *                kv_stride_{block,token,head} (elements of the cache type; channel stride 1), so the
 *                head-major pool [num_blocks, Hkv, page_size, D] and a contiguous [B, Hkv, T, D] cache
 *                (block b*T/P + t/P, head stride T*D) use the same kernels.
 *   k/v_scale    fp32; PER_HEAD: [Hkv]; PER_TOKEN_HEAD: strides scale_stride_{block,token,head}
 *   block_table  [B, max_blocks_per_seq] (row stride table_stride_b) physical page of each logical page
 *   context_lens [B] int32: tokens in the cache for each sequence, the Q new ones included. Query i of
 *                sequence b sits at position context_lens[b] - Q + i and sees slots 0 .. that position.
 *                NULL: every sequence holds max_context tokens.
 *   out          [B, Q, Hq, D] (strides out_stride_{b,q,h}), BF16, F16 or F32
 *
 * max_context bounds context_lens and sizes the launch (no device->host read); lengths above it, or
 * above max_blocks_per_seq * page_size, are truncated to that bound. Page ids are clamped into
 * [0, num_blocks). batch is at most 4096.
 *
 * Split-K: each (sequence, KV head) is cut into partitions whose log-sum-exp partials are combined exactly
 * inside the same launch. num_splits = 0 balances the whole batch over the launched workgroups (ragged
 * lengths included); num_splits = S > 0 cuts a max_context-long sequence into S partitions (shorter ones
 * into proportionally fewer).
 *
 * Buffers: bpt_decode_plan reports the size of `workspace` (the split-K partials; any content) and of
 * `counters` (one uint32 arrival counter per (sequence, KV head, row group)). The counters must be zero
 * before the first call (allocate them zeroed) and every completed call leaves them zero again, so one
 * pair serves any number of calls issued in order on one stream, whatever their shapes. Calls that may
 * overlap (different streams) need separate buffers. q rows and the caches must be 16-byte aligned.
 */
typedef struct {
  uint32_t struct_size; /* sizeof(bpt_decode_args): guards against a stale binding */
  int32_t kv_dtype;     /* bpt_kv_dtype   */
  int32_t scale_kind;   /* bpt_scale_kind */
  int32_t q_dtype;      /* bpt_float_dtype */
  int32_t out_dtype;    /* bpt_float_dtype */
  int32_t table_dtype;  /* bpt_index_dtype */

  int32_t batch, num_queries, num_q_heads, num_kv_heads, head_dim, page_size;
  int32_t num_blocks, max_blocks_per_seq, max_context;
  int32_t num_splits;   /* in: 0 = balance automatically, S > 0 = S partitions of a max_context sequence */
  int32_t chunk_tokens; /* out of bpt_decode_plan: tokens one wave streams per step */
  int32_t grid_groups;  /* out of bpt_decode_plan: workgroups launched */
  int32_t rows_per_group; /* out of bpt_decode_plan: query rows computed together per KV head; 16 = the
                             matrix-core kernel (FP8 caches, 2..16 rows), 1/2/4 = the vector kernel */
  float sm_scale;

  const void* q;
  int64_t q_stride_b, q_stride_q, q_stride_h;
  const void* k_cache;
  const void* v_cache;
  int64_t kv_stride_block, kv_stride_token, kv_stride_head;
  const float* k_scale;
  const float* v_scale;
  int64_t scale_stride_block, scale_stride_token, scale_stride_head;
  const void* block_table;
  int64_t table_stride_b;
  const int32_t* context_lens;
  void* out;
  int64_t out_stride_b, out_stride_q, out_stride_h;
  void* workspace;        /* split-K partials, 256-byte aligned */
  size_t workspace_bytes;
  void* counters;         /* uint32 arrival counters, zero before first use and after every call */
  size_t counters_bytes;

  /* Cascade (a prefix shared by several sequences attended once, then each sequence's own tokens): */
  int32_t flags;           /* BPT_DECODE_NONCAUSAL: every query sees all of its sequence's tokens */
  int32_t len_offset;      /* tokens subtracted from every context length (and from every query position) */
  float* lse_out;          /* optional contiguous float32 [B, Q, Hq]: each row's log-sum-exp (natural log) */
  const float* merge_out;  /* optional contiguous float32 [B, Q, Hq, D]: a partial over other tokens ... */
  const float* merge_lse;  /* ... and its log-sum-exp [B, Q, Hq] (natural log, -inf if empty), merged into
                              out (and lse_out) exactly, as kernels/reference.py:205-211 merges parts */
} bpt_decode_args;

#define BPT_DECODE_NONCAUSAL 1

/*
 * Plan constants for tuning sweeps, process-wide (bench.py --tune). A field at its neutral value keeps the
 * library's own choice; NULL restores every default. Calls planned on other threads meanwhile see either
 * setting. No counterpart in the reference's kernel interface: it is what fastserve's tuning sweep
 * (experiments/m7.py:292-335, over the launcher's split and num_warps arguments) varies, for the knobs this
 * launch has instead (workgroups per CU, the per-segment charge, the minimum chunks per workgroup).
 */
typedef struct {
  uint32_t struct_size;  /* sizeof(bpt_tuning) */
  int32_t groups_per_cu; /* workgroups per CU of the auto plan, paged and KIVI (0: built-in) */
  int32_t piece_cost;    /* line units charged per segment start (-1: built-in) */
  int32_t min_chunks;    /* chunks per workgroup below which the auto plan launches fewer, paged and KIVI
                            (0: built-in) */
} bpt_tuning;
int bpt_set_tuning(const bpt_tuning* t);

/*
 * New K/V rows written into the paged pools, quantized on the way (store-before-attend).
 *
 *   k, v           [B, Q, Hkv, D] rows (strides new_stride_{b,q,h}), BF16 / F16 / F32
 *   write_blocks   [B, Q] physical page of each row (negative = skip the row), strides slot_stride_{b,q}
 *   write_offsets  [B, Q] slot inside that page
 *   FP8:  code = e4m3fn(clamp(x / scale[h], -448, 448)), scale read from k/v_scale[Hkv]
 *   INT8: s = max(amax|x| / 127, 1e-12); code = clamp(rint(x / s), -128, 127); s written to the
 *         per-token-head scale pools at the row's slot
 *   BF16: the row is stored as is.
 * Rows whose block is outside [0, num_blocks) or whose offset is outside [0, page_size) are skipped.
 */
typedef struct {
  uint32_t struct_size;
  int32_t kv_dtype, scale_kind, src_dtype, slot_dtype;
  int32_t batch, num_queries, num_kv_heads, head_dim, page_size, num_blocks;
  const void* k;
  const void* v;
  int64_t new_stride_b, new_stride_q, new_stride_h;
  const void* write_blocks;
  const void* write_offsets;
  int64_t slot_stride_b, slot_stride_q;
  void* k_cache;
  void* v_cache;
  int64_t kv_stride_block, kv_stride_token, kv_stride_head;
  float* k_scale; /* FP8: read [Hkv]; INT8: written per token-head */
  float* v_scale;
  int64_t scale_stride_block, scale_stride_token, scale_stride_head;
} bpt_append_args;

/* storage format of a KIVI cache (kernels/reference.py:66-100 QuantKV; bits 4, 8 or 16) */
typedef enum {
  BPT_KIVI_INT4 = 0, /* uint8 [B, Hkv, T, D/2]: channel d in the low nibble, d + D/2 in the high one      */
  BPT_KIVI_INT8 = 1, /* uint8 [B, Hkv, T, D]                                                           */
  BPT_KIVI_F16 = 2,  /* bits 16: float16 keys and values [B, Hkv, T, D], no grids                      */
  BPT_KIVI_BF16 = 3, /* bits 16: bfloat16 keys and values, no grids                                    */
  BPT_KIVI_F32 = 4   /* bits 16: float32 keys and values, no grids (a float32 model's cache)             */
} bpt_kivi_format;

/*
 * Decode attention of one query per head over a KIVI cache, one partial result per split.
 *
 *   q            [B, Hq, D] (strides q_stride_{b,h}; channel stride 1), BF16 / F16 / F32
 *   k/v_codes    [B, Hkv, T, D] codes (INT4: D/2 bytes per token), strides code_stride_{b,h,t} in elements
 *                of the stored type (bytes for INT4 / INT8, halves for F16 / BF16); channel stride 1
 *   k_scale/zero float16 [B, Hkv, num_groups, D], strides kgrid_stride_{b,h,g}: the key grid of tokens
 *                g*group .. g*group + group - 1 (INT4 / INT8 only); key = scale * (code - zero)
 *   v_scale/zero float16 [B, Hkv, T], strides vgrid_stride_{b,h}: one grid per token; value likewise
 *   lengths      [B] int32: tokens visible to each row's query (clamped to T and to num_splits * split)
 *   out          float32 [B, Hq, S, D] (strides out_stride_{b,h,s}): split s's softmax-weighted average of
 *                the values of tokens s*split .. min((s+1)*split, length) - 1, 0 for an empty split
 *   lse          float32 [B, Hq, S] (strides lse_stride_{b,h,s}): log sum exp (natural log) of that split's
 *                scores sm_scale * q.k, -inf for an empty split
 *
 * Hq a multiple of Hkv with at most 16 query heads per KV head; split a multiple of group; for INT4 / INT8,
 * T a multiple of group and num_groups * group >= T.
 * Two kernels. D = 128 with INT4 / INT8 / F16 / BF16 codes takes the matrix-core kernel: T and split
 * multiples of 32, for INT4 / INT8 group a power of two of at least 32; one KV head's codes must span less
 * than 2 GiB; code tensors and grids 16-byte aligned, code strides multiples of 16 bytes, key-grid strides
 * multiples of 8 elements and value-grid strides multiples of 4. Every cached byte is read once for all query
 * heads of its KV head; the tokens are shared out over the launched workgroups regardless of the split, and
 * a split that several workgroups cover is combined exactly in the same launch (buffers: as for
 * bpt_paged_decode; bpt_kivi_plan gives the sizes; counters zero before the first call and left zero by every
 * call). Any other even D up to 256, and F32 caches, take a float32 kernel with one workgroup per (sequence,
 * KV head, split); group a power of two; it needs no workspace or counters (bpt_kivi_plan reports 0 bytes).
 */
typedef struct {
  uint32_t struct_size; /* sizeof(bpt_kivi_args) */
  int32_t format;       /* bpt_kivi_format */
  int32_t q_dtype;      /* bpt_float_dtype */
  int32_t batch, num_q_heads, num_kv_heads, head_dim;
  int32_t tokens;       /* T: tokens laid out per (sequence, KV head) */
  int32_t group;        /* tokens per key grid */
  int32_t num_groups;   /* key grids laid out per (sequence, KV head) */
  int32_t split;        /* tokens per split */
  int32_t num_splits;   /* S >= 1 */
  int32_t grid_groups;  /* out of bpt_kivi_plan: workgroups launched */
  float sm_scale;

  const void* q;
  int64_t q_stride_b, q_stride_h;
  const void* k_codes;
  const void* v_codes;
  int64_t code_stride_b, code_stride_h, code_stride_t;
  const void* k_scale; /* float16 */
  const void* k_zero;
  int64_t kgrid_stride_b, kgrid_stride_h, kgrid_stride_g;
  const void* v_scale; /* float16 */
  const void* v_zero;
  int64_t vgrid_stride_b, vgrid_stride_h;
  const int32_t* lengths;
  float* out;
  int64_t out_stride_b, out_stride_h, out_stride_s;
  float* lse;
  int64_t lse_stride_b, lse_stride_h, lse_stride_s;
  void* workspace;
  size_t workspace_bytes;
  void* counters;
  size_t counters_bytes;

  /* Full-precision tail (optional; tail_len = 0 for none): the tokens whose key group is not complete yet,
     as fastserve's QuantizedKVCache keeps them (integration/kv_cache.py:139-158), attended in the same launch
     and merged into the result (its :172-185: partial_attention over the tail, then merge_partials). Every
     row sees all tail_len tokens; a row with no codes gets the tail's attention alone. num_splits must be 1.
       tail_k, tail_v  [B, Hkv, tail_len, D] (strides tail_stride_{b,h,t} in elements; channel stride 1),
                       BF16 / F16 / F32 (tail_dtype); at most 64 tokens. */
  const void* tail_k;
  const void* tail_v;
  int64_t tail_stride_b, tail_stride_h, tail_stride_t;
  int32_t tail_dtype; /* bpt_float_dtype */
  int32_t tail_len;
} bpt_kivi_args;

/*
 * Per-forward paged metadata from device positions (engine/kv_cache.py:140-156 PagedKVCache.prepare, built on
 * the device). The cache keeps each live sequence's block table as one row ("slot") of `table` [num_slots,
 * table_stride] int32 and the number of blocks reserved for it in `reserved` [num_slots] int32.
 *   slots         [B] int32: the slot of each row of this forward pass (clamped into the table)
 *   positions     [B, Q] int32 / int64 (strides pos_stride_{b,q}): the positions this pass writes and queries
 *   block_table   out [B, n_blocks] int32: the slot's blocks, 0 past the reserved ones (fastserve's padding)
 *   context_lens  out [B] int32: the last position + 1, clamped to the reserved tokens
 *   write_blocks  out [B, Q] int32: the block of each position that is token context_len - Q + i of its row
 *                 (the step's new rows are the row's last Q tokens) inside the reserved blocks, else -1
 *                 (skipped by bpt_quant_append). Consecutive positions inside the reservation all get their
 *                 block; positions past it (the length is then clamped) or out of order get none, so a step
 *                 never stores a row it does not attend as new.
 *   write_offsets out [B, Q] int32: position % page_size
 * page_size a power of two; max_blocks (<= table_stride) bounds the blocks read per slot. Nothing is read
 * back to the host: the call is one launch and can be captured in a graph.
 */
typedef struct {
  uint32_t struct_size; /* sizeof(bpt_prepare_args) */
  int32_t batch, num_queries, n_blocks, num_slots, max_blocks, page_size;
  int32_t positions_dtype; /* bpt_index_dtype */
  const int32_t* table;
  int64_t table_stride;
  const int32_t* reserved;
  const int32_t* slots;
  const void* positions;
  int64_t pos_stride_b, pos_stride_q;
  int32_t* block_table;
  int32_t* write_blocks;
  int32_t* write_offsets;
  int32_t* context_lens;
} bpt_prepare_args;

/*
 * KIVI quantize-on-write (kernels/reference.py:103-160 quantize_kv): keys and values [B, Hkv, T, D] stored as
 * asymmetric `bits`-bit codes with float16 grids, one grid per key channel per `group` tokens and one per value
 * token: lo = min(min x, 0), hi = max(max x, 0), scale = f16((hi - lo) / (2^bits - 1)) (1 where not > 0),
 * zero = clamp(round_half_even(-lo / scale), 0, 2^bits - 1), code = clamp(round_half_even(x / scale) + zero,
 * 0, 2^bits - 1), float32 IEEE divisions: bit-exact with the reference formulas. 4-bit codes pair channel d
 * (low nibble) with d + D/2 (high nibble).
 *   k, v          [B, Hkv, T, D] BF16 / F16 / F32 (strides src_stride_{b,h,t} in elements, channel stride 1)
 *   k/v_codes     uint8 [B, Hkv, T, D] (bits 8) or [B, Hkv, T, D/2] (bits 4), strides code_stride_{b,h,t} bytes
 *   k_scale/zero  float16 [B, Hkv, T/group, D], strides kgrid_stride_{b,h,g} (channel stride 1)
 *   v_scale/zero  float16 [B, Hkv, T], strides vgrid_stride_{b,h} (token stride 1)
 * bits 4 or 8; D a power of two up to 256; T a whole number of groups (the outputs may be views into a larger
 * cache at any token offset that is a multiple of group).
 */
typedef struct {
  uint32_t struct_size; /* sizeof(bpt_kivi_quant_args) */
  int32_t bits, src_dtype;
  int32_t batch, num_kv_heads, tokens, head_dim, group;
  const void* k;
  const void* v;
  int64_t src_stride_b, src_stride_h, src_stride_t;
  void* k_codes;
  void* v_codes;
  int64_t code_stride_b, code_stride_h, code_stride_t;
  void* k_scale; /* float16 */
  void* k_zero;
  int64_t kgrid_stride_b, kgrid_stride_h, kgrid_stride_g;
  void* v_scale; /* float16 */
  void* v_zero;
  int64_t vgrid_stride_b, vgrid_stride_h;
} bpt_kivi_quant_args;

/*
 * RMSNorm + per-token symmetric INT8, one pass over each row, float32 arithmetic:
 *   y = x * rsqrt(mean(x^2) + eps) * weight;  scale = max(max|y| / 127, 1e-12);
 *   codes = clamp(round_half_even(y / scale), -128, 127)
 *   x       [rows, d] (row stride x_stride_row elements, channel stride 1), BF16 / F16 / F32
 *   weight  [d], BF16 / F16 / F32
 *   codes   int8 [rows, d] (row stride codes_stride_row), scale float32 [rows]
 */
typedef struct {
  uint32_t struct_size; /* sizeof(bpt_norm_quant_args) */
  int32_t x_dtype, weight_dtype; /* bpt_float_dtype */
  int32_t rows, d;
  float eps;
  const void* x;
  int64_t x_stride_row;
  const void* weight;
  int8_t* codes;
  int64_t codes_stride_row;
  float* scale;
} bpt_norm_quant_args;

/* ---- entry points ------------------------------------------------------------------------------- */

/* Host-only: validate args, fill chunk_tokens / grid_groups, report the workspace and counter sizes in
 * bytes. Touches no GPU. */
int bpt_decode_plan(bpt_decode_args* args, size_t* workspace_bytes, size_t* counters_bytes);

/* Paged decode attention: one kernel launch, split-K partials combined in the same launch. */
int bpt_paged_decode(const bpt_decode_args* args, void* stream);

/* bpt_paged_decode with no caller workspace: the split-K partials and arrival counters live in a device-
 * resident array of the library (30 MiB of partials and 2 MiB of counters on each GPU it runs on, held until the
 * process ends), so the call allocates nothing: for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). No counterpart in the reference. The
 * workspace and counters fields of args are ignored; a call whose bpt_decode_plan sizes exceed the array's
 * returns BPT_ERR_INVALID_ARGUMENT. Calls on one GPU share the array: calls that may overlap (different
 * streams) race and must not be issued. */
int bpt_paged_decode_noalloc(const bpt_decode_args* args, void* stream);

/* Per-forward paged metadata (block tables, write slots, context lengths) from device positions: one launch. */
int bpt_paged_prepare(const bpt_prepare_args* args, void* stream);

/* Quantize-on-write of new K/V rows into their (page, slot). */
int bpt_quant_append(const bpt_append_args* args, void* stream);

/* Store, then attend (replaces integration/kv_cache.py:160-192, the cache's attend: _append then the decode
 * call). The rows of `append` ([batch, num_queries] of the decode) are the last Q tokens of each sequence: row
 * i of sequence b is token context_lens[b] - Q + i. A row is stored, as bpt_quant_append stores it, when its
 * slot is where the decode reads that token (the token's block-table page, clamped into the pool as the
 * decode clamps it, and its offset); rows with no slot or a slot anywhere else are not stored. `decode` then
 * attends the pools with the stored rows in place. When the decode runs on the matrix-core kernel with
 * per-head scales over the same pools, the rows are bf16 (16-byte aligned), Q <= 8, head dim 128, no
 * len_offset and no merge partial, one launch does both: it stores the rows and uses their codes for those
 * tokens directly. Otherwise two launches (the store, then bpt_paged_decode), with the same results. Every
 * argument of both halves is checked before anything is launched: a refused call writes nothing. */
int bpt_paged_append_decode(const bpt_append_args* append, const bpt_decode_args* decode, void* stream);

/* Host-only: validate a KIVI call, fill grid_groups, report workspace and counter sizes in bytes. */
int bpt_kivi_plan(bpt_kivi_args* args, size_t* workspace_bytes, size_t* counters_bytes);

/* Decode attention over a KIVI cache: one launch, every split's (out, lse) written. */
int bpt_kivi_decode(const bpt_kivi_args* args, void* stream);

/* KIVI quantize-on-write of completed key groups (one launch): replaces kernels/reference.py:132-160
 * quantize_kv where integration/kv_cache.py:147 QuantizedKVCache._append calls it. */
int bpt_kivi_quantize(const bpt_kivi_quant_args* args, void* stream);

/* RMSNorm fused with per-token INT8 quantization (one launch). */
int bpt_rms_norm_int8(const bpt_norm_quant_args* args, void* stream);

/* Thread-local message of the last failing call ("" when none). */
const char* bpt_last_error(void);

/* BPT_ABI_VERSION of the built library. */
int bpt_abi_version(void);

/* Hash of the sources the library was compiled from (the .hip and .h files of csrc and include), so that a binding
 * can refuse a library built from other sources. No reference counterpart. */
const char* bpt_source_hash(void);

/* ---- conversion and measurement primitives (used by the tests and the benchmark) ---------------- */

/* out[i] = float(e4m3fn code i) for i in 0..255, decoded by the same device routine the kernels use. */
int bpt_fp8_decode_table(float* out256, void* stream);

/* out[i] = e4m3fn(clamp(x[i] / scale, -448, 448)), the FP8 write-path encoder, for n floats. */
int bpt_fp8_encode(const float* x, float scale, uint8_t* out, int64_t n, void* stream);

/* bpt_paged_decode whose kernel launch also records two HIP events (hipEvent_t, created with timing) around
 * the kernel's own execution, through hipExtLaunchKernel: the benchmark's per-call kernel time, free of the
 * cost of separate event records. No reference counterpart. With nothing to launch (batch 0) both events
 * are recorded on the stream at once. */
int bpt_paged_decode_timed(const bpt_decode_args* args, void* stream, void* start_event, void* stop_event);

/* Streaming read of `bytes` (multiple of 16) from buf; one float per workgroup into partial_sums. The
 * measured-peak probe, and the cache flush run before cold timings. Returns the workgroup count used
 * in *num_groups so the caller can size partial_sums (call with partial_sums = NULL to query). */
int bpt_read_probe(const void* buf, uint64_t bytes, float* partial_sums, int64_t* num_groups,
                   void* stream);

/* bpt_read_probe of `bytes` (a positive multiple of 16) whose launch records two HIP events around the kernel's
 * own execution, as bpt_paged_decode_timed does: the contiguous-read floor for a byte count, timed the way
 * the decode kernel is. partial_sums holds the workgroup count bpt_read_probe reports. No reference
 * counterpart. */
int bpt_read_probe_timed(const void* buf, uint64_t bytes, float* partial_sums, void* stream, void* start_event,
                         void* stop_event);

/* The page-read probe: every K and V row (and per-token scale) that bpt_paged_decode over the same args
 * reads, fetched through the same block table and context lengths, in the decode's own order (its segments,
 * workgroup ranges and chunks, the same number of workgroups) with no attention math and no merges (one float
 * per workgroup into partial_sums). It is the read floor of a decode call's own access pattern. Call with
 * partial_sums = NULL to get the workgroup count in *num_groups. Optional events as bpt_read_probe_timed
 * (both or neither). Uses the shape, cache, scale, table and length fields of args. No reference
 * counterpart. */
int bpt_page_read_probe(const bpt_decode_args* args, float* partial_sums, int64_t* num_groups, void* stream,
                        void* start_event, void* stop_event);

/* dst <- src, `bytes` a multiple of 16: the known-size kernel that calibrates HBM byte counters. */
int bpt_copy_probe(void* dst, const void* src, uint64_t bytes, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* BPT_AMD_H */
