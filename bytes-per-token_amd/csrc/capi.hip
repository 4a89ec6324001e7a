// The C ABI (include/bpt_amd.h): argument checks, the split-K plan, kernel dispatch, error reporting.
//
// Argument checks run on the host before anything is launched and report BPT_ERR_INVALID_ARGUMENT with a
// message; nothing here reads device memory, so every call stays asynchronous and graph-capturable.
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <string>

#include "../../include/bpt_amd.h"
#include "bpt_device.h"
#include "bpt_internal.h"

namespace {

thread_local std::string g_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_error = buf;
  return code;
}

int hip_fail(const char* where, hipError_t e) {
  return fail(BPT_ERR_HIP, "%s: HIP error %d (%s)", where, (int)e, hipGetErrorString(e));
}

bool is_pow2(int64_t x) { return x > 0 && (x & (x - 1)) == 0; }
int log2i(int64_t x) {
  int r = 0;
  while ((int64_t(1) << r) < x) ++r;
  return r;
}
bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }
int float_bytes(int dt) { return dt == BPT_F_F32 ? 4 : 2; }
bool aligned_to(const void* p, int64_t stride_b, int64_t stride_q, int64_t stride_h, int elem) {
  return ((uintptr_t)p % 16 == 0) && (stride_b * elem) % 16 == 0 && (stride_q * elem) % 16 == 0 &&
         (stride_h * elem) % 16 == 0;
}

struct Plan {
  bool mfma;  // the matrix-core kernel (all rows of a KV head in one 16-row group)
  int rows, rows_per_group, n_rg, HR, chunk, grid, len_cap;
  int64_t per_forced;
  int equal_grid;  // workgroups that take equal partitions when all lengths are equal (0: none)
  int piece_cost;  // line units charged per segment start
  int waves;       // matrix-core kernel: waves per workgroup
  size_t ws_out_floats, ws_lse_floats, workspace, counters;
};

// Plan constants set by bpt_set_tuning (sweeps); a field at its neutral value keeps the built-in choice.
bpt_tuning g_tuning = {sizeof(bpt_tuning), 0, -1, 0};
std::mutex g_tuning_mutex;

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

int make_plan(const bpt_decode_args* a, Plan* pl) {
  const char* fn = "bpt_decode_plan";
  if (!a) return fail(BPT_ERR_INVALID_ARGUMENT, "%s: args is NULL", fn);
  if (a->struct_size != sizeof(bpt_decode_args))
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: struct_size %u != %zu (stale binding)", fn, a->struct_size,
                sizeof(bpt_decode_args));
  if (a->kv_dtype < BPT_KV_BF16 || a->kv_dtype > BPT_KV_INT8)
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: unknown kv_dtype %d", fn, a->kv_dtype);
  if (a->kv_dtype == BPT_KV_BF16 && a->scale_kind != BPT_SCALE_NONE)
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: a bf16 cache takes no scales", fn);
  if (a->kv_dtype != BPT_KV_BF16 && a->scale_kind != BPT_SCALE_PER_HEAD && a->scale_kind != BPT_SCALE_PER_TOKEN_HEAD)
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: a quantized cache needs per-head or per-token-head scales", fn);
  if (a->q_dtype < BPT_F_BF16 || a->q_dtype > BPT_F_F32 || a->out_dtype < BPT_F_BF16 || a->out_dtype > BPT_F_F32)
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: q_dtype/out_dtype must be bf16, f16 or f32", fn);
  if (a->table_dtype != BPT_IDX_I32 && a->table_dtype != BPT_IDX_I64)
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: block table must be int32 or int64", fn);
  if (a->batch < 0 || a->num_queries < 1 || a->num_q_heads < 1 || a->num_kv_heads < 1)
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: batch >= 0, num_queries, num_q_heads, num_kv_heads >= 1", fn);
  if (a->batch > bpt::kMaxBatch)
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: batch %d exceeds %d", fn, a->batch, bpt::kMaxBatch);
  if (a->num_q_heads % a->num_kv_heads)
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: %d query heads are not a multiple of %d KV heads", fn,
                a->num_q_heads, a->num_kv_heads);
  if (a->head_dim != bpt::kHeadDim)
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: head_dim %d not supported (128)", fn, a->head_dim);
  if (!is_pow2(a->page_size) || a->page_size > 1024)
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: page_size %d must be a power of two <= 1024", fn, a->page_size);
  if (a->num_blocks < 1 || a->max_blocks_per_seq < 1 || a->max_context < 0)
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: num_blocks, max_blocks_per_seq >= 1 and max_context >= 0", fn);
  if (a->num_splits < 0) return fail(BPT_ERR_INVALID_ARGUMENT, "%s: num_splits must be >= 0", fn);
  if (!std::isfinite(a->sm_scale)) return fail(BPT_ERR_INVALID_ARGUMENT, "%s: sm_scale must be finite", fn);

  const int G = a->num_q_heads / a->num_kv_heads;
  pl->rows = a->num_queries * G;
  // The matrix-core kernel reads every page once for up to 16 rows (the vector kernel once per group of at
  // most 4) and shares its per-token work among them: FP8 heads with 2..16 rows go there, INT8 heads only
  // from 5 rows on (with fewer, the vector kernel reads each page once too and its INT8 decode is cheaper).
  pl->mfma = pl->rows <= bpt::kMfmaRows && ((a->kv_dtype == BPT_KV_FP8_E4M3FN && pl->rows >= bpt::kMfmaMinRows) ||
                                            (a->kv_dtype == BPT_KV_INT8 && pl->rows >= bpt::kMfmaMinRowsInt8));
  pl->rows_per_group = pl->mfma ? bpt::kMfmaRows : (pl->rows <= 1 ? 1 : (pl->rows <= 2 ? 2 : 4));
  pl->n_rg = (pl->rows + pl->rows_per_group - 1) / pl->rows_per_group;
  const int64_t hr = (int64_t)a->num_kv_heads * pl->n_rg;
  if (hr > (1 << 20)) return fail(BPT_ERR_INVALID_ARGUMENT, "%s: too many KV heads x row groups", fn);
  pl->HR = (int)hr;
  pl->chunk = pl->mfma ? bpt::kMfmaChunk : bpt::decode_chunk_tokens(a->kv_dtype, pl->rows_per_group);
  const int64_t table_cap = (int64_t)a->max_blocks_per_seq * a->page_size;
  pl->len_cap = (int)(a->max_context < table_cap ? a->max_context : table_cap);
  const int64_t max_nb = (pl->len_cap + pl->chunk - 1) / pl->chunk;
  bpt_tuning tune;
  {
    std::lock_guard<std::mutex> lock(g_tuning_mutex);
    tune = g_tuning;
  }
  const int64_t seq_chunks = (int64_t)a->batch * max_nb;  // bound on the chunk prefix sum
  const int64_t max_cost = tune.piece_cost > bpt::kMaxPieceCost ? tune.piece_cost : bpt::kMaxPieceCost;
  const int64_t seq_cost = (int64_t)a->batch * (max_nb + max_cost);  // and on the line's
  if (seq_cost > 0x7fffffffLL / (hr > 0 ? hr : 1))
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: batch x context x heads too large", fn);
  const int64_t bound_c = seq_chunks * hr;
  pl->waves = !pl->mfma ? bpt::kDecodeWaves
              : pl->rows >= bpt::kManyRows ? bpt::kMfmaManyRowWaves
              : a->num_splits == 0 && (int64_t)a->batch * hr >= bpt::kMfmaPairMinSegments ? bpt::kMfmaPairWaves
                                                                                      : bpt::kDecodeWaves;
  const bool pair = pl->waves == bpt::kMfmaPairWaves;
  const int groups_per_cu =
      tune.groups_per_cu > 0 ? tune.groups_per_cu
      : pair ? bpt::kMfmaPairGroupsPerCu
      : pl->mfma ? bpt::mfma_groups_per_cu(pl->rows)
                 : bpt::decode_groups_per_cu(a->kv_dtype == BPT_KV_INT8, pl->rows_per_group,
                                             a->page_size >= bpt::decode_rows_per_load(a->kv_dtype),
                                             a->q_dtype != BPT_F_BF16);
  pl->equal_grid = 0;
  if (a->num_splits > 0) {
    // num_splits partitions for a max_context sequence. When that gives more partitions than resident
    // workgroups, each workgroup takes several consecutive ones whole: inside a workgroup the online
    // softmax simply continues across their boundary (the log-sum-exp merge of the two partials, done in
    // registers), so the partials that go through memory are those of the resident workgroups.
    const int64_t max_grid = (int64_t)bpt::kComputeUnits * groups_per_cu;
    int64_t per = (max_nb + a->num_splits - 1) / a->num_splits;
    if (per < 1) per = 1;
    const int64_t parts = (bound_c + per - 1) / per;
    if (parts > max_grid) per *= (parts + max_grid - 1) / max_grid;
    pl->per_forced = per;
    int64_t grid = (bound_c + pl->per_forced - 1) / pl->per_forced;
    pl->grid = (int)(grid < 1 ? 1 : grid);
  } else {
    pl->per_forced = 0;
    int64_t grid = (int64_t)bpt::kComputeUnits * groups_per_cu;
    const int64_t min_chunks = tune.min_chunks > 0 ? tune.min_chunks
                               : bpt::decode_min_chunks(pl->mfma, pl->rows, a->kv_dtype == BPT_KV_INT8, bound_c);
    const int64_t fill = (bound_c + min_chunks - 1) / min_chunks;
    if (fill < grid) grid = fill;
    if (!pl->mfma && bound_c > 0 &&
        ((a->kv_dtype == BPT_KV_BF16 && bound_c <= bpt::kAlignedMaxChunksBf16) ||
         (a->kv_dtype == BPT_KV_INT8 && bound_c <= bpt::kAlignedMaxChunksInt8))) {
      // About 4 sqrt(chunks) workgroups (at most 512) take equal partitions of a power-of-two number of
      // chunks when every sequence has the same length (the kernel checks); the launch keeps the line
      // cut's workgroups for ragged batches, the rest of them leaving at once otherwise. One sequence
      // is never ragged: its partitions are fixed here (no piece cost, no check in the kernel).
      int64_t target = (int64_t)(4.0 * std::sqrt((double)bound_c));
      target = target < 1 ? 1 : (target > bpt::kAlignedMaxGrid ? bpt::kAlignedMaxGrid : target);
      int64_t per = 1;
      while (per * 2 <= bound_c / target) per *= 2;
      const int64_t parts = (bound_c + per - 1) / per;
      if (parts > bpt::kAlignedMaxGrid) per *= (parts + bpt::kAlignedMaxGrid - 1) / bpt::kAlignedMaxGrid;
      const int64_t equal = (bound_c + per - 1) / per;
      if (a->batch == 1) {
        pl->per_forced = per;
        grid = equal;
      } else {
        pl->equal_grid = (int)equal;
        if (equal > grid) grid = equal;
      }
    }
    pl->grid = (int)(grid < 1 ? 1 : grid);
  }
  // One sequence: its segments (one per KV head) are equally long, so the line's equal ranges need no charge
  // for the merges (measured on the matrix-core kernel at 512 / 2943 tokens: 11.1 -> 9.5, 12.9 -> 12.0 us).
  pl->piece_cost = pl->per_forced > 0 ? 0
                   : tune.piece_cost >= 0 ? tune.piece_cost
                   : a->batch == 1 ? 0
                   : pair ? bpt::kMfmaPairPieceCost
                   : (pl->mfma && pl->rows >= bpt::kManyRows ? bpt::kManyRowPieceCost : bpt::kDecodePieceCost);
  const size_t slots = (size_t)a->batch * pl->HR + pl->grid;
  pl->ws_out_floats = slots * pl->rows_per_group * a->head_dim;
  pl->ws_lse_floats = slots * pl->rows_per_group;
  pl->workspace = align256((pl->ws_out_floats + pl->ws_lse_floats) * sizeof(float));
  pl->counters = align256((size_t)a->batch * pl->HR * sizeof(unsigned));
  return BPT_OK;
}

struct KiviPlan {
  bool any;  // the float32 kernel for head dims other than 128 and float32 caches (kivi_any.hip)
  int G, grid, len_cap, eb;
  size_t ws_out_floats, ws_lse_floats, workspace, counters;
};

int make_kivi_plan(const bpt_kivi_args* a, KiviPlan* pl) {
  const char* fn = "bpt_kivi_plan";
  if (!a) return fail(BPT_ERR_INVALID_ARGUMENT, "%s: args is NULL", fn);
  if (a->struct_size != sizeof(bpt_kivi_args))
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: struct_size %u != %zu (stale binding)", fn, a->struct_size,
                sizeof(bpt_kivi_args));
  if (a->format < BPT_KIVI_INT4 || a->format > BPT_KIVI_F32)
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: unknown format %d", fn, a->format);
  if (a->q_dtype < BPT_F_BF16 || a->q_dtype > BPT_F_F32)
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: q_dtype must be bf16, f16 or f32", fn);
  if (a->batch < 0 || a->num_q_heads < 1 || a->num_kv_heads < 1 || a->tokens < 0)
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: batch, tokens >= 0 and num_q_heads, num_kv_heads >= 1", fn);
  if (a->batch > bpt::kMaxBatch)
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: batch %d exceeds %d", fn, a->batch, bpt::kMaxBatch);
  if (a->num_q_heads % a->num_kv_heads)
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: %d query heads are not a multiple of %d KV heads", fn,
                a->num_q_heads, a->num_kv_heads);
  pl->G = a->num_q_heads / a->num_kv_heads;
  if (pl->G > 16)
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: %d query heads per KV head (at most 16)", fn, pl->G);
  if (a->head_dim < 2 || a->head_dim > 256 || a->head_dim % 2)
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: head_dim %d not supported (an even number up to 256)", fn,
                a->head_dim);
  const bool quant = a->format == BPT_KIVI_INT4 || a->format == BPT_KIVI_INT8;
  pl->any = a->head_dim != bpt::kHeadDim || a->format == BPT_KIVI_F32;
  if (a->group < 1 || a->split < 1 || a->split % a->group)
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: split %d must be a multiple of the key group %d", fn, a->split,
                a->group);
  if (a->num_splits < 1) return fail(BPT_ERR_INVALID_ARGUMENT, "%s: num_splits must be >= 1", fn);
  if (!pl->any) {
    if (a->split % bpt::kMfmaChunk)
      return fail(BPT_ERR_INVALID_ARGUMENT, "%s: split %d must be a multiple of %d tokens", fn, a->split,
                  bpt::kMfmaChunk);
    if (a->tokens % bpt::kMfmaChunk)
      return fail(BPT_ERR_INVALID_ARGUMENT, "%s: the cache's %d tokens must be a multiple of %d", fn, a->tokens,
                  bpt::kMfmaChunk);
  }
  if (quant) {
    if (!is_pow2(a->group) || (!pl->any && a->group % bpt::kMfmaChunk))
      return fail(BPT_ERR_INVALID_ARGUMENT, "%s: key group %d must be a power of two%s", fn, a->group,
                  pl->any ? "" : " of at least 32 tokens");
    if (a->tokens % a->group)
      return fail(BPT_ERR_INVALID_ARGUMENT, "%s: %d tokens are not a whole number of groups of %d", fn, a->tokens,
                  a->group);
    if ((int64_t)a->num_groups * a->group < a->tokens)
      return fail(BPT_ERR_INVALID_ARGUMENT, "%s: %d key groups do not cover %d tokens", fn, a->num_groups,
                  a->tokens);
  }
  if (!std::isfinite(a->sm_scale)) return fail(BPT_ERR_INVALID_ARGUMENT, "%s: sm_scale must be finite", fn);
  pl->eb = quant ? 1 : (a->format == BPT_KIVI_F32 ? 4 : 2);
  const int64_t reach = (int64_t)a->num_splits * a->split;
  pl->len_cap = (int)(reach < a->tokens ? reach : a->tokens);
  const int64_t segs = (int64_t)a->batch * a->num_kv_heads * a->num_splits;
  if (segs > 0x7fffffffLL) return fail(BPT_ERR_INVALID_ARGUMENT, "%s: batch x heads x splits too large", fn);
  if (pl->any) {  // one workgroup per (sequence, KV head, split); no partials cross workgroups
    pl->grid = (int)segs;
    pl->ws_out_floats = pl->ws_lse_floats = 0;
    pl->workspace = pl->counters = 0;
    return BPT_OK;
  }
  const int64_t max_nb = (pl->len_cap + bpt::kMfmaChunk - 1) / bpt::kMfmaChunk;
  const int64_t seq_chunks = (int64_t)a->batch * max_nb;
  if (seq_chunks > 0x7fffffffLL / a->num_kv_heads)
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: batch x tokens x heads too large", fn);
  bpt_tuning tune;
  {
    std::lock_guard<std::mutex> lock(g_tuning_mutex);
    tune = g_tuning;
  }
  const int64_t seq_heads = (int64_t)a->batch * a->num_kv_heads;
  const bool few_long = seq_heads <= bpt::kKiviFewSegments && max_nb >= bpt::kKiviLongSegmentChunks;
  const int default_gpc = few_long ? 1 : bpt::kDecodeGroupsPerCu;
  int64_t grid = (int64_t)bpt::kComputeUnits * (tune.groups_per_cu > 0 ? tune.groups_per_cu : default_gpc);
  const int64_t bound_c = seq_chunks * a->num_kv_heads;
  const int64_t min_chunks = tune.min_chunks > 0 ? tune.min_chunks : bpt::kivi_min_chunks(bound_c, grid);
  const int64_t by_chunks = (bound_c + min_chunks - 1) / min_chunks;
  if (by_chunks < grid) grid = by_chunks;
  pl->grid = (int)(grid < 1 ? 1 : grid);
  const size_t slots = 2 * (size_t)pl->grid;
  pl->ws_out_floats = slots * pl->G * a->head_dim;
  pl->ws_lse_floats = slots * pl->G;
  pl->workspace = align256((pl->ws_out_floats + pl->ws_lse_floats) * sizeof(float));
  pl->counters = align256((size_t)segs * sizeof(unsigned));
  return BPT_OK;
}

}  // namespace

extern "C" {

const char* bpt_last_error(void) { return g_error.c_str(); }

int bpt_abi_version(void) { return BPT_ABI_VERSION; }

#ifndef BPT_SOURCE_HASH
#define BPT_SOURCE_HASH "unknown"
#endif
const char* bpt_source_hash(void) { return BPT_SOURCE_HASH; }

int bpt_decode_plan(bpt_decode_args* args, size_t* workspace_bytes, size_t* counters_bytes) {
  Plan pl;
  int rc = make_plan(args, &pl);
  if (rc) return rc;
  args->chunk_tokens = pl.chunk;
  args->grid_groups = pl.grid;
  args->rows_per_group = pl.rows_per_group;
  if (workspace_bytes) *workspace_bytes = pl.workspace;
  if (counters_bytes) *counters_bytes = pl.counters;
  return BPT_OK;
}

namespace {

// Where a call's split-K partials and arrival counters live: the caller's buffers (bpt_paged_decode) or this
// device's scratch array (bpt_paged_decode_noalloc).
struct Buffers {
  void* workspace;
  size_t workspace_bytes;
  void* counters;
  size_t counters_bytes;
};

// The launch's line fields of the kernel parameters.
void line_fields(const Plan& pl, bpt::DecodeParams* p) {
  p->grid = pl.grid;
  p->per_forced = pl.per_forced;
  p->equal_grid = pl.equal_grid;
  p->piece_cost = pl.piece_cost;
}

// Checks a decode call's arguments and buffers on the host and fills its launch parameters (*p, *pl); nothing
// is launched. *empty: a batch of zero (nothing to launch).
int decode_setup(const bpt_decode_args* a, const char* fn, const Buffers* own, bpt::DecodeParams* out, Plan* plan,
                 bool* empty) {
  Plan& pl = *plan;
  int rc = make_plan(a, &pl);
  if (rc) return rc;
  const Buffers buf = own ? *own : Buffers{a->workspace, a->workspace_bytes, a->counters, a->counters_bytes};
  *empty = a->batch == 0;
  if (*empty) return BPT_OK;
  if (!a->q || !a->k_cache || !a->v_cache || !a->block_table || !a->out)
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: q, caches, block_table and out must be non-NULL", fn);
  if ((a->merge_out == nullptr) != (a->merge_lse == nullptr))
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: merge_out and merge_lse go together", fn);
  if (a->flags & ~BPT_DECODE_NONCAUSAL) return fail(BPT_ERR_INVALID_ARGUMENT, "%s: unknown flags %d", fn, a->flags);
  if (a->len_offset < 0) return fail(BPT_ERR_INVALID_ARGUMENT, "%s: len_offset must be >= 0", fn);
  if (a->kv_dtype != BPT_KV_BF16 && (!a->k_scale || !a->v_scale))
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: k_scale and v_scale are required for a quantized cache", fn);
  const int eb = a->kv_dtype == BPT_KV_BF16 ? 2 : 1;
  if (!aligned16(a->k_cache) || !aligned16(a->v_cache) || (a->kv_stride_block * eb) % 16 ||
      (a->kv_stride_token * eb) % 16 || (a->kv_stride_head * eb) % 16)
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: cache pointers and strides must be 16-byte aligned", fn);
  if (!buf.workspace || buf.workspace_bytes < pl.workspace || ((uintptr_t)buf.workspace & 255u))
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: a 256-byte aligned workspace of %zu bytes is required (got %zu)", fn,
                pl.workspace, buf.workspace_bytes);
  if (!buf.counters || buf.counters_bytes < pl.counters || ((uintptr_t)buf.counters & 3u))
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: a zeroed counter buffer of %zu bytes is required (got %zu)", fn,
                pl.counters, buf.counters_bytes);
  if (!aligned_to(a->q, a->q_stride_b, a->q_stride_q, a->q_stride_h, float_bytes(a->q_dtype)))
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: q rows must be 16-byte aligned (pointer and strides)", fn);

  bpt::DecodeParams p{};
  p.q = a->q;
  p.q_sb = a->q_stride_b;
  p.q_sq = a->q_stride_q;
  p.q_sh = a->q_stride_h;
  p.k = (const uint8_t*)a->k_cache;
  p.v = (const uint8_t*)a->v_cache;
  p.kv_sblk = a->kv_stride_block * eb;
  p.kv_stok = a->kv_stride_token * eb;
  p.kv_shead = a->kv_stride_head * eb;
  p.ks = a->k_scale;
  p.vs = a->v_scale;
  p.sc_sblk = a->scale_stride_block;
  p.sc_stok = a->scale_stride_token;
  p.sc_shead = a->scale_stride_head;
  p.table = a->block_table;
  p.table_sb = a->table_stride_b;
  p.lens = a->context_lens;
  p.out = a->out;
  p.o_sb = a->out_stride_b;
  p.o_sq = a->out_stride_q;
  p.o_sh = a->out_stride_h;
  p.ws_out = (float*)buf.workspace;
  p.ws_lse = (float*)buf.workspace + pl.ws_out_floats;
  p.counters = (unsigned*)buf.counters;
  p.B = a->batch;
  p.Q = a->num_queries;
  p.Hq = a->num_q_heads;
  p.Hkv = a->num_kv_heads;
  p.G = a->num_q_heads / a->num_kv_heads;
  p.P = a->page_size;
  p.logP = log2i(a->page_size);
  p.num_blocks = a->num_blocks;
  p.max_blocks = a->max_blocks_per_seq;
  p.n_rg = pl.n_rg;
  p.HR = pl.HR;
  p.waves = pl.waves;
  line_fields(pl, &p);
  p.len_cap = pl.len_cap;
  p.qscale = a->sm_scale * bpt::kLog2e;
  p.q_dtype = a->q_dtype;
  p.out_dtype = a->out_dtype;
  p.table_i64 = a->table_dtype == BPT_IDX_I64;
  p.noncausal = (a->flags & BPT_DECODE_NONCAUSAL) != 0;
  p.len_offset = a->len_offset;
  p.lse_out = a->lse_out;
  p.merge_out = a->merge_out;
  p.merge_lse = a->merge_lse;
  *out = p;
  return BPT_OK;
}

int paged_decode(const bpt_decode_args* a, void* stream, const bpt::LaunchEvents& ev, const char* fn,
                 const Buffers* own = nullptr, const bpt::AppendParams* fuse = nullptr) {
  Plan pl;
  bpt::DecodeParams p;
  bool empty;
  int rc = decode_setup(a, fn, own, &p, &pl, &empty);
  if (rc) return rc;
  if (empty) {
    if (ev.start) {  // nothing to launch: the interval is empty
      hipError_t e = hipEventRecord(ev.start, (hipStream_t)stream);
      if (e == hipSuccess) e = hipEventRecord(ev.stop, (hipStream_t)stream);
      if (e != hipSuccess) return hip_fail(fn, e);
    }
    return BPT_OK;
  }
  if (fuse) {
    p.fuse_q = fuse->Q;
    p.nk = (const uint16_t*)fuse->k;
    p.nv = (const uint16_t*)fuse->v;
    p.n_sb = fuse->n_sb;
    p.n_sq = fuse->n_sq;
    p.n_sh = fuse->n_sh;
    p.w_blocks = fuse->blocks;
    p.w_offsets = fuse->offsets;
    p.w_sb = fuse->s_sb;
    p.w_sq = fuse->s_sq;
    p.w_i64 = fuse->slot_i64;
  }
  hipError_t e = pl.mfma ? bpt::launch_decode_mfma(p, a->kv_dtype, a->scale_kind, (hipStream_t)stream, ev)
                         : bpt::launch_decode(p, a->kv_dtype, a->scale_kind, pl.rows_per_group, (hipStream_t)stream, ev);
  if (e != hipSuccess) return hip_fail(fn, e);
  return BPT_OK;
}

}  // namespace

int bpt_paged_decode(const bpt_decode_args* a, void* stream) { return paged_decode(a, stream, {}, "bpt_paged_decode"); }

int bpt_set_tuning(const bpt_tuning* t) {
  const bpt_tuning none = {sizeof(bpt_tuning), 0, -1, 0};
  if (t && t->struct_size != sizeof(bpt_tuning))
    return fail(BPT_ERR_INVALID_ARGUMENT, "bpt_set_tuning: struct_size %u != %zu (stale binding)", t->struct_size,
                sizeof(bpt_tuning));
  if (t && (t->groups_per_cu < 0 || t->groups_per_cu > 16 || t->piece_cost < -1 || t->piece_cost > 1024 ||
            t->min_chunks < 0))
    return fail(BPT_ERR_INVALID_ARGUMENT, "bpt_set_tuning: a value is out of range");
  std::lock_guard<std::mutex> lock(g_tuning_mutex);
  g_tuning = t ? *t : none;
  return BPT_OK;
}

}  // extern "C"

// ---- bpt_paged_decode_noalloc: the split-K partials and counters in a device-resident array ---------------
//
// `scratch` holds, on every GPU the library runs on, kScratchWorkspace bytes of partials followed by
// kScratchCounters bytes of arrival counters. The counters sit at a fixed offset, so the invariant that every
// completed call leaves them zero holds across calls of any shape. They start at zero: the array has static
// storage and no initializer, so the code object's loader zero-fills it on every GPU (no clear is queued, so
// a first call made under stream capture records nothing extra into the graph). In host code `scratch` names
// a host-side stand-in: its device address, different on each GPU, comes from hipGetSymbolAddress and is the
// only form passed to kernels.
namespace {

constexpr size_t kScratchWorkspace = (size_t)30 << 20;
constexpr size_t kScratchCounters = (size_t)2 << 20;
constexpr int kMaxDevices = 64;

}  // namespace

static __device__ __align__(256) uint8_t scratch[kScratchWorkspace + kScratchCounters];

namespace {

std::mutex g_scratch_mutex;
uint8_t* g_scratch[kMaxDevices];  // device address of `scratch` on each GPU, once set up

// This device's scratch address; on the device's first call, looks it up (with the device current).
int scratch_for(hipStream_t stream, uint8_t** out, const char* fn) {
  hipDevice_t dev = 0;
  hipError_t e = hipStreamGetDevice(stream, &dev);
  if (e != hipSuccess) return hip_fail(fn, e);
  if (dev < 0 || dev >= kMaxDevices) return fail(BPT_ERR_INVALID_ARGUMENT, "%s: device %d out of range", fn, (int)dev);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch[dev]) {
    int cur = 0;
    e = hipGetDevice(&cur);
    if (e == hipSuccess && cur != dev) e = hipSetDevice(dev);
    void* ptr = nullptr;
    if (e == hipSuccess) e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (cur != dev) {
      const hipError_t e2 = hipSetDevice(cur);
      if (e == hipSuccess) e = e2;
    }
    if (e != hipSuccess) return hip_fail(fn, e);
    g_scratch[dev] = (uint8_t*)ptr;
  }
  *out = g_scratch[dev];
  return BPT_OK;
}

}  // namespace

extern "C" {

int bpt_paged_decode_noalloc(const bpt_decode_args* a, void* stream) {
  const char* fn = "bpt_paged_decode_noalloc";
  Plan pl;
  int rc = make_plan(a, &pl);
  if (rc) return rc;
  if (pl.workspace > kScratchWorkspace || pl.counters > kScratchCounters)
    return fail(BPT_ERR_INVALID_ARGUMENT,
                "%s: the call needs %zu bytes of partials and %zu of counters; the device scratch holds %zu and %zu "
                "(use bpt_paged_decode with a caller workspace)",
                fn, pl.workspace, pl.counters, kScratchWorkspace, kScratchCounters);
  if (a->batch == 0) return BPT_OK;
  uint8_t* base = nullptr;
  rc = scratch_for((hipStream_t)stream, &base, fn);
  if (rc) return rc;
  const Buffers own{base, kScratchWorkspace, base + kScratchWorkspace, kScratchCounters};
  return paged_decode(a, stream, {}, fn, &own);
}

int bpt_paged_decode_timed(const bpt_decode_args* a, void* stream, void* start_event, void* stop_event) {
  const char* fn = "bpt_paged_decode_timed";
  if (!start_event || !stop_event) return fail(BPT_ERR_INVALID_ARGUMENT, "%s: both events are required", fn);
  bpt::LaunchEvents ev;
  ev.start = (hipEvent_t)start_event;
  ev.stop = (hipEvent_t)stop_event;
  return paged_decode(a, stream, ev, fn);
}

int bpt_kivi_plan(bpt_kivi_args* args, size_t* workspace_bytes, size_t* counters_bytes) {
  KiviPlan pl;
  int rc = make_kivi_plan(args, &pl);
  if (rc) return rc;
  args->grid_groups = pl.grid;
  if (workspace_bytes) *workspace_bytes = pl.workspace;
  if (counters_bytes) *counters_bytes = pl.counters;
  return BPT_OK;
}

int bpt_kivi_decode(const bpt_kivi_args* a, void* stream) {
  const char* fn = "bpt_kivi_decode";
  KiviPlan pl;
  int rc = make_kivi_plan(a, &pl);
  if (rc) return rc;
  if (a->batch == 0) return BPT_OK;
  const bool quant = a->format == BPT_KIVI_INT4 || a->format == BPT_KIVI_INT8;
  if (!a->q || !a->k_codes || !a->v_codes || !a->lengths || !a->out || !a->lse)
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: q, codes, lengths, out and lse must be non-NULL", fn);
  if (quant && (!a->k_scale || !a->k_zero || !a->v_scale || !a->v_zero))
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: 4- and 8-bit codes need their key and value grids", fn);
  if (a->tail_len < 0 || a->tail_len > bpt::kKiviMaxTail)
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: tail_len %d must be in [0, %d]", fn, a->tail_len, bpt::kKiviMaxTail);
  if (a->tail_len > 0) {
    if (!a->tail_k || !a->tail_v)
      return fail(BPT_ERR_INVALID_ARGUMENT, "%s: a tail needs tail_k and tail_v", fn);
    if (a->num_splits != 1)
      return fail(BPT_ERR_INVALID_ARGUMENT, "%s: a tail is merged into one split's result (num_splits 1)", fn);
    if (a->tail_dtype < BPT_F_BF16 || a->tail_dtype > BPT_F_F32)
      return fail(BPT_ERR_INVALID_ARGUMENT, "%s: tail_dtype must be bf16, f16 or f32", fn);
  }
  if (pl.any) {  // element-aligned tensors are enough for the float32 kernel
    if (((uintptr_t)a->k_codes | (uintptr_t)a->v_codes) % pl.eb)
      return fail(BPT_ERR_INVALID_ARGUMENT, "%s: code tensors must be aligned to their element size", fn);
  } else {
    if (!aligned16(a->k_codes) || !aligned16(a->v_codes) || (a->code_stride_b * pl.eb) % 16 ||
        (a->code_stride_h * pl.eb) % 16 || (a->code_stride_t * pl.eb) % 16)
      return fail(BPT_ERR_INVALID_ARGUMENT, "%s: code tensors and their strides must be 16-byte aligned", fn);
    if (quant && (!aligned16(a->k_scale) || !aligned16(a->k_zero) || !aligned16(a->v_scale) ||
                  !aligned16(a->v_zero) || a->kgrid_stride_b % 8 || a->kgrid_stride_h % 8 || a->kgrid_stride_g % 8 ||
                  a->vgrid_stride_b % 4 || a->vgrid_stride_h % 4))
      return fail(BPT_ERR_INVALID_ARGUMENT,
                  "%s: grids must be 16-byte aligned, key-grid strides multiples of 8 and value-grid strides of 4", fn);
    // One (sequence, KV head)'s codes and grids are addressed with 32-bit offsets.
    if ((int64_t)a->tokens * a->code_stride_t * pl.eb >= (int64_t)1 << 31 ||
        (quant && (int64_t)a->num_groups * a->kgrid_stride_g >= (int64_t)1 << 30))
      return fail(BPT_ERR_INVALID_ARGUMENT, "%s: one KV head's codes or grids span 2 GiB or more", fn);
    if (!a->workspace || a->workspace_bytes < pl.workspace || ((uintptr_t)a->workspace & 255u))
      return fail(BPT_ERR_INVALID_ARGUMENT, "%s: a 256-byte aligned workspace of %zu bytes is required (got %zu)",
                  fn, pl.workspace, a->workspace_bytes);
    if (!a->counters || a->counters_bytes < pl.counters || ((uintptr_t)a->counters & 3u))
      return fail(BPT_ERR_INVALID_ARGUMENT, "%s: a zeroed counter buffer of %zu bytes is required (got %zu)", fn,
                  pl.counters, a->counters_bytes);
  }

  bpt::KiviParams p;
  p.q = a->q;
  p.q_sb = a->q_stride_b;
  p.q_sh = a->q_stride_h;
  p.kc = (const uint8_t*)a->k_codes;
  p.vc = (const uint8_t*)a->v_codes;
  p.c_sb = a->code_stride_b * pl.eb;
  p.c_sh = a->code_stride_h * pl.eb;
  p.c_st = a->code_stride_t * pl.eb;
  p.ks = (const uint16_t*)a->k_scale;
  p.kz = (const uint16_t*)a->k_zero;
  p.g_sb = a->kgrid_stride_b;
  p.g_sh = a->kgrid_stride_h;
  p.g_sg = a->kgrid_stride_g;
  p.vs = (const uint16_t*)a->v_scale;
  p.vz = (const uint16_t*)a->v_zero;
  p.t_sb = a->vgrid_stride_b;
  p.t_sh = a->vgrid_stride_h;
  p.lens = a->lengths;
  p.out = a->out;
  p.o_sb = a->out_stride_b;
  p.o_sh = a->out_stride_h;
  p.o_ss = a->out_stride_s;
  p.lse = a->lse;
  p.l_sb = a->lse_stride_b;
  p.l_sh = a->lse_stride_h;
  p.l_ss = a->lse_stride_s;
  p.ws_out = (float*)a->workspace;
  p.ws_lse = (float*)a->workspace + pl.ws_out_floats;
  p.counters = (unsigned*)a->counters;
  p.B = a->batch;
  p.Hq = a->num_q_heads;
  p.Hkv = a->num_kv_heads;
  p.G = pl.G;
  p.S = a->num_splits;
  p.cps = a->split / bpt::kMfmaChunk;
  p.gshift = quant ? log2i(a->group / bpt::kMfmaChunk) : 0;
  p.len_offset = 0;
  p.len_cap = pl.len_cap;
  p.grid = pl.grid;
  p.qscale = a->sm_scale * bpt::kLog2e;
  p.q_dtype = a->q_dtype;
  p.D = a->head_dim;
  p.split = a->split;
  p.gshift_tokens = quant ? log2i(a->group) : 0;
  p.tk = a->tail_k;
  p.tv = a->tail_v;
  p.tk_sb = a->tail_stride_b;
  p.tk_sh = a->tail_stride_h;
  p.tk_st = a->tail_stride_t;
  p.tail_dtype = a->tail_dtype;
  p.tail_len = a->tail_len;
  hipError_t e = pl.any ? bpt::launch_kivi_any(p, a->format, (hipStream_t)stream)
                        : bpt::launch_kivi(p, a->format, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(fn, e);
  return BPT_OK;
}

int bpt_paged_prepare(const bpt_prepare_args* a, void* stream) {
  const char* fn = "bpt_paged_prepare";
  if (!a) return fail(BPT_ERR_INVALID_ARGUMENT, "%s: args is NULL", fn);
  if (a->struct_size != sizeof(bpt_prepare_args))
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: struct_size %u != %zu (stale binding)", fn, a->struct_size,
                sizeof(bpt_prepare_args));
  if (a->batch < 0 || a->num_queries < 1 || a->n_blocks < 0 || a->num_slots < 1 || a->max_blocks < 0 ||
      a->table_stride < a->max_blocks)
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: bad sizes (table_stride must cover max_blocks)", fn);
  if (!is_pow2(a->page_size)) return fail(BPT_ERR_INVALID_ARGUMENT, "%s: page_size must be a power of two", fn);
  if (a->positions_dtype != BPT_IDX_I32 && a->positions_dtype != BPT_IDX_I64)
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: positions must be int32 or int64", fn);
  if (a->batch == 0) return BPT_OK;
  if (!a->table || !a->reserved || !a->slots || !a->positions || !a->write_blocks || !a->write_offsets ||
      !a->context_lens || (a->n_blocks > 0 && !a->block_table))
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: tables, slots, positions and outputs must be non-NULL", fn);
  bpt::PrepareParams p;
  p.table = a->table;
  p.table_stride = a->table_stride;
  p.reserved = a->reserved;
  p.slots = a->slots;
  p.positions = a->positions;
  p.pos_sb = a->pos_stride_b;
  p.pos_sq = a->pos_stride_q;
  p.pos_i64 = a->positions_dtype == BPT_IDX_I64;
  p.block_table = a->block_table;
  p.write_blocks = a->write_blocks;
  p.write_offsets = a->write_offsets;
  p.context_lens = a->context_lens;
  p.B = a->batch;
  p.Q = a->num_queries;
  p.n_blocks = a->n_blocks;
  p.num_slots = a->num_slots;
  p.max_blocks = a->max_blocks;
  p.P = a->page_size;
  p.logP = log2i(a->page_size);
  hipError_t e = bpt::launch_paged_prepare(p, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(fn, e);
  return BPT_OK;
}

int bpt_kivi_quantize(const bpt_kivi_quant_args* a, void* stream) {
  const char* fn = "bpt_kivi_quantize";
  if (!a) return fail(BPT_ERR_INVALID_ARGUMENT, "%s: args is NULL", fn);
  if (a->struct_size != sizeof(bpt_kivi_quant_args))
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: struct_size %u != %zu (stale binding)", fn, a->struct_size,
                sizeof(bpt_kivi_quant_args));
  if (a->bits != 4 && a->bits != 8) return fail(BPT_ERR_INVALID_ARGUMENT, "%s: bits must be 4 or 8, got %d", fn, a->bits);
  if (a->src_dtype < BPT_F_BF16 || a->src_dtype > BPT_F_F32)
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: keys and values must be bf16, f16 or f32", fn);
  if (a->batch < 0 || a->num_kv_heads < 1 || a->tokens < 0 || a->group < 1)
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: batch, tokens >= 0; num_kv_heads, group >= 1", fn);
  if (!is_pow2(a->head_dim) || a->head_dim < 2 || a->head_dim > 256)
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: head_dim %d must be a power of two up to 256", fn, a->head_dim);
  if (a->tokens % a->group)
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: %d tokens are not a whole number of groups of %d", fn, a->tokens,
                a->group);
  if ((int64_t)a->batch * a->num_kv_heads * (a->tokens / a->group) >= (int64_t)1 << 31)
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: too many key groups", fn);
  if ((int64_t)a->batch * a->num_kv_heads * a->tokens == 0) return BPT_OK;
  if (!a->k || !a->v || !a->k_codes || !a->v_codes || !a->k_scale || !a->k_zero || !a->v_scale || !a->v_zero)
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: inputs, codes and grids must be non-NULL", fn);
  bpt::KiviQuantParams p;
  p.k = a->k;
  p.v = a->v;
  p.x_sb = a->src_stride_b;
  p.x_sh = a->src_stride_h;
  p.x_st = a->src_stride_t;
  p.src_dtype = a->src_dtype;
  p.kc = (uint8_t*)a->k_codes;
  p.vc = (uint8_t*)a->v_codes;
  p.c_sb = a->code_stride_b;
  p.c_sh = a->code_stride_h;
  p.c_st = a->code_stride_t;
  p.ks = (uint16_t*)a->k_scale;
  p.kz = (uint16_t*)a->k_zero;
  p.g_sb = a->kgrid_stride_b;
  p.g_sh = a->kgrid_stride_h;
  p.g_sg = a->kgrid_stride_g;
  p.vs = (uint16_t*)a->v_scale;
  p.vz = (uint16_t*)a->v_zero;
  p.t_sb = a->vgrid_stride_b;
  p.t_sh = a->vgrid_stride_h;
  p.B = a->batch;
  p.Hkv = a->num_kv_heads;
  p.T = a->tokens;
  p.D = a->head_dim;
  p.group = a->group;
  p.bits = a->bits;
  hipError_t e = bpt::launch_kivi_quantize(p, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(fn, e);
  return BPT_OK;
}

int bpt_rms_norm_int8(const bpt_norm_quant_args* a, void* stream) {
  const char* fn = "bpt_rms_norm_int8";
  if (!a) return fail(BPT_ERR_INVALID_ARGUMENT, "%s: args is NULL", fn);
  if (a->struct_size != sizeof(bpt_norm_quant_args))
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: struct_size %u != %zu (stale binding)", fn, a->struct_size,
                sizeof(bpt_norm_quant_args));
  if (a->x_dtype < BPT_F_BF16 || a->x_dtype > BPT_F_F32 || a->weight_dtype < BPT_F_BF16 || a->weight_dtype > BPT_F_F32)
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: x and weight must be bf16, f16 or f32", fn);
  if (a->rows < 0 || a->d < 1) return fail(BPT_ERR_INVALID_ARGUMENT, "%s: rows >= 0 and d >= 1", fn);
  if (!(a->eps >= 0.0f) || !std::isfinite(a->eps)) return fail(BPT_ERR_INVALID_ARGUMENT, "%s: eps must be finite and >= 0", fn);
  if (a->rows == 0) return BPT_OK;
  if (!a->x || !a->weight || !a->codes || !a->scale)
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: x, weight, codes and scale must be non-NULL", fn);
  if (a->x_stride_row < a->d || a->codes_stride_row < a->d)
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: row strides must be at least d", fn);
  const int xb = float_bytes(a->x_dtype), wb = float_bytes(a->weight_dtype);
  // 8 elements per lane per step when every row and the weight start on 16 bytes (codes on 8).
  const bool vec8 = a->d % 8 == 0 && aligned16(a->x) && (a->x_stride_row * xb) % 16 == 0 && aligned16(a->weight) &&
                    ((uintptr_t)a->codes % 8) == 0 && a->codes_stride_row % 8 == 0;
  (void)wb;
  bpt::NormQuantParams p;
  p.x = a->x;
  p.x_rs = a->x_stride_row;
  p.w = a->weight;
  p.codes = a->codes;
  p.c_rs = a->codes_stride_row;
  p.scale = a->scale;
  p.rows = a->rows;
  p.d = a->d;
  p.eps = a->eps;
  p.x_dtype = a->x_dtype;
  p.w_dtype = a->weight_dtype;
  hipError_t e = bpt::launch_norm_quant(p, vec8, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(fn, e);
  return BPT_OK;
}

namespace {

// Checks bpt_append_args and fills p; *empty: nothing to write.
int append_params(const bpt_append_args* a, bpt::AppendParams* out, bool* empty, const char* fn) {
  *empty = false;
  if (!a) return fail(BPT_ERR_INVALID_ARGUMENT, "%s: args is NULL", fn);
  if (a->struct_size != sizeof(bpt_append_args))
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: struct_size %u != %zu (stale binding)", fn, a->struct_size,
                sizeof(bpt_append_args));
  if (a->kv_dtype < BPT_KV_BF16 || a->kv_dtype > BPT_KV_INT8)
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: unknown kv_dtype %d", fn, a->kv_dtype);
  if (a->kv_dtype == BPT_KV_BF16 && a->scale_kind != BPT_SCALE_NONE)
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: a bf16 cache takes no scales", fn);
  if (a->kv_dtype != BPT_KV_BF16 && a->scale_kind != BPT_SCALE_PER_HEAD && a->scale_kind != BPT_SCALE_PER_TOKEN_HEAD)
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: a quantized cache needs per-head or per-token-head scales", fn);
  if (a->src_dtype < BPT_F_BF16 || a->src_dtype > BPT_F_F32)
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: new rows must be bf16, f16 or f32", fn);
  if (a->slot_dtype != BPT_IDX_I32 && a->slot_dtype != BPT_IDX_I64)
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: write_blocks/write_offsets must be int32 or int64", fn);
  if (a->batch < 0 || a->num_queries < 0 || a->num_kv_heads < 1 || a->num_blocks < 1 || a->page_size < 1)
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: bad sizes", fn);
  if (a->head_dim != 64 && a->head_dim != 128 && a->head_dim != 256)
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: head_dim %d not supported (64, 128, 256)", fn, a->head_dim);
  if ((int64_t)a->batch * a->num_queries * a->num_kv_heads == 0) {
    *empty = true;
    return BPT_OK;
  }
  if (!a->k || !a->v || !a->write_blocks || !a->write_offsets || !a->k_cache || !a->v_cache)
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: rows, slots and caches must be non-NULL", fn);
  if (a->kv_dtype != BPT_KV_BF16 && (!a->k_scale || !a->v_scale))
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: k_scale and v_scale are required for a quantized cache", fn);
  if ((int64_t)a->batch * a->num_queries * a->num_kv_heads * 2 / 8 >= (int64_t)0x7fffffff)
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: too many rows", fn);

  const int eb = a->kv_dtype == BPT_KV_BF16 ? 2 : 1;
  bpt::AppendParams p;
  p.k = a->k;
  p.v = a->v;
  p.n_sb = a->new_stride_b;
  p.n_sq = a->new_stride_q;
  p.n_sh = a->new_stride_h;
  p.blocks = a->write_blocks;
  p.offsets = a->write_offsets;
  p.s_sb = a->slot_stride_b;
  p.s_sq = a->slot_stride_q;
  p.kc = (uint8_t*)a->k_cache;
  p.vc = (uint8_t*)a->v_cache;
  p.kv_sblk = a->kv_stride_block * eb;
  p.kv_stok = a->kv_stride_token * eb;
  p.kv_shead = a->kv_stride_head * eb;
  p.ks = a->k_scale;
  p.vs = a->v_scale;
  p.sc_sblk = a->scale_stride_block;
  p.sc_stok = a->scale_stride_token;
  p.sc_shead = a->scale_stride_head;
  p.B = a->batch;
  p.Q = a->num_queries;
  p.Hkv = a->num_kv_heads;
  p.P = a->page_size;
  p.num_blocks = a->num_blocks;
  p.src_dtype = a->src_dtype;
  p.slot_i64 = a->slot_dtype == BPT_IDX_I64;
  p.in_place = 0;
  p.table = nullptr;
  p.table_sb = 0;
  p.table_i64 = p.max_blocks = p.logP = 0;
  p.lens = nullptr;
  *out = p;
  return BPT_OK;
}

// Whether the matrix-core decode of d can store a's rows itself: the same caches and shapes, per-head scales,
// bf16 rows (16-byte aligned) for the last Q <= 8 tokens of every sequence, lengths given and not offset,
// head dim 128, no caller partial to merge.
bool fusable(const bpt_append_args* a, const bpt_decode_args* d) {
  Plan pl;
  if (make_plan(d, &pl) != BPT_OK) return false;
  const bool rows_aligned = aligned16(a->k) && aligned16(a->v) && (a->new_stride_b * 2) % 16 == 0 &&
                            (a->new_stride_q * 2) % 16 == 0 && (a->new_stride_h * 2) % 16 == 0;
  return pl.mfma && a->kv_dtype == d->kv_dtype && a->kv_dtype != BPT_KV_BF16 && a->scale_kind == BPT_SCALE_PER_HEAD &&
         d->scale_kind == BPT_SCALE_PER_HEAD && a->k_cache == d->k_cache && a->v_cache == d->v_cache &&
         a->k_scale == d->k_scale && a->v_scale == d->v_scale && a->kv_stride_block == d->kv_stride_block &&
         a->kv_stride_token == d->kv_stride_token && a->kv_stride_head == d->kv_stride_head &&
         a->num_blocks == d->num_blocks && a->page_size == d->page_size && a->num_kv_heads == d->num_kv_heads &&
         a->head_dim == 128 && d->head_dim == 128 && a->batch == d->batch && a->num_queries == d->num_queries &&
         a->num_queries >= 1 && a->num_queries <= 8 && a->src_dtype == BPT_F_BF16 && rows_aligned &&
         d->context_lens != nullptr && d->len_offset == 0 && d->merge_out == nullptr;
}

}  // namespace

int bpt_quant_append(const bpt_append_args* a, void* stream) {
  const char* fn = "bpt_quant_append";
  bpt::AppendParams p;
  bool empty;
  int rc = append_params(a, &p, &empty, fn);
  if (rc || empty) return rc;
  hipError_t e = bpt::launch_append(p, a->kv_dtype, a->scale_kind, a->head_dim, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(fn, e);
  return BPT_OK;
}

int bpt_paged_append_decode(const bpt_append_args* append, const bpt_decode_args* decode, void* stream) {
  const char* fn = "bpt_paged_append_decode";
  bpt::AppendParams p;
  bool empty;
  int rc = append_params(append, &p, &empty, fn);
  if (rc) return rc;
  if (!decode) return fail(BPT_ERR_INVALID_ARGUMENT, "%s: decode args is NULL", fn);
  // Every check of the decode half runs before anything is launched: a refused call writes nothing.
  bpt::DecodeParams dp;
  Plan pl;
  bool no_decode;
  rc = decode_setup(decode, fn, nullptr, &dp, &pl, &no_decode);
  if (rc) return rc;
  if (!empty && !no_decode && !decode->context_lens)
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: context_lens are required (the new rows are the last tokens)", fn);
  if (!empty && fusable(append, decode)) return paged_decode(decode, stream, {}, fn, nullptr, &p);
  if (!empty && !no_decode) {
    if (append->batch != decode->batch || append->num_queries != decode->num_queries)
      return fail(BPT_ERR_INVALID_ARGUMENT, "%s: the new rows must be [batch, num_queries] of the decode", fn);
    // The rule of the fused launch: only rows stored where the decode reads token len - Q + qi.
    p.in_place = 1;
    p.table = decode->block_table;
    p.table_sb = decode->table_stride_b;
    p.table_i64 = decode->table_dtype == BPT_IDX_I64;
    p.max_blocks = decode->max_blocks_per_seq;
    p.logP = log2i(decode->page_size);
    p.lens = decode->context_lens;
    if (append->page_size != decode->page_size || append->num_blocks != decode->num_blocks)
      return fail(BPT_ERR_INVALID_ARGUMENT, "%s: append and decode must describe the same pools", fn);
  }
  if (!empty) {
    hipError_t e = bpt::launch_append(p, append->kv_dtype, append->scale_kind, append->head_dim, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(fn, e);
  }
  return paged_decode(decode, stream, {}, fn);
}

int bpt_fp8_decode_table(float* out256, void* stream) {
  if (!out256) return fail(BPT_ERR_INVALID_ARGUMENT, "bpt_fp8_decode_table: out is NULL");
  hipError_t e = bpt::launch_fp8_table(out256, (hipStream_t)stream);
  return e == hipSuccess ? BPT_OK : hip_fail("bpt_fp8_decode_table", e);
}

int bpt_fp8_encode(const float* x, float scale, uint8_t* out, int64_t n, void* stream) {
  if (n < 0 || (n > 0 && (!x || !out))) return fail(BPT_ERR_INVALID_ARGUMENT, "bpt_fp8_encode: bad buffers");
  if (!(scale > 0.0f) || !std::isfinite(scale))
    return fail(BPT_ERR_INVALID_ARGUMENT, "bpt_fp8_encode: scale must be positive and finite");
  hipError_t e = bpt::launch_fp8_encode(x, scale, out, n, (hipStream_t)stream);
  return e == hipSuccess ? BPT_OK : hip_fail("bpt_fp8_encode", e);
}

int bpt_read_probe(const void* buf, uint64_t bytes, float* partial_sums, int64_t* num_groups, void* stream) {
  if (bytes % 16) return fail(BPT_ERR_INVALID_ARGUMENT, "bpt_read_probe: bytes must be a multiple of 16");
  const int64_t g = bpt::read_probe_groups(bytes);
  if (num_groups) *num_groups = g;
  if (!partial_sums) return BPT_OK;
  if (!buf || !aligned16(buf)) return fail(BPT_ERR_INVALID_ARGUMENT, "bpt_read_probe: buffer must be 16-byte aligned");
  hipError_t e = bpt::launch_read_probe(buf, bytes, partial_sums, (hipStream_t)stream);
  return e == hipSuccess ? BPT_OK : hip_fail("bpt_read_probe", e);
}

int bpt_read_probe_timed(const void* buf, uint64_t bytes, float* partial_sums, void* stream, void* start_event,
                         void* stop_event) {
  const char* fn = "bpt_read_probe_timed";
  if (bytes % 16 || bytes == 0) return fail(BPT_ERR_INVALID_ARGUMENT, "%s: bytes must be a positive multiple of 16", fn);
  if (!buf || !aligned16(buf) || !partial_sums)
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: a 16-byte aligned buffer and partial_sums are required", fn);
  if (!start_event || !stop_event) return fail(BPT_ERR_INVALID_ARGUMENT, "%s: both events are required", fn);
  bpt::LaunchEvents ev;
  ev.start = (hipEvent_t)start_event;
  ev.stop = (hipEvent_t)stop_event;
  hipError_t e = bpt::launch_read_probe(buf, bytes, partial_sums, (hipStream_t)stream, ev);
  return e == hipSuccess ? BPT_OK : hip_fail(fn, e);
}

int bpt_page_read_probe(const bpt_decode_args* a, float* partial_sums, int64_t* num_groups, void* stream,
                        void* start_event, void* stop_event) {
  const char* fn = "bpt_page_read_probe";
  Plan pl;
  int rc = make_plan(a, &pl);
  if (rc) return rc;
  const int64_t g = a->batch > 0 ? pl.grid : 0;  // the decode's workgroups
  if (num_groups) *num_groups = g;
  if (!partial_sums) return BPT_OK;
  if (!a->k_cache || !a->v_cache || !a->block_table)
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: caches and block_table must be non-NULL", fn);
  const bool per_token = a->kv_dtype != BPT_KV_BF16 && a->scale_kind == BPT_SCALE_PER_TOKEN_HEAD;
  if (per_token && (!a->k_scale || !a->v_scale))
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: per-token scales are required for this cache", fn);
  const int eb = a->kv_dtype == BPT_KV_BF16 ? 2 : 1;
  if (!aligned16(a->k_cache) || !aligned16(a->v_cache) || (a->kv_stride_block * eb) % 16 ||
      (a->kv_stride_token * eb) % 16 || (a->kv_stride_head * eb) % 16)
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: cache pointers and strides must be 16-byte aligned", fn);
  if ((start_event == nullptr) != (stop_event == nullptr))
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: give both events or neither", fn);
  bpt::DecodeParams p{};
  p.k = (const uint8_t*)a->k_cache;
  p.v = (const uint8_t*)a->v_cache;
  p.kv_sblk = a->kv_stride_block * eb;
  p.kv_stok = a->kv_stride_token * eb;
  p.kv_shead = a->kv_stride_head * eb;
  p.ks = a->k_scale;
  p.vs = a->v_scale;
  p.sc_sblk = a->scale_stride_block;
  p.sc_stok = a->scale_stride_token;
  p.sc_shead = a->scale_stride_head;
  p.table = a->block_table;
  p.table_sb = a->table_stride_b;
  p.table_i64 = a->table_dtype == BPT_IDX_I64;
  p.lens = a->context_lens;
  p.B = a->batch;
  p.Hkv = a->num_kv_heads;
  p.P = a->page_size;
  p.logP = log2i(a->page_size);
  p.num_blocks = a->num_blocks;
  p.len_cap = pl.len_cap;
  p.len_offset = a->len_offset;
  p.HR = pl.HR;
  p.n_rg = pl.n_rg;
  p.waves = pl.waves;
  p.grid = (int)g;
  bpt::LaunchEvents ev;
  ev.start = (hipEvent_t)start_event;
  ev.stop = (hipEvent_t)stop_event;
  if (g == 0 && ev.start) {
    hipError_t e = hipEventRecord(ev.start, (hipStream_t)stream);
    if (e == hipSuccess) e = hipEventRecord(ev.stop, (hipStream_t)stream);
    return e == hipSuccess ? BPT_OK : hip_fail(fn, e);
  }
  // A chunk is read as whole 16-byte loads over 64 lanes: rows per load divide it, 1, 2, 4 or 8 loads per
  // lane, and one lane per token for the scales.
  const int rows_per_load = 64 / (a->head_dim * eb / 16);
  const int loads = pl.chunk / rows_per_load;
  if (pl.chunk % rows_per_load || loads > 8 || (loads & (loads - 1)) || pl.chunk > 64)
    return fail(BPT_ERR_INVALID_ARGUMENT, "%s: %d-token chunks of %d-byte rows are not read by this probe", fn,
                pl.chunk, a->head_dim * eb);
  hipError_t e = bpt::launch_page_read_probe(p, a->head_dim * eb, pl.chunk, per_token, partial_sums,
                                             (hipStream_t)stream, ev);
  return e == hipSuccess ? BPT_OK : hip_fail(fn, e);
}

int bpt_copy_probe(void* dst, const void* src, uint64_t bytes, void* stream) {
  if (bytes % 16 || !dst || !src || !aligned16(dst) || !aligned16(src))
    return fail(BPT_ERR_INVALID_ARGUMENT, "bpt_copy_probe: 16-byte aligned buffers, bytes a multiple of 16");
  if (bytes == 0) return BPT_OK;
  hipError_t e = bpt::launch_copy_probe(dst, src, bytes, (hipStream_t)stream);
  return e == hipSuccess ? BPT_OK : hip_fail("bpt_copy_probe", e);
}

}  // extern "C"
