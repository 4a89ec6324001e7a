// Kernel parameter blocks and launchers shared between the kernel files and the C-ABI layer.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace bpt {

// Upper bound on the pages one split stages into LDS (split_tokens / page_size + 1).
constexpr int kMaxSplitPages = 512;
// Waves per workgroup of the split kernel, and 16-byte loads per lane per K (and per V) chunk.
constexpr int kDecodeWaves = 4;
constexpr int kDecodeLoads = 4;

// Derived, launch-ready form of bpt_decode_args (strides of the caches in bytes).
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
  float* part_out;  // [B, Q, Hq, S, D]
  float* part_lse;  // [B, Q, Hq, S], log2 units
  int B, Q, Hq, Hkv, G, P, logP, num_blocks, max_blocks, S, split_tokens, n_rg, len_cap;
  float qscale;  // sm_scale * log2(e)
  int q_dtype, out_dtype, table_i64;
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
};

// Chunk of tokens one wave consumes per loop iteration for a KV element type (fp8/int8: 1 byte).
inline int decode_chunk_tokens(int kv_dtype, int head_dim) {
  int vec = kv_dtype == 0 ? 8 : 16;  // elements per 16-byte load
  int lanes_per_token = head_dim / vec;
  return kDecodeLoads * (64 / lanes_per_token);
}

hipError_t launch_decode(const DecodeParams& p, int kv_dtype, int scale_kind, int head_dim, int rows_per_group,
                         hipStream_t stream, hipEvent_t mid_event);
hipError_t launch_append(const AppendParams& p, int kv_dtype, int scale_kind, int head_dim, hipStream_t stream);
hipError_t launch_fp8_table(float* out, hipStream_t stream);
hipError_t launch_fp8_encode(const float* x, float scale, uint8_t* out, int64_t n, hipStream_t stream);
int64_t read_probe_groups(uint64_t bytes);
hipError_t launch_read_probe(const void* buf, uint64_t bytes, float* partial, hipStream_t stream);
hipError_t launch_copy_probe(void* dst, const void* src, uint64_t bytes, hipStream_t stream);

}  // namespace bpt
