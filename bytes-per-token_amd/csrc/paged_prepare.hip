// Per-forward paged-cache metadata built on the device: fastserve's PagedKVCache.prepare
// (engine/kv_cache.py:140-156) without its host round trip (int(positions.max()), a Python table build and an
// H2D copy every step), so a decode step that starts from device positions can be captured in a HIP graph.
//
// The cache keeps every live sequence's block table as one row ("slot") of a device table, written when blocks
// are reserved, with the number of reserved blocks per slot. From the rows' slots and their positions [B, Q]:
//   block_table[b, j]   = table[slot_b, j] for j < reserved_b, else 0 (fastserve pads with block 0)
//   context_lens[b]     = positions[b, Q - 1] + 1, clamped to [0, reserved_b * P]
//   write_blocks[b, i]  = table[slot_b, positions[b, i] / P] when positions[b, i] is token context_lens[b] - Q + i
//                         (the row's last Q tokens, which the decode attends as the step's new rows) inside the
//                         reserved blocks, else -1: the quantize-on-write kernels skip those rows. With
//                         consecutive positions inside the reservation that is every row; positions past it
//                         (the context is then clamped) or out of order get no slot, so a step never stores a
//                         row where it does not also attend it.
//   write_offsets[b, i] = positions[b, i] % P
// Index work only: one launch of a grid-stride loop; HBM-bound at B * (n_blocks + 2 Q + 1) * 4 bytes written.
#include "bpt_device.h"
#include "bpt_internal.h"

namespace bpt {

constexpr int kPrepareThreads = 256;

// Slot indices come from device memory: kept inside the table whatever they hold.
__device__ __forceinline__ int clamp_slot(const PrepareParams& p, int s) {
  return s < 0 ? 0 : (s >= p.num_slots ? p.num_slots - 1 : s);
}

// Row b's context length: its last position + 1, clamped to [0, reserved tokens].
__device__ __forceinline__ int64_t context_len(const PrepareParams& p, int b, int reserved) {
  const int64_t cap = (int64_t)max(reserved, 0) * p.P;
  const int64_t last = load_index(p.positions, (int64_t)b * p.pos_sb + (int64_t)(p.Q - 1) * p.pos_sq, p.pos_i64);
  const int64_t len = last + 1;
  return len < 0 ? 0 : (len > cap ? cap : len);
}

__global__ __launch_bounds__(kPrepareThreads) void paged_prepare_kernel(const PrepareParams p) {
  const int64_t n_table = (int64_t)p.B * p.n_blocks;
  const int64_t n_write = (int64_t)p.B * p.Q;
  const int64_t total = n_table + n_write + p.B;
  for (int64_t i = (int64_t)blockIdx.x * kPrepareThreads + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * kPrepareThreads) {
    if (i < n_table) {
      const int b = (int)(i / p.n_blocks), j = (int)(i - (int64_t)b * p.n_blocks);
      const int slot = clamp_slot(p, p.slots[b]);
      const int reserved = min(p.reserved[slot], p.max_blocks);
      p.block_table[(int64_t)b * p.n_blocks + j] = j < reserved ? p.table[(int64_t)slot * p.table_stride + j] : 0;
    } else if (i < n_table + n_write) {
      const int64_t w = i - n_table;
      const int b = (int)(w / p.Q), qi = (int)(w - (int64_t)b * p.Q);
      const int slot = clamp_slot(p, p.slots[b]);
      const int reserved = min(p.reserved[slot], p.max_blocks);
      const int64_t pos = load_index(p.positions, (int64_t)b * p.pos_sb + (int64_t)qi * p.pos_sq, p.pos_i64);
      const int64_t blk = pos >> p.logP;
      const int64_t len = context_len(p, b, reserved);
      const bool new_token = pos == len - p.Q + qi;
      p.write_blocks[w] = pos >= 0 && blk < reserved && new_token ? p.table[(int64_t)slot * p.table_stride + blk] : -1;
      p.write_offsets[w] = (int)(pos & (p.P - 1));
    } else {
      const int b = (int)(i - n_table - n_write);
      const int slot = clamp_slot(p, p.slots[b]);
      p.context_lens[b] = (int)context_len(p, b, min(p.reserved[slot], p.max_blocks));
    }
  }
}

hipError_t launch_paged_prepare(const PrepareParams& p, hipStream_t stream) {
  const int64_t total = (int64_t)p.B * (p.n_blocks + p.Q + 1);
  if (total == 0) return hipSuccess;
  int64_t groups = (total + kPrepareThreads - 1) / kPrepareThreads;
  if (groups > 1024) groups = 1024;
  hipLaunchKernelGGL(paged_prepare_kernel, dim3((unsigned)groups), dim3(kPrepareThreads), 0, stream, p);
  return hipGetLastError();
}

}  // namespace bpt
