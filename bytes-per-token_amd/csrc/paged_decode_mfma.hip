// Paged decode attention on the matrix cores, for KV heads that serve 2..16 query rows per sequence (G query
// heads x Q queries, up to the speculative-verify case), over an FP8 (e4m3fn) KV cache.
//
// Follows fastserve kernels/kv_attention.py:56-175 (G heads of one KV head per program, online softmax,
// split-K) with engine/attention.py:12-20's causal rule for several queries, like the vector kernel; the
// work decomposition, workspace exchange and combine are the vector kernel's (decode_common.h). What
// differs is the chunk math: all rows of a segment go through the matrix cores together, so every page is
// read once for all of them.
//
// One chunk = 32 tokens = two 16-token tiles; rows are padded to 16 (the MFMA N dimension). With
// l = lane, n = l % 16 (this lane's row), kq = l / 16:
//  * scores S^T = K Q^T with v_mfma_f32_16x16x32_bf16, four K-steps of 32 channels per tile. A = K rows
//    (lane: token 16 t + n, channels 32 kq + 8 s .. + 7 at step s: 32 contiguous bytes per lane, FP8
//    decoded to bf16 exactly; loaded as whole 128-byte rows and rearranged through LDS); B = Q^T (lane:
//    row n, the same channels, from registers). The result gives lane l the scores of row n for tokens
//    16 t + 4 kq + i (i < 4), t = 0, 1: eight per lane.
//  * online softmax per row over those eight values; the row's four lanes agree on the maximum through
//    two shuffles and keep partial weight sums that are added at the end.
//  * output O^T += V^T P^T with v_mfma_f32_16x16x32_f16: the contraction index k = 8 kq + j is mapped to
//    the lane's own score tokens (j < 4: 4 kq + j, j >= 4: 16 + 4 kq + j - 4), so P^T comes straight
//    from this lane's weights, as f16 plus a second product with their f16 rounding remainders (22
//    significant bits, float32-accurate outputs). V^T needs tokens contiguous per lane: V rows are loaded whole like K
//    and passed through the same LDS tile, from which the lane reads channels 8 n' .. 8 n' + 7
//    (n' = l % 16) of its eight tokens (8 bytes each); it transposes 4 x 4 byte blocks with v_perm and
//    decodes FP8 -> f16 exactly; M-tile mu holds channels 8 n' + mu. The accumulator then gives lane l
//    row n, channels 32 kq + 8 i + mu (i < 4, mu < 8): 32 contiguous channels.
// Scales: sm_scale * log2(e) and a per-head K scale multiply the scores, per-token K / V scales the scores
// and weights, a per-head V scale the output. Softmax is in base 2 with the same lazy reference point as
// the vector kernel.
#include <type_traits>

#include "decode_common.h"

namespace bpt {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kMRows = 16;   // rows per segment, padded: the MFMA N dimension
constexpr int kMChunk = 32;  // tokens per chunk: two 16-token tiles

// This lane's share of one chunk: K for its token of each tile, V for its eight score tokens.
struct MChunk {
  U4 k[2][2];          // tile t, load j: token 16 t + 8 j + l / 8, bytes 16 (l % 8) .. 16 (l % 8) + 15
  U4 v[2][2];          // tile t, load j: V of token 16 t + 8 j + l / 8, bytes 16 (l % 8) .. + 15 (as k)
  float sc1;           // per-token scales: lane l holds tile l / 32's token l % 16, K (l / 16 even) or V
  // Fused writes: the bf16 channels 16 (l % 8) .. + 15 of a new token among this lane's four load rows
  // (at most one when fuse_q <= 8), and which load (2 t + j) it replaces, or -1.
  U4 nk[2], nv[2];
  int nsel_k, nsel_v;
};

// The new token among this lane's four rows of chunk kk (first_new: the sequence's first new token), as
// 2 t + j with its index among the new rows, or -1. Only rows stored in place (bit qi of in_place) count.
__device__ __forceinline__ int new_row(int kk, int len, int first_new, unsigned in_place, int lane, int& qi) {
  const int T0 = kk * kMChunk;
  int sel = -1;
  qi = 0;
  if (T0 + kMChunk > first_new) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int tok = T0 + 16 * t + 8 * j + (lane >> 3);
        if (tok >= first_new && tok < len && ((in_place >> (tok - first_new)) & 1u)) {
          sel = 2 * t + j;
          qi = tok - first_new;
        }
      }
    }
  }
  return sel;
}

// 16 new channels (bf16, in order) -> their codes under scale s, as quant_append_kernel computes them
// (IEEE quotient; FP8: clamp to +-448 and round to nearest even; INT8: rint and clamp).
template <int KV>
__device__ __forceinline__ U4 quantize16(const U4 (&x)[2], float s) {
  uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const U4& h = x[i >> 3];
    const uint32_t word = ((i >> 1) & 3) == 0 ? h.x : ((i >> 1) & 3) == 1 ? h.y : ((i >> 1) & 3) == 2 ? h.z : h.w;
    const float f = __uint_as_float((i & 1) ? (word & 0xffff0000u) : (word << 16));
    const float y = __fdiv_rn(f, s);
    uint32_t code;
    if constexpr (KV == kKvFp8) {
      code = f32_to_fp8(clamp_fp8_range(y));
    } else {
      float r = rintf(y);
      r = r > 127.0f ? 127.0f : (r < -128.0f ? -128.0f : r);
      code = (uint32_t)(int32_t)r & 0xffu;
    }
    w[i >> 2] |= code << (8 * (i & 3));
  }
  return U4{w[0], w[1], w[2], w[3]};
}

template <int KV>
__device__ __forceinline__ void substitute(U4 (&rows)[2][2], const U4 (&x)[2], int sel, float s) {
  if (sel < 0) return;
  const U4 c = quantize16<KV>(x, s);
#pragma unroll
  for (int t = 0; t < 2; ++t) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      if (sel == 2 * t + j) rows[t][j] = c;
    }
  }
}

// This launch's share of the new rows' writes: B x fuse_q x Hkv rows of K and of V, one per half-wave,
// 32 lanes x 4 channels, to the caller's (block, offset) slots: the bytes quant_append_kernel stores.
template <int KV, int NT>
__device__ __forceinline__ void fused_append(const DecodeParams& p) {
  const int lane = threadIdx.x & 31;
  const int64_t ntask = (int64_t)p.B * p.fuse_q * p.Hkv * 2;
  for (int64_t task = (int64_t)blockIdx.x * (NT / 32) + (threadIdx.x >> 5); task < ntask;
       task += (int64_t)gridDim.x * (NT / 32)) {
    const int which = (int)(task & 1);
    const int64_t row = task >> 1;
    const int h = (int)(row % p.Hkv);
    const int64_t bq = row / p.Hkv;
    const int qi = (int)(bq % p.fuse_q);
    const int b = (int)(bq / p.fuse_q);
    const int64_t si = (int64_t)b * p.w_sb + (int64_t)qi * p.w_sq;
    const int64_t blk = load_index(p.w_blocks, si, p.w_i64 != 0);
    const int64_t off = load_index(p.w_offsets, si, p.w_i64 != 0);
    if (blk < 0 || blk >= p.num_blocks || off < 0 || off >= p.P) continue;
    if (!slot_is_token(p.table, (int64_t)b * p.table_sb, p.table_i64 != 0, p.max_blocks, p.num_blocks, p.logP,
                       (int64_t)p.lens[b] - p.fuse_q + qi, blk, off))
      continue;
    const uint16_t* src = (which ? p.nv : p.nk) + (int64_t)b * p.n_sb + (int64_t)qi * p.n_sq + (int64_t)h * p.n_sh + 4 * lane;
    const float s = (which ? p.vs : p.ks)[h];
    uint32_t w = 0u;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float y = __fdiv_rn(__uint_as_float((uint32_t)src[i] << 16), s);
      uint32_t code;
      if constexpr (KV == kKvFp8) {
        code = f32_to_fp8(clamp_fp8_range(y));
      } else {
        float r = rintf(y);
        r = r > 127.0f ? 127.0f : (r < -128.0f ? -128.0f : r);
        code = (uint32_t)(int32_t)r & 0xffu;
      }
      w |= code << (8 * i);
    }
    uint8_t* dst = (uint8_t*)(which ? p.v : p.k) + blk * p.kv_sblk + off * p.kv_stok + (int64_t)h * p.kv_shead + 4 * lane;
    *(uint32_t*)dst = w;
  }
}

__device__ __forceinline__ int clamp_page(const DecodeParams& p, int e) {
  return e < 0 ? 0 : (e >= p.num_blocks ? p.num_blocks - 1 : e);
}
__device__ __forceinline__ int clamp_page_u(const DecodeParams& p, int e) { return sread(clamp_page(p, e)); }

// Which of sequence b's new rows (the last fuse_q tokens of its length: row qi is token first_new + qi) are
// stored where the decode reads that token (slot_is_token): bit qi. Rows aimed anywhere else are neither
// stored by this launch nor used by it, so no workgroup ever reads a slot another one may be writing. Scalar
// loads, once per piece.
__device__ __forceinline__ unsigned fused_in_place(const DecodeParams& p, int b, int first_new) {
  unsigned mask = 0u;
  const int ws = p.w_i64 != 0 ? 1 : 0;
  for (int qi = 0; qi < p.fuse_q; ++qi) {
    // Both words of both slot fields at once (an int32 slot's second load repeats its first).
    const int64_t si = (int64_t)b * p.w_sb + (int64_t)qi * p.w_sq;
    const int32_t* wb = (const int32_t*)p.w_blocks + (si << ws);
    const int32_t* wo = (const int32_t*)p.w_offsets + (si << ws);
    const int32_t b_lo = load_uniform(wb), b_hi = load_uniform(wb + ws);
    const int32_t o_lo = load_uniform(wo), o_hi = load_uniform(wo + ws);
    const int64_t blk = ws ? (int64_t)(((uint64_t)(uint32_t)b_hi << 32) | (uint32_t)b_lo) : (int64_t)b_lo;
    const int64_t off = ws ? (int64_t)(((uint64_t)(uint32_t)o_hi << 32) | (uint32_t)o_lo) : (int64_t)o_lo;
    const int64_t tok = (int64_t)first_new + qi;
    if (tok < 0 || (tok >> p.logP) >= p.max_blocks || blk < 0 || blk >= p.num_blocks) continue;
    const int e = clamp_page_u(p, load_uniform((const int32_t*)p.table + table_word(p, b, (int)(tok >> p.logP))));
    if (blk == e && off == (tok & (p.P - 1))) mask |= 1u << qi;
  }
  return mask;
}

// Issue chunk kk's K loads (mfma_issue_k) or V loads and per-token scales (mfma_issue_v). Tokens at or past
// len read the sequence's last token instead (valid memory, never weighted). PU: a 16-token tile lies
// inside one page (page_size >= 16), whose id is read once per tile with a scalar load; otherwise every
// token looks up its own page.
template <bool PU>
__device__ __forceinline__ int mfma_page(const DecodeParams& p, int b, int tile_first, int tok, int len) {
  const int32_t* table = (const int32_t*)p.table;
  if constexpr (PU) return clamp_page(p, load_uniform(table + table_word(p, b, min(tile_first, len - 1) >> p.logP)));
  return clamp_page(p, table[table_word(p, b, tok >> p.logP)]);
}

// K rows are loaded whole: each load instruction covers eight tokens' 128-byte rows (lane l: token
// l / 8, 16 bytes at 16 (l % 8)), which the memory pipeline serves faster than the operand layout's half
// rows of sixteen tokens; mfma_k_operand then rearranges them through LDS.
template <bool PU, bool FUSE>
__device__ __forceinline__ void mfma_issue_k(const DecodeParams& p, int b, int h, int kk, int len, int lane, int first_new,
                                             unsigned in_place, MChunk& c) {
  const int T0 = kk * kMChunk;
  const int r = lane >> 3, sg = lane & 7;
  const int64_t head_off = (int64_t)h * p.kv_shead + 16 * sg;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int tok = min(T0 + 16 * t + 8 * j + r, len - 1);
      const int e = mfma_page<PU>(p, b, T0 + 16 * t, tok, len);
      c.k[t][j] = load16(p.k + (int64_t)e * p.kv_sblk + (int64_t)(tok & (p.P - 1)) * p.kv_stok + head_off);
    }
  }
  if constexpr (FUSE) {
    int qi;
    c.nsel_k = new_row(kk, len, first_new, in_place, lane, qi);
    if (c.nsel_k >= 0) {
      const uint16_t* src = p.nk + (int64_t)b * p.n_sb + (int64_t)qi * p.n_sq + (int64_t)h * p.n_sh + 16 * sg;
      c.nk[0] = load16((const uint8_t*)src);
      c.nk[1] = load16((const uint8_t*)(src + 8));
    }
  }
}

// The score MFMAs' K operand from the loaded rows: lane l gets token 16 t + n, bytes 32 kq .. 32 kq + 31
// (n = l % 16, kq = l / 16), through this wave's LDS tile sk. The 16-byte segments of row x sit at
// segment ^ (x % 8) ^ (x / 8): every 8 lanes of a store (one row) or of a load (rows n .. n + 7) and every
// 16 (two rows; rows n .. n + 15) touch distinct banks.
__device__ __forceinline__ void mfma_k_operand(const MChunk& c, U4 (&sk)[2][16][8], int lane, U4 (&kr)[2][2]) {
  const int r = lane >> 3, sg = lane & 7;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
#pragma unroll
    for (int j = 0; j < 2; ++j) sk[t][8 * j + r][sg ^ r ^ j] = c.k[t][j];
  }
  const int n = lane & 15, kq = lane >> 4;
  const int sw = (n & 7) ^ (n >> 3);
#pragma unroll
  for (int t = 0; t < 2; ++t) {
#pragma unroll
    for (int j = 0; j < 2; ++j) kr[t][j] = sk[t][n][(2 * kq + j) ^ sw];
  }
}

template <int SK, bool PU, bool FUSE>
__device__ __forceinline__ void mfma_issue_v(const DecodeParams& p, int b, int h, int kk, int len, int lane, int first_new,
                                             unsigned in_place, MChunk& c) {
  const int T0 = kk * kMChunk;
  {
    const int r = lane >> 3, sg = lane & 7;
    const int64_t head_off = (int64_t)h * p.kv_shead + 16 * sg;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int tok = min(T0 + 16 * t + 8 * j + r, len - 1);
        const int e = mfma_page<PU>(p, b, T0 + 16 * t, tok, len);
        c.v[t][j] = load16(p.v + (int64_t)e * p.kv_sblk + (int64_t)(tok & (p.P - 1)) * p.kv_stok + head_off);
      }
    }
  }
  if constexpr (SK == kScaleTokenHead) {
    // One scale per lane (32 tokens x K and V); mfma_compute spreads them through LDS.
    const int t = lane >> 5;
    const int tok = min(T0 + 16 * t + (lane & 15), len - 1);
    const int e = mfma_page<PU>(p, b, T0 + 16 * t, tok, len);
    const int64_t so = (int64_t)e * p.sc_sblk + (int64_t)(tok & (p.P - 1)) * p.sc_stok + (int64_t)h * p.sc_shead;
    c.sc1 = ((lane >> 4) & 1 ? p.vs : p.ks)[so];
  }
  if constexpr (FUSE) {
    int qi;
    c.nsel_v = new_row(kk, len, first_new, in_place, lane, qi);
    if (c.nsel_v >= 0) {
      const uint16_t* src = p.nv + (int64_t)b * p.n_sb + (int64_t)qi * p.n_sq + (int64_t)h * p.n_sh + 16 * (lane & 7);
      c.nv[0] = load16((const uint8_t*)src);
      c.nv[1] = load16((const uint8_t*)(src + 8));
    }
  }
}

// The new rows' loads of chunk kk (fused writes), after its K / V loads: which lanes hold a new token and
// their bf16 channels, as mfma_issue_k / mfma_issue_v request them.
__device__ __forceinline__ void mfma_issue_new(const DecodeParams& p, int b, int h, int kk, int len, int lane,
                                               int first_new, unsigned in_place, MChunk& c) {
  int qi;
  c.nsel_k = c.nsel_v = new_row(kk, len, first_new, in_place, lane, qi);
  if (c.nsel_k >= 0) {
    const int64_t row = (int64_t)b * p.n_sb + (int64_t)qi * p.n_sq + (int64_t)h * p.n_sh + 16 * (lane & 7);
    c.nk[0] = load16((const uint8_t*)(p.nk + row));
    c.nk[1] = load16((const uint8_t*)(p.nk + row + 8));
    c.nv[0] = load16((const uint8_t*)(p.nv + row));
    c.nv[1] = load16((const uint8_t*)(p.nv + row + 8));
  }
}

template <int SK, bool PU, bool FUSE>
__device__ __forceinline__ void mfma_issue(const DecodeParams& p, int b, int h, int kk, int len, int lane, int first_new,
                                           unsigned in_place, MChunk& c) {
  mfma_issue_k<PU, FUSE>(p, b, h, kk, len, lane, first_new, in_place, c);
  mfma_issue_v<SK, PU, FUSE>(p, b, h, kk, len, lane, first_new, in_place, c);
}

// 4 x 4 byte transpose: w[i] byte j -> out[j] byte i.
__device__ __forceinline__ void transpose4(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3, uint32_t (&o)[4]) {
  const uint32_t t0 = __builtin_amdgcn_perm(w1, w0, 0x05010400u);  // w0.0 w1.0 w0.1 w1.1
  const uint32_t t1 = __builtin_amdgcn_perm(w3, w2, 0x05010400u);  // w2.0 w3.0 w2.1 w3.1
  const uint32_t t2 = __builtin_amdgcn_perm(w1, w0, 0x07030602u);  // w0.2 w1.2 w0.3 w1.3
  const uint32_t t3 = __builtin_amdgcn_perm(w3, w2, 0x07030602u);  // w2.2 w3.2 w2.3 w3.3
  o[0] = __builtin_amdgcn_perm(t1, t0, 0x05040100u);
  o[1] = __builtin_amdgcn_perm(t1, t0, 0x07060302u);
  o[2] = __builtin_amdgcn_perm(t3, t2, 0x05040100u);
  o[3] = __builtin_amdgcn_perm(t3, t2, 0x07060302u);
}

__device__ __forceinline__ bf16x8 fp8x8_to_bf16(uint32_t w0, uint32_t w1) {
  typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
  const bf16x2v a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.0f, false);
  const bf16x2v b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.0f, true);
  const bf16x2v c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.0f, false);
  const bf16x2v d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.0f, true);
  return bf16x8{a.x, a.y, b.x, b.y, c.x, c.y, d.x, d.y};
}

__device__ __forceinline__ f16x8 fp8x8_to_f16(uint32_t w0, uint32_t w1) {
  typedef _Float16 f16x2v __attribute__((ext_vector_type(2)));
  const f16x2v a = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w0, 1.0f, false);
  const f16x2v b = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w0, 1.0f, true);
  const f16x2v c = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w1, 1.0f, false);
  const f16x2v d = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w1, 1.0f, true);
  return f16x8{a.x, a.y, b.x, b.y, c.x, c.y, d.x, d.y};
}

// Eight int8 codes (bytes of w0 then w1) -> f16, exactly: the bits 0x6400 | (b ^ 0x80) are the f16 value
// 1152 + b, from which 1152 is subtracted.
__device__ __forceinline__ f16x8 int8x8_to_f16(uint32_t w0, uint32_t w1) {
  typedef _Float16 f16x2v __attribute__((ext_vector_type(2)));
  const f16x2v bias = {(_Float16)1152.0f, (_Float16)1152.0f};
  const f16x2v a = __builtin_bit_cast(f16x2v, __builtin_amdgcn_perm(0u, w0, 0x0c010c00u) ^ 0x64806480u) - bias;
  const f16x2v b = __builtin_bit_cast(f16x2v, __builtin_amdgcn_perm(0u, w0, 0x0c030c02u) ^ 0x64806480u) - bias;
  const f16x2v c = __builtin_bit_cast(f16x2v, __builtin_amdgcn_perm(0u, w1, 0x0c010c00u) ^ 0x64806480u) - bias;
  const f16x2v d = __builtin_bit_cast(f16x2v, __builtin_amdgcn_perm(0u, w1, 0x0c030c02u) ^ 0x64806480u) - bias;
  return f16x8{a.x, a.y, b.x, b.y, c.x, c.y, d.x, d.y};
}

// The q operand of the score MFMAs: bf16 for FP8 codes (exact bf16 values), f16 for INT8 codes (exact f16
// values); hi parts for the four K-steps, plus the rounding remainders (lo, QS) when q carries more bits
// than that type: an f16 / f32 q on the bf16 path, an f32 q on the f16 path. (A bf16 q converts to f16
// exactly in f16's normal range; below 2^-14 the dropped remainder is at most 2^-25.)
template <int KV, bool QS>
struct MQ {
  static constexpr bool kF16 = KV == kKvInt8;
  static constexpr int kOps = QS ? 8 : 4;
  typedef typename std::conditional<kF16, f16x8, bf16x8>::type T;
};

// Fold chunk kk into this lane's state: m (row n's reference point, shared by the row's four lanes),
// l (this lane's partial weight sum) and o[mu] (row n, channels 32 kq + 8 i + mu).
// `after_scores` runs once the chunk's K registers are consumed (the caller issues the next chunk's K loads
// there, so they fly during this chunk's softmax and value products).
template <int KV, int SK, bool QS, bool FUSE, typename AfterScores>
__device__ __forceinline__ void mfma_compute(MChunk& c, U4 (&sk)[2][16][8], float (&ssc)[64], int kk, int lane,
                                             const typename MQ<KV, QS>::T (&qb)[MQ<KV, QS>::kOps], float qscale,
                                             int rlen, float& m, float& l, f32x4 (&o)[8], float ks_new, float vs_new,
                                             AfterScores after_scores) {
  const int T0 = kk * kMChunk;
  const int kq = lane >> 4;
  if constexpr (FUSE) substitute<KV>(c.k, c.nk, c.nsel_k, ks_new);
  U4 kr[2][2];
  mfma_k_operand(c, sk, lane, kr);
  // Per-token scales of this lane's score tokens 16 t + 4 kq + i: ks4[t][i] (K), vs4[t][i] (V).
  f32x4 ks4[2], vs4[2];
  if constexpr (SK == kScaleTokenHead) {
    ssc[lane] = c.sc1;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      ks4[t] = *(const f32x4*)&ssc[32 * t + 4 * kq];
      vs4[t] = *(const f32x4*)&ssc[32 * t + 16 + 4 * kq];
    }
  }
  float sc[8];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    f32x4 st = {0.0f, 0.0f, 0.0f, 0.0f};
    const uint32_t w[8] = {kr[t][0].x, kr[t][0].y, kr[t][0].z, kr[t][0].w,
                           kr[t][1].x, kr[t][1].y, kr[t][1].z, kr[t][1].w};
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      if constexpr (MQ<KV, QS>::kF16) {
        const f16x8 a = int8x8_to_f16(w[2 * s], w[2 * s + 1]);
        st = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qb[s], st, 0, 0, 0);
        if constexpr (QS) st = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qb[4 + s], st, 0, 0, 0);
      } else {
        const bf16x8 a = fp8x8_to_bf16(w[2 * s], w[2 * s + 1]);
        st = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qb[s], st, 0, 0, 0);
        if constexpr (QS) st = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qb[4 + s], st, 0, 0, 0);
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int tok = T0 + 16 * t + 4 * kq + i;
      float x = st[i] * qscale;
      if constexpr (SK == kScaleTokenHead) x *= ks4[t][i];
      sc[4 * t + i] = tok < rlen ? x : kNegInf;
    }
  }
  after_scores();

  // ---- online softmax of row n over this chunk's 32 tokens (8 here, 24 on the row's other lanes) -------
  // With per-token value scales the reference point tracks score + vscale_bound(vscale), so that the f16
  // weights e * vscale stay below 2^(kSlack + kBias).
  float mx = kNegInf;
#pragma unroll
  for (int j = 0; j < 8; ++j)
    mx = fmaxf(mx, SK == kScaleTokenHead ? sc[j] + vscale_bound(vs4[j >> 2][j & 3]) : sc[j]);
  mx = max_xor<32>(max_xor<16>(mx));
  const bool move = mx > m + kSlack;
  if (__any(move)) {
    const float mn = move ? mx : m;
    const float alpha = move ? fast_exp2(m - mn) : 1.0f;  // 0 when m was -inf
    l *= alpha;
#pragma unroll
    for (int mu = 0; mu < 8; ++mu) o[mu] *= alpha;
    m = mn;
  }
  const float base = (m == kNegInf ? 0.0f : m) - kBias;
  f16x8 pb, pr;  // the weights in f16 and their rounding remainders: 22 significant bits between them
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float e = fast_exp2(sc[j] - base);
    l += e;
    const float w = SK == kScaleTokenHead ? e * vs4[j >> 2][j & 3] : e;
    pb[j] = (_Float16)w;
    pr[j] = (_Float16)(w - (float)pb[j]);
  }

  // ---- O^T += V^T P^T: eight M-tiles of 16 channels (tile mu: channels 8 n' + mu) -------------------------
  uint32_t lo[2][4], hi[2][4];  // [tile][j]: channel 8 n' + j (lo) or 8 n' + 4 + j (hi), bytes = tokens i
  // V rows through the wave's LDS tile (the K operand's reads are done): lane (n', kq) reads channels
  // 8 n' .. 8 n' + 7 of its score tokens 16 t + 4 kq + i, with the K tile's segment swizzle.
  u32x2 vw[2][4];
  if constexpr (FUSE) substitute<KV>(c.v, c.nv, c.nsel_v, vs_new);
  {
    const int r = lane >> 3, sg = lane & 7;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int j = 0; j < 2; ++j) sk[t][8 * j + r][sg ^ r ^ j] = c.v[t][j];
    }
    const int np = lane & 15;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = 4 * kq + i;
        vw[t][i] = ((const u32x2*)&sk[t][row][(np >> 1) ^ (row & 7) ^ (row >> 3)])[np & 1];
      }
    }
  }
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    transpose4(vw[t][0].x, vw[t][1].x, vw[t][2].x, vw[t][3].x, lo[t]);
    transpose4(vw[t][0].y, vw[t][1].y, vw[t][2].y, vw[t][3].y, hi[t]);
  }
#pragma unroll
  for (int mu = 0; mu < 8; ++mu) {
    const uint32_t d0 = mu < 4 ? lo[0][mu & 3] : hi[0][mu & 3];
    const uint32_t d1 = mu < 4 ? lo[1][mu & 3] : hi[1][mu & 3];
    const f16x8 a = KV == kKvInt8 ? int8x8_to_f16(d0, d1) : fp8x8_to_f16(d0, d1);
    o[mu] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, pb, o[mu], 0, 0, 0);
    o[mu] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, pr, o[mu], 0, 0, 0);
  }
}

// Row n's q (channels 32 kq .. 32 kq + 31) as MFMA B operands for the four K-steps; an f16 / f32 q (QS) also
// gets the bf16 rounding remainder (steps 4 .. 7). Rows past `rows` are zero and see no tokens.
template <int KV, bool QS>
__device__ __forceinline__ void mfma_load_q(const DecodeParams& p, int b, int h, int rows, int len, int lane,
                                            typename MQ<KV, QS>::T (&qb)[MQ<KV, QS>::kOps], int& rlen) {
  typedef typename MQ<KV, QS>::T T;
  typedef typename std::remove_reference<decltype(qb[0][0])>::type E;
  const int kq = lane >> 4, n = lane & 15;
  const bool in = n < rows;
  const int qi = in ? n / p.G : 0;
  const int hq = in ? h * p.G + (n - qi * p.G) : 0;
  rlen = in ? len - (p.noncausal ? 0 : p.Q - 1 - qi) : 0;
  const int64_t base = (int64_t)b * p.q_sb + (int64_t)qi * p.q_sq + (int64_t)hq * p.q_sh + 32 * kq;
  if constexpr (!QS && !MQ<KV, QS>::kF16) {
    // bf16 q on the bf16 path: the words already are the operands.
    const U4* src = (const U4*)((const uint16_t*)p.q + base);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const U4 w = src[s];
      const U4 z = in ? w : U4{0, 0, 0, 0};
      qb[s] = __builtin_bit_cast(T, z);
    }
  } else {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      float f[8];
      load_q<8>(p, base + 8 * s, 1.0f, f);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float x = in ? f[j] : 0.0f;
        const E hbits = (E)x;
        qb[s][j] = hbits;
        if constexpr (QS) qb[4 + s][j] = (E)(x - (float)hbits);
      }
    }
  }
}

template <int KV, int SK, bool PU, bool QS, int NW, bool FUSE>
__global__ __launch_bounds__(NW * 64, kMfmaWavesPerSimd) void decode_mfma_kernel(const DecodeParams p) {
  constexpr int NT = NW * 64;
  constexpr int D = kHeadDim;
  constexpr int RG = kMRows;

  extern __shared__ int s_dyn[];  // [B + 1] line cost per sequence (exclusive prefix sum), then [B] lengths
  int* s_prefix = s_dyn;
  int* s_len = s_dyn + p.B + 1;
  __shared__ int s_wsum[NW];
  __shared__ int s_last;
  __shared__ float s_m[NW][RG];
  __shared__ float s_l[NW][RG];
  // Rows padded by 16 bytes: the merge stores put lane (n, kq) at row n, byte 128 kq (+ 32 i), so unpadded
  // 512-byte rows would send the 16 rows of one store to the same banks (many-row segments store them all).
  __shared__ __attribute__((aligned(16))) float s_o[NW][RG][D + 4];
  __shared__ U4 s_k[NW][2][16][8];  // each wave's K rows of one chunk, on their way to the operand layout
  __shared__ float s_sc[NW][64];    // each wave's per-token scales of one chunk

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = sread(tid >> 6);
  const int kq = lane >> 4, n = lane & 15;
  const int B = p.B;

  if constexpr (FUSE) fused_append<KV, NT>(p);
  build_segment_line<NW, kMChunk>(p, s_prefix, s_len, s_wsum, p.piece_cost);
  zero_empty_sequences<NT>(p, s_prefix);

  // ---- this workgroup's range of chunks (segments are (sequence, KV head): HR = Hkv) ---------------------
  // Segments lie sequence-major on the line, or head-major (HM: all sequences of KV head 0, then of head 1,
  // ...) for many-row segments: with the line numbered XCD-major, the sequences of one KV head then run
  // on one XCD, so pages they share (a common prefix) are fetched from HBM once into that XCD's L2. On the
  // verify workload (16 sequences sharing a 1024-token prefix) that took the fetched bytes from 1.54x to
  // 1.12x the unique bytes and the call from 24.3 to 23.5 us; for 2-row segments sequence-major order,
  // which keeps a sequence's KV heads (one page holds them all) in one L2, is the faster one.
  constexpr bool HM = NW == kMfmaManyRowWaves;
  const int HR = p.HR;
  const int64_t SB = s_prefix[B];  // one KV head's line units
  const int64_t C = (int64_t)HR * SB;
  if (C == 0) return;
  const int64_t per = p.per_forced > 0 ? p.per_forced : (C + gridDim.x - 1) / gridDim.x;
  const int64_t g = line_index(gridDim.x);
  const int64_t c_begin = g * per;
  if (c_begin >= C) return;
  const int64_t c_end = min(c_begin + per, C);
  int64_t c = c_begin;

  int b, h;
  {
    const int64_t hc = HM ? c / SB : 0;  // head-major: the KV head whose stretch holds c
    const int64_t cb = HM ? c - hc * SB : c;
    int lo = 0, hi = B - 1;  // largest b with prefix[b] <= cb (HM), HR * prefix[b] <= cb (sequence-major)
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if ((HM ? 1 : (int64_t)HR) * s_prefix[mid] <= cb) lo = mid; else hi = mid - 1;
    }
    b = sread(lo);
    h = (int)hc;
  }
  // A segment spans X line units, then its nb chunks; a range that starts among the X units starts with
  // the segment's first chunk.
  const int X = p.piece_cost;
  int span = sread(s_prefix[b + 1] - s_prefix[b]);
  int nb = span - X;
  auto seg_start = [&](int sb, int sh, int sspan) -> int64_t {
    return HM ? (int64_t)sh * SB + s_prefix[sb] : (int64_t)HR * s_prefix[sb] + (int64_t)sh * sspan;
  };
  int k;
  {
    if (!HM) h = sread((int)((c - (int64_t)HR * s_prefix[b]) / span));
    k = sread(max((int)(c - seg_start(b, h, span)) - X, 0));
  }
  const int rows = p.Q * p.G;
  {
    // A range that holds no chunk (it lies within one segment's X units) has nothing to do.
    const int64_t seg_c0 = seg_start(b, h, span);
    if (min(c_end, seg_c0 + span) - seg_c0 - X <= k) return;
  }

  // The first piece's q rows and first chunk are requested before the loop; every later piece's while the
  // previous piece's waves are merged.
  typename MQ<KV, QS>::T qb[MQ<KV, QS>::kOps];
  int rlen;
  MChunk cr;
  int len = sread(s_len[b]);
  // Fused writes: the sequence's first new token (its new rows are the last fuse_q of its length) and the
  // head's scales, which quantize them.
  int first_new = 0;
  unsigned in_place = 0u;
  float ks_new = FUSE ? load_uniform(p.ks + h) : 1.0f, vs_new = FUSE ? load_uniform(p.vs + h) : 1.0f;
  float qscale = p.qscale * (SK == kScaleHead ? load_uniform(p.ks + h) : 1.0f);
  // The head's V scale is read with the piece, not at its merge: after a cold start that read is a full
  // memory round trip, which at a workgroup's last merge would stand between its last chunk and its end.
  float vscale = SK == kScaleHead ? load_uniform(p.vs + h) : 1.0f;
  mfma_load_q<KV, QS>(p, b, h, rows, len, lane, qb, rlen);
  {
    const int64_t seg_c0 = seg_start(b, h, span);
    const int k_end = (int)(min(c_end, seg_c0 + span) - seg_c0 - X);
    // Fused writes: the first chunk's K / V loads go out before the lookup of which new rows are stored in
    // place (a chain of scalar loads), which then runs while they are in flight.
    if (k + wave < k_end) mfma_issue<SK, PU, false>(p, b, h, k + wave, len, lane, 0, 0u, cr);
    if constexpr (FUSE) {
      first_new = load_uniform(p.lens + b) - p.fuse_q;
      in_place = fused_in_place(p, b, first_new);
      cr.nsel_k = cr.nsel_v = -1;
      if (k + wave < k_end) mfma_issue_new(p, b, h, k + wave, len, lane, first_new, in_place, cr);
    }
  }

  for (;;) {
    const int64_t seg_c0 = seg_start(b, h, span);
    const int64_t pe = min(c_end, seg_c0 + span);
    const int k_end = (int)(pe - seg_c0 - X);  // this piece's chunks: [k, k_end)

    float m = kNegInf, l = 0.0f;
    f32x4 o[8];
#pragma unroll
    for (int mu = 0; mu < 8; ++mu) o[mu] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    // Chunks k + wave, k + wave + NW, ... of this piece: chunk kk is in flight on entry to its iteration;
    // the next chunk's K loads are issued as soon as kk's scores are done, its V loads after kk's values.
    for (int kk = k + wave; kk < k_end;) {
      const int kn = kk + NW;
      mfma_compute<KV, SK, QS, FUSE>(cr, s_k[wave], s_sc[wave], kk, lane, qb, qscale, rlen, m, l, o, ks_new, vs_new,
                                     [&]() {
                                       if (kn < k_end)
                                         mfma_issue_k<PU, FUSE>(p, b, h, kn, len, lane, first_new, in_place, cr);
                                     });
      if (kn < k_end) mfma_issue_v<SK, PU, FUSE>(p, b, h, kn, len, lane, first_new, in_place, cr);
      kk = kn;
    }

    // The next piece (if the range holds chunks of the next segment): its q rows and this wave's first
    // chunk go in flight now.
    const int b_cur = b, h_cur = h, nb_cur = nb;
    const float vscale_head = vscale;
    const int64_t c_next = pe;
    bool more = false;
    if (c_next < c_end) {
      k = 0;
      if constexpr (HM) {  // the next sequence of this KV head holding chunks, else the next head's first
        do {
          ++b;
        } while (b < B && s_prefix[b + 1] == s_prefix[b]);
        if (b == B) {
          ++h;
          b = 0;
          while (s_prefix[b + 1] == s_prefix[b]) ++b;
        }
        b = sread(b);
        span = sread(s_prefix[b + 1] - s_prefix[b]);
        nb = span - X;
      } else {
        ++h;
        if (h == HR) {
          h = 0;
          do {
            ++b;
          } while (s_prefix[b + 1] == s_prefix[b]);
          b = sread(b);
          span = sread(s_prefix[b + 1] - s_prefix[b]);
          nb = span - X;
        }
      }
      const int kn_end = (int)min((int64_t)nb, c_end - c_next - X);
      more = kn_end > 0;
      if (more) {
        len = sread(s_len[b]);
        if constexpr (FUSE) {
          ks_new = load_uniform(p.ks + h);
          vs_new = load_uniform(p.vs + h);
        }
        qscale = p.qscale * (SK == kScaleHead ? load_uniform(p.ks + h) : 1.0f);
        vscale = SK == kScaleHead ? load_uniform(p.vs + h) : 1.0f;
        mfma_load_q<KV, QS>(p, b, h, rows, len, lane, qb, rlen);
        if (wave < kn_end) mfma_issue<SK, PU, false>(p, b, h, wave, len, lane, 0, 0u, cr);
        if constexpr (FUSE) {
          first_new = load_uniform(p.lens + b) - p.fuse_q;
          in_place = fused_in_place(p, b, first_new);
          cr.nsel_k = cr.nsel_v = -1;
          if (wave < kn_end) mfma_issue_new(p, b, h, wave, len, lane, first_new, in_place, cr);
        }
      }
    }

    // This wave's state of row n: the four lanes' weight sums added, stored for the workgroup merge.
    l = sum_xor<32>(sum_xor<16>(l));
    if (kq == 0) {
      s_m[wave][n] = m;
      s_l[wave][n] = l;
    }
    if (n < rows) {  // the merge reads real rows only
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        *(f32x4*)&s_o[wave][n][32 * kq + 8 * i] = f32x4{o[0][i], o[1][i], o[2][i], o[3][i]};
        *(f32x4*)&s_o[wave][n][32 * kq + 8 * i + 4] = f32x4{o[4][i], o[5][i], o[6][i], o[7][i]};
      }
    }
    __syncthreads();

    // ---- merge the waves; write the segment's output, or this piece's partial ---------------------
    // The segment's number in line order: workspace slots seg + g stay distinct across segments only when
    // segments are numbered in the order the line holds them.
    const int seg = HM ? h_cur * B + b_cur : b_cur * HR + h_cur;
    const int64_t g_first = (seg_c0 + X) / per;  // the workgroups holding the segment's first and last chunks
    const int64_t g_last = (seg_c0 + X + nb_cur - 1) / per;
    const bool whole = g_first == g_last;
    const int64_t wslot = (int64_t)seg + g;
    // Four channels of one row per thread, rows < `rows` only.
    for (int idx = tid; idx < rows * (D / 4); idx += NT) {
      const int r = idx / (D / 4);
      const int ch = 4 * (idx - r * (D / 4));
      float M = kNegInf;
#pragma unroll
      for (int w = 0; w < NW; ++w) M = fmaxf(M, s_m[w][r]);
      const float mu = M == kNegInf ? 0.0f : M;
      float L = 0.0f;
      f32x4 A = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        const float lw = s_l[w][r];
        const float e = lw > 0.0f ? fast_exp2(s_m[w][r] - mu) : 0.0f;
        L += lw * e;
        if (lw > 0.0f) A += *(const f32x4*)&s_o[w][r][ch] * e;
      }
      const float f = L > 0.0f ? vscale_head / L : 0.0f;
      const float lse2 = L > 0.0f ? M - kBias + __log2f(L) : kNegInf;
      if (whole) {
        const int qi = r / p.G;
        const int hq = h_cur * p.G + (r - qi * p.G);
#pragma unroll
        for (int j = 0; j < 4; ++j) write_out(p, b_cur, qi, hq, ch + j, A[j] * f, lse2);
      } else {
#pragma unroll
        for (int j = 0; j < 4; j += 2) ws_store2(p.ws_out + (wslot * RG + r) * D + ch + j, A[j] * f, A[j + 1] * f);
        if (ch == 0) ws_store(p.ws_lse + wslot * RG + r, lse2);
      }
    }
    if (!whole) {
      ws_publish();
      __syncthreads();
      arrive_and_combine<RG, NT>(p, seg, b_cur, h_cur, g_first, (int)(g_last - g_first + 1), rows, tid, &s_last);
    }
    if (!more) break;
    c = c_next;
    __syncthreads();  // the LDS merge buffers are rewritten by the next piece
  }
}

template <int KV, int SK, int NW, bool FUSE>
static hipError_t launch_mfma_nw(const DecodeParams& p, bool pu, bool qs, hipStream_t stream, const LaunchEvents& ev) {
  dim3 grid(p.grid), block(NW * 64);
  const size_t lds = (size_t)(2 * p.B + 1) * sizeof(int);
  if (pu && !qs) launch_kernel(decode_mfma_kernel<KV, SK, true, false, NW, FUSE>, grid, block, lds, stream, ev, p);
  else if (pu) launch_kernel(decode_mfma_kernel<KV, SK, true, true, NW, FUSE>, grid, block, lds, stream, ev, p);
  else if (!qs) launch_kernel(decode_mfma_kernel<KV, SK, false, false, NW, FUSE>, grid, block, lds, stream, ev, p);
  else launch_kernel(decode_mfma_kernel<KV, SK, false, true, NW, FUSE>, grid, block, lds, stream, ev, p);
  return hipGetLastError();
}

template <int KV, int SK>
static hipError_t launch_mfma_sk(const DecodeParams& p, bool pu, bool qs, hipStream_t stream, const LaunchEvents& ev) {
  // The plan's waves per workgroup: 8 for many-row segments, 2 for few-row calls over many segments, else 4.
  const bool many = p.waves == kMfmaManyRowWaves, pair = p.waves == kMfmaPairWaves;
  if (!many && !pair && p.waves != kDecodeWaves) return hipErrorInvalidValue;
  if (many != (p.Q * p.G >= kManyRows)) return hipErrorInvalidValue;
  if constexpr (SK == kScaleHead) {
    if (p.fuse_q > 0) {
      if (many) return launch_mfma_nw<KV, SK, kMfmaManyRowWaves, true>(p, pu, qs, stream, ev);
      if (pair) return launch_mfma_nw<KV, SK, kMfmaPairWaves, true>(p, pu, qs, stream, ev);
      return launch_mfma_nw<KV, SK, kDecodeWaves, true>(p, pu, qs, stream, ev);
    }
  } else {
    if (p.fuse_q > 0) return hipErrorInvalidValue;  // fused writes take per-head scales
  }
  if (many) return launch_mfma_nw<KV, SK, kMfmaManyRowWaves, false>(p, pu, qs, stream, ev);
  if (pair) return launch_mfma_nw<KV, SK, kMfmaPairWaves, false>(p, pu, qs, stream, ev);
  return launch_mfma_nw<KV, SK, kDecodeWaves, false>(p, pu, qs, stream, ev);
}

hipError_t launch_decode_mfma(const DecodeParams& p, int kv_dtype, int scale_kind, hipStream_t stream,
                              const LaunchEvents& ev) {
  const bool pu = p.P >= 16;
  // q needs the hi + lo split when it carries more bits than the score MFMA's type.
  const bool qs = kv_dtype == kKvInt8 ? p.q_dtype == kFF32 : p.q_dtype != kFBf16;
  if (kv_dtype == kKvFp8 && scale_kind == kScaleHead) return launch_mfma_sk<kKvFp8, kScaleHead>(p, pu, qs, stream, ev);
  if (kv_dtype == kKvFp8 && scale_kind == kScaleTokenHead)
    return launch_mfma_sk<kKvFp8, kScaleTokenHead>(p, pu, qs, stream, ev);
  if (kv_dtype == kKvInt8 && scale_kind == kScaleHead) return launch_mfma_sk<kKvInt8, kScaleHead>(p, pu, qs, stream, ev);
  if (kv_dtype == kKvInt8 && scale_kind == kScaleTokenHead)
    return launch_mfma_sk<kKvInt8, kScaleTokenHead>(p, pu, qs, stream, ev);
  return hipErrorInvalidValue;
}

}  // namespace bpt
