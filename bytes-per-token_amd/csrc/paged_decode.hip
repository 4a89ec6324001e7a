// Paged decode attention over a BF16, FP8 (e4m3fn) or INT8 KV cache, dequantized in registers: one launch.
//
// Algorithm (follows fastserve kernels/kv_attention.py:56-175, kernels/reference.py:186-211): the rows of a
// KV head are its G query heads times the sequence's Q queries, so each cached page is read from HBM once
// for all of them. Keys and values stream through in chunks; every lane keeps an online softmax (running
// max m, weight sum l, weighted value sum acc) over the tokens it saw, and states are merged exactly with
// the log-sum-exp algebra of reference.merge_partials.
//
// Work decomposition (stream-K): a segment is one (sequence, KV head, row group) and owns ceil(len / CHUNK)
// chunks, preceded on the line by a few units that stand for the cost of one more piece merge; segments are
// laid end to end (sequence-major) and the launched workgroups split that line into equal contiguous
// ranges (numbered XCD-major), so ragged batches and long contexts balance to within one chunk. Each
// workgroup computes the chunk counts' prefix sum itself and keeps it, with the lengths, in LDS (lengths
// stay on the device), then walks its range segment by segment ("pieces"). The waves of a workgroup take
// a piece's chunks round-robin; each chunk's block-table entries are read while the previous chunk is
// computed. The next piece's q rows and first chunk are requested before the current piece's waves are
// merged, so the merge overlaps their latency. A segment covered by one workgroup is written directly;
// otherwise every workgroup writes its piece's normalized output and log2-sum-exp to a workspace slot as
// soon as the piece is done, bumps the segment's arrival counter, and the last arriver combines all
// pieces and resets the counter to zero (no waiting on other workgroups anywhere).
//
// Wave layout (D = 128, one-byte codes): lane = slot * 8 + part. `part` owns channels [16 part, 16 part + 16)
// and loads them with one 16-byte load per token row; one load instruction covers 8 token rows. Scores are
// summed over the 8 lanes of a slot with DPP. BF16 pools use 16 lanes per row (8 channels each).
//
// Compute: FP8 and BF16 keys are dotted with q held as bf16 pairs (v_dot2_f32_bf16; FP8 codes convert to
// bf16 exactly), and so are INT8 keys when q is bf16 (codes converted exactly through f32); FP8 values are
// decoded to f16 two tokens at a time and accumulated with v_dot2_f32_f16 over token pairs, the weights as
// f16 plus their f16 rounding remainders (22 significant bits); INT8 values (and INT8 keys under an f16 /
// f32 q) use f32 FMAs. Scales fold out of the inner loop: a per-head K scale and
// sm_scale * log2(e) multiply the reduced score, a per-head V scale multiplies the final output, per-token
// scales multiply the reduced score (K) and the softmax weight (V). Softmax runs in base 2 with a lazily
// moved reference point; the workspace lse is in log2 units.
#include "decode_common.h"

namespace bpt {

template <int KV>
struct KvTraits {
  static constexpr int kBytes = KV == kKvBf16 ? 2 : 1;
  static constexpr int kVec = 16 / kBytes;          // elements in one 16-byte load
  static constexpr int kLanesPerRow = kHeadDim / kVec;
  static constexpr int kRowsPerLoad = 64 / kLanesPerRow;
};

// 16 bytes of cache -> kVec floats (codes, not yet scaled).
template <int KV>
__device__ __forceinline__ void unpack16(const U4& r, float* f) {
  const uint32_t w[4] = {r.x, r.y, r.z, r.w};
  if constexpr (KV == kKvFp8) {
#pragma unroll
    for (int j = 0; j < 4; ++j) fp8x4_to_f32(w[j], f + 4 * j);
  } else if constexpr (KV == kKvInt8) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int b = 0; b < 4; ++b) f[4 * j + b] = (float)(int8_t)((w[j] >> (8 * b)) & 0xffu);
    }
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      f[2 * j] = __uint_as_float(w[j] << 16);
      f[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
    }
  }
}

// One chunk of one lane's K and V rows (and per-token scales), and the physical page of each of its loads.
template <int CL>
struct ChunkRegs {
  U4 k[CL];
  U4 v[CL];
  float ks[CL];
  float vs[CL];
};

template <int CL>
struct ChunkPages {
  int e[CL];
};

// Physical pages of chunk kk's loads. PU: a page holds whole load rows (page_size >= rows per load), so each
// load's page is wave-uniform and read with a scalar load; otherwise every lane reads its own row's page.
template <int KV, int CL, bool PU>
__device__ __forceinline__ void fetch_pages(const DecodeParams& p, int b, int kk, int len, int slot, ChunkPages<CL>& g) {
  constexpr int RPL = KvTraits<KV>::kRowsPerLoad;
  const int tb = kk * CL * RPL;
  const int32_t* table = (const int32_t*)p.table;
#pragma unroll
  for (int i = 0; i < CL; ++i) {
    int e;
    if constexpr (PU) {
      const int t0 = tb + i * RPL;  // wave-uniform
      e = t0 < len ? load_uniform(table + table_word(p, b, t0 >> p.logP)) : 0;
    } else {
      const int t = tb + i * RPL + slot;
      e = t < len ? table[table_word(p, b, t >> p.logP)] : 0;
    }
    g.e[i] = e < 0 ? 0 : (e >= p.num_blocks ? p.num_blocks - 1 : e);
  }
}

// Issue chunk kk's 16-byte K and V loads (and per-token scales) into c. PU: each load's page and the row
// offset of its first token are wave-uniform, so the address is a scalar base plus this lane's constant
// 32-bit offset (slot rows down, part * 16 bytes across).
// Rows at or past len: INT8 codes are loaded anyway from the (valid) page fetch_pages chose, since any byte
// is a finite code, their scores are masked and their value scale is zeroed, so they weigh nothing; this
// keeps the loads unconditional. FP8 and BF16 rows there are zero-filled instead (stale bytes could hold
// NaN codes, and NaN times a zero weight is NaN).
template <int KV, int SK, int CL, bool PU>
__device__ __forceinline__ void issue_chunk(const DecodeParams& p, const ChunkPages<CL>& g, int h, int kk, int len,
                                            int slot, int part, ChunkRegs<CL>& c) {
  constexpr int RPL = KvTraits<KV>::kRowsPerLoad;
  const int tb = kk * CL * RPL;
  const int64_t head_off = (int64_t)h * p.kv_shead;
#pragma unroll
  for (int i = 0; i < CL; ++i) {
    const int t = tb + i * RPL + slot;
    c.ks[i] = 1.0f;
    c.vs[i] = 1.0f;
    if (KV == kKvInt8 || t < len) {
      if constexpr (PU) {
        const int w0 = (tb + i * RPL) & (p.P - 1);  // wave-uniform: this lane's row is w0 + slot
        const int64_t base = (int64_t)g.e[i] * p.kv_sblk + (int64_t)w0 * p.kv_stok + head_off;
        const uint32_t lane_off = (uint32_t)(slot * p.kv_stok) + (uint32_t)part * 16u;
        c.k[i] = load16(p.k + base + lane_off);
        c.v[i] = load16(p.v + base + lane_off);
        if constexpr (SK == kScaleTokenHead) {
          const int64_t sb = (int64_t)g.e[i] * p.sc_sblk + (int64_t)w0 * p.sc_stok + (int64_t)h * p.sc_shead;
          const uint32_t so = (uint32_t)(slot * p.sc_stok);
          c.ks[i] = p.ks[sb + so];
          c.vs[i] = t < len ? p.vs[sb + so] : 0.0f;
        }
      } else {
        const int within = t & (p.P - 1);
        const int64_t off = (int64_t)g.e[i] * p.kv_sblk + (int64_t)within * p.kv_stok + head_off + part * 16;
        c.k[i] = load16(p.k + off);
        c.v[i] = load16(p.v + off);
        if constexpr (SK == kScaleTokenHead) {
          const int64_t so = (int64_t)g.e[i] * p.sc_sblk + (int64_t)within * p.sc_stok + (int64_t)h * p.sc_shead;
          c.ks[i] = p.ks[so];
          c.vs[i] = t < len ? p.vs[so] : 0.0f;
        }
      }
    } else {
      c.k[i] = U4{0, 0, 0, 0};
      c.v[i] = U4{0, 0, 0, 0};
    }
  }
}

// The query rows of a piece in the form the score path consumes. Dot-product paths (FP8, BF16 caches)
// keep q unscaled as bf16 pairs: exact for a bf16 q; for an f16 / f32 q (QS) a second pair holds the
// rounding remainder, so hi + lo carries 16 significant bits. INT8 caches under an f16 / f32 q keep
// pre-scaled floats instead.
template <int KV, int RG, bool QS>
struct QRows {
  static constexpr int VEC = KvTraits<KV>::kVec;
  static constexpr bool kDot = KV != kKvInt8 || !QS;  // INT8 with a bf16 q: codes made bf16, q exact
  bf16x2 hi[RG][kDot ? VEC / 2 : 1];
  bf16x2 lo[RG][(kDot && QS) ? VEC / 2 : 1];
  float f[RG][kDot ? 1 : VEC];
  float scale;  // applied to each reduced score
};

// Fold chunk kk into this lane's online-softmax state.
template <int KV, int SK, int RG, int CL, bool QS>
__device__ __forceinline__ void compute_chunk(const ChunkRegs<CL>& c, int kk, int slot, const QRows<KV, RG, QS>& q,
                                              const int (&rlen)[RG], float (&m)[RG], float (&l)[RG],
                                              float (&acc)[RG][KvTraits<KV>::kVec]) {
  constexpr int VEC = KvTraits<KV>::kVec;
  constexpr int LPR = KvTraits<KV>::kLanesPerRow;
  constexpr int RPL = KvTraits<KV>::kRowsPerLoad;
  constexpr int CH = CL * RPL;
  constexpr bool kDotK = QRows<KV, RG, QS>::kDot;  // scores from packed bf16 dot products
  constexpr bool kDotV = KV == kKvFp8;   // values through packed f16 dot products over token pairs
  static_assert(!kDotV || CL % 2 == 0, "token pairs need an even number of loads per chunk");
  const int tb = kk * CH + slot;

  // ---- scores: this lane's partial dot products, summed over the lanes of each token row ------------
  float s[CL][RG];
#pragma unroll
  for (int i = 0; i < CL; ++i) {
    const uint32_t w[4] = {c.k[i].x, c.k[i].y, c.k[i].z, c.k[i].w};
    if constexpr (kDotK) {
      bf16x2 kp[VEC / 2];
      if constexpr (KV == kKvFp8) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          kp[2 * j] = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[j], 1.0f, false);
          kp[2 * j + 1] = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[j], 1.0f, true);
        }
      } else if constexpr (KV == kKvInt8) {
        // int8 -> f32 (exact), then the high halves of two f32 values form one bf16 pair (exact: |code| <= 128
        // needs 8 significant bits).
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float f[4];
#pragma unroll
          for (int b = 0; b < 4; ++b) f[b] = (float)(int8_t)((w[j] >> (8 * b)) & 0xffu);
          kp[2 * j] = __builtin_bit_cast(bf16x2, __builtin_amdgcn_perm(__float_as_uint(f[1]), __float_as_uint(f[0]), 0x07060302u));
          kp[2 * j + 1] = __builtin_bit_cast(bf16x2, __builtin_amdgcn_perm(__float_as_uint(f[3]), __float_as_uint(f[2]), 0x07060302u));
        }
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) kp[j] = __builtin_bit_cast(bf16x2, w[j]);
      }
#pragma unroll
      for (int r = 0; r < RG; ++r) {
        float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
        for (int j = 0; j < VEC / 2; j += 2) {
          a0 = __builtin_amdgcn_fdot2_f32_bf16(q.hi[r][j], kp[j], a0, false);
          a1 = __builtin_amdgcn_fdot2_f32_bf16(q.hi[r][j + 1], kp[j + 1], a1, false);
          if constexpr (QS) {
            a0 = __builtin_amdgcn_fdot2_f32_bf16(q.lo[r][j], kp[j], a0, false);
            a1 = __builtin_amdgcn_fdot2_f32_bf16(q.lo[r][j + 1], kp[j + 1], a1, false);
          }
        }
        s[i][r] = a0 + a1;
      }
    } else {
      float kf[VEC];
      unpack16<KV>(c.k[i], kf);
#pragma unroll
      for (int r = 0; r < RG; ++r) {
        float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
        for (int v = 0; v < VEC; v += 2) {
          a0 = fmaf(q.f[r][v], kf[v], a0);
          a1 = fmaf(q.f[r][v + 1], kf[v + 1], a1);
        }
        s[i][r] = a0 + a1;
      }
    }
  }
#pragma unroll
  for (int i = 0; i < CL; ++i) {
    const int t = tb + i * RPL;
#pragma unroll
    for (int r = 0; r < RG; ++r) {
      float x = group_sum<LPR>(s[i][r]) * q.scale;
      if constexpr (SK == kScaleTokenHead) x *= c.ks[i];
      s[i][r] = t < rlen[r] ? x : kNegInf;
    }
  }

  // ---- online softmax. m is a reference point, moved only when a score passes it by kSlack: weights
  // are 2^(score - m + kBias) <= 2^(kSlack + kBias), so the accumulators are rarely rescaled and the
  // packed f16 weights never overflow. Per-token value scales ride in the f16 weights of the FP8 path, so
  // there m tracks score + vscale_bound(vscale) (the weight sums keep the bare exponentials). ------------
  constexpr bool kScaledF16 = kDotV && SK == kScaleTokenHead;
  float pw[CL][RG];
#pragma unroll
  for (int r = 0; r < RG; ++r) {
    float mc = kNegInf;
#pragma unroll
    for (int i = 0; i < CL; ++i) mc = fmaxf(mc, kScaledF16 ? s[i][r] + vscale_bound(c.vs[i]) : s[i][r]);
    const bool move = mc > m[r] + kSlack;
    if (__any(move)) {
      const float mn = move ? mc : m[r];
      const float alpha = move ? fast_exp2(m[r] - mn) : 1.0f;  // 0 when m was -inf
      l[r] *= alpha;
#pragma unroll
      for (int v = 0; v < VEC; ++v) acc[r][v] *= alpha;
      m[r] = mn;
    }
    const float mu = (m[r] == kNegInf ? 0.0f : m[r]) - kBias;
    float lsum = l[r];
#pragma unroll
    for (int i = 0; i < CL; ++i) {
      const float e = fast_exp2(s[i][r] - mu);
      lsum += e;
      pw[i][r] = e * c.vs[i];
    }
    l[r] = lsum;
  }

  // ---- values ------------------------------------------------------------------------------------------
  if constexpr (kDotV) {
    // Two token rows of this lane at a time: bytes of rows a and b are interleaved so one f16 pair holds
    // channel c of both rows, and one dot product adds both rows' weighted contributions to channel c.
#pragma unroll
    for (int i = 0; i < CL; i += 2) {
      f16x2 pp[RG], pr[RG];  // weights in f16 and their rounding remainders (22 significant bits together)
#pragma unroll
      for (int r = 0; r < RG; ++r) {
        pp[r] = f16x2{(_Float16)pw[i][r], (_Float16)pw[i + 1][r]};
        pr[r] = f16x2{(_Float16)(pw[i][r] - (float)pp[r].x), (_Float16)(pw[i + 1][r] - (float)pp[r].y)};
      }
      const uint32_t a[4] = {c.v[i].x, c.v[i].y, c.v[i].z, c.v[i].w};
      const uint32_t b[4] = {c.v[i + 1].x, c.v[i + 1].y, c.v[i + 1].z, c.v[i + 1].w};
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const uint32_t lo = __builtin_amdgcn_perm(b[d], a[d], 0x05010400u);  // a.c0 b.c0 a.c1 b.c1
        const uint32_t hi = __builtin_amdgcn_perm(b[d], a[d], 0x07030602u);  // a.c2 b.c2 a.c3 b.c3
        const f16x2 v0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(lo, 1.0f, false);
        const f16x2 v1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(lo, 1.0f, true);
        const f16x2 v2 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(hi, 1.0f, false);
        const f16x2 v3 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(hi, 1.0f, true);
#pragma unroll
        for (int r = 0; r < RG; ++r) {
          acc[r][4 * d + 0] = __builtin_amdgcn_fdot2(v0, pp[r], acc[r][4 * d + 0], false);
          acc[r][4 * d + 1] = __builtin_amdgcn_fdot2(v1, pp[r], acc[r][4 * d + 1], false);
          acc[r][4 * d + 2] = __builtin_amdgcn_fdot2(v2, pp[r], acc[r][4 * d + 2], false);
          acc[r][4 * d + 3] = __builtin_amdgcn_fdot2(v3, pp[r], acc[r][4 * d + 3], false);
          acc[r][4 * d + 0] = __builtin_amdgcn_fdot2(v0, pr[r], acc[r][4 * d + 0], false);
          acc[r][4 * d + 1] = __builtin_amdgcn_fdot2(v1, pr[r], acc[r][4 * d + 1], false);
          acc[r][4 * d + 2] = __builtin_amdgcn_fdot2(v2, pr[r], acc[r][4 * d + 2], false);
          acc[r][4 * d + 3] = __builtin_amdgcn_fdot2(v3, pr[r], acc[r][4 * d + 3], false);
        }
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < CL; ++i) {
      float vf[VEC];
      unpack16<KV>(c.v[i], vf);
#pragma unroll
      for (int r = 0; r < RG; ++r) {
#pragma unroll
        for (int v = 0; v < VEC; ++v) acc[r][v] = fmaf(pw[i][r], vf[v], acc[r][v]);
      }
    }
  }
}

// Merge the online-softmax states of the wave's slots (same channels, disjoint tokens) and store the
// wave's state for one segment: m and l per row, acc per row and channel.
template <int KV, int RG>
__device__ __forceinline__ void close_state(float (&m)[RG], float (&l)[RG], float (&acc)[RG][KvTraits<KV>::kVec],
                                            int slot, int part, float* sm, float* sl, float* sacc) {
  constexpr int VEC = KvTraits<KV>::kVec;
  constexpr int LPR = KvTraits<KV>::kLanesPerRow;
#pragma unroll
  for (int off = LPR; off < 64; off <<= 1) {
#pragma unroll
    for (int r = 0; r < RG; ++r) {
      const float mo = shfl_xor_f(m[r], off);
      const float lo = shfl_xor_f(l[r], off);
      const float mn = fmaxf(m[r], mo);
      const float mu = mn == kNegInf ? 0.0f : mn;
      const float a = l[r] > 0.0f ? fast_exp2(m[r] - mu) : 0.0f;
      const float e = lo > 0.0f ? fast_exp2(mo - mu) : 0.0f;
      l[r] = l[r] * a + lo * e;
#pragma unroll
      for (int v = 0; v < VEC; ++v) {
        const float other = shfl_xor_f(acc[r][v], off);
        acc[r][v] = (a > 0.0f ? acc[r][v] * a : 0.0f) + (e > 0.0f ? other * e : 0.0f);
      }
      m[r] = mn;
    }
  }
  if (slot == 0) {
#pragma unroll
    for (int r = 0; r < RG; ++r) {
#pragma unroll
      for (int v = 0; v < VEC; ++v) sacc[r * kHeadDim + part * VEC + v] = acc[r][v];
      if (part == 0) {
        sm[r] = m[r];
        sl[r] = l[r];
      }
    }
  }
}

// The q rows of segment (b, KV head h, row group rg): bf16 pairs for the dot-product paths, pre-scaled
// floats for INT8; and the tokens each row sees (query i of Q sits at position len - Q + i).
template <int KV, int RG, bool QS>
__device__ __forceinline__ void load_q_rows(const DecodeParams& p, QRows<KV, RG, QS>& q, int (&rlen)[RG], int b, int h,
                                            int rg, int rows, int part, int len, float kscale_head) {
  constexpr int VEC = KvTraits<KV>::kVec;
  q.scale = QRows<KV, RG, QS>::kDot ? p.qscale * kscale_head : 1.0f;
#pragma unroll
  for (int r = 0; r < RG; ++r) {
    const int gr = rg * RG + r;
    float qf[VEC];
    if (gr < rows) {
      const int qi = gr / p.G;
      const int hq = h * p.G + (gr - qi * p.G);
      const int64_t base = (int64_t)b * p.q_sb + (int64_t)qi * p.q_sq + (int64_t)hq * p.q_sh + part * VEC;
      load_q<VEC>(p, base, QRows<KV, RG, QS>::kDot ? 1.0f : p.qscale * kscale_head, qf);
      rlen[r] = len - (p.noncausal ? 0 : p.Q - 1 - qi);
    } else {
#pragma unroll
      for (int v = 0; v < VEC; ++v) qf[v] = 0.0f;
      rlen[r] = 0;
    }
    if constexpr (QRows<KV, RG, QS>::kDot) {
#pragma unroll
      for (int j = 0; j < VEC / 2; ++j) {
        q.hi[r][j] = pack_bf16(qf[2 * j], qf[2 * j + 1]);
        if constexpr (QS)
          q.lo[r][j] = pack_bf16(qf[2 * j] - (float)q.hi[r][j].x, qf[2 * j + 1] - (float)q.hi[r][j].y);
      }
    } else {
#pragma unroll
      for (int v = 0; v < VEC; ++v) q.f[r][v] = qf[v];
    }
  }
}

template <int KV, int SK, int RG, bool PU, bool QS>
__global__ __launch_bounds__(kDecodeWaves * 64,
                             decode_groups_per_cu(KV == kKvInt8, RG, PU, QS) == kDecodeGroupsPerCuInt8 ? 3 : 1)
void decode_kernel(const DecodeParams p) {
  constexpr int NW = kDecodeWaves;
  constexpr int NT = NW * 64;
  constexpr int D = kHeadDim;
  constexpr int VEC = KvTraits<KV>::kVec;
  constexpr int LPR = KvTraits<KV>::kLanesPerRow;
  constexpr int CL = decode_loads(RG);
  constexpr int CH = CL * KvTraits<KV>::kRowsPerLoad;

  extern __shared__ int s_dyn[];  // [B + 1] line cost per sequence (exclusive prefix sum), then [B] lengths
  int* s_prefix = s_dyn;
  int* s_len = s_dyn + p.B + 1;
  __shared__ int s_wsum[NW];
  __shared__ int s_last;
  __shared__ float s_m[NW][RG];
  __shared__ float s_l[NW][RG];
  __shared__ float s_acc[NW][RG][D];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = sread(tid >> 6);
  const int B = p.B;

  // Equal partitions when the plan asked for them and every sequence has the same length: no piece cost, the
  // first equal_grid workgroups each take the smallest power-of-two number of chunks that they cover between
  // them, and the rest of the launch leaves. Otherwise the whole launch shares the line cut.
  const SegmentLine line = build_segment_line<NW, CH>(p, s_prefix, s_len, s_wsum, p.piece_cost, p.equal_grid > 0);
  const int X = sread(line.piece_cost);
  const bool equal = sread(line.uniform ? 1 : 0) != 0;
  zero_empty_sequences<NT>(p, s_prefix);

  // ---- this workgroup's range of chunks -----------------------------------------------------------
  const int HR = p.HR;
  const int64_t C = (int64_t)HR * s_prefix[B];
  if (C == 0) return;
  const int n_line = equal ? p.equal_grid : (int)gridDim.x;
  if ((int)blockIdx.x >= n_line) return;
  int64_t per = p.per_forced > 0 ? p.per_forced : (C + n_line - 1) / n_line;
  if (equal) {
    int64_t pw = 1;
    while (pw < per) pw *= 2;
    per = pw;
  }
  const int64_t g = line_index(n_line);
  const int64_t c_begin = g * per;
  if (c_begin >= C) return;
  const int64_t c_end = min(c_begin + per, C);
  int64_t c = c_begin;

  int b;
  {
    int lo = 0, hi = B - 1;  // largest b with HR * prefix[b] <= c
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if ((int64_t)HR * s_prefix[mid] <= c) lo = mid; else hi = mid - 1;
    }
    b = sread(lo);
  }
  // A segment spans X line units, then its nb chunks; a range that starts among the X units starts with
  // the segment's first chunk.
  int span = sread(s_prefix[b + 1] - s_prefix[b]);
  int nb = span - X;
  int hr, k;
  {
    const int64_t r = c - (int64_t)HR * s_prefix[b];
    hr = sread((int)(r / span));
    k = sread(max((int)(r - (int64_t)hr * span) - X, 0));
  }
  {
    // A range that holds no chunk (it lies within one segment's X units) has nothing to do.
    const int64_t seg_c0 = (int64_t)HR * s_prefix[b] + (int64_t)hr * span;
    if (min(c_end, seg_c0 + span) - seg_c0 - X <= k) return;
  }

  const int slot = lane / LPR;
  const int part = lane - slot * LPR;
  const int rows = p.Q * p.G;

  // The first piece's q rows and first chunk are requested before the loop; every later piece's are
  // requested while the previous piece's waves are merged, so that merge overlaps their latency.
  QRows<KV, RG, QS> q;
  int rlen[RG];
  ChunkRegs<CL> cr;
  ChunkPages<CL> gp;
  int len = sread(s_len[b]);
  // The head's V scale is read with the piece, not at its merge (after a cold start, a full memory round
  // trip between a workgroup's last chunk and its end).
  float vscale = SK == kScaleHead ? load_uniform(p.vs + hr / p.n_rg) : 1.0f;
  {
    const int h = hr / p.n_rg;
    load_q_rows<KV, RG, QS>(p, q, rlen, b, h, hr - h * p.n_rg, rows, part, len,
                            SK == kScaleHead ? load_uniform(p.ks + h) : 1.0f);
    const int64_t seg_c0 = (int64_t)HR * s_prefix[b] + (int64_t)hr * span;
    const int k_end = (int)(min(c_end, seg_c0 + span) - seg_c0 - X);
    if (k + wave < k_end) {
      fetch_pages<KV, CL, PU>(p, b, k + wave, len, slot, gp);
      issue_chunk<KV, SK, CL, PU>(p, gp, h, k + wave, len, slot, part, cr);
    }
  }

  // ---- pieces: the parts of segments inside [c_begin, c_end) -------------------------------------------
  for (;;) {
    const int64_t seg_c0 = (int64_t)HR * s_prefix[b] + (int64_t)hr * span;
    const int64_t pe = min(c_end, seg_c0 + span);
    const int k_end = (int)(pe - seg_c0 - X);  // this piece's chunks: [k, k_end)
    const int h = hr / p.n_rg;
    const int rg = hr - h * p.n_rg;

    float m[RG], l[RG], acc[RG][VEC];
#pragma unroll
    for (int r = 0; r < RG; ++r) {
      m[r] = kNegInf;
      l[r] = 0.0f;
#pragma unroll
      for (int v = 0; v < VEC; ++v) acc[r][v] = 0.0f;
    }

    // Chunks k + wave, k + wave + NW, ... of this piece; chunk kk's loads are in flight on entry to its
    // iteration, the next chunk's pages are fetched while it is computed, then its loads are issued. The
    // last chunk is peeled off so that the loop body issues unconditionally (no register copies of the
    // chunk buffer for a skipped issue).
    int kk = k + wave;
    for (; kk + NW < k_end; kk += NW) {
      const int kn = kk + NW;
      fetch_pages<KV, CL, PU>(p, b, kn, len, slot, gp);
      compute_chunk<KV, SK, RG, CL, QS>(cr, kk, slot, q, rlen, m, l, acc);
      issue_chunk<KV, SK, CL, PU>(p, gp, h, kn, len, slot, part, cr);
    }
    if (kk < k_end) compute_chunk<KV, SK, RG, CL, QS>(cr, kk, slot, q, rlen, m, l, acc);

    // The next piece (if the range holds chunks of the next segment): its q rows and this wave's first
    // chunk go in flight now.
    const int b_cur = b, hr_cur = hr, nb_cur = nb;
    const float vscale_head = vscale;
    const int64_t c_next = pe;
    bool more = false;
    if (c_next < c_end) {
      ++hr;
      k = 0;
      if (hr == HR) {
        hr = 0;
        do {
          ++b;
        } while (s_prefix[b + 1] == s_prefix[b]);
        b = sread(b);
        span = sread(s_prefix[b + 1] - s_prefix[b]);
        nb = span - X;
      }
      const int kn_end = (int)min((int64_t)nb, c_end - c_next - X);
      more = kn_end > 0;
      if (more) {
        len = sread(s_len[b]);
        const int hn = hr / p.n_rg;
        load_q_rows<KV, RG, QS>(p, q, rlen, b, hn, hr - hn * p.n_rg, rows, part, len,
                                SK == kScaleHead ? load_uniform(p.ks + hn) : 1.0f);
        vscale = SK == kScaleHead ? load_uniform(p.vs + hn) : 1.0f;
        if (wave < kn_end) {
          fetch_pages<KV, CL, PU>(p, b, wave, len, slot, gp);
          issue_chunk<KV, SK, CL, PU>(p, gp, hn, wave, len, slot, part, cr);
        }
      }
    }

    close_state<KV, RG>(m, l, acc, slot, part, &s_m[wave][0], &s_l[wave][0], &s_acc[wave][0][0]);
    __syncthreads();

    // ---- merge the waves; write the segment's output, or this piece's partial ---------------------
    const int seg = b_cur * HR + hr_cur;
    const int64_t g_first = (seg_c0 + X) / per;  // the workgroups holding the segment's first and last chunks
    const int64_t g_last = (seg_c0 + X + nb_cur - 1) / per;
    const bool whole = g_first == g_last;
    const int64_t wslot = (int64_t)seg + g;
    for (int idx = tid; idx < RG * D; idx += NT) {
      const int r = idx / D;
      const int ch = idx - r * D;
      const int gr = rg * RG + r;
      if (gr >= rows) continue;
      float M = kNegInf;
#pragma unroll
      for (int w = 0; w < NW; ++w) M = fmaxf(M, s_m[w][r]);
      const float mu = M == kNegInf ? 0.0f : M;
      float L = 0.0f, A = 0.0f;
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        const float lw = s_l[w][r];
        const float e = lw > 0.0f ? fast_exp2(s_m[w][r] - mu) : 0.0f;
        L += lw * e;
        A += lw > 0.0f ? s_acc[w][r][ch] * e : 0.0f;
      }
      const float o = L > 0.0f ? A / L * vscale_head : 0.0f;
      if (whole) {
        const int qi = gr / p.G;
        const int hq = h * p.G + (gr - qi * p.G);
        write_out(p, b_cur, qi, hq, ch, o, L > 0.0f ? M - kBias + __log2f(L) : kNegInf);
      } else {
        ws_store(p.ws_out + (wslot * RG + r) * D + ch, o);
        if (ch == 0) ws_store(p.ws_lse + wslot * RG + r, L > 0.0f ? M - kBias + __log2f(L) : kNegInf);
      }
    }
    if (!whole) {
      // Publish the piece now: partials travel as device-coherent accesses, so the only ordering needed is
      // that this workgroup's stores have completed before its arrival is counted.
      ws_publish();
      __syncthreads();
      arrive_and_combine<RG, NT>(p, seg, b_cur, hr_cur, g_first, (int)(g_last - g_first + 1), rows, tid, &s_last);
    }
    if (!more) break;
    c = c_next;
    __syncthreads();  // the LDS merge buffers are rewritten by the next piece
  }
}

template <int KV, int SK, int RG>
static hipError_t launch_t(const DecodeParams& p, bool page_uniform, hipStream_t stream, const LaunchEvents& ev) {
  dim3 grid(p.grid), block(kDecodeWaves * 64);
  const size_t lds = (size_t)(2 * p.B + 1) * sizeof(int);  // the line's cost prefix sum and the lengths
  // A non-bf16 q needs the hi + lo split on the FP8 / BF16 dot-product paths; INT8 caches take the dot path
  // with a bf16 q (exact) and otherwise read q as pre-scaled floats.
  const bool qs = p.q_dtype != kFBf16;
  if (page_uniform && !qs)
    launch_kernel(decode_kernel<KV, SK, RG, true, false>, grid, block, lds, stream, ev, p);
  else if (page_uniform)
    launch_kernel(decode_kernel<KV, SK, RG, true, true>, grid, block, lds, stream, ev, p);
  else if (!qs)
    launch_kernel(decode_kernel<KV, SK, RG, false, false>, grid, block, lds, stream, ev, p);
  else
    launch_kernel(decode_kernel<KV, SK, RG, false, true>, grid, block, lds, stream, ev, p);
  return hipGetLastError();
}

template <int KV, int SK>
static hipError_t launch_rg(const DecodeParams& p, int rg, bool pu, hipStream_t stream, const LaunchEvents& ev) {
  switch (rg) {
    case 1: return launch_t<KV, SK, 1>(p, pu, stream, ev);
    case 2: return launch_t<KV, SK, 2>(p, pu, stream, ev);
    case 4: return launch_t<KV, SK, 4>(p, pu, stream, ev);
    default: return hipErrorInvalidValue;
  }
}

int decode_chunk_tokens(int kv_dtype, int rows_per_group) {
  return decode_loads(rows_per_group) * decode_rows_per_load(kv_dtype);
}

int decode_rows_per_load(int kv_dtype) {
  return kv_dtype == kKvBf16 ? KvTraits<kKvBf16>::kRowsPerLoad : KvTraits<kKvFp8>::kRowsPerLoad;
}

hipError_t launch_decode(const DecodeParams& p, int kv_dtype, int scale_kind, int rows_per_group, hipStream_t stream,
                         const LaunchEvents& ev) {
  const bool pu = p.P >= decode_rows_per_load(kv_dtype);
  if (kv_dtype == kKvBf16) return launch_rg<kKvBf16, kScaleNone>(p, rows_per_group, pu, stream, ev);
  if (kv_dtype == kKvFp8 && scale_kind == kScaleHead) return launch_rg<kKvFp8, kScaleHead>(p, rows_per_group, pu, stream, ev);
  if (kv_dtype == kKvFp8 && scale_kind == kScaleTokenHead)
    return launch_rg<kKvFp8, kScaleTokenHead>(p, rows_per_group, pu, stream, ev);
  if (kv_dtype == kKvInt8 && scale_kind == kScaleHead) return launch_rg<kKvInt8, kScaleHead>(p, rows_per_group, pu, stream, ev);
  if (kv_dtype == kKvInt8 && scale_kind == kScaleTokenHead)
    return launch_rg<kKvInt8, kScaleTokenHead>(p, rows_per_group, pu, stream, ev);
  return hipErrorInvalidValue;
}

}  // namespace bpt
