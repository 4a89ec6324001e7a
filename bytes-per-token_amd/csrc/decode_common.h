// Device helpers shared by the paged decode kernels (vector and matrix-core paths).
#pragma once

#include "bpt_device.h"
#include "bpt_internal.h"

namespace bpt {

__device__ __forceinline__ int sread(int x) { return __builtin_amdgcn_readfirstlane(x); }

// Cross-workgroup exchange of split-K partials. Workgroups run on different XCDs, whose L2 caches are not
// coherent with each other. Every access to a partial is an agent-scope relaxed (monotonic) atomic, which
// gfx950 performs coherently at the memory side (the sc1 bit: stores write through the L2, loads miss it), so
// no access races. The order between a partial's stores and the arrival that announces it is kept at the
// instruction level, by what LLVM's release / acquire lowering for this target does minus its whole-L2
// writeback and invalidate (which only non-atomic accesses need):
//  * ws_publish: every thread waits until its partial stores have completed at the memory side
//    (s_waitcnt vmcnt(0)) before the workgroup barrier that precedes the counter's fetch-add;
//  * ws_acquire: the last arriver issues its partial loads only after the fetch-add has returned (and the
//    barrier that broadcasts it); the statement keeps the compiler from hoisting them.
// Both are compiler barriers ("memory" clobbers). The memory model's own fences (release: buffer_wbl2 sc1 +
// s_waitcnt vmcnt(0), acquire: buffer_inv sc1, per arrival) were measured at 4.3x the headline call's time
// (37.9 -> 164 us). tests/test_exchange_isa.py checks the emitted sequence on every build.

__device__ __forceinline__ void ws_store(float* ptr, float v) {
  __hip_atomic_store(ptr, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Two adjacent floats (8-byte aligned) in one coherent 8-byte load.
__device__ __forceinline__ void ws_load2(const float* ptr, float& a, float& b) {
  const uint64_t bits = __hip_atomic_load((const uint64_t*)ptr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  a = __uint_as_float((uint32_t)bits);
  b = __uint_as_float((uint32_t)(bits >> 32));
}

// Two adjacent floats (8-byte aligned) in one coherent 8-byte store.
__device__ __forceinline__ void ws_store2(float* ptr, float a, float b) {
  const uint64_t bits = (uint64_t)__float_as_uint(a) | ((uint64_t)__float_as_uint(b) << 32);
  __hip_atomic_store((uint64_t*)ptr, bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ float ws_load(const float* ptr) {
  return __hip_atomic_load(ptr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Every partial store of this wave has completed (and is visible at the memory side).
__device__ __forceinline__ void ws_publish() { __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Keeps the compiler from hoisting the partial loads above the arrival that licenses them.
__device__ __forceinline__ void ws_acquire() { __asm__ volatile("" ::: "memory"); }

// Counts one arrival at a segment's counter (coherently, at the memory side); returns the count before it.
__device__ __forceinline__ unsigned ws_arrive(unsigned* counter) {
  return __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// A load the whole wave makes from one address, through the scalar cache (the data is read-only here).
template <typename T>
__device__ __forceinline__ T load_uniform(const T* ptr) {
  return *(const __attribute__((address_space(4))) T*)ptr;
}

// Block-table entry `idx` of row `row`: int32 tables directly, int64 tables by their low word (page ids
// are below 2^31; anything else is clamped into the pool by the caller).
__device__ __forceinline__ int64_t table_word(const DecodeParams& p, int b, int idx) {
  return ((int64_t)b * p.table_sb + idx) << p.table_i64;
}

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// Softmax weights are 2^(score - m + kBias) with the reference point m kept within kSlack of the largest
// score seen (log2 units): weights stay below 2^12, well inside f16, and small ones keep f16 precision.
constexpr float kBias = 4.0f;
constexpr float kSlack = 8.0f;

// Per-token value scales ride in the f16 weights (w = 2^(score - base) * vscale). The reference point then
// tracks score + vscale_bound(vscale) instead of the score, where vscale < 2^vscale_bound: the f16 weights
// stay below 2^(kSlack + kBias) whatever the scale, and scales far below one keep the weights' precision.
// The weight sums (f32) keep the bare 2^(score - base), so the log-sum-exp is unchanged. The bound is
// clamped to [-kVscaleExpMax, kVscaleExpMax] so those sums stay finite: scales up to 2^64 are exact.
constexpr int kVscaleExpMax = 64;
__device__ __forceinline__ float vscale_bound(float vscale) {
  const int e = __builtin_amdgcn_frexp_expf(vscale);  // vscale = m * 2^e with m in [0.5, 1); 0 for 0
  return (float)(e < -kVscaleExpMax ? -kVscaleExpMax : (e > kVscaleExpMax ? kVscaleExpMax : e));
}

// Round-to-nearest-even float -> bf16 pair.
__device__ __forceinline__ bf16x2 pack_bf16(float a, float b) {
  return bf16x2{(__bf16)a, (__bf16)b};
}

// This lane's VEC query channels of row (b, qi, hq), loaded as 16-byte vectors (unscaled floats).
template <int VEC>
__device__ __forceinline__ void load_q(const DecodeParams& p, int64_t base, float cs, float* q) {
  const uint8_t* src = (const uint8_t*)p.q;
  if (p.q_dtype == kFF32) {
    const U4* v = (const U4*)(src + base * 4);
    U4 raw[VEC / 4];
#pragma unroll
    for (int j = 0; j < VEC / 4; ++j) raw[j] = v[j];
#pragma unroll
    for (int j = 0; j < VEC / 4; ++j) {
      q[4 * j] = __uint_as_float(raw[j].x) * cs;
      q[4 * j + 1] = __uint_as_float(raw[j].y) * cs;
      q[4 * j + 2] = __uint_as_float(raw[j].z) * cs;
      q[4 * j + 3] = __uint_as_float(raw[j].w) * cs;
    }
  } else {
    const U4* v = (const U4*)(src + base * 2);
    U4 raw[VEC / 8];
#pragma unroll
    for (int j = 0; j < VEC / 8; ++j) raw[j] = v[j];
#pragma unroll
    for (int j = 0; j < VEC / 8; ++j) {
      const uint32_t w[4] = {raw[j].x, raw[j].y, raw[j].z, raw[j].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float lo, hi;
        if (p.q_dtype == kFBf16) {
          lo = __uint_as_float(w[e] << 16);
          hi = __uint_as_float(w[e] & 0xffff0000u);
        } else {
          lo = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[e] & 0xffffu));
          hi = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[e] >> 16));
        }
        q[8 * j + 2 * e] = lo * cs;
        q[8 * j + 2 * e + 1] = hi * cs;
      }
    }
  }
}

// Lengths (clamped to the launch's cap), the cost of each sequence's segments and its exclusive prefix sum
// over the batch (the segment line: sequence b's segments start at HR * prefix[b]), computed by the whole
// workgroup into LDS: s_prefix[B + 1], s_len[B]; s_wsum holds one int per wave. A segment of a non-empty
// sequence costs its chunks plus piece_cost units, which stand for the merge of one more piece and sit
// at the segment's start, ahead of its chunks. With check_uniform set, a batch whose sequences all have
// the same length gets no piece cost. Returns the piece cost the line was built with and whether the
// lengths were found equal (the same in every thread). Params: any parameter block with B, lens (NULL:
// every sequence is len_cap long), len_offset and len_cap.
struct SegmentLine {
  int piece_cost;
  bool uniform;
};
template <int NW, int CH, typename Params>
__device__ __forceinline__ SegmentLine build_segment_line(const Params& p, int* s_prefix, int* s_len, int* s_wsum,
                                                          int piece_cost = 0, bool check_uniform = false) {
  constexpr int NT = NW * 64;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int B = p.B;
  const int per_thread = (B + NT - 1) / NT;
  const int lo = min(tid * per_thread, B);
  const int hi = min(lo + per_thread, B);
  int sum = 0;
  for (int b = lo; b < hi; ++b) {
    int len = (p.lens ? p.lens[b] : p.len_cap + p.len_offset) - p.len_offset;  // no lengths: all full
    len = len < 0 ? 0 : (len > p.len_cap ? p.len_cap : len);
    s_len[b] = len;
    sum += len > 0 ? (len + CH - 1) / CH + piece_cost : 0;
  }
  int x = sum;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(x, off, 64);
    if (lane >= off) x += y;
  }
  __shared__ int s_uniform;  // cleared by any thread that sees a length other than the first
  if (lane == 63) s_wsum[tid >> 6] = x;
  if (check_uniform && tid == 0) s_uniform = 1;
  __syncthreads();
  int run = 0;
  for (int w = 0; w < (tid >> 6); ++w) run += s_wsum[w];
  run += x - sum;
  int same = 1;
  if (check_uniform) {
    const int len0 = s_len[0];
    for (int b = lo; b < hi; ++b) same &= s_len[b] == len0;
  }
  for (int b = lo; b < hi; ++b) {
    s_prefix[b] = run;
    run += s_len[b] > 0 ? (s_len[b] + CH - 1) / CH + piece_cost : 0;
  }
  if (tid == 0) {
    int total = 0;
    for (int w = 0; w < NW; ++w) total += s_wsum[w];
    s_prefix[B] = total;
  }
  if (check_uniform && !same) s_uniform = 0;
  __syncthreads();
  if (!check_uniform || !s_uniform) return {piece_cost, false};
  if (piece_cost == 0) return {0, true};
  // Equal lengths: every segment is the same number of chunks, with no piece cost.
  const int len0 = s_len[0];
  const int nb = len0 > 0 ? (len0 + CH - 1) / CH : 0;
  for (int b = lo; b < hi; ++b) s_prefix[b] = b * nb;
  if (tid == 0) s_prefix[B] = B * nb;
  __syncthreads();
  return {0, true};
}

constexpr float kLn2 = 0.69314718055994531f;

// Final value of output element (b, qi, hq, ch) from this launch's normalized result o, whose base-2
// log-sum-exp is lse2 (-inf: the row saw no token): merged with the caller's partial of another token
// range when one is given (kernels/reference.py:205-211 for two parts), then stored; the row's natural-log
// log-sum-exp goes to lse_out (once per row) when asked for.
__device__ __forceinline__ void write_out(const DecodeParams& p, int b, int qi, int hq, int ch, float o, float lse2) {
  const int64_t row = ((int64_t)b * p.Q + qi) * p.Hq + hq;
  if (p.merge_out) {
    const float other = p.merge_lse[row] * kLog2e;
    const float m = fmaxf(lse2, other);
    if (m != kNegInf) {
      const float a = fast_exp2(lse2 - m), c = fast_exp2(other - m);
      o = (a * o + c * p.merge_out[row * kHeadDim + ch]) / (a + c);
      lse2 = m + __log2f(a + c);
    }
  }
  store_float(p.out, (int64_t)b * p.o_sb + (int64_t)qi * p.o_sq + (int64_t)hq * p.o_sh + ch, p.out_dtype, o);
  if (p.lse_out && ch == 0) p.lse_out[row] = lse2 == kNegInf ? kNegInf : lse2 * kLn2;
}

// This workgroup's place on the stream-K line. Workgroups are dispatched to the 8 XCDs round-robin (block x
// runs on XCD x % 8, each XCD with its own L2), and the line is numbered XCD-major: XCD k takes one
// contiguous stretch of it. Neighbouring ranges then meet in one L2: the KV heads of a sequence (one page
// holds all of them, and per-token scales share cache lines across them) and the ranges of one segment.
// n: the workgroups that share the line (the first n of the launch).
__device__ __forceinline__ int64_t line_index(int n) {
  const int x = blockIdx.x;
  const int q = n >> 3, r = n & 7, k = x & 7;
  return (int64_t)k * q + min(k, r) + (x >> 3);
}

// Sequences with no tokens get zero output, or the caller's partial (workgroups take them round-robin).
template <int NT>
__device__ __forceinline__ void zero_empty_sequences(const DecodeParams& p, const int* s_prefix) {
  constexpr int D = kHeadDim;
  const int row_elems = p.Q * p.Hq * D;
  for (int b = blockIdx.x; b < p.B; b += gridDim.x) {
    if (s_prefix[b + 1] != s_prefix[b]) continue;
    for (int i = threadIdx.x; i < row_elems; i += NT) {
      const int ch = i % D;
      const int hq = (i / D) % p.Hq;
      const int qi = i / (D * p.Hq);
      write_out(p, b, qi, hq, ch, 0.0f, kNegInf);
    }
  }
}

// The combine of one segment's n pieces (workspace slots seg + first ..), CPC channels per thread.
template <int RG, int NT, int CPC>
__device__ __forceinline__ void combine_rows(const DecodeParams& p, int seg, int b, int hh, int rg, int64_t first,
                                             int n, int live, int tid) {
  constexpr int D = kHeadDim;
  for (int idx = tid; idx < live * (D / CPC); idx += NT) {
    const int r = idx / (D / CPC);
    const int ch = CPC * (idx - r * (D / CPC));
    const int gr = rg * RG + r;
    const float* lse = p.ws_lse + ((int64_t)seg + first) * RG + r;
    const float* prt = p.ws_out + (((int64_t)seg + first) * RG + r) * D + ch;
    float M = kNegInf, W = 0.0f;  // running maximum and weight
    float O[CPC];                 // weighted outputs
#pragma unroll
    for (int c = 0; c < CPC; ++c) O[c] = 0.0f;
    for (int j0 = 0; j0 < n; j0 += 8) {
      float lv[8], ov[8][CPC];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const bool in = j0 + j < n;
        lv[j] = in ? ws_load(lse + (int64_t)(j0 + j) * RG) : kNegInf;
        if constexpr (CPC % 2 == 0) {
#pragma unroll
          for (int c = 0; c < CPC; c += 2) {
            ov[j][c] = ov[j][c + 1] = 0.0f;
            if (in) ws_load2(prt + (int64_t)(j0 + j) * RG * D + c, ov[j][c], ov[j][c + 1]);
          }
        } else {
#pragma unroll
          for (int c = 0; c < CPC; ++c) ov[j][c] = in ? ws_load(prt + (int64_t)(j0 + j) * RG * D + c) : 0.0f;
        }
      }
      float bm = lv[0];
#pragma unroll
      for (int j = 1; j < 8; ++j) bm = fmaxf(bm, lv[j]);
      const float nm = fmaxf(M, bm);
      const float mu = nm == kNegInf ? 0.0f : nm;
      const float alpha = W > 0.0f ? fast_exp2(M - mu) : 0.0f;
      W *= alpha;
#pragma unroll
      for (int c = 0; c < CPC; ++c) O[c] *= alpha;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float e = fast_exp2(lv[j] - mu);  // 0 for empty pieces (lse -inf)
        W += e;
#pragma unroll
        for (int c = 0; c < CPC; ++c) O[c] = fmaf(e, ov[j][c], O[c]);
      }
      M = nm;
    }
    const int qi = gr / p.G;
    const int hq = hh * p.G + (gr - qi * p.G);
    const float inv = W > 0.0f ? 1.0f / W : 0.0f;
    const float lse2 = W > 0.0f ? M + __log2f(W) : kNegInf;
#pragma unroll
    for (int c = 0; c < CPC; ++c) write_out(p, b, qi, hq, ch + c, O[c] * inv, lse2);
  }
}

// The combine of segment `seg` by the last of its n pieces to arrive (the whole workgroup), which then
// resets the segment's counter.
template <int RG, int NT>
__device__ __forceinline__ void combine_segment(const DecodeParams& p, int seg, int b, int hr, int64_t first, int n,
                                                int rows, int tid) {
  constexpr int D = kHeadDim;
  ws_acquire();
  const int hh = hr / p.n_rg;
  const int rg = hr - hh * p.n_rg;
  const int live = min(RG, rows - rg * RG);  // this row group's real rows
  // CPC channels of one row per thread, every piece's loads issued before they are combined: the fewest that
  // still cover the rows in one pass of the workgroup (four at most). A second pass would issue its loads
  // only after the first pass's have returned: one more memory round trip at the end of the segment (3 rows
  // over 128 threads with two channels each took 1 us longer than with four).
  if (live * D > 2 * NT) combine_rows<RG, NT, 4>(p, seg, b, hh, rg, first, n, live, tid);
  else if (live * D > NT) combine_rows<RG, NT, 2>(p, seg, b, hh, rg, first, n, live, tid);
  else combine_rows<RG, NT, 1>(p, seg, b, hh, rg, first, n, live, tid);
  if (tid == 0) __hip_atomic_store(p.counters + seg, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Count this workgroup's arrival at segment `seg` (its partial is stored and complete); the last of its n
// pieces (workspace slots seg + first ...) to arrive combines them, as reference.merge_partials does (base
// 2), writes the rows and resets the counter. Called by the whole workgroup; s_flag is one LDS int.
template <int RG, int NT>
__device__ __forceinline__ void arrive_and_combine(const DecodeParams& p, int seg, int b, int hr, int64_t first, int n,
                                                   int rows, int tid, int* s_flag) {
  if (tid == 0) {
    *s_flag = ws_arrive(p.counters + seg) == (unsigned)n - 1u;
  }
  __syncthreads();
  if (*s_flag) combine_segment<RG, NT>(p, seg, b, hr, first, n, rows, tid);
}

}  // namespace bpt
