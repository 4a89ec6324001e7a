// Paged decode attention over a BF16, FP8 (e4m3fn) or INT8 KV cache, dequantized in registers.
//
// Algorithm (follows fastserve kernels/kv_attention.py:56-175 and kernels/reference.py:186-211): one
// workgroup per (sequence, KV head, row group, split). Its rows are the G query heads of the KV head times
// the Q queries of the sequence, so each cached page is read from HBM once for all of them. Each split
// writes its own normalized output and log-sum-exp; a second kernel combines the splits exactly.
//
// Layout inside a wave (D = 128, one-byte codes): lane = slot * 8 + part. `part` owns channels
// [16*part, 16*part + 16) and loads them with one 16-byte load per token; the 8 lanes of a slot cover one
// token row (128 contiguous bytes), so one load instruction moves 8 whole token rows. Scores are summed
// over the 8 lanes of a slot with DPP (quad_perm, row_half_mirror). Every slot keeps its own online-softmax
// state (running max m, weight sum l, weighted value sum acc) over the tokens it saw; slots, then waves
// (through LDS), are merged at the end with the same log-sum-exp algebra as the split combine.
//
// Scales fold out of the inner loop: a per-head K scale and sm_scale * log2(e) go into q once, a per-head V
// scale multiplies the final output, and per-token scales multiply the reduced score (K) and the softmax
// weight (V). Softmax runs in base 2 (exp2 of log2-scaled scores); lse is stored in log2 units.
#include "bpt_device.h"
#include "bpt_internal.h"

namespace bpt {

template <int KV>
struct KvTraits {
  static constexpr int kBytes = KV == kKvBf16 ? 2 : 1;
  static constexpr int kVec = 16 / kBytes;  // elements in one 16-byte load
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

template <int KV, int SK, int D, int RG, int NW, int CL>
__global__ __launch_bounds__(NW * 64) void decode_split_kernel(const DecodeParams p) {
  constexpr int VEC = KvTraits<KV>::kVec;
  constexpr int EB = KvTraits<KV>::kBytes;
  constexpr int LPT = D / VEC;  // lanes per token row
  constexpr int TPL = 64 / LPT; // token rows per load instruction
  constexpr int CHUNK = CL * TPL;
  static_assert(D % VEC == 0 && 64 % LPT == 0, "head_dim must split into 16-byte lanes");

  __shared__ int s_pages[kMaxSplitPages];
  __shared__ float s_m[NW][RG];
  __shared__ float s_l[NW][RG];
  __shared__ float s_acc[NW][RG][D];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int split = blockIdx.x;
  const int h = blockIdx.y / p.n_rg;
  const int rg = blockIdx.y - h * p.n_rg;
  const int b = blockIdx.z;

  int len = p.lens[b];
  len = len < 0 ? 0 : (len > p.len_cap ? p.len_cap : len);
  const int t0 = split * p.split_tokens;
  if (p.S > 1 && t0 >= len) return;  // nothing to write: the combine reads splits below len only
  const int t_end = min(t0 + p.split_tokens, len);

  // Stage the split's page ids in LDS, clamped into the pool.
  const int p0 = t0 >> p.logP;
  const int np = t_end > t0 ? ((t_end - 1) >> p.logP) - p0 + 1 : 0;
  for (int i = threadIdx.x; i < np; i += NW * 64) {
    int64_t e = load_index(p.table, (int64_t)b * p.table_sb + p0 + i, p.table_i64 != 0);
    e = e < 0 ? 0 : (e >= p.num_blocks ? p.num_blocks - 1 : e);
    s_pages[i] = (int)e;
  }

  const int slot = lane / LPT;
  const int part = lane - slot * LPT;
  const int rows = p.Q * p.G;

  // This lane's slice of each row's query, pre-scaled.
  float q[RG][VEC];
  int rlen[RG];
  float kscale_head = 1.0f;
  if constexpr (SK == kScaleHead) kscale_head = p.ks[h];
#pragma unroll
  for (int r = 0; r < RG; ++r) {
    const int gr = rg * RG + r;
    if (gr < rows) {
      const int qi = gr / p.G;
      const int hq = h * p.G + (gr - qi * p.G);
      const int64_t base = (int64_t)b * p.q_sb + (int64_t)qi * p.q_sq + (int64_t)hq * p.q_sh + part * VEC;
      const float c = p.qscale * kscale_head;
#pragma unroll
      for (int v = 0; v < VEC; ++v) q[r][v] = load_float(p.q, base + v, p.q_dtype) * c;
      rlen[r] = len - (p.Q - 1 - qi);
    } else {
#pragma unroll
      for (int v = 0; v < VEC; ++v) q[r][v] = 0.0f;
      rlen[r] = 0;
    }
  }

  float m[RG], l[RG], acc[RG][VEC];
#pragma unroll
  for (int r = 0; r < RG; ++r) {
    m[r] = kNegInf;
    l[r] = 0.0f;
#pragma unroll
    for (int v = 0; v < VEC; ++v) acc[r][v] = 0.0f;
  }

  __syncthreads();

  const int64_t lane_off = (int64_t)h * p.kv_shead + part * 16;
  const int pmask = p.P - 1;

  for (int c0 = t0 + wave * CHUNK; c0 < t_end; c0 += NW * CHUNK) {
    U4 kr[CL], vr[CL];
    float ksc[CL], vsc[CL];
    int tok[CL];
#pragma unroll
    for (int i = 0; i < CL; ++i) {
      const int t = c0 + i * TPL + slot;
      tok[i] = t;
      ksc[i] = 1.0f;
      vsc[i] = 1.0f;
      if (t < t_end) {
        const int page = s_pages[(t >> p.logP) - p0];
        const int within = t & pmask;
        const int64_t off = (int64_t)page * p.kv_sblk + (int64_t)within * p.kv_stok + lane_off;
        kr[i] = load16(p.k + off);
        vr[i] = load16(p.v + off);
        if constexpr (SK == kScaleTokenHead) {
          const int64_t so = (int64_t)page * p.sc_sblk + (int64_t)within * p.sc_stok + (int64_t)h * p.sc_shead;
          ksc[i] = p.ks[so];
          vsc[i] = p.vs[so];
        }
      } else {
        kr[i] = U4{0, 0, 0, 0};
        vr[i] = U4{0, 0, 0, 0};
      }
    }

    // Scores of every row against the chunk's tokens.
    float s[CL][RG];
#pragma unroll
    for (int i = 0; i < CL; ++i) {
      float kf[VEC];
      unpack16<KV>(kr[i], kf);
#pragma unroll
      for (int r = 0; r < RG; ++r) {
        float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
        for (int v = 0; v < VEC; v += 2) {
          a0 = fmaf(q[r][v], kf[v], a0);
          a1 = fmaf(q[r][v + 1], kf[v + 1], a1);
        }
        s[i][r] = a0 + a1;
      }
    }
#pragma unroll
    for (int i = 0; i < CL; ++i) {
#pragma unroll
      for (int r = 0; r < RG; ++r) {
        float x = group_sum<LPT>(s[i][r]);
        if constexpr (SK == kScaleTokenHead) x *= ksc[i];
        s[i][r] = tok[i] < rlen[r] ? x : kNegInf;
      }
    }

    // Online softmax over the chunk, per slot.
    float pw[CL][RG];
#pragma unroll
    for (int r = 0; r < RG; ++r) {
      float mc = s[0][r];
#pragma unroll
      for (int i = 1; i < CL; ++i) mc = fmaxf(mc, s[i][r]);
      const float mn = fmaxf(m[r], mc);
      const float mu = mn == kNegInf ? 0.0f : mn;
      const float alpha = fast_exp2(m[r] - mu);
      m[r] = mn;
      float lsum = l[r] * alpha;
#pragma unroll
      for (int i = 0; i < CL; ++i) {
        const float e = fast_exp2(s[i][r] - mu);
        lsum += e;
        pw[i][r] = e * vsc[i];
      }
      l[r] = lsum;
#pragma unroll
      for (int v = 0; v < VEC; ++v) acc[r][v] *= alpha;
    }
#pragma unroll
    for (int i = 0; i < CL; ++i) {
      float vf[VEC];
      unpack16<KV>(vr[i], vf);
#pragma unroll
      for (int r = 0; r < RG; ++r) {
#pragma unroll
        for (int v = 0; v < VEC; ++v) acc[r][v] = fmaf(pw[i][r], vf[v], acc[r][v]);
      }
    }
  }

  // Merge the slots of the wave: lanes with the same part hold states over disjoint tokens.
#pragma unroll
  for (int off = LPT; off < 64; off <<= 1) {
#pragma unroll
    for (int r = 0; r < RG; ++r) {
      const float mo = shfl_xor_f(m[r], off);
      const float lo = shfl_xor_f(l[r], off);
      const float mn = fmaxf(m[r], mo);
      const float mu = mn == kNegInf ? 0.0f : mn;
      const float a = fast_exp2(m[r] - mu);
      const float c = fast_exp2(mo - mu);
      l[r] = l[r] * a + lo * c;
#pragma unroll
      for (int v = 0; v < VEC; ++v) acc[r][v] = acc[r][v] * a + shfl_xor_f(acc[r][v], off) * c;
      m[r] = mn;
    }
  }
  if (slot == 0) {
#pragma unroll
    for (int r = 0; r < RG; ++r) {
#pragma unroll
      for (int v = 0; v < VEC; ++v) s_acc[wave][r][part * VEC + v] = acc[r][v];
      if (part == 0) {
        s_m[wave][r] = m[r];
        s_l[wave][r] = l[r];
      }
    }
  }
  __syncthreads();

  // Merge the waves and write this split's result.
  const float vscale_head = SK == kScaleHead ? p.vs[h] : 1.0f;
  for (int idx = threadIdx.x; idx < RG * D; idx += NW * 64) {
    const int r = idx / D;
    const int ch = idx - r * D;
    const int gr = rg * RG + r;
    if (gr >= rows) continue;
    float M = s_m[0][r];
#pragma unroll
    for (int w = 1; w < NW; ++w) M = fmaxf(M, s_m[w][r]);
    const float mu = M == kNegInf ? 0.0f : M;
    float L = 0.0f, A = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float e = fast_exp2(s_m[w][r] - mu);
      L += s_l[w][r] * e;
      A += s_acc[w][r][ch] * e;
    }
    const float o = L > 0.0f ? A / L * vscale_head : 0.0f;
    const int qi = gr / p.G;
    const int hq = h * p.G + (gr - qi * p.G);
    if (p.S == 1) {
      const int64_t oi = (int64_t)b * p.o_sb + (int64_t)qi * p.o_sq + (int64_t)hq * p.o_sh + ch;
      store_float(p.out, oi, p.out_dtype, o);
    } else {
      const int64_t row = ((int64_t)b * p.Q + qi) * p.Hq + hq;
      p.part_out[(row * p.S + split) * D + ch] = o;
      if (ch == 0) p.part_lse[row * p.S + split] = L > 0.0f ? M + __log2f(L) : kNegInf;
    }
  }
  (void)EB;
}

// Exact combine of the splits (reference.merge_partials): out = sum_s 2^(lse_s - M) out_s / sum_s 2^(lse_s - M).
// One wave per (sequence, query, head) row; only splits that start below the sequence's length exist.
template <int D>
__global__ __launch_bounds__(256) void decode_combine_kernel(const DecodeParams p) {
  constexpr int PER = D / 64;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t nrows = (int64_t)p.B * p.Q * p.Hq;
  if (row >= nrows) return;
  const int b = (int)(row / ((int64_t)p.Q * p.Hq));
  const int rem = (int)(row - (int64_t)b * p.Q * p.Hq);
  const int qi = rem / p.Hq;
  const int hq = rem - qi * p.Hq;
  int len = p.lens[b];
  len = len < 0 ? 0 : (len > p.len_cap ? p.len_cap : len);
  const int ns = min((len + p.split_tokens - 1) / p.split_tokens, p.S);

  const float* lse = p.part_lse + row * p.S;
  float M = kNegInf;
  for (int s = lane; s < ns; s += 64) M = fmaxf(M, lse[s]);
  M = wave_max(M);
  const float mu = M == kNegInf ? 0.0f : M;

  float o[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) o[j] = 0.0f;
  float W = 0.0f;
  const float* part = p.part_out + row * p.S * D + lane * PER;
  for (int s = 0; s < ns; ++s) {
    const float w = fast_exp2(lse[s] - mu);
    W += w;
#pragma unroll
    for (int j = 0; j < PER; ++j) o[j] = fmaf(w, part[(int64_t)s * D + j], o[j]);
  }
  const float inv = W > 0.0f ? 1.0f / W : 0.0f;
  const int64_t oi = (int64_t)b * p.o_sb + (int64_t)qi * p.o_sq + (int64_t)hq * p.o_sh + lane * PER;
#pragma unroll
  for (int j = 0; j < PER; ++j) store_float(p.out, oi + j, p.out_dtype, o[j] * inv);
}

template <int KV, int SK, int D, int RG>
static hipError_t launch_split_t(const DecodeParams& p, hipStream_t stream) {
  dim3 grid(p.S, p.Hkv * p.n_rg, p.B);
  dim3 block(kDecodeWaves * 64);
  hipLaunchKernelGGL((decode_split_kernel<KV, SK, D, RG, kDecodeWaves, kDecodeLoads>), grid, block, 0, stream, p);
  return hipGetLastError();
}

template <int KV, int SK, int D>
static hipError_t launch_split_rg(const DecodeParams& p, int rg, hipStream_t stream) {
  switch (rg) {
    case 1: return launch_split_t<KV, SK, D, 1>(p, stream);
    case 2: return launch_split_t<KV, SK, D, 2>(p, stream);
    case 4: return launch_split_t<KV, SK, D, 4>(p, stream);
    default: return hipErrorInvalidValue;
  }
}

template <int D>
static hipError_t launch_split_d(const DecodeParams& p, int kv, int sk, int rg, hipStream_t stream) {
  if (kv == kKvBf16) return launch_split_rg<kKvBf16, kScaleNone, D>(p, rg, stream);
  if (kv == kKvFp8 && sk == kScaleHead) return launch_split_rg<kKvFp8, kScaleHead, D>(p, rg, stream);
  if (kv == kKvFp8 && sk == kScaleTokenHead) return launch_split_rg<kKvFp8, kScaleTokenHead, D>(p, rg, stream);
  if (kv == kKvInt8 && sk == kScaleHead) return launch_split_rg<kKvInt8, kScaleHead, D>(p, rg, stream);
  if (kv == kKvInt8 && sk == kScaleTokenHead) return launch_split_rg<kKvInt8, kScaleTokenHead, D>(p, rg, stream);
  return hipErrorInvalidValue;
}

hipError_t launch_decode(const DecodeParams& p, int kv_dtype, int scale_kind, int head_dim, int rows_per_group,
                         hipStream_t stream, hipEvent_t mid_event) {
  hipError_t e;
  switch (head_dim) {
    case 128: e = launch_split_d<128>(p, kv_dtype, scale_kind, rows_per_group, stream); break;
    default: return hipErrorInvalidValue;
  }
  if (e != hipSuccess) return e;
  if (mid_event) {
    e = hipEventRecord(mid_event, stream);
    if (e != hipSuccess) return e;
  }
  if (p.S > 1) {
    const int64_t nrows = (int64_t)p.B * p.Q * p.Hq;
    dim3 grid((unsigned)((nrows + 3) / 4));
    hipLaunchKernelGGL(decode_combine_kernel<128>, grid, dim3(256), 0, stream, p);
    e = hipGetLastError();
  }
  return e;
}

}  // namespace bpt
