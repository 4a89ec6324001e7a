// KIVI decode attention for the head sizes and cache dtypes the matrix-core kernel (kivi_decode.hip) does not
// take: any even head dim up to 256 (fastserve's tiny test model has 16) and float32 bits-16 caches.
//
// Same call surface and results as kivi_decode.hip (fastserve kernels/kv_attention.py:56-175 and :190-245):
// one partial attention per split of `split` tokens, out = softmax-weighted average of the split's values
// (0 for an empty split), lse = natural-log log-sum-exp of its scores (-inf when empty). Keys are
// scale * (code - zero) with one float16 grid per channel per `group` tokens, values with one per token;
// 4-bit codes pair channel d (low nibble) with d + D/2 (high nibble); bits-16 caches hold the values.
//
// One workgroup per (sequence, KV head, split); the split's tokens stream through in blocks of 256, one token
// per thread for the scores of all G query heads of the KV head, then an online softmax per head (base 2)
// and the value sums, each thread owning a few (head, channel) accumulators. Everything is float32: these
// are small shapes (tests and tiny models), where a launch is a few microseconds whatever the layout.
#include "bpt_device.h"
#include "bpt_internal.h"

namespace bpt {

constexpr int kAnyThreads = 256;
constexpr int kAnyMaxD = 256;
constexpr int kAnyMaxG = 16;
constexpr int kAnyAcc = kAnyMaxD * kAnyMaxG / kAnyThreads;  // accumulators per thread

__device__ __forceinline__ float half_at(const uint16_t* p, int64_t i) {
  return (float)__builtin_bit_cast(_Float16, p[i]);
}

// Element (token t, channel c) of one (sequence, KV head)'s keys or values: `codes` points at its first token;
// `scale` / `zero` at the grid that token reads (quantized formats only).
template <int FMT>
__device__ __forceinline__ float kivi_element(const uint8_t* codes, int64_t c_st, int t, int c, int D, float scale,
                                              float zero) {
  if constexpr (FMT == kKivi8) return scale * ((float)codes[t * c_st + c] - zero);
  if constexpr (FMT == kKivi4) {
    const int half = D / 2;
    const uint32_t byte = codes[t * c_st + (c < half ? c : c - half)];
    return scale * ((float)(c < half ? byte & 15u : byte >> 4) - zero);
  }
  if constexpr (FMT == kKiviF16) return (float)((const _Float16*)codes)[t * c_st + c];
  if constexpr (FMT == kKiviBf16) return bf16_bits_to_f32(((const uint16_t*)codes)[t * c_st + c]);
  return ((const float*)codes)[t * c_st + c];
}

template <int FMT>
__global__ __launch_bounds__(kAnyThreads) void kivi_any_kernel(const KiviParams p) {
  constexpr bool kQuant = FMT == kKivi4 || FMT == kKivi8;
  constexpr int NW = kAnyThreads / 64;
  __shared__ float s_q[kAnyMaxG][kAnyMaxD];        // q rows, scaled by sm_scale * log2(e)
  __shared__ float s_p[kAnyMaxG][kAnyThreads];     // a block's scores, then its softmax weights
  __shared__ float s_m[kAnyMaxG], s_l[kAnyMaxG], s_alpha[kAnyMaxG];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int s = blockIdx.x % p.S;
  const int bh = blockIdx.x / p.S;
  const int h = bh % p.Hkv, b = bh / p.Hkv;
  const int D = p.D, G = p.G;
  const int len = max(min(p.lens[b], p.len_cap), 0);
  const int lo = s * p.split, hi = min(lo + p.split, len);

  for (int i = tid; i < G * D; i += kAnyThreads) {
    const int g = i / D, c = i - g * D;
    s_q[g][c] = load_float(p.q, (int64_t)b * p.q_sb + (int64_t)(h * G + g) * p.q_sh + c, p.q_dtype) * p.qscale;
  }
  if (tid < G) {
    s_m[tid] = kNegInf;
    s_l[tid] = 0.0f;
  }
  float acc[kAnyAcc];
#pragma unroll
  for (int k = 0; k < kAnyAcc; ++k) acc[k] = 0.0f;
  __syncthreads();

  const uint8_t* kc = p.kc + (int64_t)b * p.c_sb + (int64_t)h * p.c_sh;
  const uint8_t* vc = p.vc + (int64_t)b * p.c_sb + (int64_t)h * p.c_sh;
  const int64_t c_st = p.c_st / (FMT == kKiviF32 ? 4 : (FMT == kKiviF16 || FMT == kKiviBf16 ? 2 : 1));
  const uint16_t* ks = kQuant ? p.ks + (int64_t)b * p.g_sb + (int64_t)h * p.g_sh : nullptr;
  const uint16_t* kz = kQuant ? p.kz + (int64_t)b * p.g_sb + (int64_t)h * p.g_sh : nullptr;
  const uint16_t* vs = kQuant ? p.vs + (int64_t)b * p.t_sb + (int64_t)h * p.t_sh : nullptr;
  const uint16_t* vz = kQuant ? p.vz + (int64_t)b * p.t_sb + (int64_t)h * p.t_sh : nullptr;

  // One block of n <= 256 tokens: key(i, c) and value(i, c) give channel c of the block's token i.
  auto block = [&](int n, auto key, auto value) {
    // ---- scores of this thread's token for every head ---------------------------------------------------
    {
      float sc[kAnyMaxG];
#pragma unroll
      for (int g = 0; g < kAnyMaxG; ++g) sc[g] = 0.0f;
      if (tid < n) {
        for (int c = 0; c < D; ++c) {
          const float x = key(tid, c);
#pragma unroll
          for (int g = 0; g < kAnyMaxG; ++g) sc[g] = g < G ? fmaf(s_q[g][c], x, sc[g]) : sc[g];
        }
      }
#pragma unroll
      for (int g = 0; g < kAnyMaxG; ++g)
        if (g < G) s_p[g][tid] = tid < n ? sc[g] : kNegInf;
    }
    __syncthreads();
    // ---- online softmax per head: wave w takes heads w, w + NW, ... -------------------------------------
    for (int g = wave; g < G; g += NW) {
      float mx = kNegInf;
      for (int i = lane; i < kAnyThreads; i += 64) mx = fmaxf(mx, s_p[g][i]);
      mx = wave_max(mx);
      const float m_old = s_m[g];
      const float m_new = fmaxf(m_old, mx);
      float sum = 0.0f;
      for (int i = lane; i < kAnyThreads; i += 64) {
        const float e = m_new == kNegInf ? 0.0f : fast_exp2(s_p[g][i] - m_new);  // 0 for masked tokens
        s_p[g][i] = e;
        sum += e;
      }
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) sum += shfl_xor_f(sum, off);
      if (lane == 0) {
        const float alpha = m_old == kNegInf ? 0.0f : fast_exp2(m_old - m_new);
        s_alpha[g] = alpha;
        s_l[g] = s_l[g] * alpha + sum;
        s_m[g] = m_new;
      }
    }
    __syncthreads();
    // ---- value sums: thread tid owns (head, channel) entries tid, tid + 256, ... ------------------------
#pragma unroll
    for (int k = 0; k < kAnyAcc; ++k) {
      const int e = tid + k * kAnyThreads;
      if (e < G * D) {
        const int g = e / D, c = e - g * D;
        float a = acc[k] * s_alpha[g];
        for (int i = 0; i < n; ++i) a = fmaf(s_p[g][i], value(i, c), a);
        acc[k] = a;
      }
    }
    __syncthreads();
  };

  for (int t0 = lo; t0 < hi; t0 += kAnyThreads) {
    block(
        min(kAnyThreads, hi - t0),
        [&](int i, int c) {
          const int t = t0 + i;
          const int64_t go = (int64_t)(t >> p.gshift_tokens) * p.g_sg;
          return kivi_element<FMT>(kc, c_st, t, c, D, kQuant ? half_at(ks, go + c) : 1.0f,
                                   kQuant ? half_at(kz, go + c) : 0.0f);
        },
        [&](int i, int c) {
          const int t = t0 + i;
          return kivi_element<FMT>(vc, c_st, t, c, D, kQuant ? half_at(vs, t) : 1.0f, kQuant ? half_at(vz, t) : 0.0f);
        });
  }
  // The full-precision tail (one split: it goes with the last), one more block (fastserve
  // integration/kv_cache.py:172-185 attends it separately and merges; the online softmax is that merge).
  if (p.tail_len > 0 && s == p.S - 1) {
    const int64_t t0 = (int64_t)b * p.tk_sb + (int64_t)h * p.tk_sh;
    block(
        p.tail_len, [&](int i, int c) { return load_float(p.tk, t0 + (int64_t)i * p.tk_st + c, p.tail_dtype); },
        [&](int i, int c) { return load_float(p.tv, t0 + (int64_t)i * p.tk_st + c, p.tail_dtype); });
  }

  // ---- the split's output and log-sum-exp (natural log) -----------------------------------------------
#pragma unroll
  for (int k = 0; k < kAnyAcc; ++k) {
    const int e = tid + k * kAnyThreads;
    if (e < G * D) {
      const int g = e / D, c = e - g * D;
      const float L = s_l[g];
      const int hq = h * G + g;
      p.out[(int64_t)b * p.o_sb + (int64_t)hq * p.o_sh + (int64_t)s * p.o_ss + c] = L > 0.0f ? acc[k] / L : 0.0f;
      if (c == 0)
        p.lse[(int64_t)b * p.l_sb + (int64_t)hq * p.l_sh + (int64_t)s * p.l_ss] =
            L > 0.0f ? (s_m[g] + __log2f(L)) * 0.69314718055994531f : kNegInf;
    }
  }
}

hipError_t launch_kivi_any(const KiviParams& p, int fmt, hipStream_t stream) {
  const int64_t groups = (int64_t)p.B * p.Hkv * p.S;
  if (groups == 0) return hipSuccess;
  dim3 grid((unsigned)groups), block(kAnyThreads);
  switch (fmt) {
    case kKivi4: hipLaunchKernelGGL(kivi_any_kernel<kKivi4>, grid, block, 0, stream, p); break;
    case kKivi8: hipLaunchKernelGGL(kivi_any_kernel<kKivi8>, grid, block, 0, stream, p); break;
    case kKiviF16: hipLaunchKernelGGL(kivi_any_kernel<kKiviF16>, grid, block, 0, stream, p); break;
    case kKiviBf16: hipLaunchKernelGGL(kivi_any_kernel<kKiviBf16>, grid, block, 0, stream, p); break;
    case kKiviF32: hipLaunchKernelGGL(kivi_any_kernel<kKiviF32>, grid, block, 0, stream, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace bpt
