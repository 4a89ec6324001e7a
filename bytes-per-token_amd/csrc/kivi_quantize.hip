// KIVI quantize-on-write: keys and values [B, Hkv, T, D] -> asymmetric 4 / 8-bit codes with float16 grids, the
// write half of fastserve's kernel-2 cache (kernels/reference.py:103-160 quantize_kv, called for every completed
// key group by integration/kv_cache.py:139-158 QuantizedKVCache._append).
//
// Per grid (keys: one channel over `group` tokens; values: one token over its D channels):
//   lo = min(min x, 0), hi = max(max x, 0), scale = f16((hi - lo) / (2^bits - 1)) (1 where that is not > 0),
//   zero = clamp(round(-lo / scale), 0, 2^bits - 1), code = clamp(round(x / scale) + zero, 0, 2^bits - 1),
// the scale rounded to float16 before the zero point and codes are computed from it; divisions are IEEE
// float32 and rounding is half to even, so codes and grids are bit-exact with the reference formulas. 4-bit
// codes pair channel d (low nibble) with d + D/2 (high nibble).
//
// One wave per (sequence, KV head, key group): lane l owns channels l, l + 64, ... (D a power of two up to 256);
// the key grids are column reductions over the group's tokens within each lane, the value grids wave
// reductions over each token's channels. Roofline: HBM, 2 * D * esize bytes read and 2 * D * bits / 8 + 4 *
// (D / group + 1) written per token, a launch-bound kernel at decode sizes.
#include "bpt_device.h"
#include "bpt_internal.h"

namespace bpt {

constexpr int kQuantWaves = 4;
constexpr int kQuantMaxChannels = 4;  // per lane: D <= 256

// torch.clamp / numpy.clip semantics: a value equal to a bound (including -0.0 against 0) is kept as is.
__device__ __forceinline__ float clamp_keep(float x, float lo, float hi) { return x < lo ? lo : (x > hi ? hi : x); }

struct Grid {
  float scale, zero;  // as stored (float16 values)
};

__device__ __forceinline__ Grid make_grid(float mn, float mx, float qmax) {
  const float lo = mn < 0.0f ? mn : 0.0f;  // the range always holds 0, so a real 0 stays 0
  const float hi = mx > 0.0f ? mx : 0.0f;
  float s = (float)(_Float16)__fdiv_rn(hi - lo, qmax);
  if (!(s > 0.0f)) s = 1.0f;
  const float z = clamp_keep(rintf(__fdiv_rn(-lo, s)), 0.0f, qmax);
  return Grid{s, z};
}

__device__ __forceinline__ uint32_t kivi_code(float x, const Grid& g, float qmax) {
  return (uint32_t)clamp_keep(rintf(__fdiv_rn(x, g.scale)) + g.zero, 0.0f, qmax);
}

__device__ __forceinline__ uint16_t f16_bits(float x) { return __builtin_bit_cast(uint16_t, (_Float16)x); }

// Store this lane's codes of one token row: code[j] is channel lane + 64 j. 8 bits: one byte per channel.
// 4 bits: byte c (< D / 2) = channel c | channel c + D / 2 << 4; the partner sits in this lane (D >= 128) or
// in lane + D / 2 (D <= 64).
template <int BITS>
__device__ __forceinline__ void store_codes(uint8_t* row, const uint32_t (&code)[kQuantMaxChannels], int D, int lane) {
  const int nc = D >= 64 ? D / 64 : 1;
  if constexpr (BITS == 8) {
#pragma unroll
    for (int j = 0; j < kQuantMaxChannels; ++j)
      if (j < nc && lane + 64 * j < D) row[lane + 64 * j] = (uint8_t)code[j];
  } else if (D >= 128) {
#pragma unroll
    for (int j = 0; j < kQuantMaxChannels / 2; ++j)
      if (j < nc / 2) row[lane + 64 * j] = (uint8_t)(code[j] | (code[j + nc / 2] << 4));
  } else {
    const uint32_t hi = (uint32_t)__shfl((int)code[0], (lane + D / 2) & 63, 64);
    if (lane < D / 2) row[lane] = (uint8_t)(code[0] | (hi << 4));
  }
}

template <int BITS>
__global__ __launch_bounds__(kQuantWaves * 64) void kivi_quantize_kernel(const KiviQuantParams p) {
  constexpr float kQmax = BITS == 4 ? 15.0f : 255.0f;
  const int lane = threadIdx.x & 63;
  const int64_t item = (int64_t)blockIdx.x * kQuantWaves + (threadIdx.x >> 6);  // (b, h, key group)
  const int groups = p.T / p.group;
  if (item >= (int64_t)p.B * p.Hkv * groups) return;
  const int g = (int)(item % groups);
  const int bh = (int)(item / groups);
  const int h = bh % p.Hkv, b = bh / p.Hkv;
  const int D = p.D;
  const int nc = D >= 64 ? D / 64 : 1;
  const int64_t src = (int64_t)b * p.x_sb + (int64_t)h * p.x_sh;
  const int t0 = g * p.group;

  // ---- keys: one grid per channel over the group's tokens ---------------------------------------------
  {
    float mn[kQuantMaxChannels], mx[kQuantMaxChannels];
#pragma unroll
    for (int j = 0; j < kQuantMaxChannels; ++j) {
      mn[j] = __builtin_huge_valf();
      mx[j] = -__builtin_huge_valf();
    }
    for (int t = 0; t < p.group; ++t) {
      const int64_t row = src + (int64_t)(t0 + t) * p.x_st;
#pragma unroll
      for (int j = 0; j < kQuantMaxChannels; ++j) {
        const int c = lane + 64 * j;
        if (j < nc && c < D) {
          const float x = load_float(p.k, row + c, p.src_dtype);
          mn[j] = fminf(mn[j], x);
          mx[j] = fmaxf(mx[j], x);
        }
      }
    }
    Grid gr[kQuantMaxChannels];
    const int64_t go = (int64_t)b * p.g_sb + (int64_t)h * p.g_sh + (int64_t)g * p.g_sg;
#pragma unroll
    for (int j = 0; j < kQuantMaxChannels; ++j) {
      const int c = lane + 64 * j;
      gr[j] = make_grid(mn[j], mx[j], kQmax);
      if (j < nc && c < D) {
        p.ks[go + c] = f16_bits(gr[j].scale);
        p.kz[go + c] = f16_bits(gr[j].zero);
      }
    }
    for (int t = 0; t < p.group; ++t) {
      const int64_t row = src + (int64_t)(t0 + t) * p.x_st;
      uint32_t code[kQuantMaxChannels];
#pragma unroll
      for (int j = 0; j < kQuantMaxChannels; ++j) {
        const int c = lane + 64 * j;
        code[j] = (j < nc && c < D) ? kivi_code(load_float(p.k, row + c, p.src_dtype), gr[j], kQmax) : 0u;
      }
      store_codes<BITS>(p.kc + (int64_t)b * p.c_sb + (int64_t)h * p.c_sh + (int64_t)(t0 + t) * p.c_st, code, D, lane);
    }
  }

  // ---- values: one grid per token over its channels -----------------------------------------------------
  for (int t = 0; t < p.group; ++t) {
    const int64_t row = src + (int64_t)(t0 + t) * p.x_st;
    float x[kQuantMaxChannels];
    float mn = __builtin_huge_valf(), mx = -__builtin_huge_valf();
#pragma unroll
    for (int j = 0; j < kQuantMaxChannels; ++j) {
      const int c = lane + 64 * j;
      x[j] = (j < nc && c < D) ? load_float(p.v, row + c, p.src_dtype) : 0.0f;
      if (j < nc && c < D) {
        mn = fminf(mn, x[j]);
        mx = fmaxf(mx, x[j]);
      }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      mn = fminf(mn, shfl_xor_f(mn, off));
      mx = fmaxf(mx, shfl_xor_f(mx, off));
    }
    const Grid gr = make_grid(mn, mx, kQmax);
    const int64_t vo = (int64_t)b * p.t_sb + (int64_t)h * p.t_sh + t0 + t;
    if (lane == 0) {
      p.vs[vo] = f16_bits(gr.scale);
      p.vz[vo] = f16_bits(gr.zero);
    }
    uint32_t code[kQuantMaxChannels];
#pragma unroll
    for (int j = 0; j < kQuantMaxChannels; ++j) code[j] = kivi_code(x[j], gr, kQmax);
    store_codes<BITS>(p.vc + (int64_t)b * p.c_sb + (int64_t)h * p.c_sh + (int64_t)(t0 + t) * p.c_st, code, D, lane);
  }
}

hipError_t launch_kivi_quantize(const KiviQuantParams& p, hipStream_t stream) {
  const int64_t items = (int64_t)p.B * p.Hkv * (p.T / p.group);
  if (items == 0) return hipSuccess;
  dim3 grid((unsigned)((items + kQuantWaves - 1) / kQuantWaves)), block(kQuantWaves * 64);
  if (p.bits == 4) hipLaunchKernelGGL(kivi_quantize_kernel<4>, grid, block, 0, stream, p);
  else hipLaunchKernelGGL(kivi_quantize_kernel<8>, grid, block, 0, stream, p);
  return hipGetLastError();
}

}  // namespace bpt
