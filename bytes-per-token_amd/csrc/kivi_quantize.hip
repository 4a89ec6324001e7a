// KIVI quantize-on-write: keys and values [B, Hkv, T, D] -> asymmetric 4 / 8-bit codes with float16 grids, the
// write half of fastserve's kernel-2 cache (kernels/reference.py:103-160 quantize_kv, called for every completed
// key group by integration/kv_cache.py:139-158 QuantizedKVCache._append).
//
// Per grid (keys: one channel over `group` tokens; values: one token over its D channels):
//   lo = min(min x, 0), hi = max(max x, 0), scale = f16((hi - lo) / (2^bits - 1)) (1 where that is not > 0),
//   zero = clamp(round(-lo / scale), 0, 2^bits - 1), code = clamp(round(x / scale) + zero, 0, 2^bits - 1),
// the scale rounded to float16 before the zero point and codes are computed from it; every quotient rounds as
// IEEE float32 division does (the rows kernel takes x times the scale's reciprocal and divides only where
// that lands near a half-way point, see rint_code) and rounding is half to even, so codes and grids are
// bit-exact with the reference formulas. 4-bit codes pair channel d (low nibble) with d + D/2 (high nibble).
//
// Two kernels, one wave per (sequence, KV head, key group) in both:
// * kivi_quantize_rows_kernel, for key groups of 32 tokens whose rows start on 16 bytes and span 32 .. 512
//   bytes (bf16 / f16 D = 16 .. 256, f32 D = 8 .. 128): lane l reads 16-byte pieces, E = 16 / esize channels
//   (l % L) E .. + E - 1 of tokens l / L + R k (L = D / E lanes per row, R = 64 / L rows per wave-wide load,
//   k < 32 / R), every key and value piece of the group requested before any arithmetic. Key grids: min / max
//   over the lane's tokens, then across the R lanes holding the same channels; value grids: over the lane's E
//   channels, then across the row's L lanes; each grid is then made by one lane of each share and shuffled to
//   the others. Codes leave as E bytes per lane in nontemporal stores (4-bit: the lane holding channels
//   c .. c + E - 1 takes its partner's codes for c + D / 2 .. with one shuffle and stores the pairs).
// * kivi_quantize_kernel, any other group, head dim or alignment: lane l owns channels l, l + 64, ... and
//   walks the group's tokens one row at a time (2- or 4-byte loads and byte stores).
// Roofline: HBM, 2 * D * esize bytes read and 2 * D * bits / 8 + 4 * (D / group + 1) written per token.
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

// ---- rows kernel: 32-token key groups, 16-byte rows ------------------------------------------------------

constexpr int kRowsGroup = 32;

template <int SRC>
constexpr int src_bytes() {
  return SRC == kFF32 ? 4 : 2;
}

// 16 bytes of source elements -> E floats, in channel order.
template <int SRC, int E>
__device__ __forceinline__ void unpack16(const U4& u, float (&x)[E]) {
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if constexpr (SRC == kFF32) {
      x[i] = __uint_as_float(w[i]);
    } else if constexpr (SRC == kFBf16) {
      x[2 * i] = __uint_as_float(w[i] << 16);
      x[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    } else {
      x[2 * i] = (float)__builtin_bit_cast(_Float16, (uint16_t)w[i]);
      x[2 * i + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[i] >> 16));
    }
  }
}

// rint(x / s) + z with x / s the IEEE quotient (the reference's round(x / scale) + zero), given
// inv = v_rcp_f32(s) and the integer zero point z. q = fma(x, inv, z) is within 2^-23 |x / s| (rcp: 1 ulp)
// plus half an ulp of |q| of x / s + z. A scale is the float16 rounding of (hi - lo) / qmax (1 if that is 0),
// never below 2/3 of it, so |x / s| <= 1.5 qmax and |q| < 1024: q is within 7.7e-5 of x / s + z, and the IEEE
// quotient within 3.1e-5 of x / s. Farther than 2^-12 from every half-integer, q and the IEEE quotient
// (shifted by the integer z) lie in the same unit interval around an integer and round to it; nearer (about
// one value in two thousand), the IEEE division decides. NaN and infinite q keep q, as the division would give.
__device__ __forceinline__ float rint_code(float x, float s, float inv, float z) {
  const float q = fmaf(x, inv, z);
  float n = rintf(q);
  if (fabsf(q - n) >= 0.5f - 0x1p-12f) n = rintf(__fdiv_rn(x, s)) + z;
  return n;
}

// E codes of one piece (integer-valued floats in [0, qmax], so the byte conversion is exact) -> E bytes.
// Grid j of the piece's element j is g[j * g_step], with inv[j * g_step] = v_rcp_f32 of its scale.
template <int E>
__device__ __forceinline__ void code_bytes(const float (&x)[E], const Grid* g, const float* inv, int g_step,
                                           float qmax, uint32_t (&w)[E / 4]) {
#pragma unroll
  for (int i = 0; i < E / 4; ++i) {
    uint32_t a = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = (4 * i + j) * g_step;
      const float n = rint_code(x[4 * i + j], g[e].scale, inv[e], g[e].zero);
      a = __builtin_amdgcn_cvt_pk_u8_f32(__builtin_amdgcn_fmed3f(n, 0.0f, qmax), j, a);
    }
    w[i] = a;
  }
}

// Min and max over aligned groups of N lanes (N a power of two up to 64), every lane left holding them:
// DPP inside rows of 16, shuffles across rows.
template <int N>
__device__ __forceinline__ void group_min_max(float& mn, float& mx) {
  if constexpr (N >= 2) {
    mn = fminf(mn, dpp_mov<kDppXor1>(mn));
    mx = fmaxf(mx, dpp_mov<kDppXor1>(mx));
  }
  if constexpr (N >= 4) {
    mn = fminf(mn, dpp_mov<kDppXor2>(mn));
    mx = fmaxf(mx, dpp_mov<kDppXor2>(mx));
  }
  if constexpr (N >= 8) {
    mn = fminf(mn, dpp_mov<kDppHalfMirror>(mn));
    mx = fmaxf(mx, dpp_mov<kDppHalfMirror>(mx));
  }
  if constexpr (N >= 16) {
    mn = fminf(mn, dpp_mov<kDppRowMirror>(mn));
    mx = fmaxf(mx, dpp_mov<kDppRowMirror>(mx));
  }
#pragma unroll
  for (int m = 16; m < N; m <<= 1) {
    mn = fminf(mn, shfl_xor_f(mn, m));
    mx = fmaxf(mx, shfl_xor_f(mx, m));
  }
}

// Codes and grids are written once and not read again by this call: nontemporal stores (measured against
// ordinary ones at 64 x 8192 tokens: INT8 572 -> 544 us, INT4 515 -> 507 us).
template <int N>
__device__ __forceinline__ void store_words(void* dst, const uint32_t (&w)[N]) {
  typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
  typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
  if constexpr (N == 1) {
    __builtin_nontemporal_store(w[0], (uint32_t*)dst);
  } else if constexpr (N == 2) {
    __builtin_nontemporal_store(u32x2_t{w[0], w[1]}, (u32x2_t*)dst);
  } else {
    static_assert(N == 4, "1, 2 or 4 words");
    __builtin_nontemporal_store(u32x4_t{w[0], w[1], w[2], w[3]}, (u32x4_t*)dst);
  }
}

// One piece's codes to its row: 8 bits as they are; 4 bits paired with the partner lane L / 2 away, which
// holds the channels D / 2 higher, and stored by the lower lane (byte c = channel c | channel c + D / 2 << 4).
template <int BITS, int L, int NW>
__device__ __forceinline__ void store_piece(uint8_t* dst, uint32_t (&w)[NW], int cp) {
  if constexpr (BITS == 4) {
#pragma unroll
    for (int i = 0; i < NW; ++i) w[i] |= (uint32_t)__shfl_xor((int)w[i], L / 2, 64) << 4;
    if (cp < L / 2) store_words(dst, w);
  } else {
    store_words(dst, w);
  }
}

template <int BITS, int SRC, int D>
__global__ __launch_bounds__(kQuantWaves * 64) void kivi_quantize_rows_kernel(const KiviQuantParams p) {
  constexpr int ES = src_bytes<SRC>();
  constexpr int E = 16 / ES;
  constexpr int L = D / E;
  constexpr int R = 64 / L;
  constexpr int NV = kRowsGroup / R;
  constexpr float kQmax = BITS == 4 ? 15.0f : 255.0f;
  static_assert(L >= 2 && L <= 32 && NV * R == kRowsGroup, "rows of 32 .. 512 bytes");
  const int lane = threadIdx.x & 63;
  const int64_t item = (int64_t)blockIdx.x * kQuantWaves + (threadIdx.x >> 6);  // (b, h, key group)
  const int groups = p.T / kRowsGroup;
  if (item >= (int64_t)p.B * p.Hkv * groups) return;
  const int g = (int)(item % groups);
  const int bh = (int)(item / groups);
  const int h = bh % p.Hkv, b = bh / p.Hkv;
  const int cp = lane % L, r0 = lane / L;
  const int t = g * kRowsGroup + r0;  // this lane's first token; then every R-th
  const int64_t src = ((int64_t)b * p.x_sb + (int64_t)h * p.x_sh + (int64_t)t * p.x_st) * ES + cp * 16;
  const int64_t src_step = (int64_t)R * p.x_st * ES;
  U4 kr[NV], vr[NV];
#pragma unroll
  for (int k = 0; k < NV; ++k) kr[k] = load16((const uint8_t*)p.k + src + k * src_step);
#pragma unroll
  for (int k = 0; k < NV; ++k) vr[k] = load16((const uint8_t*)p.v + src + k * src_step);
  const int64_t code = (int64_t)b * p.c_sb + (int64_t)h * p.c_sh + (int64_t)t * p.c_st + cp * E;
  const int64_t code_step = (int64_t)R * p.c_st;

  // ---- keys: per channel over the group's 32 tokens ----------------------------------------------------
  {
    float mn[E], mx[E];
    {
      float x[E];
      unpack16<SRC>(kr[0], x);
#pragma unroll
      for (int e = 0; e < E; ++e) mn[e] = mx[e] = x[e];
    }
#pragma unroll
    for (int k = 1; k < NV; ++k) {
      float x[E];
      unpack16<SRC>(kr[k], x);
#pragma unroll
      for (int e = 0; e < E; ++e) {
        mn[e] = fminf(mn[e], x[e]);
        mx[e] = fmaxf(mx[e], x[e]);
      }
    }
#pragma unroll
    for (int m = L; m < 64; m <<= 1) {
#pragma unroll
      for (int e = 0; e < E; ++e) {
        mn[e] = fminf(mn[e], shfl_xor_f(mn[e], m));
        mx[e] = fmaxf(mx[e], shfl_xor_f(mx[e], m));
      }
    }
    // The R lanes of a channel column now hold the same E ranges: lane r0 makes the grids of channels
    // r0 % RE + RE j only, and every lane takes the E grids from their makers.
    constexpr int RE = R < E ? R : E;
    constexpr int KG = E / RE;
    const int sub = r0 % RE;
    Grid own[KG];
#pragma unroll
    for (int j = 0; j < KG; ++j) {
      float lo = mn[j * RE], hi = mx[j * RE];
#pragma unroll
      for (int u = 1; u < RE; ++u) {
        lo = sub == u ? mn[j * RE + u] : lo;
        hi = sub == u ? mx[j * RE + u] : hi;
      }
      own[j] = make_grid(lo, hi, kQmax);
    }
    Grid gr[E];
    float inv[E];
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int maker = (e % RE) * L + cp;
      gr[e].scale = __shfl(own[e / RE].scale, maker, 64);
      gr[e].zero = __shfl(own[e / RE].zero, maker, 64);
      inv[e] = __builtin_amdgcn_rcpf(gr[e].scale);
    }
    if (r0 == 0) {
      uint32_t sw[E / 2], zw[E / 2];
#pragma unroll
      for (int i = 0; i < E / 2; ++i) {
        sw[i] = f16_bits(gr[2 * i].scale) | (uint32_t)f16_bits(gr[2 * i + 1].scale) << 16;
        zw[i] = f16_bits(gr[2 * i].zero) | (uint32_t)f16_bits(gr[2 * i + 1].zero) << 16;
      }
      const int64_t go = (int64_t)b * p.g_sb + (int64_t)h * p.g_sh + (int64_t)g * p.g_sg + cp * E;
      store_words(p.ks + go, sw);
      store_words(p.kz + go, zw);
    }
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      float x[E];
      unpack16<SRC>(kr[k], x);
      uint32_t w[E / 4];
      code_bytes(x, gr, inv, 1, kQmax, w);
      store_piece<BITS, L>(p.kc + code + k * code_step, w, cp);
    }
  }

  // ---- values: per token over its D channels ------------------------------------------------------------
  // Ranges of the lane's NV rows first; the row's L lanes then hold the same NV ranges, and lane cp makes
  // the grid of row cp % NV only (NV = L / 2: two makers per row), stores it, and every lane takes its NV
  // rows' grids from their makers.
  float vmn[NV], vmx[NV];
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    float x[E];
    unpack16<SRC>(vr[k], x);
    float mn = x[0], mx = x[0];
#pragma unroll
    for (int e = 1; e < E; ++e) {
      mn = fminf(mn, x[e]);
      mx = fmaxf(mx, x[e]);
    }
    group_min_max<L>(mn, mx);
    vmn[k] = mn;
    vmx[k] = mx;
  }
  static_assert(2 * NV == L, "two makers per row");
  const int vsub = cp % NV;
  Grid vown;
  {
    float lo = vmn[0], hi = vmx[0];
#pragma unroll
    for (int u = 1; u < NV; ++u) {
      lo = vsub == u ? vmn[u] : lo;
      hi = vsub == u ? vmx[u] : hi;
    }
    vown = make_grid(lo, hi, kQmax);
  }
  if (cp < NV) {
    const int64_t vo = (int64_t)b * p.t_sb + (int64_t)h * p.t_sh + t + (int64_t)cp * R;
    __builtin_nontemporal_store(f16_bits(vown.scale), p.vs + vo);
    __builtin_nontemporal_store(f16_bits(vown.zero), p.vz + vo);
  }
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int maker = r0 * L + k;
    Grid gr;
    gr.scale = __shfl(vown.scale, maker, 64);
    gr.zero = __shfl(vown.zero, maker, 64);
    const float inv = __builtin_amdgcn_rcpf(gr.scale);
    float x[E];
    unpack16<SRC>(vr[k], x);
    uint32_t w[E / 4];
    code_bytes(x, &gr, &inv, 0, kQmax, w);
    store_piece<BITS, L>(p.vc + code + k * code_step, w, cp);
  }
}

// The rows kernel's layout conditions: 32-token groups; rows of 32 .. 512 bytes; sources, codes (E bytes per
// lane) and key grids (E halves per lane) aligned for the lanes' vector accesses at every (b, h, token).
static bool rows_kernel_fits(const KiviQuantParams& p) {
  const int es = p.src_dtype == kFF32 ? 4 : 2;
  const int e = 16 / es;
  const int64_t rb = (int64_t)p.D * es;
  auto al = [](const void* ptr, int n) { return (uintptr_t)ptr % n == 0; };
  return p.group == kRowsGroup && rb >= 32 && rb <= 512 && al(p.k, 16) && al(p.v, 16) &&
         (p.x_sb * es) % 16 == 0 && (p.x_sh * es) % 16 == 0 && (p.x_st * es) % 16 == 0 && al(p.kc, e) &&
         al(p.vc, e) && p.c_sb % e == 0 && p.c_sh % e == 0 && p.c_st % e == 0 && al(p.ks, 2 * e) &&
         al(p.kz, 2 * e) && p.g_sb % e == 0 && p.g_sh % e == 0 && p.g_sg % e == 0;
}

template <int BITS, int SRC>
static hipError_t launch_rows(const KiviQuantParams& p, dim3 grid, dim3 block, hipStream_t stream) {
  constexpr int ES = src_bytes<SRC>();
  switch (p.D * ES) {
    case 32: hipLaunchKernelGGL((kivi_quantize_rows_kernel<BITS, SRC, 32 / ES>), grid, block, 0, stream, p); break;
    case 64: hipLaunchKernelGGL((kivi_quantize_rows_kernel<BITS, SRC, 64 / ES>), grid, block, 0, stream, p); break;
    case 128: hipLaunchKernelGGL((kivi_quantize_rows_kernel<BITS, SRC, 128 / ES>), grid, block, 0, stream, p); break;
    case 256: hipLaunchKernelGGL((kivi_quantize_rows_kernel<BITS, SRC, 256 / ES>), grid, block, 0, stream, p); break;
    case 512: hipLaunchKernelGGL((kivi_quantize_rows_kernel<BITS, SRC, 512 / ES>), grid, block, 0, stream, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <int BITS>
static hipError_t launch_rows_bits(const KiviQuantParams& p, dim3 grid, dim3 block, hipStream_t stream) {
  if (p.src_dtype == kFBf16) return launch_rows<BITS, kFBf16>(p, grid, block, stream);
  if (p.src_dtype == kFF16) return launch_rows<BITS, kFF16>(p, grid, block, stream);
  return launch_rows<BITS, kFF32>(p, grid, block, stream);
}

hipError_t launch_kivi_quantize(const KiviQuantParams& p, hipStream_t stream) {
  const int64_t items = (int64_t)p.B * p.Hkv * (p.T / p.group);
  if (items == 0) return hipSuccess;
  dim3 grid((unsigned)((items + kQuantWaves - 1) / kQuantWaves)), block(kQuantWaves * 64);
  if (rows_kernel_fits(p))
    return p.bits == 4 ? launch_rows_bits<4>(p, grid, block, stream) : launch_rows_bits<8>(p, grid, block, stream);
  if (p.bits == 4) hipLaunchKernelGGL(kivi_quantize_kernel<4>, grid, block, 0, stream, p);
  else hipLaunchKernelGGL(kivi_quantize_kernel<8>, grid, block, 0, stream, p);
  return hipGetLastError();
}

}  // namespace bpt
