// Decode attention over a KIVI cache on the matrix cores: asymmetric 4- or 8-bit codes with float16 grids
// (keys: one (scale, zero) per channel per key group of tokens; values: one per token), or float16 /
// bfloat16 keys and values (the unquantized control). One query per head, the G query heads of a KV head
// computed together so every cached byte is read once; one partial result per split of the tokens.
//
// Follows fastserve kernels/kv_attention.py:56-175 (decode_attention_kernel: grids folded out of the inner
// product, online softmax, one partial (out, lse) per split) and :190-245 (the launcher's split rule), over
// the format of kernels/reference.py:66-160. The work is cut differently: the tokens of every (sequence,
// KV head) are a line of 32-token chunks that the launched workgroups share out evenly (stream-K), so the
// chip fills whatever the caller's split; a split covered by several workgroups is combined exactly
// (kernels/reference.py:205-211's algebra) by the last one to finish.
//
// Chunk math (l = lane, n = l % 16, kq = l / 16; rows padded to 16, the MFMA N dimension):
//  * scores S^T = K Q^T with 16x16x32 f16 (bf16 for a bfloat16 cache) MFMAs, four K-steps per 16-token
//    tile. A = this lane's token 16 t + n: the codes turned into f16 (1024 + code, by placing the code
//    under the f16 exponent of 1024) minus (1024 + zero) of their channel, i.e. code - zero exactly.
//    B = q * key scale, folded once per chunk (its key group) in a compact layout (RP rows x 128
//    channels over 64 lanes), scaled by a power of two so its largest element sits in [2^13, 2^14), split
//    into an f16 high part and the f16 rounding remainder (22 significant bits), and handed to the MFMA
//    layout through LDS. Each row's score is the MFMA result times sm_scale * log2(e) / that power of two.
//  * online softmax in base 2 per row (the row's four lanes agree through two shuffles). Each token's value
//    scale is folded into its weight, w = 2^(s - base) * vscale; the reference point tracks the largest
//    score plus a power-of-two bound on the chunk's value scales, so every w stays below 2^12 (inside f16)
//    whatever the value scales.
//  * output O^T += V^T W^T, contraction over the lane's own eight score tokens. V^T comes from 4 x 4 byte
//    (or 2 x 2 half) transposes, turned into code - value zero exactly as for keys; W = f16 high part plus
//    remainder, two MFMAs per M-tile.
#include <type_traits>

#include "decode_common.h"

namespace bpt {

namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kChunk = 32;  // tokens per chunk: two 16-token tiles

template <int FMT>
struct KF {
  static constexpr bool kQuant = FMT == kKivi4 || FMT == kKivi8;
  // Value products over offset codes with the zero points taken out afterwards (compute, value_zero_out):
  // always for 4-bit codes; for 8-bit codes but at 16 rows, where the extra accumulator would spill.
  template <int CPL>
  static constexpr bool kZeroFold = FMT == kKivi4 || (FMT == kKivi8 && CPL < 32);
  static constexpr bool kBf16 = FMT == kKiviBf16;
  static constexpr int kKU4 = FMT == kKivi4 ? 1 : (FMT == kKivi8 ? 2 : 4);  // 16-byte K loads per lane per tile
  static constexpr int kVWords = FMT == kKivi4 ? 1 : (FMT == kKivi8 ? 2 : 4);  // V dwords per lane per token
  typedef typename std::conditional<kBf16, bf16x8, f16x8>::type T;  // MFMA operand
  typedef typename std::conditional<kBf16, __bf16, _Float16>::type E;
};

// Position of channel c in the score contraction order (k = 32 kq + 8 s + i). Byte-wide formats use the
// identity (lane kq reads channels 32 kq .. 32 kq + 31); 4-bit codes pair channel d with d + 64 in a byte,
// so lane kq's 16 bytes hold channels 16 kq + j and 64 + 16 kq + j, and K-step s takes byte word s:
// [16 kq + 4 s + 0..3 (low nibbles), 64 + 16 kq + 4 s + 0..3 (high nibbles)].
template <int FMT>
__device__ __forceinline__ int kpos(int c) {
  if constexpr (FMT == kKivi4) {
    const int cc = c & 63;
    return 2 * (cc & ~3) + (c >= 64 ? 4 : 0) + (cc & 3);
  }
  return c;
}

// Output channel held by lane (kq, i) in M-tile mu of the value product.
template <int FMT>
__device__ __forceinline__ int out_channel(int kq, int i, int mu) {
  if constexpr (FMT == kKivi4) return (mu < 4 ? 0 : 64) + 16 * kq + 4 * i + (mu & 3);
  return 32 * kq + 8 * i + mu;
}

template <int FMT, int CPL>
struct KChunk {
  U4 k[2][KF<FMT>::kKU4];                 // tile t: token 16 t + n
  uint32_t v[2][4][KF<FMT>::kVWords];     // tile t, token 16 t + 4 kq + i
  u32x2 vs[2], vz[2];                     // f16 value grids of tokens 16 t + 4 kq + 0..3
  uint32_t gs[CPL / 2], gz[CPL / 2];      // f16 key grid of this lane's fold channels
};

__device__ __forceinline__ f32x4 mfma(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Bytes 0, 1 (pair_lo) or 2, 3 (pair_hi) of w as the f16 pair (1024 + b0, 1024 + b1): exact for 0..255.
__device__ __forceinline__ uint32_t pair_lo(uint32_t w) { return __builtin_amdgcn_perm(0x64006400u, w, 0x07010500u); }
__device__ __forceinline__ uint32_t pair_hi(uint32_t w) { return __builtin_amdgcn_perm(0x64006400u, w, 0x07030502u); }

typedef _Float16 h2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t sub_h2(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, a) - __builtin_bit_cast(h2, b));
}

// (1024 + byte) - z, pair by pair (packed f16 subtractions): the code minus its zero point, exactly. The zero
// points z travel as f16 pairs in plain dwords.
__device__ __forceinline__ f16x8 bytes8_minus(uint32_t w0, uint32_t w1, const uint32_t (&z)[4]) {
  const u32x4 r = {sub_h2(pair_lo(w0), z[0]), sub_h2(pair_hi(w0), z[1]), sub_h2(pair_lo(w1), z[2]),
                   sub_h2(pair_hi(w1), z[3])};
  return __builtin_bit_cast(f16x8, r);
}

// The f16 pair (1024 + b0, 1024 + b1) from bytes 0 and 1 (pair_lo) or 2 and 3 (pair_hi), for the value
// product, which takes codes with the 1024 left in (the zero points are taken out after it).
__device__ __forceinline__ f16x8 bytes8(uint32_t w0, uint32_t w1) {
  const u32x4 r = {pair_lo(w0), pair_hi(w0), pair_lo(w1), pair_hi(w1)};
  return __builtin_bit_cast(f16x8, r);
}

// Byte j of token words a (first) and b as the low half and the high half of one dword, the other bytes 0:
// 4-bit codes of one channel pair for two tokens, split into f16 pairs by nib_lo / nib_hi.
__device__ __forceinline__ uint32_t byte_pair(uint32_t a, uint32_t b, int j) {
  return __builtin_amdgcn_perm(b, a, 0x0c000c00u | ((uint32_t)(4 + j) << 16) | (uint32_t)j);
}
// (1024 + low nibble) and (1024 + 16 * high nibble) of both halves, as f16 pairs: one v_and_or_b32 each,
// the mask from a scalar register and 0x64006400 (f16 1024, 1024) from a vector register `k` that the caller
// keeps (a VOP3 instruction takes no literal here, and reads one scalar register at most; left to itself
// the compiler splits the AND and the OR into two instructions with literals).
__device__ __forceinline__ uint32_t and_or_k(uint32_t x, uint32_t mask, uint32_t k) {
  uint32_t r;
  __asm__("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "s"(mask), "v"(k));
  return r;
}
__device__ __forceinline__ uint32_t nib_lo(uint32_t x, uint32_t k) { return and_or_k(x, 0x000F000Fu, k); }
__device__ __forceinline__ uint32_t nib_hi(uint32_t x, uint32_t k) { return and_or_k(x, 0x00F000F0u, k); }

// x = hi + lo with hi, lo f16 (hi rounded toward zero, lo the rounded remainder, which x - hi holds
// exactly): 22 significant bits of each of two floats, as two f16 pairs.
__device__ __forceinline__ void split_pair(float x0, float x1, uint32_t& hi, uint32_t& lo) {
  const auto h = __builtin_amdgcn_cvt_pkrtz(x0, x1);
  hi = __builtin_bit_cast(uint32_t, h);
  lo = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(x0 - (float)h[0], x1 - (float)h[1]));
}

// Bytes 0, 1 (HI false) or 2, 3 of x, each 0 .. 15, as the f16 pair (b0, b1): FP8 e4m3 times 2^9.
template <bool HI>
__device__ __forceinline__ uint32_t codes_f16(uint32_t x) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(x, 512.0f, HI));
}

// 4 x 4 byte transpose: w[i] byte j -> o[j] byte i.
__device__ __forceinline__ void transpose4(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3, uint32_t (&o)[4]) {
  const uint32_t t0 = __builtin_amdgcn_perm(w1, w0, 0x05010400u);
  const uint32_t t1 = __builtin_amdgcn_perm(w3, w2, 0x05010400u);
  const uint32_t t2 = __builtin_amdgcn_perm(w1, w0, 0x07030602u);
  const uint32_t t3 = __builtin_amdgcn_perm(w3, w2, 0x07030602u);
  o[0] = __builtin_amdgcn_perm(t1, t0, 0x05040100u);
  o[1] = __builtin_amdgcn_perm(t1, t0, 0x07060302u);
  o[2] = __builtin_amdgcn_perm(t3, t2, 0x05040100u);
  o[3] = __builtin_amdgcn_perm(t3, t2, 0x07060302u);
}

// The (sequence, KV head)'s tensors (wave-uniform) and this lane's constant offsets into them (32-bit:
// one head's codes and grids span less than 2 GiB, checked on the host).
struct Head {
  const uint8_t* k;
  const uint8_t* v;
  const uint16_t* ks;
  const uint16_t* kz;
  const uint16_t* vs;
  const uint16_t* vz;
};

struct LaneOffsets {
  uint32_t k, v;  // bytes: K row of token n at byte 16 kq * (K loads); V row of token 4 kq at byte n * (V bytes)
  uint32_t g;     // elements: this lane's fold channels in a key grid
  uint32_t t;     // elements: token 4 kq in a value grid
};

__device__ __forceinline__ Head head_of(const KiviParams& p, int b, int h) {
  const int64_t c = (int64_t)b * p.c_sb + (int64_t)h * p.c_sh;
  const int64_t g = (int64_t)b * p.g_sb + (int64_t)h * p.g_sh;
  const int64_t t = (int64_t)b * p.t_sb + (int64_t)h * p.t_sh;
  return Head{p.kc + c, p.vc + c, p.ks + g, p.kz + g, p.vs + t, p.vz + t};
}

template <int FMT, int RP, int CPL>
__device__ __forceinline__ LaneOffsets lane_offsets(const KiviParams& p, int lane) {
  typedef KF<FMT> F;
  const uint32_t st = (uint32_t)p.c_st;
  const int kq = lane >> 4, n = lane & 15;
  return LaneOffsets{n * st + kq * (16 * F::kKU4), 4 * kq * st + n * (4 * F::kVWords), (uint32_t)((lane % (64 / RP)) * CPL),
                     (uint32_t)(4 * kq)};
}

// Chunk kk's key-grid, K and value-grid loads (issued together, in the order they are consumed) and its V
// loads. The chunk's 32 tokens all lie inside the laid-out T (a multiple of 32); those at or past the
// row's length are masked after loading.
template <int FMT, int CPL>
__device__ __forceinline__ void issue_k(const KiviParams& p, const Head& hd, const LaneOffsets& lo, int kk, KChunk<FMT, CPL>& c) {
  typedef KF<FMT> F;
  const uint32_t T0 = (uint32_t)kk * kChunk;
  const uint32_t st = (uint32_t)p.c_st;
  if constexpr (F::kQuant) {
    const uint32_t go = (uint32_t)(kk >> p.gshift) * (uint32_t)p.g_sg + lo.g;
    if constexpr (CPL == 4) {
      const u32x2 s = *(const u32x2*)(hd.ks + go);
      const u32x2 z = *(const u32x2*)(hd.kz + go);
      c.gs[0] = s.x; c.gs[1] = s.y;
      c.gz[0] = z.x; c.gz[1] = z.y;
    } else {
#pragma unroll
      for (int j = 0; j < CPL / 8; ++j) {
        const u32x4 s = *(const u32x4*)(hd.ks + go + 8 * j);
        const u32x4 z = *(const u32x4*)(hd.kz + go + 8 * j);
        c.gs[4 * j] = s.x; c.gs[4 * j + 1] = s.y; c.gs[4 * j + 2] = s.z; c.gs[4 * j + 3] = s.w;
        c.gz[4 * j] = z.x; c.gz[4 * j + 1] = z.y; c.gz[4 * j + 2] = z.z; c.gz[4 * j + 3] = z.w;
      }
    }
  }
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const uint32_t off = lo.k + (T0 + 16 * t) * st;
#pragma unroll
    for (int j = 0; j < F::kKU4; ++j) c.k[t][j] = load16(hd.k + off + 16 * j);
  }
  if constexpr (F::kQuant) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      c.vs[t] = *(const u32x2*)(hd.vs + T0 + 16 * t + lo.t);
      c.vz[t] = *(const u32x2*)(hd.vz + T0 + 16 * t + lo.t);
    }
  }
}

template <int FMT, int CPL>
__device__ __forceinline__ void issue_v(const KiviParams& p, const Head& hd, const LaneOffsets& lo, int kk, KChunk<FMT, CPL>& c) {
  typedef KF<FMT> F;
  const uint32_t T0 = (uint32_t)kk * kChunk;
  const uint32_t st = (uint32_t)p.c_st;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint8_t* src = hd.v + (lo.v + (T0 + 16 * t + i) * st);
      if constexpr (F::kVWords == 1) {
        c.v[t][i][0] = __builtin_nontemporal_load((const uint32_t*)src);
      } else if constexpr (F::kVWords == 2) {
        const u32x2 x = __builtin_nontemporal_load((const u32x2*)src);
        c.v[t][i][0] = x.x;
        c.v[t][i][1] = x.y;
      } else {
        const U4 x = load16(src);
        c.v[t][i][0] = x.x;
        c.v[t][i][1] = x.y;
        c.v[t][i][2] = x.z;
        c.v[t][i][3] = x.w;
      }
    }
  }
}

// The compact fold: lane l covers row fr = l / LPR, channels fc .. fc + CPL - 1 (fc = (l % LPR) * CPL).
// x = q * key scale (1 for the unquantized formats); the row's largest |x| picks the power of two f; the
// f-scaled x goes to LDS as high part + remainder at its contraction position, qscale / f to s_inv; for
// 8-bit codes 1024 + key zero goes to s_kz (row 0's lanes), for 4-bit codes the row's sum of key zero x
// f-scaled x to s_zc (the scores start from minus it).
template <int FMT, int RP, int CPL>
__device__ __forceinline__ void fold(const float (&qf)[CPL], const uint32_t (&gs)[CPL / 2], const uint32_t (&gz)[CPL / 2],
                                     float qscale, int lane, uint16_t (*s_qh)[kHeadDim], uint16_t (*s_ql)[kHeadDim],
                                     uint16_t* s_kz, float* s_inv, float* s_zc) {
  typedef KF<FMT> F;
  typedef typename F::E E;
  constexpr int LPR = 64 / RP;
  const int fr = lane / LPR;
  const int fc = (lane % LPR) * CPL;
  float x[CPL];
  float mx = 0.0f;
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    float s = 1.0f;
    if constexpr (F::kQuant) {
      const uint32_t w = gs[c >> 1];
      s = (float)__builtin_bit_cast(_Float16, (uint16_t)((c & 1) ? (w >> 16) : (w & 0xffffu)));
    }
    x[c] = qf[c] * s;
    mx = fmaxf(mx, fabsf(x[c]));
  }
  // The row's largest |x| over its LPR lanes (an aligned group of 4 .. 32): DPP within rows of 16, then the
  // row pair through v_permlane16_swap (no LDS round trips on the chunk's path).
  static_assert(LPR >= 4 && LPR <= 32, "4 .. 32 lanes per fold row");
  mx = fmaxf(mx, dpp_mov<kDppXor1>(mx));
  mx = fmaxf(mx, dpp_mov<kDppXor2>(mx));
  if constexpr (LPR >= 8) mx = fmaxf(mx, dpp_mov<kDppHalfMirror>(mx));
  if constexpr (LPR >= 16) mx = fmaxf(mx, dpp_mov<kDppRowMirror>(mx));
  if constexpr (LPR >= 32) mx = max_xor<16>(mx);
  int e = 0;
  if (mx > 0.0f) (void)frexpf(mx, &e);
  e = e < -100 ? -100 : e;
  const float f = ldexpf(1.0f, 14 - e);
  float zc = 0.0f;  // 4-bit codes: this lane's share of the row's sum of key zero x f-scaled x
  if constexpr (FMT == kKivi4) {
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const uint32_t w = gz[c >> 1];
      zc += (float)__builtin_bit_cast(_Float16, (uint16_t)((c & 1) ? (w >> 16) : (w & 0xffffu))) * (x[c] * f);
    }
    zc += dpp_mov<kDppXor1>(zc);
    zc += dpp_mov<kDppXor2>(zc);
    if constexpr (LPR >= 8) zc += dpp_mov<kDppHalfMirror>(zc);
    if constexpr (LPR >= 16) zc += dpp_mov<kDppRowMirror>(zc);
    if constexpr (LPR >= 32) zc = sum_xor<16>(zc);
  }
#pragma unroll
  for (int c0 = 0; c0 < CPL; c0 += 4) {
    uint32_t hw[2], lw[2];
    if constexpr (std::is_same<E, _Float16>::value) {
#pragma unroll
      for (int c = 0; c < 4; c += 2) split_pair(x[c0 + c] * f, x[c0 + c + 1] * f, hw[c >> 1], lw[c >> 1]);
    } else {
      uint16_t hb[4], lb[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float y = x[c0 + c] * f;
        const E hi = (E)y;
        const E lo = (E)(y - (float)hi);
        hb[c] = __builtin_bit_cast(uint16_t, hi);
        lb[c] = __builtin_bit_cast(uint16_t, lo);
      }
      hw[0] = hb[0] | ((uint32_t)hb[1] << 16);
      hw[1] = hb[2] | ((uint32_t)hb[3] << 16);
      lw[0] = lb[0] | ((uint32_t)lb[1] << 16);
      lw[1] = lb[2] | ((uint32_t)lb[3] << 16);
    }
    const int pos = kpos<FMT>(fc + c0);  // four consecutive channels stay consecutive
    *(u32x2*)&s_qh[fr][pos] = u32x2{hw[0], hw[1]};
    *(u32x2*)&s_ql[fr][pos] = u32x2{lw[0], lw[1]};
    if constexpr (FMT == kKivi8) {
      if (fr == 0) {
        typedef _Float16 h2 __attribute__((ext_vector_type(2)));
        const h2 k1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
        const h2 z0 = __builtin_bit_cast(h2, gz[c0 >> 1]) + k1024;
        const h2 z1 = __builtin_bit_cast(h2, gz[(c0 >> 1) + 1]) + k1024;
        *(u32x2*)&s_kz[pos] = u32x2{__builtin_bit_cast(uint32_t, z0), __builtin_bit_cast(uint32_t, z1)};
      }
    }
  }
  if ((lane % LPR) == 0) {
    s_inv[fr] = ldexpf(qscale, e - 14);  // qscale / f
    if constexpr (FMT == kKivi4) s_zc[fr] = zc;
  }
}

// Row n's score operands for the four K-steps, its score factor (0 past the G rows) and, for 8-bit codes,
// 1024 + key zero in this lane's contraction order, for 4-bit codes the row's zero term zc.
template <int FMT, int RP>
__device__ __forceinline__ void read_fold(int n, int kq, int G, const uint16_t (*s_qh)[kHeadDim],
                                          const uint16_t (*s_ql)[kHeadDim], const uint16_t* s_kz, const float* s_inv,
                                          const float* s_zc, typename KF<FMT>::T (&qh)[4], typename KF<FMT>::T (&ql)[4],
                                          uint32_t (&kzp)[4][4], float& inv, float& zc) {
  typedef typename KF<FMT>::T T;
  const bool in = n < G;
  const int r = in ? n : 0;  // padded rows compute row 0's scores, scaled by 0 and never stored
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    qh[s] = *(const T*)&s_qh[r][32 * kq + 8 * s];
    ql[s] = *(const T*)&s_ql[r][32 * kq + 8 * s];
    if constexpr (FMT == kKivi8) {
      const u32x4 z = *(const u32x4*)&s_kz[32 * kq + 8 * s];
      kzp[s][0] = z.x;
      kzp[s][1] = z.y;
      kzp[s][2] = z.z;
      kzp[s][3] = z.w;
    }
  }
  inv = in ? s_inv[r] : 0.0f;
  zc = FMT == kKivi4 ? s_zc[r] : 0.0f;
}

// Score operand A of K-step s, tile t: code - zero (quantized) or the stored halves.
template <int FMT, int CPL>
__device__ __forceinline__ typename KF<FMT>::T k_operand(const KChunk<FMT, CPL>& c, int t, int s, const uint32_t (&kz)[4]) {
  typedef typename KF<FMT>::T T;
  if constexpr (FMT == kKivi8) {
    const U4 q = c.k[t][s >> 1];
    const uint32_t w0 = (s & 1) ? q.z : q.x;
    const uint32_t w1 = (s & 1) ? q.w : q.y;
    return bytes8_minus(w0, w1, kz);
  } else if constexpr (FMT == kKivi4) {
    // The codes themselves (the zero points go into the scores' starting value): a byte holding 0 .. 15,
    // read as FP8 e4m3, is code x 2^-9 exactly (the subnormals and the first binade step by 2^-9), and the
    // FP8 -> f16 conversion scaled by 2^9 gives the code.
    const U4 q = c.k[t][0];
    const uint32_t w = s == 0 ? q.x : (s == 1 ? q.y : (s == 2 ? q.z : q.w));
    const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
    const u32x4 r = {codes_f16<false>(lo), codes_f16<true>(lo), codes_f16<false>(hi), codes_f16<true>(hi)};
    return __builtin_bit_cast(T, r);
  } else {
    return __builtin_bit_cast(T, c.k[t][s]);
  }
}

// Fold chunk kk into this lane's state: m (row n's reference point, shared by its four lanes), l (this
// lane's partial weight sum), o[mu] (row n, channels out_channel(kq, i, mu)) and, for codes, oz: the value
// products take 1024 + code (4-bit high nibbles: 1024 + 16 code), and oz gathers what that adds, the sum
// over tokens of weight x (1024 + value zero) (1024 + 16 zero in rows 8 .. 15 of its tile), which
// value_zero_out takes out. The weights are positive, so the offset costs no precision that matters: the
// products stay within 2^11 of their sum without it.
template <int FMT, int CPL, typename AfterScores>
__device__ __forceinline__ void compute(KChunk<FMT, CPL>& c, int kk, int len, int lane, const typename KF<FMT>::T (&qh)[4],
                                        const typename KF<FMT>::T (&ql)[4], const uint32_t (&kzp)[4][4], float inv, float zc,
                                        float& m, float& l, f32x4 (&o)[8], f32x4& oz, AfterScores after_scores) {
  typedef KF<FMT> F;
  typedef typename F::T T;
  typedef typename F::E E;
  const int T0 = kk * kChunk;
  const int kq = lane >> 4;
  float sc[8];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    f32x4 st = {-zc, -zc, -zc, -zc};  // 0 but for 4-bit codes
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const T a = k_operand<FMT, CPL>(c, t, s, kzp[s]);
      st = mfma(a, qh[s], st);
      st = mfma(a, ql[s], st);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) sc[4 * t + i] = st[i] * inv;
  }

  // Value grids of the lane's eight tokens (j < 4: tile 0, token 4 kq + j; j >= 4: tile 1, 4 kq + j - 4).
  uint32_t sw[4] = {0u, 0u, 0u, 0u}, zw[4] = {0u, 0u, 0u, 0u};
  if constexpr (F::kQuant) {
    sw[0] = c.vs[0].x; sw[1] = c.vs[0].y; sw[2] = c.vs[1].x; sw[3] = c.vs[1].y;
    zw[0] = c.vz[0].x; zw[1] = c.vz[0].y; zw[2] = c.vz[1].x; zw[3] = c.vz[1].y;
  }
  if (T0 + kChunk > len) {  // the row's last chunk: tokens past its length are loaded but may hold anything
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (T0 + 16 * (j >> 2) + 4 * kq + (j & 3) >= len) {
        sc[j] = kNegInf;
        if constexpr (F::kQuant) {
          const uint32_t keep = (j & 1) ? 0x0000ffffu : 0xffff0000u;
          sw[j >> 1] &= keep;
          zw[j >> 1] &= keep;
        } else {
#pragma unroll
          for (int w = 0; w < F::kVWords; ++w) c.v[j >> 2][j & 3][w] = 0u;  // finite values under weight 0
        }
      }
    }
  }
  float vsf[8];
  float ev = 0.0f;  // this lane's tokens have value scales below 2^ev
  uint32_t vzp[4];  // 1024 + value zero of the lane's eight tokens (x 16 first in 4-bit rows 8 .. 15), f16 pairs
  if constexpr (F::kQuant) {
    typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
    const u16x2 m01 = __builtin_elementwise_max(__builtin_bit_cast(u16x2, sw[0]), __builtin_bit_cast(u16x2, sw[1]));
    const u16x2 m23 = __builtin_elementwise_max(__builtin_bit_cast(u16x2, sw[2]), __builtin_bit_cast(u16x2, sw[3]));
    const u16x2 mm = __builtin_elementwise_max(m01, m23);
    const uint32_t top = mm.x > mm.y ? mm.x : mm.y;  // positive f16: bit order is value order
    ev = (float)((int)((top >> 10) & 31u) - 14);
    const h2 k1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t bits = (j & 1) ? (sw[j >> 1] >> 16) : (sw[j >> 1] & 0xffffu);
      vsf[j] = (float)__builtin_bit_cast(_Float16, (uint16_t)bits);
    }
    if constexpr (FMT == kKivi4) {
      const _Float16 z16 = (lane & 15) < 8 ? (_Float16)1.0f : (_Float16)16.0f;
      const h2 zs = {z16, z16};
#pragma unroll
      for (int j = 0; j < 4; ++j) vzp[j] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, zw[j]) * zs + k1024);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) vzp[j] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, zw[j]) + k1024);
    }
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) vsf[j] = 1.0f;
  }
  after_scores();

  // ---- online softmax of row n over this chunk (8 scores here, 24 on the row's other lanes) -------------
  float mx = kNegInf;
#pragma unroll
  for (int j = 0; j < 8; ++j) mx = fmaxf(mx, sc[j]);
  mx += ev;
  mx = max_xor<32>(max_xor<16>(mx));
  const bool move = mx > m + kSlack;
  if (__any(move)) {
    const float mn = move ? mx : m;
    const float alpha = move ? fast_exp2(m - mn) : 1.0f;  // 0 when m was -inf
    l *= alpha;
#pragma unroll
    for (int mu = 0; mu < 8; ++mu) o[mu] *= alpha;
    if constexpr (F::template kZeroFold<CPL>) oz *= alpha;
    m = mn;
  }
  const float base = (m == kNegInf ? 0.0f : m) - kBias;
  T ph, pl;
  if constexpr (std::is_same<E, _Float16>::value) {
    u32x4 hw, lw;
#pragma unroll
    for (int j = 0; j < 8; j += 2) {
      const float e0 = fast_exp2(sc[j] - base), e1 = fast_exp2(sc[j + 1] - base);
      l += e0;
      l += e1;
      uint32_t hi, lo;
      split_pair(e0 * vsf[j], e1 * vsf[j + 1], hi, lo);
      hw[j >> 1] = hi;
      lw[j >> 1] = lo;
    }
    ph = __builtin_bit_cast(T, hw);
    pl = __builtin_bit_cast(T, lw);
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float e = fast_exp2(sc[j] - base);
      l += e;
      const float w = e * vsf[j];
      const E hi = (E)w;
      ph[j] = hi;
      pl[j] = (E)(w - (float)hi);
    }
  }

  // ---- O^T += V^T W^T: eight M-tiles -------------------------------------------------------------------
  if constexpr (FMT == kKivi8) {
    uint32_t lo[2][4], hi[2][4];  // [tile][j]: channel 8 n' + j (lo) or 8 n' + 4 + j (hi); bytes = tokens
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      transpose4(c.v[t][0][0], c.v[t][1][0], c.v[t][2][0], c.v[t][3][0], lo[t]);
      transpose4(c.v[t][0][1], c.v[t][1][1], c.v[t][2][1], c.v[t][3][1], hi[t]);
    }
    constexpr bool ZF = F::template kZeroFold<CPL>;
#pragma unroll
    for (int mu = 0; mu < 8; ++mu) {
      const uint32_t d0 = mu < 4 ? lo[0][mu & 3] : hi[0][mu & 3];
      const uint32_t d1 = mu < 4 ? lo[1][mu & 3] : hi[1][mu & 3];
      const f16x8 a = ZF ? bytes8(d0, d1) : bytes8_minus(d0, d1, vzp);
      o[mu] = mfma(a, ph, o[mu]);
      o[mu] = mfma(a, pl, o[mu]);
    }
    if constexpr (ZF) {
      const f16x8 az = __builtin_bit_cast(f16x8, u32x4{vzp[0], vzp[1], vzp[2], vzp[3]});
      oz = mfma(az, ph, oz);
      oz = mfma(az, pl, oz);
    }
  } else if constexpr (FMT == kKivi4) {
    // Byte j of the lane's token words holds channels 4 n' + j (low nibble) and 64 + 4 n' + j (high):
    // M-tiles j and 4 + j take it, for tokens (0, 1) and (2, 3) of each tile.
    const uint32_t k1024 = 0x64006400u;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t pr[2][2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        pr[t][0] = byte_pair(c.v[t][0][0], c.v[t][1][0], j);
        pr[t][1] = byte_pair(c.v[t][2][0], c.v[t][3][0], j);
      }
      const f16x8 al = __builtin_bit_cast(
          f16x8, u32x4{nib_lo(pr[0][0], k1024), nib_lo(pr[0][1], k1024), nib_lo(pr[1][0], k1024), nib_lo(pr[1][1], k1024)});
      const f16x8 ah = __builtin_bit_cast(
          f16x8, u32x4{nib_hi(pr[0][0], k1024), nib_hi(pr[0][1], k1024), nib_hi(pr[1][0], k1024), nib_hi(pr[1][1], k1024)});
      o[j] = mfma(al, ph, o[j]);
      o[j] = mfma(al, pl, o[j]);
      o[4 + j] = mfma(ah, ph, o[4 + j]);
      o[4 + j] = mfma(ah, pl, o[4 + j]);
    }
    const f16x8 az = __builtin_bit_cast(f16x8, u32x4{vzp[0], vzp[1], vzp[2], vzp[3]});
    oz = mfma(az, ph, oz);
    oz = mfma(az, pl, oz);
  } else {
    // Halves: token pair (i, i + 1) of tile t at channel 8 n' + mu, as one dword.
#pragma unroll
    for (int mu = 0; mu < 8; ++mu) {
      const uint32_t sel = (mu & 1) ? 0x07060302u : 0x05040100u;
      const int wd = mu >> 1;
      const u32x4 r = {__builtin_amdgcn_perm(c.v[0][1][wd], c.v[0][0][wd], sel),
                       __builtin_amdgcn_perm(c.v[0][3][wd], c.v[0][2][wd], sel),
                       __builtin_amdgcn_perm(c.v[1][1][wd], c.v[1][0][wd], sel),
                       __builtin_amdgcn_perm(c.v[1][3][wd], c.v[1][2][wd], sel)};
      const T a = __builtin_bit_cast(T, r);
      o[mu] = mfma(a, ph, o[mu]);
      o[mu] = mfma(a, pl, o[mu]);
    }
  }
}

// Takes out of o what the offset value codes added (oz: row n's sum of weight x (1024 + zero), the same in
// every row of the lane's tile; for 4-bit codes rows 0 .. 7 hold the low channels' sum and rows 8 .. 15 the
// high channels' (1024 + 16 zero), whose products also carry a factor 16).
template <int FMT>
__device__ __forceinline__ void value_zero_out(int kq, const f32x4& oz, f32x4 (&o)[8]) {
  if constexpr (FMT == kKivi4) {
    const float own = oz[0];
    const float other = __shfl_xor(own, 32, 64);  // lanes kq and kq ^ 2: one holds each half
    const float zl = kq < 2 ? own : other, zh = kq < 2 ? other : own;
#pragma unroll
    for (int mu = 0; mu < 4; ++mu) o[mu] -= zl;
#pragma unroll
    for (int mu = 4; mu < 8; ++mu) o[mu] = (o[mu] - zh) * 0.0625f;
  } else {
#pragma unroll
    for (int mu = 0; mu < 8; ++mu) o[mu] -= oz[0];
  }
}

// This lane's fold inputs: q of row fr (h * G + fr), channels fc .. fc + CPL - 1, unscaled; zero past G.
template <int RP, int CPL>
__device__ __forceinline__ void load_q_fold(const KiviParams& p, int b, int h, int lane, float (&qf)[CPL]) {
  constexpr int LPR = 64 / RP;
  const int fr = lane / LPR;
  const bool in = fr < p.G;
  const int64_t base = (int64_t)b * p.q_sb + (int64_t)(h * p.G + (in ? fr : 0)) * p.q_sh + (lane % LPR) * CPL;
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const float x = load_float(p.q, base + c, p.q_dtype);
    qf[c] = in ? x : 0.0f;
  }
}

__device__ __forceinline__ int64_t out_index(const KiviParams& p, int b, int hq, int j) {
  return (int64_t)b * p.o_sb + (int64_t)hq * p.o_sh + (int64_t)j * p.o_ss;
}

__device__ __forceinline__ int64_t lse_index(const KiviParams& p, int b, int hq, int j) {
  return (int64_t)b * p.l_sb + (int64_t)hq * p.l_sh + (int64_t)j * p.l_ss;
}

// Splits past a row's length: out 0, lse -inf (workgroups take the rows round-robin).
// The attention state of the full-precision tail for the G query heads of (b, h), in the wave states' form
// (base 2, reference point m, bias kBias): s_tm[r] = m_r = max_t s_rt, s_tl[r] = sum_t 2^(s_rt - m_r + kBias),
// s_to[r D + ch] = sum_t 2^(s_rt - m_r + kBias) v_t[ch], where s_rt = sm_scale log2(e) q_r . k_t over the
// tail_len tokens (fastserve integration/kv_cache.py:179-182: partial_attention over the tail, in float32).
// s_tp: G x kKiviMaxTail floats of scratch. The whole workgroup calls it; it ends with a barrier.
template <int NT>
__device__ __forceinline__ void tail_state(const KiviParams& p, int b, int h, float* s_tp, float* s_tm, float* s_tl,
                                           float* s_to) {
  constexpr int D = kHeadDim;
  const int T = p.tail_len, G = p.G;
  const int64_t kv0 = (int64_t)b * p.tk_sb + (int64_t)h * p.tk_sh;
  for (int i = threadIdx.x; i < G * T; i += NT) {
    const int r = i / T, t = i - r * T;
    const int64_t qo = (int64_t)b * p.q_sb + (int64_t)(h * G + r) * p.q_sh;
    const int64_t ko = kv0 + (int64_t)t * p.tk_st;
    float acc = 0.0f;
#pragma unroll 8
    for (int c = 0; c < D; ++c) acc = fmaf(load_float(p.q, qo + c, p.q_dtype), load_float(p.tk, ko + c, p.tail_dtype), acc);
    s_tp[r * kKiviMaxTail + t] = acc * p.qscale;
  }
  __syncthreads();
  for (int r = threadIdx.x; r < G; r += NT) {
    float m = kNegInf;
    for (int t = 0; t < T; ++t) m = fmaxf(m, s_tp[r * kKiviMaxTail + t]);
    float l = 0.0f;
    for (int t = 0; t < T; ++t) {
      const float w = fast_exp2(s_tp[r * kKiviMaxTail + t] - m + kBias);
      s_tp[r * kKiviMaxTail + t] = w;
      l += w;
    }
    s_tm[r] = m;
    s_tl[r] = l;
  }
  __syncthreads();
  for (int i = threadIdx.x; i < G * D; i += NT) {
    const int r = i / D, ch = i - r * D;
    float o = 0.0f;
    for (int t = 0; t < T; ++t) o = fmaf(s_tp[r * kKiviMaxTail + t], load_float(p.tv, kv0 + (int64_t)t * p.tk_st + ch, p.tail_dtype), o);
    s_to[r * D + ch] = o;
  }
  __syncthreads();
}

template <int NT, bool TAIL>
__device__ __forceinline__ void zero_empty_splits(const KiviParams& p, const int* s_prefix, float* s_tp, float* s_tm,
                                                  float* s_tl, float* s_to) {
  constexpr int D = kHeadDim;
  for (int b = blockIdx.x; b < p.B; b += gridDim.x) {
    const int nb = s_prefix[b + 1] - s_prefix[b];
    if (TAIL && nb == 0) {  // no codes: the result is the tail's attention alone (one split)
      for (int h = 0; h < p.Hkv; ++h) {
        tail_state<NT>(p, b, h, s_tp, s_tm, s_tl, s_to);
        for (int i = threadIdx.x; i < p.G * D; i += NT) {
          const int r = i / D, ch = i - r * D;
          const int hq = h * p.G + r;
          p.out[out_index(p, b, hq, 0) + ch] = s_to[r * D + ch] / s_tl[r];
          if (ch == 0) p.lse[lse_index(p, b, hq, 0)] = (s_tm[r] - kBias + __log2f(s_tl[r])) * kLn2;
        }
        __syncthreads();  // the tail buffers are rewritten by the next head
      }
      continue;
    }
    const int active = (nb + p.cps - 1) / p.cps;
    const int per_head = (p.S - active) * D;
    for (int i = threadIdx.x; i < p.Hq * per_head; i += NT) {
      const int hq = i / per_head;
      const int r = i - hq * per_head;
      const int j = active + r / D;
      const int ch = r % D;
      p.out[out_index(p, b, hq, j) + ch] = 0.0f;
      if (ch == 0) p.lse[lse_index(p, b, hq, j)] = kNegInf;
    }
  }
}

// Count this workgroup's arrival at split segment `seg`; the last of its n pieces to arrive combines them
// (slots: the piece of workgroup gg is in slot 2 gg if it was that workgroup's first piece, else 2 gg + 1),
// writes the split's out and lse (natural log) and resets the counter.
template <int NT>
__device__ __forceinline__ void arrive_and_combine(const KiviParams& p, int seg, int b, int h, int j, int sc0,
                                                   int per, int g_first, int n, int tid, int* s_flag) {
  constexpr int D = kHeadDim;
  if (tid == 0) {
    *s_flag = ws_arrive(p.counters + seg) == (unsigned)n - 1u;
  }
  __syncthreads();
  if (!*s_flag) return;
  ws_acquire();
  const int G = p.G;
  for (int idx = tid; idx < G * D; idx += NT) {
    const int r = idx / D;
    const int ch = idx - r * D;
    float M = kNegInf, W = 0.0f, O = 0.0f;
    // kJ pieces' loads in flight per round: a split over many workgroups is combined in few round trips.
    constexpr int kJ = 16;
    for (int i0 = 0; i0 < n; i0 += kJ) {
      float lv[kJ], ov[kJ];
#pragma unroll
      for (int i = 0; i < kJ; ++i) {
        const int gg = g_first + i0 + i;
        const int64_t slot = (i0 + i == 0 && sc0 != gg * per) ? 2 * gg + 1 : 2 * gg;
        const bool in = i0 + i < n;
        lv[i] = in ? ws_load(p.ws_lse + slot * G + r) : kNegInf;
        ov[i] = in ? ws_load(p.ws_out + (slot * G + r) * D + ch) : 0.0f;
      }
      float bm = lv[0];
#pragma unroll
      for (int i = 1; i < kJ; ++i) bm = fmaxf(bm, lv[i]);
      const float nm = fmaxf(M, bm);
      const float mu = nm == kNegInf ? 0.0f : nm;
      const float alpha = W > 0.0f ? fast_exp2(M - mu) : 0.0f;
      W *= alpha;
      O *= alpha;
#pragma unroll
      for (int i = 0; i < kJ; ++i) {
        const float e = fast_exp2(lv[i] - mu);
        W += e;
        O = fmaf(e, ov[i], O);
      }
      M = nm;
    }
    const int hq = h * G + r;
    p.out[out_index(p, b, hq, j) + ch] = W > 0.0f ? O / W : 0.0f;
    if (ch == 0) p.lse[lse_index(p, b, hq, j)] = W > 0.0f ? (M + __log2f(W)) * kLn2 : kNegInf;
  }
  if (tid == 0) __hip_atomic_store(p.counters + seg, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

template <int FMT, int RP, bool TAIL>
__global__ __launch_bounds__(kDecodeWaves * 64, 2) void kivi_decode_kernel(const KiviParams p) {
  constexpr int NW = kDecodeWaves;
  constexpr int NT = NW * 64;
  constexpr int D = kHeadDim;
  constexpr int LPR = 64 / RP;
  constexpr int CPL = D / LPR;
  typedef KF<FMT> F;
  typedef typename F::T T;

  extern __shared__ int s_dyn[];  // [B + 1] chunks per sequence (exclusive prefix sum), then [B] lengths
  int* s_prefix = s_dyn;
  int* s_len = s_dyn + p.B + 1;
  __shared__ int s_wsum[NW];
  __shared__ int s_last;
  __shared__ __align__(16) uint16_t s_qh[NW][RP][D];  // score operands, high parts, contraction order
  __shared__ __align__(16) uint16_t s_ql[NW][RP][D];  // and remainders
  __shared__ __align__(16) uint16_t s_kz[NW][D];      // 1024 + key zero (f16), contraction order
  __shared__ float s_inv[NW][RP];
  __shared__ float s_zc[NW][RP];                      // 4-bit codes: each row's key zero term
  __shared__ float s_m[NW][RP];
  __shared__ float s_l[NW][RP];
  __shared__ float s_o[NW][RP][D + 1];  // rows padded by one word: a merge store's rows land on distinct banks
  __shared__ float s_tm[RP], s_tl[RP];  // the tail's state (tail_state); its scratch and sums reuse the fold buffers
  static_assert(sizeof(s_qh) >= RP * kKiviMaxTail * sizeof(float) && sizeof(s_ql) >= RP * D * sizeof(float),
                "the fold buffers hold the tail's scratch");
  float* const s_tp = (float*)&s_qh[0][0][0];
  float* const s_to = (float*)&s_ql[0][0][0];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = sread(tid >> 6);
  const int kq = lane >> 4, n = lane & 15;
  const int B = p.B;
  const int HR = p.Hkv;
  const int G = p.G;

  build_segment_line<NW, kChunk>(p, s_prefix, s_len, s_wsum);
  zero_empty_splits<NT, TAIL>(p, s_prefix, s_tp, s_tm, s_tl, s_to);

  // ---- this workgroup's range of chunks on the line of (sequence, KV head) segments ---------------------
  const int C = HR * s_prefix[B];  // < 2^31, checked on the host
  if (C == 0) return;
  const int per = (C + (int)gridDim.x - 1) / (int)gridDim.x;
  const int g = blockIdx.x;
  const int c_begin = g * per;
  if (c_begin >= C) return;
  const int c_end = min(c_begin + per, C);
  int c = c_begin;

  int b;
  {
    int lo = 0, hi = B - 1;  // largest b with HR * prefix[b] <= c
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (HR * s_prefix[mid] <= c) lo = mid; else hi = mid - 1;
    }
    b = sread(lo);
  }
  int nb = sread(s_prefix[b + 1] - s_prefix[b]);
  int h, k;
  {
    const int r = c - HR * s_prefix[b];
    h = sread(r / nb);
    k = sread(r - h * nb);
  }

  // Chunks [k, k_end) of (b, h) form this piece: up to the split's end, the segment's end or the range's.
  auto piece_end = [&](int k0, int c0) {
    const int split_end = min((k0 / p.cps + 1) * p.cps, nb);
    const int seg_c0 = HR * s_prefix[b] + h * nb;
    return k0 + (min(c_end, seg_c0 + split_end) - c0);
  };

  // Chunks in flight per wave. A 4-bit chunk is 4 KiB: with one in flight, the chip's waves hold too few bytes
  // in flight to cover the memory latency, so each wave keeps two chunks going (a second register set; there
  // is room for it at up to 2 rows, 255 VGPRs).
  constexpr int DEPTH = (FMT == kKivi4 && RP <= 2) ? 2 : 1;
  float qf[CPL];
  KChunk<FMT, CPL> cr, cr2;
  const LaneOffsets lo = lane_offsets<FMT, RP, CPL>(p, lane);
  Head hd = head_of(p, b, h);
  int len = sread(s_len[b]);
  load_q_fold<RP, CPL>(p, b, h, lane, qf);
  // Two sets: the piece's first chunks of this wave go in flight, k0 + wave into cr, k0 + wave + NW into cr2.
  // Every load is issued (a wave without the chunk loads chunk k0 again) and in the loop's order (the grids
  // and K, then V; cr, then cr2): the compiler sizes the loop's waits for the loads on every path into it,
  // so a skipped or reordered load here would make every chunk of the loop wait for more of the loads behind.
  auto prime2 = [&](int k0, int k_end0) __attribute__((always_inline)) {
    const int c0 = k0 + wave < k_end0 ? k0 + wave : k0;
    const int c1 = k0 + wave + NW < k_end0 ? k0 + wave + NW : k0;
    issue_k<FMT, CPL>(p, hd, lo, c0, cr);
    __builtin_amdgcn_sched_barrier(0);
    issue_v<FMT, CPL>(p, hd, lo, c0, cr);
    __builtin_amdgcn_sched_barrier(0);
    issue_k<FMT, CPL>(p, hd, lo, c1, cr2);
    __builtin_amdgcn_sched_barrier(0);
    issue_v<FMT, CPL>(p, hd, lo, c1, cr2);
  };
  {
    const int k_end = piece_end(k, c);
    if constexpr (DEPTH == 2) {
      prime2(k, k_end);
    } else if (k + wave < k_end) {
      issue_k<FMT, CPL>(p, hd, lo, k + wave, cr);
      issue_v<FMT, CPL>(p, hd, lo, k + wave, cr);
    }
  }

  for (;;) {
    const int j_cur = k / p.cps;
    const int k_first = k;
    const int k_end = piece_end(k, c);
    const int seg_c0 = HR * s_prefix[b] + h * nb;
    const int split_end = min((j_cur + 1) * p.cps, nb);

    float m = kNegInf, l = 0.0f;
    f32x4 o[8], oz = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int mu = 0; mu < 8; ++mu) o[mu] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    T qh[4], ql[4];
    uint32_t kzp[4][4];
    float inv = 0.0f, zc = 0.0f;
    if constexpr (!F::kQuant) {  // unquantized: one fold serves the whole piece
      const uint32_t unit[CPL / 2] = {};
      fold<FMT, RP, CPL>(qf, unit, unit, p.qscale, lane, s_qh[wave], s_ql[wave], s_kz[wave], s_inv[wave], s_zc[wave]);
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      read_fold<FMT, RP>(n, kq, G, s_qh[wave], s_ql[wave], s_kz[wave], s_inv[wave], s_zc[wave], qh, ql, kzp, inv, zc);
    }

    if constexpr (DEPTH == 1) {
      // Chunks k + wave, k + wave + NW, ... of this piece: chunk kk is in flight on entry to its iteration;
      // the next chunk's grids and K go out once kk's scores are done, its V after kk's value products.
      for (int kk = k + wave; kk < k_end;) {
        const int kn = kk + NW;
        if constexpr (F::kQuant) {
          fold<FMT, RP, CPL>(qf, cr.gs, cr.gz, p.qscale, lane, s_qh[wave], s_ql[wave], s_kz[wave], s_inv[wave], s_zc[wave]);
          __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
          __builtin_amdgcn_wave_barrier();
          __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
          read_fold<FMT, RP>(n, kq, G, s_qh[wave], s_ql[wave], s_kz[wave], s_inv[wave], s_zc[wave], qh, ql, kzp, inv, zc);
        }
        compute<FMT, CPL>(cr, kk, len, lane, qh, ql, kzp, inv, zc, m, l, o, oz, [&]() {
          if (kn < k_end) issue_k<FMT, CPL>(p, hd, lo, kn, cr);
        });
        if (kn < k_end) issue_v<FMT, CPL>(p, hd, lo, kn, cr);
        kk = kn;
        if constexpr (F::kQuant) __builtin_amdgcn_wave_barrier();  // the LDS fold buffers are rewritten next
      }
    } else {
      // The same with two sets: chunk kk is in flight in set cur on entry to its step, and chunk kk + 2 NW
      // takes the set over (past the piece, chunk kk again, as in prime2). The sets alternate, cr first on
      // every piece: pairs, then an odd last chunk. (A loop that may leave between its two steps makes the
      // compiler assume a path on which cr2's loads were not issued, and wait for them before every pair.)
      auto step = [&](KChunk<FMT, CPL>& cur, int kk) __attribute__((always_inline)) {
        const int kn = kk + 2 * NW;
        const int kl = kn < k_end ? kn : kk;
        fold<FMT, RP, CPL>(qf, cur.gs, cur.gz, p.qscale, lane, s_qh[wave], s_ql[wave], s_kz[wave], s_inv[wave], s_zc[wave]);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        read_fold<FMT, RP>(n, kq, G, s_qh[wave], s_ql[wave], s_kz[wave], s_inv[wave], s_zc[wave], qh, ql, kzp, inv, zc);
        compute<FMT, CPL>(cur, kk, len, lane, qh, ql, kzp, inv, zc, m, l, o, oz, [&]() { issue_k<FMT, CPL>(p, hd, lo, kl, cur); });
        issue_v<FMT, CPL>(p, hd, lo, kl, cur);
        __builtin_amdgcn_wave_barrier();  // the LDS fold buffers are rewritten next
      };
      const int first = k + wave;
      const int cnt = first < k_end ? (k_end - first + NW - 1) / NW : 0;
      int kk = first;
      for (int i = 1; i < cnt; i += 2, kk += 2 * NW) {
        step(cr, kk);
        step(cr2, kk + NW);
      }
      if (cnt & 1) step(cr, kk);
    }

    // The next piece (if any): its first chunk (and q rows, for a new KV head) go in flight now.
    const int b_cur = b, h_cur = h;
    const int c_piece = c;
    const int c_next = c + (k_end - k);
    if (c_next < c_end) {
      if (k_end < nb) {
        k = k_end;  // the same (sequence, KV head): the next split
      } else {
        ++h;
        k = 0;
        if (h == HR) {
          h = 0;
          do {
            ++b;
          } while (s_prefix[b + 1] == s_prefix[b]);
          b = sread(b);
          nb = sread(s_prefix[b + 1] - s_prefix[b]);
        }
        len = sread(s_len[b]);
        hd = head_of(p, b, h);
        load_q_fold<RP, CPL>(p, b, h, lane, qf);
      }
      const int k_next_end = piece_end(k, c_next);
      if constexpr (DEPTH == 2) {
        prime2(k, k_next_end);
      } else if (k + wave < k_next_end) {
        issue_k<FMT, CPL>(p, hd, lo, k + wave, cr);
        issue_v<FMT, CPL>(p, hd, lo, k + wave, cr);
      }
    }

    // This wave's state of row n: the value zero points taken out, the four lanes' weight sums added,
    // stored for the workgroup merge.
    if constexpr (F::template kZeroFold<CPL>) value_zero_out<FMT>(kq, oz, o);
    l = sum_xor<32>(sum_xor<16>(l));
    if (n < RP) {
      if (kq == 0) {
        s_m[wave][n] = m;
        s_l[wave][n] = l;
      }
#pragma unroll
      for (int mu = 0; mu < 8; ++mu) {
#pragma unroll
        for (int i = 0; i < 4; ++i) s_o[wave][n][out_channel<FMT>(kq, i, mu)] = o[mu][i];
      }
    }
    __syncthreads();
    // The piece that starts the segment also holds the tail's tokens (one split: the tail goes with it).
    const bool with_tail = TAIL && k_first == 0;
    if (with_tail) tail_state<NT>(p, b_cur, h_cur, s_tp, s_tm, s_tl, s_to);

    // ---- merge the waves; write the split's result, or this piece's partial ---------------------------
    const int seg = (b_cur * HR + h_cur) * p.S + j_cur;
    const int sc0 = seg_c0 + j_cur * p.cps;
    const int g_first = sc0 / per;
    const int g_last = (seg_c0 + split_end - 1) / per;
    const bool whole = g_first == g_last;
    const int slot = c_piece == c_begin ? 2 * g : 2 * g + 1;
    for (int idx = tid; idx < RP * D; idx += NT) {
      const int r = idx / D;
      const int ch = idx - r * D;
      if (r >= G) continue;
      float M = kNegInf;
#pragma unroll
      for (int w = 0; w < NW; ++w) M = fmaxf(M, s_m[w][r]);
      if (with_tail) M = fmaxf(M, s_tm[r]);
      const float mu = M == kNegInf ? 0.0f : M;
      float L = 0.0f, A = 0.0f;
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        const float lw = s_l[w][r];
        const float e = lw > 0.0f ? fast_exp2(s_m[w][r] - mu) : 0.0f;
        L += lw * e;
        A += lw > 0.0f ? s_o[w][r][ch] * e : 0.0f;
      }
      if (with_tail) {
        const float e = fast_exp2(s_tm[r] - mu);
        L += s_tl[r] * e;
        A += s_to[r * D + ch] * e;
      }
      const float out = L > 0.0f ? A / L : 0.0f;
      const float lse2 = L > 0.0f ? M - kBias + __log2f(L) : kNegInf;
      if (whole) {
        const int hq = h_cur * G + r;
        p.out[out_index(p, b_cur, hq, j_cur) + ch] = out;
        if (ch == 0) p.lse[lse_index(p, b_cur, hq, j_cur)] = L > 0.0f ? lse2 * kLn2 : kNegInf;
      } else {
        ws_store(p.ws_out + (slot * G + r) * D + ch, out);
        if (ch == 0) ws_store(p.ws_lse + slot * G + r, lse2);
      }
    }
    if (!whole) {
      ws_publish();
      __syncthreads();
      arrive_and_combine<NT>(p, seg, b_cur, h_cur, j_cur, sc0, per, g_first, g_last - g_first + 1, tid, &s_last);
    }
    if (c_next >= c_end) break;
    c = c_next;
    __syncthreads();  // the LDS merge buffers are rewritten by the next piece
  }
}

template <int FMT, bool TAIL>
static hipError_t launch_fmt(const KiviParams& p, hipStream_t stream) {
  dim3 grid(p.grid), block(kDecodeWaves * 64);
  const size_t lds = (size_t)(2 * p.B + 1) * sizeof(int);
  if (p.G <= 2) hipLaunchKernelGGL((kivi_decode_kernel<FMT, 2, TAIL>), grid, block, lds, stream, p);
  else if (p.G <= 4) hipLaunchKernelGGL((kivi_decode_kernel<FMT, 4, TAIL>), grid, block, lds, stream, p);
  else if (p.G <= 8) hipLaunchKernelGGL((kivi_decode_kernel<FMT, 8, TAIL>), grid, block, lds, stream, p);
  else hipLaunchKernelGGL((kivi_decode_kernel<FMT, 16, TAIL>), grid, block, lds, stream, p);
  return hipGetLastError();
}

// Calls with a full-precision tail run their own instantiation: the tail's merge costs the others nothing.
template <int FMT>
static hipError_t launch_fmt(const KiviParams& p, hipStream_t stream) {
  return p.tail_len > 0 ? launch_fmt<FMT, true>(p, stream) : launch_fmt<FMT, false>(p, stream);
}

hipError_t launch_kivi(const KiviParams& p, int fmt, hipStream_t stream) {
  if (p.G < 1 || p.G > 16) return hipErrorInvalidValue;
  switch (fmt) {
    case kKivi4: return launch_fmt<kKivi4>(p, stream);
    case kKivi8: return launch_fmt<kKivi8>(p, stream);
    case kKiviF16: return launch_fmt<kKiviF16>(p, stream);
    case kKiviBf16: return launch_fmt<kKiviBf16>(p, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace bpt
