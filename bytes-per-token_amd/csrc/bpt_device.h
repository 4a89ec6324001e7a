// Device helpers for the gfx950 kernels: element conversions, 8-lane DPP reductions, 16-byte loads.
//
// FP8 here is OCP e4m3fn (sign, 4 exponent bits with bias 7, 3 mantissa bits; no infinities; 0x7F and
// 0xFF are NaN; largest finite value 448). gfx950's v_cvt_pk_f32_fp8 / v_cvt_pk_fp8_f32 use this
// encoding (gfx942 used the FNUZ variant instead); the 256-code decode table and the encoder are checked
// against torch.float8_e4m3fn on the GPU.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace bpt {

typedef float float2_v __attribute__((ext_vector_type(2)));

constexpr int kKvBf16 = 0;
constexpr int kKvFp8 = 1;
constexpr int kKvInt8 = 2;

constexpr int kScaleNone = 0;
constexpr int kScaleHead = 1;
constexpr int kScaleTokenHead = 2;

constexpr int kFBf16 = 0;
constexpr int kFF16 = 1;
constexpr int kFF32 = 2;

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegInf = -__builtin_huge_valf();

// ---- floats ------------------------------------------------------------------------------------------

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) { return __uint_as_float(bits16 << 16); }

// Round-to-nearest-even float -> bfloat16 bits, quiet NaN kept (the rounding torch's .to(bfloat16) does).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float load_float(const void* base, int64_t idx, int dtype) {
  if (dtype == kFBf16) return bf16_bits_to_f32(((const uint16_t*)base)[idx]);
  if (dtype == kFF16) return (float)((const _Float16*)base)[idx];
  return ((const float*)base)[idx];
}

__device__ __forceinline__ void store_float(void* base, int64_t idx, int dtype, float x) {
  if (dtype == kFBf16)
    ((uint16_t*)base)[idx] = f32_to_bf16_bits(x);
  else if (dtype == kFF16)
    ((_Float16*)base)[idx] = (_Float16)x;
  else
    ((float*)base)[idx] = x;
}

// ---- FP8 e4m3fn --------------------------------------------------------------------------------------

// Four e4m3fn codes packed in a dword (byte j = element j) -> four floats, exact.
__device__ __forceinline__ void fp8x4_to_f32(uint32_t w, float* out) {
  float2_v lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false);
  float2_v hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true);
  out[0] = lo.x;
  out[1] = lo.y;
  out[2] = hi.x;
  out[3] = hi.y;
}

// clamp(x, -448, 448) with NaN passed through, as torch.clamp does (fminf/fmaxf would drop the NaN).
__device__ __forceinline__ float clamp_fp8_range(float x) {
  x = x > 448.0f ? 448.0f : x;
  x = x < -448.0f ? -448.0f : x;
  return x;
}

// One float in [-448, 448] (or NaN) -> e4m3fn code, round to nearest even. NaN -> 0x7F with the input's
// sign, which is what torch's float8_e4m3fn cast produces.
__device__ __forceinline__ uint32_t f32_to_fp8(float x) {
  if (x != x) return 0x7fu | ((__float_as_uint(x) >> 24) & 0x80u);
  int packed = __builtin_amdgcn_cvt_pk_fp8_f32(x, 0.0f, 0, false);
  return (uint32_t)packed & 0xffu;
}

// ---- cross-lane --------------------------------------------------------------------------------------

template <int CTRL>
__device__ __forceinline__ float dpp_mov(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xf, 0xf, true));
}

constexpr int kDppXor1 = 0xB1;         // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;         // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;  // lane i <-> 7 - i inside each group of 8
constexpr int kDppRowMirror = 0x140;   // lane i <-> 15 - i inside each row of 16

// Sum over aligned groups of N lanes (N = 4, 8 or 16), every lane of a group left holding the sum.
template <int N>
__device__ __forceinline__ float group_sum(float x) {
  static_assert(N == 4 || N == 8 || N == 16, "group of 4, 8 or 16 lanes");
  x += dpp_mov<kDppXor1>(x);
  x += dpp_mov<kDppXor2>(x);
  if (N >= 8) x += dpp_mov<kDppHalfMirror>(x);
  if (N >= 16) x += dpp_mov<kDppRowMirror>(x);
  return x;
}

__device__ __forceinline__ float shfl_xor_f(float x, int mask) { return __shfl_xor(x, mask, 64); }

// Lane l's value and lane (l ^ 16)'s (XOR16) or (l ^ 32)'s (XOR32), in some order, in every lane: gfx950's
// v_permlane16_swap / v_permlane32_swap, VALU instructions with no LDS round trip (unlike __shfl_xor's
// ds_bpermute). Both lanes of a pair get the same two values, so max and sum agree between them.
template <int XOR>
__device__ __forceinline__ void lane_pair(float x, float& a, float& b) {
  static_assert(XOR == 16 || XOR == 32, "rows of 16 or halves of 32");
  const unsigned u = __float_as_uint(x);
  if constexpr (XOR == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    a = __uint_as_float(r[0]);
    b = __uint_as_float(r[1]);
  } else {
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    a = __uint_as_float(r[0]);
    b = __uint_as_float(r[1]);
  }
}
template <int XOR>
__device__ __forceinline__ float max_xor(float x) {
  float a, b;
  lane_pair<XOR>(x, a, b);
  return fmaxf(a, b);
}
template <int XOR>
__device__ __forceinline__ float sum_xor(float x) {
  float a, b;
  lane_pair<XOR>(x, a, b);
  return a + b;
}

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) x = fmaxf(x, shfl_xor_f(x, m));
  return x;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// rint of the IEEE quotient x / s (torch's round(x / s)), given inv = v_rcp_f32(s), s a positive normal float.
// q = x * inv is within 2^-22 |x / s| of x / s (rcp: 1 ulp, 2^-23 relative; the product: half an ulp) and the
// IEEE quotient within 2^-24 |x / s|, so both lie strictly on the same side of every half-integer farther
// than 2^-21 |q| from q, and then round to the same integer. Quotients closer to a half-integer than
// 2^-20 |q| (a few in ten thousand of random values) take the IEEE division; NaN and infinite q keep q, as
// the division would give.
__device__ __forceinline__ float rint_quotient(float x, float s, float inv) {
  const float q = x * inv;
  float n = rintf(q);
  if (0.5f - fabsf(q - n) <= fabsf(q) * 0x1p-20f) n = rintf(__fdiv_rn(x, s));
  return n;
}

// ---- memory ------------------------------------------------------------------------------------------

struct alignas(16) U4 {
  uint32_t x, y, z, w;
};

__device__ __forceinline__ U4 load16(const uint8_t* p) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  u32x4 v = __builtin_nontemporal_load((const u32x4*)p);
  return U4{v.x, v.y, v.z, v.w};
}

__device__ __forceinline__ int64_t load_index(const void* base, int64_t idx, bool i64) {
  return i64 ? ((const int64_t*)base)[idx] : (int64_t)((const int32_t*)base)[idx];
}

// Whether pool slot (blk, off) is where the paged decode reads token `tok` of the sequence whose block-table
// row starts at entry `row_entry`: blk is the token's block-table entry clamped into the pool (as the decode
// kernels clamp it) and off its offset in the page. A token before the sequence or past the table's width has
// no slot. Int64 tables are read by their low word, as the decode kernels read them.
__device__ __forceinline__ bool slot_is_token(const void* table, int64_t row_entry, bool table_i64, int max_blocks,
                                              int num_blocks, int logP, int64_t tok, int64_t blk, int64_t off) {
  if (tok < 0 || (tok >> logP) >= max_blocks) return false;
  int e = ((const int32_t*)table)[(row_entry + (tok >> logP)) << (table_i64 ? 1 : 0)];
  e = e < 0 ? 0 : (e >= num_blocks ? num_blocks - 1 : e);
  return blk == e && off == (tok & ((int64_t(1) << logP) - 1));
}

}  // namespace bpt
