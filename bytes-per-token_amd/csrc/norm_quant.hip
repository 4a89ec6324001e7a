// RMSNorm fused with per-token INT8 quantization (fastserve kernels/norm_quant.py:43-69, defined by
// kernels/reference.py:44-55): for every row x of [rows, d],
//   y = x * rsqrt(mean(x^2) + eps) * weight,  scale = max(max|y| / 127, 1e-12),
//   codes = clamp(rint(y / scale), -128, 127)
// in float32. The row is read once: one wave per row holds it and the weight in registers (VEC elements per
// lane per step, IT steps), both requested up front; the sum of squares and the largest |y| are wave
// reductions. Rows wider than the register copy (IT = 0, beyond 4096 elements) are streamed three times
// instead (the re-reads hit L2). HBM-bound: 2d (16-bit input) bytes read and d + 4 written per row.
#include "bpt_device.h"
#include "bpt_internal.h"

namespace bpt {

namespace {

constexpr int kRowsPerGroup = 4;  // one wave per row

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) x += shfl_xor_f(x, m);
  return x;
}

// VEC consecutive elements of a row starting at element e (VEC = 8: one 16-byte load for 16-bit types, two
// for float32; the caller guarantees alignment and e + 8 <= d; VEC = 1: one element, 0 past d).
template <int VEC>
__device__ __forceinline__ void load_vec(const void* base, int64_t idx, int dtype, int e, int d, float (&v)[VEC]) {
  if constexpr (VEC == 8) {
    if (dtype == kFF32) {
      const U4 a = *(const U4*)((const float*)base + idx);
      const U4 b = *(const U4*)((const float*)base + idx + 4);
      const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = __uint_as_float(w[j]);
    } else {
      const U4 a = *(const U4*)((const uint16_t*)base + idx);
      const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (dtype == kFBf16) {
          v[2 * j] = __uint_as_float(w[j] << 16);
          v[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
        } else {
          v[2 * j] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[j] & 0xffffu));
          v[2 * j + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[j] >> 16));
        }
      }
    }
  } else {
    v[0] = e < d ? load_float(base, idx, dtype) : 0.0f;
  }
}

// Codes of VEC elements of one row, written at element e; inv = v_rcp_f32(scale).
template <int VEC>
__device__ __forceinline__ void store_codes(int8_t* row, int e, int d, const float (&y)[VEC], float scale,
                                            float inv) {
  uint32_t c[VEC];
#pragma unroll
  for (int j = 0; j < VEC; ++j) {
    float q = rint_quotient(y[j], scale, inv);  // rint of the IEEE quotient, as torch's round(y / scale)
    q = q > 127.0f ? 127.0f : (q < -128.0f ? -128.0f : q);
    c[j] = (uint32_t)(int)q & 0xffu;
  }
  if constexpr (VEC == 8) {
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    // Written once: a nontemporal store (32768 x 2048: 54.3 -> 52.6 us; 4096 x 2048: 12.9 -> 11.8 us).
    __builtin_nontemporal_store(u32x2{c[0] | (c[1] << 8) | (c[2] << 16) | (c[3] << 24),
                                      c[4] | (c[5] << 8) | (c[6] << 16) | (c[7] << 24)},
                                (u32x2*)(row + e));
  } else {
    if (e < d) row[e] = (int8_t)c[0];
  }
}

}  // namespace

// IT > 0: the row (at most IT * 64 * VEC elements) stays in registers; IT == 0: any width, streamed.
template <int VEC, int IT>
__global__ __launch_bounds__(kRowsPerGroup * 64) void rms_norm_int8_kernel(const NormQuantParams p) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * kRowsPerGroup + (int)(threadIdx.x >> 6);
  if (row >= p.rows) return;  // the whole wave leaves
  const int d = p.d;
  const int64_t xr = (int64_t)row * p.x_rs;
  constexpr int STEP = 64 * VEC;
  int8_t* crow = p.codes + (int64_t)row * p.c_rs;

  if constexpr (IT > 0) {
    float v[IT][VEC], w[IT][VEC];  // the row and the weight, both requested before any reduction
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      const int e = it * STEP + lane * VEC;
      if (VEC == 1 || e < d) {
        load_vec<VEC>(p.x, xr + e, p.x_dtype, e, d, v[it]);
        load_vec<VEC>(p.w, e, p.w_dtype, e, d, w[it]);
      } else {
#pragma unroll
        for (int j = 0; j < VEC; ++j) v[it][j] = w[it][j] = 0.0f;
      }
    }
    float ss = 0.0f;
#pragma unroll
    for (int it = 0; it < IT; ++it) {
#pragma unroll
      for (int j = 0; j < VEC; ++j) ss = fmaf(v[it][j], v[it][j], ss);
    }
    ss = wave_sum(ss);
    const float r = __frsqrt_rn(__fdiv_rn(ss, (float)d) + p.eps);
    float amax = 0.0f;
#pragma unroll
    for (int it = 0; it < IT; ++it) {
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        v[it][j] = (v[it][j] * r) * w[it][j];
        amax = fmaxf(amax, fabsf(v[it][j]));
      }
    }
    amax = wave_max(amax);
    const float scale = fmaxf(__fdiv_rn(amax, 127.0f), 1e-12f);
    const float inv = __builtin_amdgcn_rcpf(scale);
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      const int e = it * STEP + lane * VEC;
      if (VEC == 1 || e < d) store_codes<VEC>(crow, e, d, v[it], scale, inv);
    }
    if (lane == 0) p.scale[row] = scale;
  } else {
    float ss = 0.0f;
    for (int e = lane * VEC; e < d; e += STEP) {
      float v[VEC];
      load_vec<VEC>(p.x, xr + e, p.x_dtype, e, d, v);
#pragma unroll
      for (int j = 0; j < VEC; ++j) ss = fmaf(v[j], v[j], ss);
    }
    ss = wave_sum(ss);
    const float r = __frsqrt_rn(__fdiv_rn(ss, (float)d) + p.eps);
    float amax = 0.0f;
    for (int e = lane * VEC; e < d; e += STEP) {
      float v[VEC], w[VEC];
      load_vec<VEC>(p.x, xr + e, p.x_dtype, e, d, v);
      load_vec<VEC>(p.w, e, p.w_dtype, e, d, w);
#pragma unroll
      for (int j = 0; j < VEC; ++j) amax = fmaxf(amax, fabsf((v[j] * r) * w[j]));
    }
    amax = wave_max(amax);
    const float scale = fmaxf(__fdiv_rn(amax, 127.0f), 1e-12f);
    const float inv = __builtin_amdgcn_rcpf(scale);
    for (int e = lane * VEC; e < d; e += STEP) {
      float v[VEC], w[VEC];
      load_vec<VEC>(p.x, xr + e, p.x_dtype, e, d, v);
      load_vec<VEC>(p.w, e, p.w_dtype, e, d, w);
#pragma unroll
      for (int j = 0; j < VEC; ++j) v[j] = (v[j] * r) * w[j];
      store_codes<VEC>(crow, e, d, v, scale, inv);
    }
    if (lane == 0) p.scale[row] = scale;
  }
}

template <int VEC>
static hipError_t launch_vec(const NormQuantParams& p, hipStream_t stream) {
  dim3 grid((p.rows + kRowsPerGroup - 1) / kRowsPerGroup), block(kRowsPerGroup * 64);
  const int steps = (p.d + 64 * VEC - 1) / (64 * VEC);
  if (steps <= 1) hipLaunchKernelGGL((rms_norm_int8_kernel<VEC, 1>), grid, block, 0, stream, p);
  else if (steps <= 2) hipLaunchKernelGGL((rms_norm_int8_kernel<VEC, 2>), grid, block, 0, stream, p);
  else if (steps <= 4) hipLaunchKernelGGL((rms_norm_int8_kernel<VEC, 4>), grid, block, 0, stream, p);
  else if (steps <= 8) hipLaunchKernelGGL((rms_norm_int8_kernel<VEC, 8>), grid, block, 0, stream, p);
  else hipLaunchKernelGGL((rms_norm_int8_kernel<VEC, 0>), grid, block, 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_norm_quant(const NormQuantParams& p, bool vec8, hipStream_t stream) {
  if (p.rows == 0) return hipSuccess;
  return vec8 ? launch_vec<8>(p, stream) : launch_vec<1>(p, stream);
}

}  // namespace bpt
