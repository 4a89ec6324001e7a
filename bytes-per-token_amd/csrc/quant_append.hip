// Quantize-on-write: new K/V rows [B, Q, Hkv, D] -> their (page, slot) in the paged pools.
//
// Follows fastserve engine/kv_cache.py:158-161 (scatter by write_blocks / write_offsets) with the
// quantizers of kv/quant.py:44-45 (FP8: clamp to +-448, cast to e4m3fn, round to nearest even) and
// quant/w8a8.py:55-74 / kernels/reference.py:44-55 (INT8: s = max(amax / 127, 1e-12),
// code = clamp(rint(x / s), -128, 127)). Divisions are IEEE round-to-nearest (__fdiv_rn), so codes and
// scales are bit-identical to the float32 formulas.
//
// Half a wave (32 lanes) per (row, K-or-V); each lane holds D / 32 consecutive channels, the row's amax
// is a 32-lane butterfly.
#include "bpt_device.h"
#include "bpt_internal.h"

namespace bpt {

template <int KV, int SK, int D>
__global__ __launch_bounds__(256) void quant_append_kernel(const AppendParams p) {
  constexpr int PER = D / 32;
  const int lane = threadIdx.x & 31;
  const int64_t task = (int64_t)blockIdx.x * 8 + (threadIdx.x >> 5);
  const int64_t ntask = (int64_t)p.B * p.Q * p.Hkv * 2;
  if (task >= ntask) return;  // whole half-wave exits together
  const int which = (int)(task & 1);  // 0 = K, 1 = V
  const int64_t row = task >> 1;
  const int h = (int)(row % p.Hkv);
  const int64_t bq = row / p.Hkv;
  const int qi = (int)(bq % p.Q);
  const int b = (int)(bq / p.Q);

  const int64_t si = (int64_t)b * p.s_sb + (int64_t)qi * p.s_sq;
  const int64_t blk = load_index(p.blocks, si, p.slot_i64 != 0);
  const int64_t off = load_index(p.offsets, si, p.slot_i64 != 0);
  if (blk < 0 || blk >= p.num_blocks || off < 0 || off >= p.P) return;
  if (p.in_place && !slot_is_token(p.table, (int64_t)b * p.table_sb, p.table_i64 != 0, p.max_blocks, p.num_blocks,
                                   p.logP, (int64_t)p.lens[b] - p.Q + qi, blk, off))
    return;

  const void* src = which ? p.v : p.k;
  const int64_t xi = (int64_t)b * p.n_sb + (int64_t)qi * p.n_sq + (int64_t)h * p.n_sh + lane * PER;
  float x[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) x[j] = load_float(src, xi + j, p.src_dtype);

  uint8_t* cache = which ? p.vc : p.kc;
  const int64_t ci = blk * p.kv_sblk + off * p.kv_stok + (int64_t)h * p.kv_shead;

  if constexpr (KV == kKvBf16) {
    uint16_t* dst = (uint16_t*)(cache + ci) + lane * PER;
#pragma unroll
    for (int j = 0; j < PER; ++j) dst[j] = f32_to_bf16_bits(x[j]);
    return;
  } else {
    float* scales = which ? p.vs : p.ks;
    float s;
    if constexpr (SK == kScaleHead) {
      s = scales[h];
    } else {
      float amax = 0.0f;
#pragma unroll
      for (int j = 0; j < PER; ++j) amax = fmaxf(amax, fabsf(x[j]));
#pragma unroll
      for (int m = 16; m >= 1; m >>= 1) amax = fmaxf(amax, __shfl_xor(amax, m, 32));
      const float qmax = KV == kKvFp8 ? 448.0f : 127.0f;
      s = __fdiv_rn(amax, qmax);
      s = s < 1e-12f ? 1e-12f : s;
      if (lane == 0) scales[blk * p.sc_sblk + off * p.sc_stok + (int64_t)h * p.sc_shead] = s;
    }
    uint8_t* dst = cache + ci + lane * PER;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const float y = __fdiv_rn(x[j], s);
      uint32_t code;
      if constexpr (KV == kKvFp8) {
        code = f32_to_fp8(clamp_fp8_range(y));
      } else {
        float r = rintf(y);
        r = r > 127.0f ? 127.0f : (r < -128.0f ? -128.0f : r);
        code = (uint32_t)(int32_t)r & 0xffu;
      }
      dst[j] = (uint8_t)code;
    }
  }
}

template <int KV, int SK>
static hipError_t launch_append_t(const AppendParams& p, int head_dim, hipStream_t stream) {
  const int64_t ntask = (int64_t)p.B * p.Q * p.Hkv * 2;
  dim3 grid((unsigned)((ntask + 7) / 8));
  switch (head_dim) {
    case 64: hipLaunchKernelGGL((quant_append_kernel<KV, SK, 64>), grid, dim3(256), 0, stream, p); break;
    case 128: hipLaunchKernelGGL((quant_append_kernel<KV, SK, 128>), grid, dim3(256), 0, stream, p); break;
    case 256: hipLaunchKernelGGL((quant_append_kernel<KV, SK, 256>), grid, dim3(256), 0, stream, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_append(const AppendParams& p, int kv_dtype, int scale_kind, int head_dim, hipStream_t stream) {
  if (kv_dtype == kKvBf16) return launch_append_t<kKvBf16, kScaleNone>(p, head_dim, stream);
  if (kv_dtype == kKvFp8 && scale_kind == kScaleHead) return launch_append_t<kKvFp8, kScaleHead>(p, head_dim, stream);
  if (kv_dtype == kKvFp8 && scale_kind == kScaleTokenHead)
    return launch_append_t<kKvFp8, kScaleTokenHead>(p, head_dim, stream);
  if (kv_dtype == kKvInt8 && scale_kind == kScaleHead) return launch_append_t<kKvInt8, kScaleHead>(p, head_dim, stream);
  if (kv_dtype == kKvInt8 && scale_kind == kScaleTokenHead)
    return launch_append_t<kKvInt8, kScaleTokenHead>(p, head_dim, stream);
  return hipErrorInvalidValue;
}

}  // namespace bpt
