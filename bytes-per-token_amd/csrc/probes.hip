// Conversion checks and bandwidth probes.
//
// The read probe is the MI355X counterpart of fastserve hw/bandwidth.py:56-89 (a streaming read that writes
// one value per workgroup): it measures the achievable HBM read rate that "% of measured peak" is quoted
// against, and evicts L2 and the Infinity Cache before cold timings. The page-read probe fetches exactly the
// K / V rows (and per-token scales) a decode call reads, through the same block table, with no attention
// math: the read floor of that call's access pattern. The copy probe moves a known number of bytes so
// rocprof's FETCH_SIZE / WRITE_SIZE counters can be calibrated.
#include "decode_common.h"

namespace bpt {

// out[i] = decoded code i. The code is replicated into all four bytes of a dword so every byte position
// and both halves of the packed converter are exercised; disagreeing positions report a sentinel.
__global__ void fp8_table_kernel(float* out) {
  const uint32_t c = threadIdx.x & 0xffu;
  const uint32_t w = c | (c << 8) | (c << 16) | (c << 24);
  float f[4];
  fp8x4_to_f32(w, f);
  bool same = true;
#pragma unroll
  for (int j = 1; j < 4; ++j) same = same && (__float_as_uint(f[j]) == __float_as_uint(f[0]));
  out[c] = same ? f[0] : -12345.0f;
}

__global__ void fp8_encode_kernel(const float* x, float scale, uint8_t* out, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  out[i] = (uint8_t)f32_to_fp8(clamp_fp8_range(__fdiv_rn(x[i], scale)));
}

constexpr int kProbeThreads = 256;
constexpr int kProbeGroupsPerCu = 8;
constexpr int kProbeCus = 256;

__global__ __launch_bounds__(kProbeThreads) void read_probe_kernel(const U4* buf, int64_t n16, float* partial) {
  const int64_t stride = (int64_t)gridDim.x * kProbeThreads;
  int64_t i = (int64_t)blockIdx.x * kProbeThreads + threadIdx.x;
  uint32_t a0 = 0, a1 = 0, a2 = 0, a3 = 0;
  for (; i + 3 * stride < n16; i += 4 * stride) {
    const U4 x0 = load16((const uint8_t*)(buf + i));
    const U4 x1 = load16((const uint8_t*)(buf + i + stride));
    const U4 x2 = load16((const uint8_t*)(buf + i + 2 * stride));
    const U4 x3 = load16((const uint8_t*)(buf + i + 3 * stride));
    a0 += x0.x ^ x0.y ^ x0.z ^ x0.w;
    a1 += x1.x ^ x1.y ^ x1.z ^ x1.w;
    a2 += x2.x ^ x2.y ^ x2.z ^ x2.w;
    a3 += x3.x ^ x3.y ^ x3.z ^ x3.w;
  }
  for (; i < n16; i += stride) {
    const U4 x0 = load16((const uint8_t*)(buf + i));
    a0 += x0.x ^ x0.y ^ x0.z ^ x0.w;
  }
  uint32_t a = a0 + a1 + a2 + a3;
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) a += (uint32_t)__shfl_xor((int)a, m, 64);
  __shared__ uint32_t s[kProbeThreads / 64];
  if ((threadIdx.x & 63) == 0) s[threadIdx.x >> 6] = a;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t t = 0;
    for (int w = 0; w < kProbeThreads / 64; ++w) t += s[w];
    partial[blockIdx.x] = (float)t;
  }
}

// One workgroup per (sequence, KV head, span of kPageReadSpan tokens); a token row is row_bytes / 16 lanes of
// one 16-byte load each for K and for V; rows past the sequence's length are not read.
constexpr int kPageReadSpan = 256;

__global__ __launch_bounds__(kProbeThreads) void page_read_probe_kernel(const DecodeParams p, int lanes_per_row,
                                                                       int spans, int with_scales, float* partial) {
  const int span = blockIdx.x % spans;
  const int bh = blockIdx.x / spans;
  const int h = bh % p.Hkv, b = bh / p.Hkv;
  const int len = min(max((p.lens ? p.lens[b] : p.len_cap) - p.len_offset, 0), p.len_cap);
  const int t0 = span * kPageReadSpan;
  const int rows_per_pass = kProbeThreads / lanes_per_row;
  const int r = threadIdx.x / lanes_per_row, part = threadIdx.x - r * lanes_per_row;
  const int32_t* table = (const int32_t*)p.table;
  uint32_t a = 0;
  const int n = min(kPageReadSpan, len - t0);
#pragma unroll 8
  for (int i = r; i < n; i += rows_per_pass) {
    const int t = t0 + i;
    int e = table[table_word(p, b, t >> p.logP)];
    e = e < 0 ? 0 : (e >= p.num_blocks ? p.num_blocks - 1 : e);
    const int within = t & (p.P - 1);
    const int64_t off = (int64_t)e * p.kv_sblk + (int64_t)within * p.kv_stok + (int64_t)h * p.kv_shead + part * 16;
    const U4 k = load16(p.k + off);
    const U4 v = load16(p.v + off);
    a += (k.x ^ k.y ^ k.z ^ k.w) + (v.x ^ v.y ^ v.z ^ v.w);
    if (with_scales && part == 0) {
      const int64_t so = (int64_t)e * p.sc_sblk + (int64_t)within * p.sc_stok + (int64_t)h * p.sc_shead;
      a += __float_as_uint(p.ks[so]) ^ __float_as_uint(p.vs[so]);
    }
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) a += (uint32_t)__shfl_xor((int)a, m, 64);
  __shared__ uint32_t s[kProbeThreads / 64];
  if ((threadIdx.x & 63) == 0) s[threadIdx.x >> 6] = a;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t t = 0;
    for (int w = 0; w < kProbeThreads / 64; ++w) t += s[w];
    partial[blockIdx.x] = (float)t;
  }
}

int64_t page_read_probe_groups(int B, int Hkv, int len_cap) {
  return (int64_t)B * Hkv * ((len_cap + kPageReadSpan - 1) / kPageReadSpan);
}

hipError_t launch_page_read_probe(const DecodeParams& p, int row_bytes, bool with_scales, float* partial,
                                  hipStream_t stream, const LaunchEvents& ev) {
  const int spans = (p.len_cap + kPageReadSpan - 1) / kPageReadSpan;
  const int64_t g = page_read_probe_groups(p.B, p.Hkv, p.len_cap);
  if (g == 0) return hipSuccess;
  launch_kernel(page_read_probe_kernel, dim3((unsigned)g), dim3(kProbeThreads), 0, stream, ev, p, row_bytes / 16,
                spans, (int)with_scales, partial);
  return hipGetLastError();
}

__global__ __launch_bounds__(kProbeThreads) void copy_probe_kernel(U4* dst, const U4* src, int64_t n16) {
  const int64_t stride = (int64_t)gridDim.x * kProbeThreads;
  for (int64_t i = (int64_t)blockIdx.x * kProbeThreads + threadIdx.x; i < n16; i += stride) dst[i] = src[i];
}

hipError_t launch_fp8_table(float* out, hipStream_t stream) {
  hipLaunchKernelGGL(fp8_table_kernel, dim3(1), dim3(256), 0, stream, out);
  return hipGetLastError();
}

hipError_t launch_fp8_encode(const float* x, float scale, uint8_t* out, int64_t n, hipStream_t stream) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(fp8_encode_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, x, scale, out, n);
  return hipGetLastError();
}

int64_t read_probe_groups(uint64_t bytes) {
  const int64_t n16 = (int64_t)(bytes / 16);
  int64_t g = (n16 + kProbeThreads - 1) / kProbeThreads;
  const int64_t cap = (int64_t)kProbeCus * kProbeGroupsPerCu;
  return g < 1 ? 1 : (g > cap ? cap : g);
}

hipError_t launch_read_probe(const void* buf, uint64_t bytes, float* partial, hipStream_t stream,
                             const LaunchEvents& ev) {
  const int64_t g = read_probe_groups(bytes);
  launch_kernel(read_probe_kernel, dim3((unsigned)g), dim3(kProbeThreads), 0, stream, ev, (const U4*)buf,
                (int64_t)(bytes / 16), partial);
  return hipGetLastError();
}

hipError_t launch_copy_probe(void* dst, const void* src, uint64_t bytes, hipStream_t stream) {
  const int64_t g = read_probe_groups(bytes);
  hipLaunchKernelGGL(copy_probe_kernel, dim3((unsigned)g), dim3(kProbeThreads), 0, stream, (U4*)dst, (const U4*)src,
                     (int64_t)(bytes / 16));
  return hipGetLastError();
}

}  // namespace bpt
