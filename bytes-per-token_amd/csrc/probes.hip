// Conversion checks and bandwidth probes.
//
// The read probe is the MI355X counterpart of fastserve hw/bandwidth.py:56-89 (a streaming read that writes
// one value per workgroup): it measures the achievable HBM read rate that "% of measured peak" is quoted
// against, and evicts L2 and the Infinity Cache before cold timings. Each workgroup reads one contiguous
// range with eight 16-byte nontemporal loads in flight per lane, sixteen workgroups per CU: measured against a
// grid-stride loop with four loads in flight (the previous form), 171.9 MB in 28.5 against 31.4 us and 4 GiB
// at 7.04 against 6.04 TB/s. The page-read probe fetches exactly the K / V rows (and per-token scales) a
// decode call reads, through the same block table and in the same order (the decode's segments, ranges and
// chunks), with no attention math and no merges: the read floor of that call's access pattern. The copy probe
// moves a known number of bytes so rocprof's FETCH_SIZE / WRITE_SIZE counters can be calibrated.
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
constexpr int kProbeGroupsPerCu = 16;
constexpr int kProbeCus = 256;
constexpr int kProbeDepth = 8;  // 16-byte loads in flight per lane

__global__ __launch_bounds__(kProbeThreads) void read_probe_kernel(const U4* buf, int64_t n16, float* partial) {
  const int64_t per = (n16 + gridDim.x - 1) / gridDim.x;
  const int64_t lo = (int64_t)blockIdx.x * per;
  const int64_t hi = lo + per < n16 ? lo + per : n16;
  int64_t i = lo + threadIdx.x;
  uint32_t a = 0;
  for (; i + (kProbeDepth - 1) * kProbeThreads < hi; i += kProbeDepth * kProbeThreads) {
    U4 x[kProbeDepth];
#pragma unroll
    for (int u = 0; u < kProbeDepth; ++u) x[u] = load16((const uint8_t*)(buf + i + u * kProbeThreads));
#pragma unroll
    for (int u = 0; u < kProbeDepth; ++u) a += x[u].x ^ x[u].y ^ x[u].z ^ x[u].w;
  }
  for (; i < hi; i += kProbeThreads) {
    const U4 x0 = load16((const uint8_t*)(buf + i));
    a += x0.x ^ x0.y ^ x0.z ^ x0.w;
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

// The decode's own work split, read only: segments (sequence, KV head, row group) of `chunk`-token chunks laid
// end to end (build_segment_line), equal contiguous ranges for the launched workgroups (numbered XCD-major, as
// the decode numbers them), the waves of a workgroup (the decode's two or four) taking a range's chunks
// round-robin; a chunk is its tokens' K and V rows (row_bytes each, 16 bytes per lane) and, with per-token
// scales, their scales. Page ids are read as the decode reads them (one scalar load per load instruction when
// a load's rows lie in one page), and each wave keeps two chunks' loads in flight. No attention math, no
// partials, no merges.
constexpr int kWalkWaves = 4;

struct WalkChunk {
  U4 k[8], v[8];
  float sc[2];
  unsigned valid;  // bit j: load j's row is a token of the sequence; bit 8: the scale pair is
};

// Issue chunk c's loads into w. `b` is the wave's cursor into the batch (chunks only move forward). Tokens at
// or past len re-read the sequence's last token, as the decode does, and are left out of the sum. The chunk's
// coordinates are made wave-uniform (readfirstlane), so that its page ids come through the scalar cache: a
// vector load there would have to complete, with every load issued before it, before the data loads go out.
// PU: rows_per_load <= page size, so the rows of one load share one page id. LOADS: load instructions per
// lane per chunk (chunk / rows_per_load). SC: per-token scales, one pair per lane (lanes past the chunk re-read
// one of its tokens' and leave it out of the sum, so that every lane issues the same loads).
template <bool PU, int LOADS, bool SC>
__device__ __forceinline__ void walk_issue(const DecodeParams& p, const int* s_prefix, const int* s_len, int64_t c,
                                           int& b, int chunk, int lanes_per_row, int lane, WalkChunk& w) {
  const int HR = p.HR;
  while ((int64_t)HR * s_prefix[b + 1] <= c) ++b;
  b = sread(b);
  const int nb = sread(s_prefix[b + 1] - s_prefix[b]);
  const int r0 = sread((int)(c - (int64_t)HR * s_prefix[b]));  // < HR * nb, an int (the plan bounds it)
  const int hr = sread(r0 / nb), kk = r0 - hr * nb;
  const int h = hr / p.n_rg;
  const int len = sread(s_len[b]);
  const int rows = 64 / lanes_per_row, r = lane / lanes_per_row, part = lane - r * lanes_per_row;
  constexpr int loads = LOADS;
  const int T0 = kk * chunk;
  const int32_t* table = (const int32_t*)p.table;
  int e[8];
  w.valid = 0u;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    if (j < loads) {
      const int t = min(T0 + j * rows + r, len - 1);
      int ej;
      if constexpr (PU) ej = load_uniform(table + table_word(p, b, min(T0 + j * rows, len - 1) >> p.logP));
      else ej = table[table_word(p, b, t >> p.logP)];
      e[j] = ej < 0 ? 0 : (ej >= p.num_blocks ? p.num_blocks - 1 : ej);
      w.valid |= (T0 + j * rows + r < len ? 1u : 0u) << j;
      const int64_t off = (int64_t)e[j] * p.kv_sblk + (int64_t)(t & (p.P - 1)) * p.kv_stok + (int64_t)h * p.kv_shead + 16 * part;
      w.k[j] = load16(p.k + off);
      w.v[j] = load16(p.v + off);
    }
  }
  if constexpr (SC) {
    const int i = lane < chunk ? lane : lane & (chunk - 1);  // chunk: a power of two
    w.valid |= (lane < chunk && T0 + i < len ? 1u : 0u) << 8;
    const int t = min(T0 + i, len - 1);
    int es;
    if constexpr (PU) {
      es = e[0];  // the page id of this token is that of load i / rows
#pragma unroll
      for (int j = 1; j < 8; ++j)
        if (j < loads && i >= j * rows) es = e[j];
    } else {
      es = table[table_word(p, b, t >> p.logP)];
      es = es < 0 ? 0 : (es >= p.num_blocks ? p.num_blocks - 1 : es);
    }
    const int64_t so = (int64_t)es * p.sc_sblk + (int64_t)(t & (p.P - 1)) * p.sc_stok + (int64_t)h * p.sc_shead;
    w.sc[0] = p.ks[so];
    w.sc[1] = p.vs[so];
  }
}

// The sum of a chunk's valid loads: XOR of each 16-byte load's words, K and V, and K ^ V of each scale pair.
template <int LOADS, bool SC>
__device__ __forceinline__ uint32_t walk_fold(const WalkChunk& w) {
  uint32_t x = 0;
#pragma unroll
  for (int j = 0; j < LOADS; ++j) {
    const uint32_t y = (w.k[j].x ^ w.k[j].y ^ w.k[j].z ^ w.k[j].w) + (w.v[j].x ^ w.v[j].y ^ w.v[j].z ^ w.v[j].w);
    x += (w.valid >> j) & 1u ? y : 0u;
  }
  if constexpr (SC) x += (w.valid >> 8) & 1u ? __float_as_uint(w.sc[0]) ^ __float_as_uint(w.sc[1]) : 0u;
  return x;
}

template <bool PU, int LOADS, bool SC, int NWALK>
__global__ __launch_bounds__(NWALK * 64) void page_read_probe_kernel(const DecodeParams p, int chunk,
                                                                         int lanes_per_row, float* partial) {
  extern __shared__ int s_dyn[];  // [B + 1] chunks per sequence (exclusive prefix sum), then [B] lengths
  int* s_prefix = s_dyn;
  int* s_len = s_dyn + p.B + 1;
  __shared__ int s_wsum[NWALK];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // The decode's segment line: `chunk`-token chunks per sequence (its prefix sum over the batch).
  {
    const int per_thread = (p.B + NWALK * 64 - 1) / (NWALK * 64);
    const int lo = min(tid * per_thread, p.B), hi = min(lo + per_thread, p.B);
    int sum = 0;
    for (int b = lo; b < hi; ++b) {
      int len = (p.lens ? p.lens[b] : p.len_cap + p.len_offset) - p.len_offset;
      len = len < 0 ? 0 : (len > p.len_cap ? p.len_cap : len);
      s_len[b] = len;
      sum += (len + chunk - 1) / chunk;
    }
    int x = sum;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int y = __shfl_up(x, off, 64);
      if (lane >= off) x += y;
    }
    if (lane == 63) s_wsum[wave] = x;
    __syncthreads();
    int run = x - sum;
    for (int w = 0; w < wave; ++w) run += s_wsum[w];
    for (int b = lo; b < hi; ++b) {
      s_prefix[b] = run;
      run += (s_len[b] + chunk - 1) / chunk;
    }
    if (tid == 0) {
      int total = 0;
      for (int w = 0; w < NWALK; ++w) total += s_wsum[w];
      s_prefix[p.B] = total;
    }
    __syncthreads();
  }
  const int64_t C = (int64_t)p.HR * s_prefix[p.B];
  const int64_t per = (C + gridDim.x - 1) / gridDim.x;
  const int64_t c0 = line_index(gridDim.x) * per;
  const int64_t c1 = min(c0 + per, C);
  uint32_t a = 0;
  // This wave's chunks: c0 + wave + NWALK i, i < n. The steady state issues unconditionally, so that
  // each fold waits for its own chunk only (a conditional issue leaves the compiler a drain of every load).
  const int64_t first = c0 + wave;
  const int n = first < c1 ? (int)((c1 - first + NWALK - 1) / NWALK) : 0;
  if (n > 0) {
    int lo = 0, hi = p.B - 1;  // the cursor: largest b with HR * prefix[b] <= first
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if ((int64_t)p.HR * s_prefix[mid] <= first) lo = mid; else hi = mid - 1;
    }
    int b = sread(lo);
    auto at = [&](int i) { return first + (int64_t)NWALK * i; };
    WalkChunk A, B;
    walk_issue<PU, LOADS, SC>(p, s_prefix, s_len, at(0), b, chunk, lanes_per_row, lane, A);
    int i = 0;
    for (; i + 2 < n; i += 2) {  // A holds chunk i
      walk_issue<PU, LOADS, SC>(p, s_prefix, s_len, at(i + 1), b, chunk, lanes_per_row, lane, B);
      a += walk_fold<LOADS, SC>(A);  // B's loads stay in flight meanwhile
      walk_issue<PU, LOADS, SC>(p, s_prefix, s_len, at(i + 2), b, chunk, lanes_per_row, lane, A);
      a += walk_fold<LOADS, SC>(B);
    }
    if (i + 2 == n) {
      walk_issue<PU, LOADS, SC>(p, s_prefix, s_len, at(i + 1), b, chunk, lanes_per_row, lane, B);
      a += walk_fold<LOADS, SC>(A);
      a += walk_fold<LOADS, SC>(B);
    } else {
      a += walk_fold<LOADS, SC>(A);
    }
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) a += (uint32_t)__shfl_xor((int)a, m, 64);
  __shared__ uint32_t s[NWALK];
  if (lane == 0) s[wave] = a;
  __syncthreads();
  if (tid == 0) {
    uint32_t t = 0;
    for (int w = 0; w < NWALK; ++w) t += s[w];
    partial[blockIdx.x] = (float)t;
  }
}

hipError_t launch_page_read_probe(const DecodeParams& p, int row_bytes, int chunk, bool with_scales, float* partial,
                                  hipStream_t stream, const LaunchEvents& ev) {
  if (p.grid <= 0) return hipSuccess;
  const size_t lds = (size_t)(2 * p.B + 1) * sizeof(int);
  const int lanes_per_row = row_bytes / 16, rows = 64 / lanes_per_row;
  // The decode's waves per workgroup: two for the matrix-core kernel's two-wave workgroups, else four.
  const bool pair = p.waves == kMfmaPairWaves;
  auto go = [&](auto pu, auto loads) {
    constexpr bool PU = decltype(pu)::value;
    constexpr int L = decltype(loads)::value;
    const dim3 grid((unsigned)p.grid), block((pair ? kMfmaPairWaves : kWalkWaves) * 64);
    if (pair && with_scales)
      launch_kernel(page_read_probe_kernel<PU, L, true, kMfmaPairWaves>, grid, block, lds, stream, ev, p, chunk,
                    lanes_per_row, partial);
    else if (pair)
      launch_kernel(page_read_probe_kernel<PU, L, false, kMfmaPairWaves>, grid, block, lds, stream, ev, p, chunk,
                    lanes_per_row, partial);
    else if (with_scales)
      launch_kernel(page_read_probe_kernel<PU, L, true, kWalkWaves>, grid, block, lds, stream, ev, p, chunk,
                    lanes_per_row, partial);
    else
      launch_kernel(page_read_probe_kernel<PU, L, false, kWalkWaves>, grid, block, lds, stream, ev, p, chunk,
                    lanes_per_row, partial);
  };
  auto by_loads = [&](auto pu) {
    switch (chunk / rows) {
      case 1: go(pu, std::integral_constant<int, 1>{}); break;
      case 2: go(pu, std::integral_constant<int, 2>{}); break;
      case 4: go(pu, std::integral_constant<int, 4>{}); break;
      case 8: go(pu, std::integral_constant<int, 8>{}); break;
      default: return false;
    }
    return true;
  };
  const bool ok = rows <= p.P ? by_loads(std::true_type{}) : by_loads(std::false_type{});
  if (!ok) return hipErrorInvalidValue;
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
