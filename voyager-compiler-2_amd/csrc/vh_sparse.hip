// The outlier path of an MX linear on gfx950: activations whose magnitude
// reaches a threshold leave the quantized tensor and travel exact in a CSR
// stream of fixed capacity (quantize_mx_outlier / filter_outlier,
// ops/quantized.py:1286-1458), CSR streams are cut into tiles
// (slice_csr_tensor, :1493-1545), and the stream is multiplied by the
// decoded weight beside the quantized GEMM (spmm_csr, :1567-1645; the
// A_data term of linear_mx / matmul_mx, :709-720 / :789-802).
//
// All of it is integer and byte work bounded by HBM (the filter) or by the
// gather of one B value per stored entry and output column (the product),
// so nothing here is shaped for MFMA:
//  - filter: one wave per 2048-element row segment writes the inliers,
//    counts the segment's stored outliers (ballot + mbcnt ranks) and keeps
//    the first 16 in a workspace; a scan per matrix turns the rows' counts
//    into row pointers, clamped at the capacity as _pad_csr does; the fill
//    copies the kept entries to their slots (row pointer + the row's earlier
//    segments), re-reading only segments with more.  Capacity slots past the stored entries are padded
//    by extra workgroups of the fill launch.
//  - column slice: the same count / scan / fill over each row's segment.
//  - product: a workgroup stages NT columns of B (all of K, 16- or 32-bit
//    as stored, 16-byte loads, rows padded 16 bytes so the NT lanes that
//    gather one column of the tile hit different banks) in LDS; each lane owns
//    one (row, column) pair and sums its row's entries in stored order in
//    float32, so 64 / NT rows share a wave and NT lanes read each entry
//    (one address per NT lanes).
#include <hip/hip_runtime.h>

#include <mutex>

#include "vh_device.h"
#include "vh_host.h"

namespace {

constexpr int ROW_WAVES = 4;        // rows per workgroup of the row kernels (one wave each)
constexpr int SCAN_THREADS = 1024;  // one workgroup per matrix
constexpr int SPMM_THREADS = 512;
constexpr int SPMM_LDS = 128 * 1024;  // B tile budget (one workgroup per CU)

template <int DT>
using raw_t = typename std::conditional<DT == VH_F32, uint32_t, uint16_t>::type;

template <int DT>
__device__ __forceinline__ float as_float(uint32_t r) {
  if constexpr (DT == VH_F32) return __uint_as_float(r);
  else if constexpr (DT == VH_F16) return __half2float(__ushort_as_half((unsigned short)r));
  else return bf2f(r);
}

__device__ __forceinline__ float raw_to_float(uint32_t r, int dt) {
  return dt == VH_F32 ? __uint_as_float(r) : dt == VH_F16 ? __half2float(__ushort_as_half((unsigned short)r)) : bf2f(r);
}

__device__ __forceinline__ uint32_t load_raw(const void* p, int64_t i, int dt) {
  return dt == VH_F32 ? ((const uint32_t*)p)[i] : (uint32_t)((const uint16_t*)p)[i];
}

__device__ __forceinline__ void store_float(void* p, int64_t i, float v, int dt) {
  if (dt == VH_F32) ((float*)p)[i] = v;
  else if (dt == VH_F16) ((__half*)p)[i] = __float2half_rn(v);
  else ((uint16_t*)p)[i] = (uint16_t)f2bf(v);
}

// Lanes below this one whose bit is set in m.
__device__ __forceinline__ int rank_below(uint64_t m) {
  return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

__device__ __forceinline__ int wave_sum(int v) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d);
  return v;
}

// Inclusive scan over the workgroup (SCAN_THREADS threads) in thread order;
// `total` receives the sum (or max) of all threads.  MAX: running maximum.
template <bool MAX>
__device__ __forceinline__ int64_t block_scan(int64_t v, int64_t* s_wave, int64_t& total) {
  constexpr int NW = SCAN_THREADS / 64;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int64_t u = __shfl_up(v, d);
    if (lane >= d) v = MAX ? (u > v ? u : v) : v + u;
  }
  if (lane == 63) s_wave[wave] = v;
  __syncthreads();
  int64_t pre = MAX ? INT64_MIN : 0, all = MAX ? INT64_MIN : 0;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    const int64_t t = s_wave[w];
    if (w < wave) pre = MAX ? (t > pre ? t : pre) : pre + t;
    all = MAX ? (t > all ? t : all) : all + t;
  }
  __syncthreads();
  total = all;
  return MAX ? (pre > v ? pre : v) : v + pre;
}

// ------------------------------------------------------------ filter
// A row is cut into segments of SEG elements, one wave each, so a prefill
// activation gives tens of thousands of waves.  Pass 1 writes the inliers,
// counts each segment's stored outliers and keeps up to SEG_STAGE of them
// (value bits and column) in the workspace; the scan turns the rows' counts
// into row pointers; pass 3 copies the kept outliers to their slots,
// re-reading only segments that held more than SEG_STAGE.
constexpr int SEG = 2048;
constexpr int SEG_STAGE = 16;
constexpr int SCAN_ITEMS = 4;  // rows per thread of the row scan

struct FilterWork {
  int32_t* seg;   // [nseg + 1] per-segment counts of stored outliers
  uint32_t* val;  // [nseg][SEG_STAGE] value bits
  int32_t* col;   // [nseg][SEG_STAGE] columns
};

__host__ __device__ inline int64_t filter_work_bytes_per_matrix(int64_t nseg) {
  return ((nseg + 1) * 4 + 15) / 16 * 16 + nseg * SEG_STAGE * 8;
}

__device__ __forceinline__ FilterWork filter_work(void* work, int64_t b, int64_t nseg) {
  uint8_t* p = (uint8_t*)work + b * filter_work_bytes_per_matrix(nseg);
  FilterWork w;
  w.seg = (int32_t*)p;
  w.val = (uint32_t*)(p + ((nseg + 1) * 4 + 15) / 16 * 16);
  w.col = (int32_t*)(w.val + nseg * SEG_STAGE);
  return w;
}

// EPV elements of a lane's 16-byte chunk (or one element when EPV == 1).
template <int DT, int EPV>
struct Chunk {
  uint32_t v[EPV];
};

template <int DT, int EPV>
__device__ __forceinline__ Chunk<DT, EPV> load_chunk(const raw_t<DT>* p) {
  Chunk<DT, EPV> c;
  if constexpr (EPV == 1) {
    c.v[0] = p[0];
  } else {
    const uint4 u = ld_stream16(p);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if constexpr (DT == VH_F32) {
        c.v[k] = w[k];
      } else {
        c.v[2 * k] = w[k] & 0xffffu;
        c.v[2 * k + 1] = w[k] >> 16;
      }
    }
  }
  return c;
}

template <int DT, int EPV>
__device__ __forceinline__ void store_chunk(raw_t<DT>* p, const Chunk<DT, EPV>& c) {
  if constexpr (EPV == 1) {
    p[0] = (raw_t<DT>)c.v[0];
  } else if constexpr (DT == VH_F32) {
    *(uint4*)p = make_uint4(c.v[0], c.v[1], c.v[2], c.v[3]);
  } else {
    *(uint4*)p = make_uint4(c.v[0] | (c.v[1] << 16), c.v[2] | (c.v[3] << 16), c.v[4] | (c.v[5] << 16),
                            c.v[6] | (c.v[7] << 16));
  }
}

// The stored outliers among a lane's chunk: bit e set for element e.
template <int DT, int EPV>
__device__ __forceinline__ uint32_t keep_bits(const Chunk<DT, EPV>& v, bool live, float thr) {
  uint32_t m = 0;
#pragma unroll
  for (int e = 0; e < EPV; ++e) {
    const float f = as_float<DT>(v.v[e]);
    if (live && fabsf(f) >= thr && f != 0.0f) m |= 1u << e;
  }
  return m;
}

// Ranks of a wave's kept elements in element order: `before` counts those
// in lanes below, `total` the wave's.
template <int EPV>
__device__ __forceinline__ void wave_ranks(uint32_t keep, int& before, int& total) {
  before = 0;
  total = 0;
#pragma unroll
  for (int e = 0; e < EPV; ++e) {
    const uint64_t m = __ballot((keep >> e) & 1u);
    before += rank_below(m);
    total += __popcll(m);
  }
}

// Pass 1: inliers; per segment the count of stored outliers and the first
// SEG_STAGE of them.
template <int DT, int EPV>
__global__ void __launch_bounds__(ROW_WAVES * 64) k_outlier_count(const raw_t<DT>* __restrict__ x, int64_t rows,
                                                                  int64_t cols, int64_t S, float thr,
                                                                  raw_t<DT>* __restrict__ inl, void* work) {
  constexpr int IT = SEG / (64 * EPV);  // chunks per lane and segment
  const int lane = threadIdx.x & 63;
  const int64_t b = blockIdx.y;
  const int64_t w = (int64_t)blockIdx.x * ROW_WAVES + (threadIdx.x >> 6);
  const int64_t nseg = rows * S;
  if (w >= nseg) return;
  const int64_t r = w / S, c_begin = (w % S) * SEG;
  const int64_t c_end = c_begin + SEG < cols ? c_begin + SEG : cols;
  const int64_t base = (b * rows + r) * cols;
  const FilterWork fw = filter_work(work, b, nseg);
  Chunk<DT, EPV> v[IT];
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    const int64_t c = c_begin + (int64_t)(it * 64 + lane) * EPV;
    if (c < c_end) {
      v[it] = load_chunk<DT, EPV>(x + base + c);
    } else {
#pragma unroll
      for (int e = 0; e < EPV; ++e) v[it].v[e] = 0u;
    }
  }
  int cnt = 0;
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    const int64_t c = c_begin + (int64_t)(it * 64 + lane) * EPV;
    const bool live = c < c_end;
    const uint32_t keep = keep_bits<DT, EPV>(v[it], live, thr);
    int before, total;
    wave_ranks<EPV>(keep, before, total);
    int mine = 0;
    Chunk<DT, EPV> o = v[it];
#pragma unroll
    for (int e = 0; e < EPV; ++e) {
      if (fabsf(as_float<DT>(o.v[e])) >= thr) o.v[e] = 0u;
      if ((keep >> e) & 1u) {
        const int s = cnt + before + mine;
        if (s < SEG_STAGE) {
          fw.val[w * SEG_STAGE + s] = v[it].v[e];
          fw.col[w * SEG_STAGE + s] = (int32_t)(c + e);
        }
        ++mine;
      }
    }
    if (live) store_chunk<DT, EPV>(inl + base + c, o);
    cnt += total;
  }
  if (lane == 0) fw.seg[w] = cnt;
}

// Pass 2 (one workgroup per matrix): row pointers from the segment counts,
// clamped at cap, plus offset (the counts stay: a segment's slots start at
// its row's pointer plus the counts of the row's earlier segments).
// SCAN_ITEMS rows per thread: serial sums, one block scan of the sums.
__global__ void __launch_bounds__(SCAN_THREADS) k_row_scan(const void* work, int64_t rows, int64_t S, int64_t cap,
                                                           int32_t offset, int32_t* __restrict__ indptr) {
  __shared__ int64_t s_wave[SCAN_THREADS / 64];
  const FilterWork fw = filter_work(const_cast<void*>(work), blockIdx.x, rows * S);
  int32_t* p = indptr + (int64_t)blockIdx.x * (rows + 1);
  int64_t carry = 0;
  for (int64_t r0 = 0; r0 < rows; r0 += (int64_t)SCAN_THREADS * SCAN_ITEMS) {
    const int64_t rb = r0 + (int64_t)threadIdx.x * SCAN_ITEMS;
    int64_t v[SCAN_ITEMS];
    int64_t sum = 0;
#pragma unroll
    for (int k = 0; k < SCAN_ITEMS; ++k) {
      v[k] = 0;
      if (rb + k < rows)
        for (int64_t sg = 0; sg < S; ++sg) v[k] += fw.seg[(rb + k) * S + sg];
      sum += v[k];
    }
    int64_t total;
    int64_t excl = block_scan<false>(sum, s_wave, total) - sum + carry;
#pragma unroll
    for (int k = 0; k < SCAN_ITEMS; ++k) {
      if (rb + k < rows) p[rb + k] = (int32_t)((excl < cap ? excl : cap) + offset);
      excl += v[k];
    }
    carry += total;
  }
  if (threadIdx.x == 0) p[rows] = (int32_t)((carry < cap ? carry : cap) + offset);
}

// Pass 3: each segment's outliers to their slots (below cap): from the
// workspace, or by re-reading a segment that held more than SEG_STAGE.
// Workgroups past the segments pad slots [nse, cap).
template <int DT, int EPV>
__global__ void __launch_bounds__(ROW_WAVES * 64) k_outlier_fill(const raw_t<DT>* __restrict__ x, int64_t rows,
                                                                 int64_t cols, int64_t S, float thr, int64_t cap,
                                                                 int32_t offset, const int32_t* __restrict__ indptr,
                                                                 const void* work, int seg_blocks,
                                                                 raw_t<DT>* __restrict__ data,
                                                                 int32_t* __restrict__ indices) {
  constexpr int IT = SEG / (64 * EPV);
  const int64_t b = blockIdx.y;
  const int64_t nseg = rows * S;
  const FilterWork fw = filter_work(const_cast<void*>(work), b, nseg);
  const int32_t* ip = indptr + b * (rows + 1);
  raw_t<DT>* d = data + b * cap;
  int32_t* ix = indices + b * cap;
  if ((int)blockIdx.x >= seg_blocks) {
    const int64_t nse = (int64_t)ip[rows] - offset;
    const int64_t step = (int64_t)(gridDim.x - seg_blocks) * blockDim.x;
    for (int64_t s = (int64_t)(blockIdx.x - seg_blocks) * blockDim.x + threadIdx.x; s < cap; s += step) {
      if (s >= nse) {
        d[s] = (raw_t<DT>)0;
        ix[s] = -1;
      }
    }
    return;
  }
  const int lane = threadIdx.x & 63;
  const int64_t w = (int64_t)blockIdx.x * ROW_WAVES + (threadIdx.x >> 6);
  if (w >= nseg) return;
  // slots start at the row's pointer (clamped: at cap, nothing of the row
  // is kept) plus the row's earlier segments' counts
  const int64_t r = w / S;
  int64_t start = (int64_t)ip[r] - offset;
  // the earlier segments' counts, eight loads in flight at a time (clamped
  // into the row and masked, so no load waits on the one before; a start
  // past cap returns below whatever the sum)
  for (int64_t s0 = r * S; s0 < w; s0 += 8) {
    int64_t cnt[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) cnt[k] = fw.seg[s0 + k < w ? s0 + k : s0];
#pragma unroll
    for (int k = 0; k < 8; ++k) start += s0 + k < w ? cnt[k] : 0;
  }
  const int64_t n = fw.seg[w];
  if (start >= cap || n == 0) return;
  if (n <= SEG_STAGE) {
    if (lane < n && start + lane < cap) {
      d[start + lane] = (raw_t<DT>)fw.val[w * SEG_STAGE + lane];
      ix[start + lane] = fw.col[w * SEG_STAGE + lane];
    }
    return;
  }
  const int64_t c_begin = (w % S) * SEG;
  const int64_t c_end = c_begin + SEG < cols ? c_begin + SEG : cols;
  const int64_t base = (b * rows + r) * cols;
  int64_t pos = start;
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    const int64_t c = c_begin + (int64_t)(it * 64 + lane) * EPV;
    const bool live = c < c_end;
    Chunk<DT, EPV> v;
    if (live) {
      v = load_chunk<DT, EPV>(x + base + c);
    } else {
#pragma unroll
      for (int e = 0; e < EPV; ++e) v.v[e] = 0u;
    }
    const uint32_t keep = keep_bits<DT, EPV>(v, live, thr);
    int before, total;
    wave_ranks<EPV>(keep, before, total);
    int mine = 0;
#pragma unroll
    for (int e = 0; e < EPV; ++e) {
      if ((keep >> e) & 1u) {
        const int64_t s = pos + before + mine;
        if (s < cap) {
          d[s] = (raw_t<DT>)v.v[e];
          ix[s] = (int32_t)(c + e);
        }
        ++mine;
      }
    }
    pos += total;
  }
}

// ------------------------------------------------------------ column slice
// Each row's entries whose column lies in [start, end): count, then fill.

// One workgroup per matrix: indptr[1 .. rows] from counts to running sums
// clamped at cap, plus offset; indptr[0] = offset.
__global__ void __launch_bounds__(SCAN_THREADS) k_rowptr_scan(int32_t* __restrict__ indptr, int64_t rows, int64_t cap,
                                                              int32_t offset) {
  __shared__ int64_t s_wave[SCAN_THREADS / 64];
  int32_t* p = indptr + (int64_t)blockIdx.x * (rows + 1);
  if (threadIdx.x == 0) p[0] = offset;
  int64_t carry = 0;
  for (int64_t i0 = 0; i0 < rows; i0 += SCAN_THREADS) {
    const int64_t i = i0 + threadIdx.x;
    const int64_t v = i < rows ? (int64_t)p[i + 1] : 0;
    int64_t total;
    const int64_t incl = block_scan<false>(v, s_wave, total) + carry;
    if (i < rows) p[i + 1] = (int32_t)((incl < cap ? incl : cap) + offset);
    carry += total;
  }
}
__global__ void __launch_bounds__(ROW_WAVES * 64) k_cols_count(const int32_t* __restrict__ indices,
                                                               const int32_t* __restrict__ indptr, int64_t rows,
                                                               int64_t cap, int64_t start, int64_t end,
                                                               int32_t* __restrict__ out_indptr) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * ROW_WAVES + (threadIdx.x >> 6);
  if (r >= rows) return;
  const int64_t j0 = max((int64_t)0, min((int64_t)indptr[r], cap));
  const int64_t j1 = max(j0, min((int64_t)indptr[r + 1], cap));
  int cnt = 0;
  for (int64_t j = j0 + lane; j < j1; j += 64) {
    const int64_t k = indices[j];
    cnt += (k >= start && k < end) ? 1 : 0;
  }
  cnt = wave_sum(cnt);
  if (lane == 0) out_indptr[r + 1] = cnt;
}

__global__ void __launch_bounds__(ROW_WAVES * 64) k_cols_fill(const void* __restrict__ data, int dt,
                                                              const int32_t* __restrict__ indices,
                                                              const int32_t* __restrict__ indptr, int64_t rows,
                                                              int64_t cap, int64_t start, int64_t end,
                                                              int64_t out_cap, const int32_t* __restrict__ out_indptr,
                                                              int row_blocks, void* __restrict__ out_data,
                                                              int32_t* __restrict__ out_indices) {
  if ((int)blockIdx.x >= row_blocks) {
    const int64_t nse = out_indptr[rows];
    const int64_t step = (int64_t)(gridDim.x - row_blocks) * blockDim.x;
    for (int64_t s = (int64_t)(blockIdx.x - row_blocks) * blockDim.x + threadIdx.x; s < out_cap; s += step) {
      if (s >= nse) {
        if (dt == VH_F32) ((uint32_t*)out_data)[s] = 0u;
        else ((uint16_t*)out_data)[s] = 0;
        out_indices[s] = -1;
      }
    }
    return;
  }
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * ROW_WAVES + (threadIdx.x >> 6);
  if (r >= rows) return;
  const int64_t j0 = max((int64_t)0, min((int64_t)indptr[r], cap));
  const int64_t j1 = max(j0, min((int64_t)indptr[r + 1], cap));
  int64_t pos = out_indptr[r];
  for (int64_t jb = j0; jb < j1 && pos < out_cap; jb += 64) {
    const int64_t j = jb + lane;
    const int64_t k = j < j1 ? (int64_t)indices[j] : -1;
    const bool keep = j < j1 && k >= start && k < end;
    const uint64_t m = __ballot(keep);
    const int64_t s = pos + rank_below(m);
    if (keep && s < out_cap) {
      if (dt == VH_F32) ((uint32_t*)out_data)[s] = ((const uint32_t*)data)[j];
      else ((uint16_t*)out_data)[s] = ((const uint16_t*)data)[j];
      out_indices[s] = (int32_t)(k - start);
    }
    pos += __popcll(m);
  }
}

// ------------------------------------------------------------ row slice
// Rows [start, end): pointers rebased on indptr[start] (clamped at out_cap
// when the span overflows it), entries copied, slots past them padded.
// Source slots outside [0, cap) read as padding.
__global__ void __launch_bounds__(256) k_rows_slice(const void* __restrict__ data, int dt,
                                                    const int32_t* __restrict__ indices,
                                                    const int32_t* __restrict__ indptr, int64_t cap, int64_t start,
                                                    int64_t end, int64_t out_cap, void* __restrict__ out_data,
                                                    int32_t* __restrict__ out_indices,
                                                    int32_t* __restrict__ out_indptr) {
  const int64_t s0 = indptr[start];
  const int64_t n = (int64_t)indptr[end] - s0;
  const int64_t nrows = end - start + 1;
  const int64_t step = (int64_t)gridDim.x * blockDim.x;
  const int64_t span = out_cap > nrows ? out_cap : nrows;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < span; i += step) {
    if (i < nrows) {
      int64_t v = (int64_t)indptr[start + i] - s0;
      if (n > out_cap && v > out_cap) v = out_cap;
      out_indptr[i] = (int32_t)v;
    }
    if (i < out_cap) {
      const int64_t src = s0 + i;
      const bool live = i < n && src >= 0 && src < cap;
      uint32_t val = 0u;
      int32_t col = -1;
      if (live) {
        val = load_raw(data, src, dt);
        col = indices[src];
      }
      if (dt == VH_F32) ((uint32_t*)out_data)[i] = val;
      else ((uint16_t*)out_data)[i] = (uint16_t)val;
      out_indices[i] = col;
    }
  }
}

// ------------------------------------------------------------ product
// work[r] = running max over r' <= r of clamp(indptr[r'] - indptr[0], 0, cap):
// the rebased, clamped, non-decreasing row pointers of the reference.
__global__ void __launch_bounds__(SCAN_THREADS) k_rowptr_rebase(const int32_t* __restrict__ indptr, int64_t rows,
                                                                int64_t cap, int32_t* __restrict__ work) {
  __shared__ int64_t s_wave[SCAN_THREADS / 64];
  const int32_t* p = indptr + (int64_t)blockIdx.x * (rows + 1);
  int32_t* w = work + (int64_t)blockIdx.x * (rows + 1);
  const int64_t first = p[0];
  int64_t carry = 0;  // every value is >= 0
  for (int64_t i0 = 0; i0 <= rows; i0 += SCAN_THREADS) {
    const int64_t i = i0 + threadIdx.x;
    int64_t v = 0;
    if (i <= rows) {
      v = (int64_t)p[i] - first;
      v = v < 0 ? 0 : v > cap ? cap : v;
    }
    int64_t total;
    int64_t incl = block_scan<true>(v, s_wave, total);
    incl = incl > carry ? incl : carry;
    if (i <= rows) w[i] = (int32_t)incl;
    carry = total > carry ? total : carry;
  }
}

// out[r, n0 + t] = round(base + sum_j float(data[j]) * B[k_j, n0 + t]).
// B tile in LDS: NT rows of KP = K + pad raw elements.
template <int NT, int ESZ>
__global__ void __launch_bounds__(SPMM_THREADS) k_spmm(const void* __restrict__ data, int data_dt,
                                                       const int32_t* __restrict__ indices,
                                                       const int32_t* __restrict__ rowptr, int64_t rows, int64_t cap,
                                                       const void* __restrict__ B, int b_dt, int b_layout, int64_t K,
                                                       int64_t N, int64_t b_stride, int64_t rows_per_block,
                                                       const float* __restrict__ base, void* __restrict__ out,
                                                       int out_dt) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  constexpr int PAD = 16 / ESZ;  // 16 bytes: tile rows stay 16-byte aligned, 4 banks apart
  constexpr int E16 = 16 / ESZ;  // elements per 16-byte load
  const int64_t KP = K + PAD;
  const int64_t b = blockIdx.z;
  const int64_t n0 = (int64_t)blockIdx.x * NT;
  const uint8_t* Bb = (const uint8_t*)B + b * b_stride * ESZ;
  // stage B[:, n0 .. n0 + NT) as [NT][KP]
  if (b_layout == 0 && K % E16 == 0 && ((uintptr_t)Bb % 16) == 0) {  // "kc", 16-byte rows
    // chunk c = t * k16 + q; eight loads in flight per thread, then their stores
    const int64_t k16 = K / E16, nchunk = NT * k16;
    for (int64_t c0 = threadIdx.x; c0 < nchunk; c0 += 8 * SPMM_THREADS) {
      uint4 v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int64_t c = c0 + u * SPMM_THREADS;
        const int64_t t = c / k16, q = c - t * k16;
        v[u] = c < nchunk && n0 + t < N ? *(const uint4*)(Bb + ((n0 + t) * K + q * E16) * ESZ)
                                        : make_uint4(0u, 0u, 0u, 0u);
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int64_t c = c0 + u * SPMM_THREADS;
        const int64_t t = c / k16, q = c - t * k16;
        if (c < nchunk) *(uint4*)(smem + (t * KP + q * E16) * ESZ) = v[u];
      }
    }
  } else if (b_layout == 0) {  // "kc": row n of B is contiguous over k
    for (int t = 0; t < NT; ++t) {
      const int64_t n = n0 + t;
      for (int64_t k = threadIdx.x; k < K; k += SPMM_THREADS) {
        const int64_t dst = t * KP + k;
        if constexpr (ESZ == 2)
          ((uint16_t*)smem)[dst] = n < N ? ((const uint16_t*)Bb)[n * K + k] : (uint16_t)0;
        else
          ((uint32_t*)smem)[dst] = n < N ? ((const uint32_t*)Bb)[n * K + k] : 0u;
      }
    }
  } else {  // "ck": B[k, n] at k * N + n; NT consecutive n per k
    for (int64_t i = threadIdx.x; i < (int64_t)NT * K; i += SPMM_THREADS) {
      const int t = (int)(i % NT);
      const int64_t k = i / NT, n = n0 + t;
      const int64_t dst = t * KP + k;
      if constexpr (ESZ == 2)
        ((uint16_t*)smem)[dst] = n < N ? ((const uint16_t*)Bb)[k * N + n] : (uint16_t)0;
      else
        ((uint32_t*)smem)[dst] = n < N ? ((const uint32_t*)Bb)[k * N + n] : 0u;
    }
  }
  __syncthreads();

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  constexpr int RPW = 64 / NT;                            // rows per wave pass
  constexpr int RPB = RPW * (SPMM_THREADS / 64);          // rows per workgroup pass
  const int t = lane % NT;
  const int64_t n = n0 + t;
  const int64_t r_begin = (int64_t)blockIdx.y * rows_per_block;
  const int64_t r_end = min(rows, r_begin + rows_per_block);
  const int32_t* rp = rowptr + b * (rows + 1);
  const int32_t* ix = indices + b * cap;
  const uint8_t* dv = (const uint8_t*)data + b * cap * (data_dt == VH_F32 ? 4 : 2);
  const uint8_t* tile = smem + t * KP * ESZ;
  for (int64_t r = r_begin + wave * RPW + lane / NT; r < r_end; r += RPB) {
    const int64_t j0 = rp[r], j1 = rp[r + 1];
    const int64_t o = (b * rows + r) * N + n;
    const float bv = (base != nullptr && n < N) ? base[o] : 0.0f;
    float acc = 0.0f;
    // entries four at a time: their loads in flight together, the sum in order
    for (int64_t j = j0; j < j1; j += 4) {
      int32_t kk[4];
      uint32_t vv[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        kk[u] = j + u < j1 ? ix[j + u] : 0;
        vv[u] = j + u < j1 ? load_raw(dv, j + u, data_dt) : 0u;
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        if (j + u < j1) {
          const int64_t k = kk[u] < 0 ? 0 : kk[u] >= K ? K - 1 : kk[u];
          const uint32_t braw = ESZ == 2 ? (uint32_t)((const uint16_t*)tile)[k] : ((const uint32_t*)tile)[k];
          acc = fmaf(raw_to_float(vv[u], data_dt), raw_to_float(braw, b_dt), acc);
        }
      }
    }
    if (n < N) store_float(out, o, base != nullptr ? acc + bv : acc, out_dt);
  }
}

template <int NT, int ESZ>
int launch_spmm(const void* data, int data_dt, const int32_t* indices, const int32_t* rowptr, int64_t batch,
                int64_t rows, int64_t cap, const void* B, int b_dt, int b_layout, int64_t K, int64_t N,
                int64_t b_stride, const float* base, void* out, int out_dt, hipStream_t st) {
  constexpr int PAD = 16 / ESZ;
  const size_t smem = (size_t)NT * (size_t)(K + PAD) * ESZ;
  static bool attr_set = false;
  if (!attr_set) {
    if (hipFuncSetAttribute((const void*)k_spmm<NT, ESZ>, hipFuncAttributeMaxDynamicSharedMemorySize,
                            SPMM_LDS + 4096) != hipSuccess) {
      vh::set_error("vh_spmm_csr: cannot reserve LDS");
      return VH_ELAUNCH;
    }
    attr_set = true;
  }
  // Column tiles x row ranges: at least one workgroup per CU where the rows
  // allow it (each row range restages its B tile).
  const int64_t tiles = (N + NT - 1) / NT;
  constexpr int64_t RPB = (64 / NT) * (SPMM_THREADS / 64);
  const int64_t passes = (rows + RPB - 1) / RPB;
  int64_t splits = (256 + tiles * batch - 1) / (tiles * batch);
  splits = splits < 1 ? 1 : splits > passes ? passes : splits;
  const int64_t per = (passes + splits - 1) / splits * RPB;
  splits = (rows + per - 1) / per;
  hipLaunchKernelGGL((k_spmm<NT, ESZ>), dim3((unsigned)tiles, (unsigned)splits, (unsigned)batch),
                     dim3(SPMM_THREADS), smem, st, data, data_dt, indices, rowptr, rows, cap, B, b_dt, b_layout, K, N,
                     b_stride, per, base, out, out_dt);
  return vh::check_launch("vh_spmm_csr");
}

bool float_dtype(int dt) { return dt == VH_BF16 || dt == VH_F16 || dt == VH_F32; }

unsigned pad_blocks(int64_t cap) {
  const int64_t b = (cap + 255) / 256;
  return (unsigned)(b < 1 ? 1 : b > 1024 ? 1024 : b);
}

template <int DT, int EPV>
int filter_launch(const void* x, int64_t batch, int64_t rows, int64_t cols, float thr, int64_t cap,
                  int32_t offset, void* data, int32_t* indices, int32_t* indptr, void* inl, void* work,
                  hipStream_t st) {
  using R = raw_t<DT>;
  const int64_t S = (cols + SEG - 1) / SEG;
  const int64_t nseg = rows * S;
  const unsigned seg_blocks = (unsigned)((nseg + ROW_WAVES - 1) / ROW_WAVES);
  if (seg_blocks > 0) {
    hipLaunchKernelGGL((k_outlier_count<DT, EPV>), dim3(seg_blocks, (unsigned)batch), dim3(ROW_WAVES * 64), 0, st,
                       (const R*)x, rows, cols, S, thr, (R*)inl, work);
    if (int e = vh::check_launch("vh_filter_outlier")) return e;
  }
  hipLaunchKernelGGL(k_row_scan, dim3((unsigned)batch), dim3(SCAN_THREADS), 0, st, (const void*)work, rows, S, cap,
                     offset, indptr);
  if (int e = vh::check_launch("vh_filter_outlier")) return e;
  const unsigned pads = cap > 0 ? pad_blocks(cap) : 0;
  if (cap == 0 || seg_blocks + pads == 0) return VH_OK;
  hipLaunchKernelGGL((k_outlier_fill<DT, EPV>), dim3(seg_blocks + pads, (unsigned)batch), dim3(ROW_WAVES * 64), 0,
                     st, (const R*)x, rows, cols, S, thr, cap, offset, (const int32_t*)indptr, (const void*)work,
                     (int)seg_blocks, (R*)data, indices);
  return vh::check_launch("vh_filter_outlier");
}

}  // namespace

extern "C" int64_t vh_filter_outlier_workspace_bytes(int64_t batch, int64_t rows, int64_t cols) {
  if (batch < 0 || rows < 0 || cols < 0) return 0;
  return batch * filter_work_bytes_per_matrix(rows * ((cols + SEG - 1) / SEG));
}

namespace {

// Everything vh_filter_outlier checks and launches, given a workspace of at
// least vh_filter_outlier_workspace_bytes(batch, rows, cols) bytes.
int filter_outlier_run(const void* x, int32_t dtype, int64_t batch, int64_t rows, int64_t cols, float threshold,
                       int64_t max_nnz, int32_t indptr_offset, void* data, int32_t* indices, int32_t* indptr,
                       void* inliers, void* work, vh_stream_t stream) {
  VH_REQUIRE(float_dtype(dtype), "vh_filter_outlier: dtype must be bf16, fp16 or fp32");
  VH_REQUIRE(batch >= 1 && batch <= 65535 && rows >= 0 && cols >= 0 && max_nnz >= 0,
             "vh_filter_outlier: bad sizes (batch %lld, rows %lld, cols %lld, max_nnz %lld)", (long long)batch,
             (long long)rows, (long long)cols, (long long)max_nnz);
  VH_REQUIRE(rows * cols < ((int64_t)1 << 31) && max_nnz < ((int64_t)1 << 31),
             "vh_filter_outlier: a matrix must hold fewer than 2**31 elements (int32 row pointers)");
  VH_REQUIRE(rows * cols == 0 || (x != nullptr && inliers != nullptr), "vh_filter_outlier: null tensor");
  const int64_t S = (cols + SEG - 1) / SEG;
  VH_REQUIRE(rows * S / ROW_WAVES < ((int64_t)1 << 31), "vh_filter_outlier: too many rows");
  const hipStream_t st = vh::as_stream(stream);
  const int epv = dtype == VH_F32 ? 4 : 8;
  const bool vec = cols % epv == 0 && ((uintptr_t)x % 16) == 0 && ((uintptr_t)inliers % 16) == 0;
#define VH_FILTER(DT, EPV)                                                                                        \
  filter_launch<DT, EPV>(x, batch, rows, cols, threshold, max_nnz, indptr_offset, data, indices, indptr, inliers, \
                         work, st)
  switch (dtype) {
    case VH_BF16: return vec ? VH_FILTER(VH_BF16, 8) : VH_FILTER(VH_BF16, 1);
    case VH_F16: return vec ? VH_FILTER(VH_F16, 8) : VH_FILTER(VH_F16, 1);
    default: return vec ? VH_FILTER(VH_F32, 4) : VH_FILTER(VH_F32, 1);
  }
#undef VH_FILTER
}

// The workspace of vh_filter_outlier_noalloc: a file-scope device array,
// one copy per GPU, held until the process ends.  Host code never passes
// the array's name to a kernel (on the host it is a stand-in, not a device
// address); it takes each device's address once with hipGetSymbolAddress.
static __device__ __align__(256) uint8_t scratch[VH_FILTER_NOALLOC_SCRATCH_BYTES];

constexpr int MAX_DEVICES = 64;
std::mutex scratch_mutex;
void* scratch_ptr[MAX_DEVICES] = {};

// This device's address of `scratch`, looked up on the device's first call.
int scratch_of_current_device(void** out) {
  int dev = -1;
  VH_REQUIRE(hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < MAX_DEVICES,
             "vh_filter_outlier_noalloc: no current device");
  std::lock_guard<std::mutex> lock(scratch_mutex);
  if (!scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    VH_REQUIRE(e == hipSuccess && p != nullptr, "vh_filter_outlier_noalloc: hipGetSymbolAddress failed: %s",
               hipGetErrorString(e));
    scratch_ptr[dev] = p;
  }
  *out = scratch_ptr[dev];
  return VH_OK;
}

}  // namespace

extern "C" int vh_filter_outlier(const void* x, int32_t dtype, int64_t batch, int64_t rows, int64_t cols,
                                 float threshold, int64_t max_nnz, int32_t indptr_offset, void* data,
                                 int32_t* indices, int32_t* indptr, void* inliers, void* work, int64_t work_bytes,
                                 vh_stream_t stream) {
  VH_REQUIRE(work != nullptr && ((uintptr_t)work % 16) == 0 &&
                 work_bytes >= vh_filter_outlier_workspace_bytes(batch, rows, cols),
             "vh_filter_outlier: workspace needs %lld bytes, 16-byte aligned",
             (long long)vh_filter_outlier_workspace_bytes(batch, rows, cols));
  return filter_outlier_run(x, dtype, batch, rows, cols, threshold, max_nnz, indptr_offset, data, indices, indptr,
                            inliers, work, stream);
}

extern "C" int vh_filter_outlier_noalloc(const void* x, int32_t dtype, int64_t batch, int64_t rows, int64_t cols,
                                         float threshold, int64_t max_nnz, int32_t indptr_offset, void* data,
                                         int32_t* indices, int32_t* indptr, void* inliers, vh_stream_t stream) {
  const int64_t need = vh_filter_outlier_workspace_bytes(batch, rows, cols);
  VH_REQUIRE(need <= VH_FILTER_NOALLOC_SCRATCH_BYTES,
             "vh_filter_outlier_noalloc: %lld x %lld x %lld needs %lld bytes of workspace, more than the %lld of the "
             "library's fixed scratch; call vh_filter_outlier with a workspace",
             (long long)batch, (long long)rows, (long long)cols, (long long)need,
             (long long)VH_FILTER_NOALLOC_SCRATCH_BYTES);
  void* work = nullptr;
  if (int e = scratch_of_current_device(&work)) return e;
  // Every workspace word a launch reads was written earlier in the same
  // call (segment counts for every segment, staged outliers below each
  // segment's count), so the scratch needs no clearing between calls.
  return filter_outlier_run(x, dtype, batch, rows, cols, threshold, max_nnz, indptr_offset, data, indices, indptr,
                            inliers, work, stream);
}

extern "C" int vh_slice_csr(const void* data, int32_t dtype, const int32_t* indices, const int32_t* indptr,
                            int64_t rows, int64_t cap, int32_t dim, int64_t start, int64_t end, int64_t out_cap,
                            void* out_data, int32_t* out_indices, int32_t* out_indptr, vh_stream_t stream) {
  VH_REQUIRE(float_dtype(dtype), "vh_slice_csr: data dtype must be bf16, fp16 or fp32");
  VH_REQUIRE(rows >= 0 && cap >= 0 && out_cap >= 0 && cap < ((int64_t)1 << 31) && out_cap < ((int64_t)1 << 31),
             "vh_slice_csr: bad sizes");
  const hipStream_t st = vh::as_stream(stream);
  if (dim == 0) {
    VH_REQUIRE(start >= 0 && start <= end && end <= rows,
               "vh_slice_csr: rows [%lld, %lld) out of range for %lld rows", (long long)start, (long long)end,
               (long long)rows);
    const int64_t span = out_cap > end - start + 1 ? out_cap : end - start + 1;
    int64_t blocks = (span + 255) / 256;
    blocks = blocks < 1 ? 1 : blocks > 4096 ? 4096 : blocks;
    hipLaunchKernelGGL(k_rows_slice, dim3((unsigned)blocks), dim3(256), 0, st, data, (int)dtype, indices, indptr, cap,
                       start, end, out_cap, out_data, out_indices, out_indptr);
    return vh::check_launch("vh_slice_csr");
  }
  VH_REQUIRE(dim == 1, "vh_slice_csr: dim must be 0 or 1");
  VH_REQUIRE(rows < (1 << 26), "vh_slice_csr: too many rows");
  const unsigned row_blocks = (unsigned)((rows + ROW_WAVES - 1) / ROW_WAVES);
  if (row_blocks > 0) {
    hipLaunchKernelGGL(k_cols_count, dim3(row_blocks), dim3(ROW_WAVES * 64), 0, st, indices, indptr, rows, cap, start,
                       end, out_indptr);
    if (int e = vh::check_launch("vh_slice_csr")) return e;
  }
  hipLaunchKernelGGL(k_rowptr_scan, dim3(1), dim3(SCAN_THREADS), 0, st, out_indptr, rows, out_cap, 0);
  if (int e = vh::check_launch("vh_slice_csr")) return e;
  const unsigned pads = out_cap > 0 ? pad_blocks(out_cap) : 0;
  if (row_blocks + pads == 0) return VH_OK;
  hipLaunchKernelGGL(k_cols_fill, dim3(row_blocks + pads), dim3(ROW_WAVES * 64), 0, st, data, (int)dtype, indices,
                     indptr, rows, cap, start, end, out_cap, (const int32_t*)out_indptr, (int)row_blocks, out_data,
                     out_indices);
  return vh::check_launch("vh_slice_csr");
}

extern "C" int vh_spmm_csr(const void* data, int32_t data_dtype, const int32_t* indices, const int32_t* indptr,
                           int64_t batch, int64_t rows, int64_t cap, const void* B, int32_t b_dtype, int32_t b_layout,
                           int64_t K, int64_t N, int64_t b_batch_stride, const float* base, void* out,
                           int32_t out_dtype, int32_t* work, vh_stream_t stream) {
  VH_REQUIRE(float_dtype(data_dtype) && float_dtype(b_dtype) && float_dtype(out_dtype),
             "vh_spmm_csr: dtypes must be bf16, fp16 or fp32");
  VH_REQUIRE(b_layout == 0 || b_layout == 1, "vh_spmm_csr: weight layout must be kc (0) or ck (1)");
  VH_REQUIRE(batch >= 1 && batch <= 65535 && rows >= 0 && rows < (1 << 26) && cap >= 0 && cap < ((int64_t)1 << 31) &&
                 K >= 1 && N >= 0,
             "vh_spmm_csr: bad sizes (batch %lld, rows %lld, cap %lld, K %lld, N %lld)", (long long)batch,
             (long long)rows, (long long)cap, (long long)K, (long long)N);
  const int esz = b_dtype == VH_F32 ? 4 : 2;
  VH_REQUIRE(K * esz + 16 <= SPMM_LDS,
             "vh_spmm_csr: K = %lld does not fit one LDS tile column (at most %d bytes per column)", (long long)K,
             SPMM_LDS);
  const hipStream_t st = vh::as_stream(stream);
  hipLaunchKernelGGL(k_rowptr_rebase, dim3((unsigned)batch), dim3(SCAN_THREADS), 0, st, indptr, rows, cap, work);
  if (int e = vh::check_launch("vh_spmm_csr")) return e;
  if (rows == 0 || N == 0) return VH_OK;
  // the widest tile of B columns whose K rows fit the LDS budget
  int nt = 16;
  while (nt > 1 && (int64_t)nt * (K * esz + 16) > SPMM_LDS) nt >>= 1;
#define VH_SPMM(NT)                                                                                                  \
  return esz == 2 ? launch_spmm<NT, 2>(data, data_dtype, indices, work, batch, rows, cap, B, b_dtype, b_layout, K, N, \
                                       b_batch_stride, base, out, out_dtype, st)                                     \
                  : launch_spmm<NT, 4>(data, data_dtype, indices, work, batch, rows, cap, B, b_dtype, b_layout, K, N, \
                                       b_batch_stride, base, out, out_dtype, st)
  switch (nt) {
    case 16: VH_SPMM(16);
    case 8: VH_SPMM(8);
    case 4: VH_SPMM(4);
    case 2: VH_SPMM(2);
    default: VH_SPMM(1);
  }
#undef VH_SPMM
}
