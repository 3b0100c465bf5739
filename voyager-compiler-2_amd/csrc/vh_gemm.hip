// GEMM core of the quantized linear / matmul ops on gfx950 MFMA.
//
//   C[M, N] = epilogue( A[M, K] . B[N, K]^T )      (layout "xc,kc->xk")
//
// Operands are K-contiguous rows.  Element formats:
//   * OP_FP8  -- OCP E4M3 bytes -> v_mfma_f32_32x32x64_f8f6f4 (fp8 rate);
//   * OP_BF16 -- bfloat16       -> v_mfma_f32_32x32x16_bf16;
//   * OP_MXI8 -- int8 codes with one power-of-two scale byte per 16 (or any
//                power-of-two `block`) K elements; decoded exactly to
//                bfloat16 (code * 2**e) while staging, then bf16 MFMA;
//   * OP_P8   -- posit8 codes; decoded through a 256-entry table in LDS.
// Two kernels.  k_gemm_f8dl (FP8 x FP8 with bf16 output) loads its stages
// straight into LDS; it is described where it is defined.  k_gemm (every
// format pair) stages through registers: the block tile is BM x BN with a
// 128-byte K stage per row, double buffered in LDS (rows padded to 144 bytes
// so a wave's 16-byte fragment reads hit distinct banks); WM x WN waves, each
// owning a (BM/WM) x (BN/WN) sub-tile of 32 x 32 MFMA tiles.  In both, tiles
// are ordered so that blocks that share operand rows run on the same XCD
// (blocks are dealt to the 8 XCDs round robin).
#include <hip/hip_runtime.h>

#include <cstring>

#include "vh_device.h"
#include "vh_host.h"

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// Exact fp16 operands (vh_gemm_mx8_f16); internal to this file, not a
// descriptor format.
constexpr int OP_F16X = 16;

constexpr int ROWB = 128;   // bytes of K per row per stage
constexpr int ROWP = 144;   // padded LDS row pitch

struct GemmArgs {
  const uint8_t* A;
  const uint8_t* B;
  void* C;
  int64_t M, N, K;           // K in elements
  int64_t lda, ldb;          // row pitch in bytes of the stored operands
  int64_t ldc;               // row pitch of C in elements
  int a_fmt, b_fmt;          // OP_* of each operand
  const uint8_t* a_scale;    // OP_MXI8: [M, K/block] biased exponent bytes
  const uint8_t* b_scale;    // OP_MXI8: [N, K/block]
  int64_t lds_a, lds_b;      // scale row pitch (blocks per row)
  int a_block, b_block;      // elements per scale byte
  int a_bias, b_bias;        // scale = 2**(byte - bias)
  const uint16_t* lut;       // OP_P8: 256 bfloat16 entries (device)
  int64_t sa, sb, sc;        // batch strides: bytes of A / B, elements of C
  int64_t ssa, ssb;          // batch strides of the scale bytes
  int group_m;               // tile-rows per column walk (tile_origin)
  vh_epilogue epi;
  const int32_t* ea;         // OP_F16X, or null: per row of A and column of B, a power of two
  const int32_t* eb;         // the accumulator is multiplied by before the epilogue
};

// ------------------------------------------------------------ staging
// Global loads go through buffer resources: an access past the resource's
// end returns zero, so tile edges in M / N need no branches.  Rows shorter
// than a stage (the last K step) are masked with a select.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr int RSRC_WORD3 = 0x00020000;

__device__ __forceinline__ rsrc_t make_rsrc(const void* p, int64_t bytes) {
  int n = bytes > 0x7fffffff ? 0x7fffffff : (int)bytes;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, n, RSRC_WORD3);
}

__device__ __forceinline__ uint4 bload16(rsrc_t r, int off) {
  auto v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
  return make_uint4(v[0], v[1], v[2], v[3]);
}

__device__ __forceinline__ uint2 bload8(rsrc_t r, int off) {
  auto v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
  return make_uint2(v[0], v[1]);
}

__device__ __forceinline__ uint32_t bload1(rsrc_t r, int off) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(r, off, 0, 0);
}

// bf16 bits of int8 code c times 2**e.  Exact: |c| <= 128 needs 8
// significant bits and the block's nonzero codes come with 2**e >= 2**-133.
__device__ __forceinline__ uint32_t mxi8_bf16(int c, int e) {
  return __float_as_uint(ldexpf((float)c, e)) >> 16;
}

__device__ __forceinline__ uint4 decode_mxi8(uint2 raw, int e) {
  uint4 o;
  o.x = mxi8_bf16((int8_t)(raw.x & 0xff), e) | (mxi8_bf16((int8_t)((raw.x >> 8) & 0xff), e) << 16);
  o.y = mxi8_bf16((int8_t)((raw.x >> 16) & 0xff), e) | (mxi8_bf16((int8_t)(raw.x >> 24), e) << 16);
  o.z = mxi8_bf16((int8_t)(raw.y & 0xff), e) | (mxi8_bf16((int8_t)((raw.y >> 8) & 0xff), e) << 16);
  o.w = mxi8_bf16((int8_t)((raw.y >> 16) & 0xff), e) | (mxi8_bf16((int8_t)(raw.y >> 24), e) << 16);
  return o;
}

__device__ __forceinline__ uint4 decode_p8(uint2 raw, const uint16_t* lut) {
  uint32_t h[8];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    h[j] = lut[(raw.x >> (8 * j)) & 0xffu];
    h[4 + j] = lut[(raw.y >> (8 * j)) & 0xffu];
  }
  return make_uint4(h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16));
}

// One operand of the block: its rows as a buffer resource.
struct Operand {
  rsrc_t data;
  rsrc_t scale;
  int ld;       // row pitch (bytes)
  int sld;      // scale row pitch (bytes)
  int64_t K;    // elements
  int block_shift;
  int bias;
};

// Raw bytes of one 16-byte LDS chunk, as loaded: the chunk itself for fp8 /
// bf16; for decoded formats 8 code bytes in x, y and the block's scale byte
// in z.  Masking (past K) and decoding wait for the LDS store, after the
// stage's MFMAs, so the loads stay in flight while the MFMAs run.
template <int FMT>
__device__ __forceinline__ uint4 fetch_raw(const Operand& o, int r, int c, int64_t k0) {
  if constexpr (FMT == OP_FP8) {
    return bload16(o.data, r * o.ld + (int)(k0 + c * 16));
  } else if constexpr (FMT == OP_BF16) {
    return bload16(o.data, r * o.ld + (int)(k0 + c * 8) * 2);
  } else {
    const int64_t k = k0 + c * 8;
    const uint2 raw = bload8(o.data, r * o.ld + (int)k);
    uint32_t sc = 0;
    if constexpr (FMT == OP_MXI8) sc = bload1(o.scale, r * o.sld + (int)(k >> o.block_shift));
    return make_uint4(raw.x, raw.y, sc, 0);
  }
}

template <int FMT>
__device__ __forceinline__ uint4 finish_raw(const uint4& w, int c, int64_t k0, const Operand& o,
                                            const uint16_t* lut) {
  const int64_t k = k0 + c * (FMT == OP_FP8 ? 16 : 8);
  const uint32_t m = k < o.K ? 0xffffffffu : 0u;
  if constexpr (FMT == OP_FP8 || FMT == OP_BF16) {
    return make_uint4(w.x & m, w.y & m, w.z & m, w.w & m);
  } else {
    const uint2 raw = make_uint2(w.x & m, w.y & m);
    if constexpr (FMT == OP_MXI8) return decode_mxi8(raw, (int)w.z - o.bias);
    else return decode_p8(raw, lut);
  }
}

// ------------------------------------------------------------ epilogue
// Wave (wm, wn) holds TM x TN 32x32 accumulator tiles of its (32 TM) x
// (32 TN) sub-tile: lane holds column lane % 32 of each tile, rows
// (r/4)*8 + (lane/32)*4 + r%4 of accumulator element r.  The caller has
// finished with the LDS stage buffers (all waves past a barrier) when the
// bf16 path reuses them.
// True when the bf16 LDS-staged epilogue applies: bf16 output whose rows
// start 16-byte aligned and hold whole 8-element chunks.
__host__ __device__ inline bool lds_epilogue_ok(const void* C, int out_dtype, int64_t ldc, int64_t N) {
  return out_dtype == VH_BF16 && ((uintptr_t)C % 16) == 0 && (ldc % 8) == 0 && (N % 8) == 0;
}

// The epilogues of the direct-to-LDS kernels: the bf16 one above, or a
// float32 result stored from the (transposed) accumulators in 16-byte runs
// of four columns (store_tile_t_f32), which needs 16-byte aligned rows.
__host__ __device__ inline bool f8dl_epilogue_ok(const void* C, int out_dtype, int64_t ldc, int64_t N) {
  if (out_dtype == VH_F32) return ((uintptr_t)C % 16) == 0 && (ldc % 4) == 0;
  return lds_epilogue_ok(C, out_dtype, ldc, N);
}

__device__ __forceinline__ float epi_scale(const vh_epilogue& e) {
  if (!e.scale) return 1.0f;
  return e.scale_dtype == VH_BF16 ? bf2f(*(const uint16_t*)e.scale) : *(const float*)e.scale;
}

// Bytes of the direct-to-LDS kernel's bf16 epilogue staging (padded rows);
// its bias instantiations keep the tile's BN biases (float32) right after.
template <int BM, int BN, int WM, int WN>
constexpr int f8dl_epi_bytes() {
  return WM * WN * (BM / WM) * (BN / WN + 8) * 2;
}

// bf16 output through LDS: each wave rounds its sub-tile (hardware
// converter, round half to even), writes it row-major to LDS (padded rows,
// WM * WN * 32 TM * (32 TN + 8) bf16 in all), and stores whole 16-byte row
// chunks.  Needs lds_epilogue_ok.
template <int TM, int TN, int WM, int WN>
__device__ __forceinline__ void store_tile_lds(const GemmArgs& g, f32x16 (&acc)[TM][TN], uint8_t* smem, int64_t m0,
                                               int64_t n0, int wave, int wm, int wn, int lane) {
  const int lrow = lane & 31;
  const int lhalf = lane >> 5;
  const vh_epilogue& e = g.epi;
  const float sc = epi_scale(e);
  constexpr int SUBM = TM * 32, SUBN = TN * 32, PITCH = SUBN + 8;  // bf16 elements
  uint16_t* ct = (uint16_t*)smem + wave * SUBM * PITCH;
  const bool round_scale = e.mode == EPI_ROUND_SCALE;
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int64_t col = n0 + wn * SUBN + j * 32 + lrow;
    float bias = 0.0f;
    if (e.bias && col < g.N)
      bias = e.bias_dtype == VH_BF16 ? bf2f(((const uint16_t*)e.bias)[col]) : ((const float*)e.bias)[col];
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        float v0 = acc[i][j][r], v1 = acc[i][j][r + 1];
        if (round_scale) {
          // dequantize(linear(xq, wq), s): round to bf16, times s, round again
          const uint32_t b = f2bf2_hw(v0, v1);
          v0 = bf2f(b & 0xffffu) * sc;
          v1 = bf2f(b >> 16) * sc;
        } else {
          if (e.scale) {
            v0 *= sc;
            v1 *= sc;
          }
          if (e.bias) {
            v0 += bias;
            v1 += bias;
          }
        }
        const uint32_t o = f2bf2_hw(v0, v1);
        const int row = i * 32 + (r >> 2) * 8 + lhalf * 4 + (r & 3);
        ct[row * PITCH + j * 32 + lrow] = (uint16_t)(o & 0xffffu);
        ct[(row + 1) * PITCH + j * 32 + lrow] = (uint16_t)(o >> 16);
      }
      // one accumulator tile at a time keeps the register demand at 16
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  constexpr int CPR = SUBN / 8;  // 16-byte chunks per row
  static_assert((SUBM * CPR) % 64 == 0, "chunks must divide among the wave");
#pragma unroll
  for (int it = 0; it < SUBM * CPR / 64; ++it) {
    const int q = lane + 64 * it;
    const int row = q / CPR, ch = q % CPR;
    const int64_t grow = m0 + wm * SUBM + row;
    const int64_t gcol = n0 + wn * SUBN + ch * 8;
    const uint4 v = *(const uint4*)(ct + row * PITCH + ch * 8);
    if (grow < g.M && gcol < g.N) *(uint4*)((uint16_t*)g.C + grow * g.ldc + gcol) = v;
  }
}

// store_tile_lds for transposed accumulators: tile (i, j) holds rows n of
// B tile j by columns m of A tile i, so lane holds output row m = lane % 32
// and, per group q of four accumulator elements, four consecutive output
// columns n = 8 q + 4 (lane / 32) + {0..3}: one 8-byte LDS write each.
// MODE: 0 round-scale (dequantize(linear(xq, wq), s): round to bf16, times
// s, round again), 1 scale only, 2 scale and bias.
// MODE 2 (scale and bias): the tile's biases sb (float32, in LDS, one per
// column of the block tile, 0 past N) added before the rounding.
template <int TM, int TN>
__device__ __forceinline__ void stage_tile_t_bias(const GemmArgs& g, f32x16 (&acc)[TM][TN], uint16_t* ct,
                                                  const float* sb, int wn, int lane) {
  const int lrow = lane & 31;
  const int lhalf = lane >> 5;
  const float sc = epi_scale(g.epi);
  constexpr int SUBN = TN * 32, PITCH = SUBN + 8;
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int j = 0; j < TN; ++j) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int nl = j * 32 + q * 8 + lhalf * 4;
        const float4 bq = *(const float4*)(sb + wn * SUBN + nl);
        const float v0 = acc[i][j][4 * q] * sc + bq.x, v1 = acc[i][j][4 * q + 1] * sc + bq.y;
        const float v2 = acc[i][j][4 * q + 2] * sc + bq.z, v3 = acc[i][j][4 * q + 3] * sc + bq.w;
        *(uint2*)(ct + (i * 32 + lrow) * PITCH + nl) = make_uint2(f2bf2_hw(v0, v1), f2bf2_hw(v2, v3));
      }
      // one accumulator tile at a time keeps the register demand at 16
      __builtin_amdgcn_sched_barrier(0);
    }
  }
}

template <int TM, int TN, int MODE>
__device__ __forceinline__ void stage_tile_t(const GemmArgs& g, f32x16 (&acc)[TM][TN], uint16_t* ct, int64_t n0,
                                             int wn, int lane) {
  const int lrow = lane & 31;
  const int lhalf = lane >> 5;
  const vh_epilogue& e = g.epi;
  const float sc = epi_scale(e);
  constexpr int SUBN = TN * 32, PITCH = SUBN + 8;
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int j = 0; j < TN; ++j) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int nl = j * 32 + q * 8 + lhalf * 4;
        float v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          v[u] = acc[i][j][4 * q + u];
          if constexpr (MODE == 0) {
            v[u] = rbf(v[u]) * sc;
          } else {
            v[u] *= sc;
            if constexpr (MODE == 2) {
              const int64_t col = n0 + wn * SUBN + nl + u;
              if (col < g.N)
                v[u] += e.bias_dtype == VH_BF16 ? bf2f(((const uint16_t*)e.bias)[col]) : ((const float*)e.bias)[col];
            }
          }
        }
        *(uint2*)(ct + (i * 32 + lrow) * PITCH + nl) = make_uint2(f2bf2_hw(v[0], v[1]), f2bf2_hw(v[2], v[3]));
      }
      // one accumulator tile at a time keeps the register demand at 16
      __builtin_amdgcn_sched_barrier(0);
    }
  }
}

template <int TM, int TN, bool BIAS>
__device__ __forceinline__ void store_tile_lds_t(const GemmArgs& g, f32x16 (&acc)[TM][TN], uint8_t* smem, int64_t m0,
                                                 int64_t n0, int wave, int wm, int wn, int lane, const float* sb) {
  constexpr int SUBM = TM * 32, SUBN = TN * 32, PITCH = SUBN + 8;  // bf16 elements
  uint16_t* ct = (uint16_t*)smem + wave * SUBM * PITCH;
  if (g.epi.mode == EPI_ROUND_SCALE) stage_tile_t<TM, TN, 0>(g, acc, ct, n0, wn, lane);
  else if constexpr (!BIAS) stage_tile_t<TM, TN, 1>(g, acc, ct, n0, wn, lane);
  else stage_tile_t_bias<TM, TN>(g, acc, ct, sb, wn, lane);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  constexpr int CPR = SUBN / 8;  // 16-byte chunks per row
  static_assert((SUBM * CPR) % 64 == 0, "chunks must divide among the wave");
#pragma unroll
  for (int it = 0; it < SUBM * CPR / 64; ++it) {
    const int q = lane + 64 * it;
    const int row = q / CPR, ch = q % CPR;
    const int64_t grow = m0 + wm * SUBM + row;
    const int64_t gcol = n0 + wn * SUBN + ch * 8;
    const uint4 v = *(const uint4*)(ct + row * PITCH + ch * 8);
    if (grow < g.M && gcol < g.N) *(uint4*)((uint16_t*)g.C + grow * g.ldc + gcol) = v;
  }
}

__device__ __forceinline__ float epi_bias(const vh_epilogue& e, int64_t col) {
  if (!e.bias) return 0.0f;
  return e.bias_dtype == VH_BF16 ? bf2f(((const uint16_t*)e.bias)[col]) : ((const float*)e.bias)[col];
}

// The epilogue of one fp32 accumulator (sc = epi_scale, bias = epi_bias).
__device__ __forceinline__ float epi_value(const vh_epilogue& e, float v, float sc, float bias) {
  if (e.mode == EPI_ROUND_SCALE) {
    // dequantize(linear(xq, wq), s): the GEMM rounds to bf16, then the bf16
    // product with the scale rounds again.
    return rbf(rbf(v) * sc);
  }
  if (e.scale) v = v * sc;
  if (e.bias) v = v + bias;
  return v;
}

// Element-wise stores (f32 output, or bf16 rows the LDS path cannot take).
template <int TM, int TN, int WM, int WN>
__device__ __forceinline__ void store_tile_direct(const GemmArgs& g, f32x16 (&acc)[TM][TN], int64_t m0, int64_t n0,
                                                  int wm, int wn, int lane) {
  const int lrow = lane & 31;
  const int lhalf = lane >> 5;
  const vh_epilogue& e = g.epi;
  const float sc = epi_scale(e);
  constexpr int SUBM = TM * 32, SUBN = TN * 32;
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int64_t col = n0 + wn * SUBN + j * 32 + lrow;
      if (col >= g.N) continue;
      const float bias = epi_bias(e, col);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = m0 + wm * SUBM + i * 32 + (r >> 2) * 8 + lhalf * 4 + (r & 3);
        if (row >= g.M) continue;
        const float v = epi_value(e, acc[i][j][r], sc, bias);
        if (e.out_dtype == VH_BF16) ((uint16_t*)g.C)[row * g.ldc + col] = (uint16_t)f2bf(v);
        else ((float*)g.C)[row * g.ldc + col] = v;
      }
    }
  }
}

// Float32 result of transposed accumulators (B was the row operand: lane l
// holds row m = l % 32 of each 32 x 32 tile, columns (r / 4) * 8 +
// (l / 32) * 4 + r % 4): four consecutive columns per 16-byte store.
template <int TM, int TN, bool BIAS>
__device__ __forceinline__ void store_tile_t_f32(const GemmArgs& g, f32x16 (&acc)[TM][TN], int64_t m0, int64_t n0,
                                                 int wm, int wn, int lane, const float* sb) {
  const int lrow = lane & 31, lhalf = lane >> 5;
  const vh_epilogue& e = g.epi;
  const float sc = epi_scale(e);
  constexpr int SUBM = TM * 32, SUBN = TN * 32;
#pragma unroll
  for (int j = 0; j < TN; ++j) {
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int64_t row = m0 + wm * SUBM + i * 32 + lrow;
      if (row >= g.M) continue;
      float* crow = (float*)g.C + row * g.ldc;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int nl = j * 32 + q * 8 + lhalf * 4;
        const int64_t col = n0 + wn * SUBN + nl;
        float v[4];
        if constexpr (BIAS) {  // the plain epilogue (launch_f8dl routes a bias here only then)
          const float4 bq = *(const float4*)(sb + wn * SUBN + nl);
          const float b4[4] = {bq.x, bq.y, bq.z, bq.w};
#pragma unroll
          for (int u = 0; u < 4; ++u) v[u] = (e.scale ? acc[i][j][4 * q + u] * sc : acc[i][j][4 * q + u]) + b4[u];
        } else {
#pragma unroll
          for (int u = 0; u < 4; ++u) v[u] = epi_value(e, acc[i][j][4 * q + u], sc, 0.0f);
        }
        if (col + 3 < g.N) {
          *(float4*)(crow + col) = make_float4(v[0], v[1], v[2], v[3]);
        } else {
#pragma unroll
          for (int u = 0; u < 4; ++u)
            if (col + u < g.N) crow[col + u] = v[u];
        }
      }
    }
  }
}

// Epilogue of a block tile: wave (wm, wn) holds TM x TN 32x32 accumulator
// tiles of its (32 TM) x (32 TN) sub-tile; lane holds column lane % 32 of
// each tile, rows (r/4)*8 + (lane/32)*4 + r%4 of accumulator element r.  The
// caller has finished with the LDS stage buffers (all waves past a barrier).
template <int TM, int TN, int WM, int WN>
__device__ __forceinline__ void store_tile(const GemmArgs& g, f32x16 (&acc)[TM][TN], uint8_t* smem, int64_t m0,
                                           int64_t n0, int wave, int wm, int wn, int lane) {
  if (lds_epilogue_ok(g.C, g.epi.out_dtype, g.ldc, g.N))
    store_tile_lds<TM, TN, WM, WN>(g, acc, smem, m0, n0, wave, wm, wn, lane);
  else
    store_tile_direct<TM, TN, WM, WN>(g, acc, m0, n0, wm, wn, lane);
}

// Block tile id -> (m0, n0).  Blocks are dealt to the 8 XCDs round robin;
// when the tile count is a multiple of 8, consecutive tile ids are
// renumbered so that each XCD gets a contiguous range of them, and groups of
// GM tile-rows are walked column by column so an XCD's blocks share operand
// panels in its L2 (group_rows picks GM).
__device__ __forceinline__ void tile_origin(int64_t M, int64_t N, int BM, int BN, int GM, int64_t& m0, int64_t& n0) {
  const int64_t tiles_m = (M + BM - 1) / BM;
  const int64_t tiles_n = (N + BN - 1) / BN;
  const int64_t ntiles = tiles_m * tiles_n;
  int64_t pid = blockIdx.x;
  if ((ntiles & 7) == 0) pid = (pid & 7) * (ntiles >> 3) + (pid >> 3);
  const int64_t group = pid / (GM * tiles_n);
  const int64_t first_m = group * GM;
  const int64_t gsize = (tiles_m - first_m) < GM ? (tiles_m - first_m) : GM;
  const int64_t tm = first_m + (pid % (GM * tiles_n)) % gsize;
  const int64_t tn = (pid % (GM * tiles_n)) / gsize;
  m0 = tm * BM;
  n0 = tn * BN;
}

// BM x BN block tile computed by WM x WN waves; MINB blocks per CU; PF
// register sets of prefetched chunks (2: loads run two steps ahead).
template <int BM, int BN, int WM, int WN, int MINB, int PF, int AF, int BF>
__global__ void __launch_bounds__(WM * WN * 64, MINB) k_gemm(GemmArgs g) {
  constexpr bool FP8 = AF == OP_FP8;
  constexpr int NT = WM * WN * 64;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  uint8_t* As = smem;                          // [2][BM][ROWP]
  uint8_t* Bs = smem + 2 * BM * ROWP;          // [2][BN][ROWP]
  uint16_t* lut = (uint16_t*)(smem + 2 * (BM + BN) * ROWP);  // [256] for OP_P8

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;

  if constexpr (AF == OP_P8 || BF == OP_P8) {
    for (int i = tid; i < 256; i += NT) lut[i] = g.lut[i];
    __syncthreads();
  }

  int64_t m0, n0;
  tile_origin(g.M, g.N, BM, BN, g.group_m, m0, n0);
  const int64_t bat = blockIdx.y;
  g.A += bat * g.sa;
  g.B += bat * g.sb;
  g.C = (uint8_t*)g.C + bat * g.sc * (g.epi.out_dtype == VH_BF16 ? 2 : 4);
  if (g.a_scale) g.a_scale += bat * g.ssa;
  if (g.b_scale) g.b_scale += bat * g.ssb;

  const int64_t rows_a = (g.M - m0) < BM ? (g.M - m0) : BM;
  const int64_t rows_b = (g.N - n0) < BN ? (g.N - n0) : BN;
  Operand oa, ob;
  oa.data = make_rsrc(g.A + m0 * g.lda, rows_a * g.lda);
  ob.data = make_rsrc(g.B + n0 * g.ldb, rows_b * g.ldb);
  oa.ld = (int)g.lda;
  ob.ld = (int)g.ldb;
  oa.K = ob.K = g.K;
  if constexpr (AF == OP_MXI8) {
    oa.scale = make_rsrc(g.a_scale + m0 * g.lds_a, rows_a * g.lds_a);
    oa.sld = (int)g.lds_a;
    oa.block_shift = __builtin_ctz(g.a_block);
    oa.bias = g.a_bias;
  }
  if constexpr (BF == OP_MXI8) {
    ob.scale = make_rsrc(g.b_scale + n0 * g.lds_b, rows_b * g.lds_b);
    ob.sld = (int)g.lds_b;
    ob.block_shift = __builtin_ctz(g.b_block);
    ob.bias = g.b_bias;
  }

  constexpr int KE = FP8 ? 128 : 64;      // K elements per stage
  constexpr int CA = BM * 8 / NT;         // 16-byte chunks per thread (A)
  constexpr int CB = BN * 8 / NT;
  static_assert(CA >= 1 && CB >= 1, "tile too small");

  // Two register sets of prefetched chunks: the loads for step k+2 are
  // issued while step k computes, so each has a whole step to land before
  // its LDS store.
  uint4 ra0[CA], rb0[CB], ra1[PF == 2 ? CA : 1], rb1[PF == 2 ? CB : 1];
  auto fetch = [&](uint4* ra, uint4* rb, int64_t k0) {
#pragma unroll
    for (int i = 0; i < CA; ++i) {
      int ch = tid + i * NT;
      ra[i] = fetch_raw<AF>(oa, ch >> 3, ch & 7, k0);
    }
#pragma unroll
    for (int i = 0; i < CB; ++i) {
      int ch = tid + i * NT;
      rb[i] = fetch_raw<BF>(ob, ch >> 3, ch & 7, k0);
    }
  };
  auto stash = [&](const uint4* ra, const uint4* rb, int s, int64_t k0) {
    uint8_t* a = As + s * BM * ROWP;
    uint8_t* b = Bs + s * BN * ROWP;
#pragma unroll
    for (int i = 0; i < CA; ++i) {
      int ch = tid + i * NT;
      *(uint4*)(a + (ch >> 3) * ROWP + (ch & 7) * 16) = finish_raw<AF>(ra[i], ch & 7, k0, oa, lut);
    }
#pragma unroll
    for (int i = 0; i < CB; ++i) {
      int ch = tid + i * NT;
      *(uint4*)(b + (ch >> 3) * ROWP + (ch & 7) * 16) = finish_raw<BF>(rb[i], ch & 7, k0, ob, lut);
    }
  };

  constexpr int TM = BM / WM / 32;  // 32-row MFMA tiles per wave
  constexpr int TN = BN / WN / 32;
  static_assert(TM >= 1 && TN >= 1 && BM % (WM * 32) == 0 && BN % (WN * 32) == 0, "bad wave layout");
  static_assert((BM * 8) % NT == 0 && (BN * 8) % NT == 0, "stage chunks must divide among threads");
  static_assert(WN * BM * (BN / WN + 8) * 2 <= 2 * (BM + BN) * ROWP, "epilogue tile does not fit the stage LDS");
  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int lrow = lane & 31;
  const int lhalf = lane >> 5;
  auto compute = [&](int s) {
    const uint8_t* a = As + s * BM * ROWP + (wm * (BM / WM) + lrow) * ROWP;
    const uint8_t* b = Bs + s * BN * ROWP + (wn * (BN / WN) + lrow) * ROWP;
    if constexpr (FP8) {
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        const int off = kk * 64 + lhalf * 32;
        i32x8 fa[TM], fb[TN];
#pragma unroll
        for (int i = 0; i < TM; ++i) {
          uint4 lo = *(const uint4*)(a + i * 32 * ROWP + off);
          uint4 hi = *(const uint4*)(a + i * 32 * ROWP + off + 16);
          fa[i] = i32x8{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
        }
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          uint4 lo = *(const uint4*)(b + j * 32 * ROWP + off);
          uint4 hi = *(const uint4*)(b + j * 32 * ROWP + off + 16);
          fb[j] = i32x8{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
        }
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fa[i], fb[j], acc[i][j], 0, 0, 0, 127, 0,
                                                                          127);
      }
    } else {
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const int off = kk * 32 + lhalf * 16;
        bf16x8 fa[TM], fb[TN];
#pragma unroll
        for (int i = 0; i < TM; ++i) fa[i] = *(const bf16x8*)(a + i * 32 * ROWP + off);
#pragma unroll
        for (int j = 0; j < TN; ++j) fb[j] = *(const bf16x8*)(b + j * 32 * ROWP + off);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
      }
    }
  };

  // Steps are taken in pairs so the two register sets have fixed names.
  // Past the end of K every chunk is masked to zero, so an odd last step
  // adds nothing.
  const int64_t nk = (g.K + KE - 1) / KE;
  if constexpr (PF == 1) {
    fetch(ra0, rb0, 0);
    stash(ra0, rb0, 0, 0);
    __syncthreads();
    for (int64_t ks = 0; ks < nk; ++ks) {
      const int st = ks & 1;
      fetch(ra0, rb0, (ks + 1) * KE);
      __builtin_amdgcn_sched_barrier(0);
      compute(st);
      __builtin_amdgcn_sched_barrier(0);
      stash(ra0, rb0, st ^ 1, (ks + 1) * KE);
      __syncthreads();
    }
  } else {
  fetch(ra0, rb0, 0);
  fetch(ra1, rb1, KE);
  stash(ra0, rb0, 0, 0);
  __syncthreads();
  for (int64_t ks = 0; ks < nk; ks += 2) {
    fetch(ra0, rb0, (ks + 2) * KE);
    __builtin_amdgcn_sched_barrier(0);
    compute(0);
    __builtin_amdgcn_sched_barrier(0);
    stash(ra1, rb1, 1, (ks + 1) * KE);
    __syncthreads();
    if (ks + 1 >= nk) break;
    fetch(ra1, rb1, (ks + 3) * KE);
    __builtin_amdgcn_sched_barrier(0);
    compute(1);
    __builtin_amdgcn_sched_barrier(0);
    stash(ra0, rb0, 0, (ks + 2) * KE);
    __syncthreads();
  }
  }

  store_tile<TM, TN, WM, WN>(g, acc, smem, m0, n0, wave, wm, wn, lane);
}

// ------------------------------------------------------------ MX-int8
// MX-int8 x MX-int8 (int8 codes, one biased power-of-two scale byte per
// block >= 16 K elements): a 64-element K stage is four 16-code chunks per
// row; each chunk is one 16-byte load plus one scale byte (a chunk never
// straddles a block), decoded exactly to bf16 (code * 2**e: at most 8
// significant bits) into LDS rows laid out as k_gemm's bf16 stages, then
// v_mfma_f32_32x32x16_bf16.  Every element is decoded once per block tile
// (2.5 VALU ops: sign-extending convert, ldexp, half a v_perm), the chunk
// offsets are computed once, and loads run two stages ahead in registers.
// gridDim.y splits K: split z covers [z kc, (z + 1) kc) and, with more than
// one split, stores its fp32 partial tile at part + z M N; k_split_reduce
// adds the partials in split order and applies the epilogue.
constexpr int MX_KE = 64;  // K elements per stage

__device__ __forceinline__ uint32_t pack_hi16(float lo, float hi) {
  return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}

// 16 int8 codes times 2**e -> 16 bf16 (truncation of an exact fp32 value).
__device__ __forceinline__ void decode16_mxi8(const uint4& raw, int e, uint4& lo, uint4& hi) {
  const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
  uint32_t o[8];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float f0 = ldexpf((float)(int8_t)(w[j] & 0xffu), e);
    const float f1 = ldexpf((float)(int8_t)((w[j] >> 8) & 0xffu), e);
    const float f2 = ldexpf((float)(int8_t)((w[j] >> 16) & 0xffu), e);
    const float f3 = ldexpf((float)(int8_t)(w[j] >> 24), e);
    o[2 * j] = pack_hi16(f0, f1);
    o[2 * j + 1] = pack_hi16(f2, f3);
  }
  lo = make_uint4(o[0], o[1], o[2], o[3]);
  hi = make_uint4(o[4], o[5], o[6], o[7]);
}

template <int BM, int BN, int WM, int WN, int P>
__global__ void __launch_bounds__(WM * WN * 64) k_gemm_mxi8(GemmArgs g, int64_t kc, float* __restrict__ part) {
  constexpr int NT = WM * WN * 64;
  constexpr int CA = BM * 4 / NT, CB = BN * 4 / NT;  // 16-code chunks per thread and stage
  static_assert(CA >= 1 && CB >= 1 && (BM * 4) % NT == 0 && (BN * 4) % NT == 0, "stage chunks must divide");
  constexpr int TM = BM / WM / 32, TN = BN / WN / 32;
  static_assert(TM >= 1 && TN >= 1 && BM % (WM * 32) == 0 && BN % (WN * 32) == 0, "bad wave layout");
  static_assert(WN * BM * (BN / WN + 8) * 2 <= 2 * (BM + BN) * ROWP, "epilogue tile does not fit the stage LDS");
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  uint8_t* As = smem;                  // [2][BM][ROWP]: 64 bf16 per row
  uint8_t* Bs = smem + 2 * BM * ROWP;  // [2][BN][ROWP]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  int64_t m0, n0;
  tile_origin(g.M, g.N, BM, BN, g.group_m, m0, n0);
  const int64_t k_lo = (int64_t)blockIdx.y * kc;
  const int64_t k_hi = (k_lo + kc) < g.K ? (k_lo + kc) : g.K;
  const int nk = (int)((k_hi - k_lo) / MX_KE);  // kc and K are multiples of MX_KE

  const int64_t rows_a = (g.M - m0) < BM ? (g.M - m0) : BM;
  const int64_t rows_b = (g.N - n0) < BN ? (g.N - n0) : BN;
  const rsrc_t ad = make_rsrc(g.A + m0 * g.lda, rows_a * g.lda);
  const rsrc_t bd = make_rsrc(g.B + n0 * g.ldb, rows_b * g.ldb);
  const rsrc_t as = make_rsrc(g.a_scale + m0 * g.lds_a, rows_a * g.lds_a);
  const rsrc_t bs = make_rsrc(g.b_scale + n0 * g.lds_b, rows_b * g.lds_b);
  const int ash = __builtin_ctz(g.a_block), bsh = __builtin_ctz(g.b_block);

  // chunk i of this thread: row ch / 4, K offset 16 (ch % 4) within the stage
  int aoff[CA], asrow[CA], ak[CA], boff[CB], bsrow[CB], bk[CB];
#pragma unroll
  for (int i = 0; i < CA; ++i) {
    const int ch = tid + i * NT, r = ch >> 2;
    ak[i] = (int)k_lo + (ch & 3) * 16;
    aoff[i] = r * (int)g.lda + ak[i];
    asrow[i] = r * (int)g.lds_a;
  }
#pragma unroll
  for (int i = 0; i < CB; ++i) {
    const int ch = tid + i * NT, r = ch >> 2;
    bk[i] = (int)k_lo + (ch & 3) * 16;
    boff[i] = r * (int)g.ldb + bk[i];
    bsrow[i] = r * (int)g.lds_b;
  }

  static_assert(P >= 2 && P % 2 == 0, "an even number of register sets");
  uint4 ra[P][CA], rb[P][CB];
  uint32_t sa[P][CA], sb[P][CB];
  // Stage s into set j (clamped to the last stage: a prefetch past the
  // split's end re-reads it and is never stored).
  auto fetch = [&](int j, int s) {
    const int kr = (s < nk ? s : nk - 1) * MX_KE;
#pragma unroll
    for (int i = 0; i < CA; ++i) {
      ra[j][i] = bload16(ad, aoff[i] + kr);
      sa[j][i] = bload1(as, asrow[i] + ((ak[i] + kr) >> ash));
    }
#pragma unroll
    for (int i = 0; i < CB; ++i) {
      rb[j][i] = bload16(bd, boff[i] + kr);
      sb[j][i] = bload1(bs, bsrow[i] + ((bk[i] + kr) >> bsh));
    }
  };
  auto stash = [&](int j, int st) {
    uint8_t* a = As + st * BM * ROWP;
    uint8_t* b = Bs + st * BN * ROWP;
#pragma unroll
    for (int i = 0; i < CA; ++i) {
      const int ch = tid + i * NT;
      uint4 lo, hi;
      decode16_mxi8(ra[j][i], (int)sa[j][i] - g.a_bias, lo, hi);
      uint8_t* d = a + (ch >> 2) * ROWP + (ch & 3) * 32;
      *(uint4*)d = lo;
      *(uint4*)(d + 16) = hi;
    }
#pragma unroll
    for (int i = 0; i < CB; ++i) {
      const int ch = tid + i * NT;
      uint4 lo, hi;
      decode16_mxi8(rb[j][i], (int)sb[j][i] - g.b_bias, lo, hi);
      uint8_t* d = b + (ch >> 2) * ROWP + (ch & 3) * 32;
      *(uint4*)d = lo;
      *(uint4*)(d + 16) = hi;
    }
  };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
  const int lrow = lane & 31;
  const int lhalf = lane >> 5;
  auto compute = [&](int st) {
    const uint8_t* a = As + st * BM * ROWP + (wm * (BM / WM) + lrow) * ROWP;
    const uint8_t* b = Bs + st * BN * ROWP + (wn * (BN / WN) + lrow) * ROWP;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int off = kk * 32 + lhalf * 16;
      bf16x8 fa[TM], fb[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) fa[i] = *(const bf16x8*)(a + i * 32 * ROWP + off);
#pragma unroll
      for (int j = 0; j < TN; ++j) fb[j] = *(const bf16x8*)(b + j * 32 * ROWP + off);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
    }
  };

  // P register sets in a ring and two LDS buffers: while stage s computes
  // from LDS buffer s % 2, stage s + 1 is decoded into the other buffer and
  // stages s + 2 .. s + P are in flight.  (Measured at M = 256: four sets,
  // or letting the decode interleave with the MFMAs, gain nothing over two.)
#pragma unroll
  for (int j = 0; j < P; ++j) fetch(j, j);
  stash(0, 0);
  __syncthreads();
  for (int ks = 0; ks < nk; ks += P) {
#pragma unroll
    for (int j = 0; j < P; ++j) {
      // stage ks + j is in LDS buffer j % 2; set j is free
      fetch(j, ks + j + P);
      __builtin_amdgcn_sched_barrier(0);
      compute(j & 1);
      __builtin_amdgcn_sched_barrier(0);
      if (ks + j + 1 >= nk) goto done;
      stash((j + 1) % P, (j + 1) & 1);
      __syncthreads();
    }
  }
done:
  __syncthreads();  // the LDS epilogue reuses the stage buffers
  if (gridDim.y == 1) {
    store_tile<TM, TN, WM, WN>(g, acc, smem, m0, n0, wave, wm, wn, lane);
  } else {
    GemmArgs p = g;
    p.C = part + (int64_t)blockIdx.y * g.M * g.N;
    p.ldc = g.N;
    p.epi.mode = EPI_PLAIN;
    p.epi.out_dtype = VH_F32;
    p.epi.scale = nullptr;
    p.epi.bias = nullptr;
    store_tile_direct<TM, TN, WM, WN>(p, acc, m0, n0, wm, wn, lane);
  }
}

// The same computation with the roles split between waves: 4 consumer
// waves (2 x 2, each a (BM/2) x (BN/2) sub-tile) run the MFMAs of stage s
// from one LDS buffer while 4 producer waves decode stage s + 1 into the
// other and have stage s + 2's loads in flight; one barrier per stage.  On a
// SIMD the consumer's matrix ops and the producer's VALU decode overlap,
// where the uniform kernel's waves all decode, then all multiply.
template <int BM, int BN>
__global__ void __launch_bounds__(512) k_gemm_mxi8_ws(GemmArgs g, int64_t kc, float* __restrict__ part) {
  constexpr int NP = 256;                            // producer threads
  constexpr int CA = BM * 4 / NP, CB = BN * 4 / NP;  // 16-code chunks per producer thread and stage
  static_assert(CA >= 1 && CB >= 1 && (BM * 4) % NP == 0 && (BN * 4) % NP == 0, "stage chunks must divide");
  constexpr int WM = 2, WN = 2;
  constexpr int TM = BM / WM / 32, TN = BN / WN / 32;
  static_assert(TM >= 1 && TN >= 1, "bad wave layout");
  static_assert(WN * BM * (BN / WN + 8) * 2 <= 2 * (BM + BN) * ROWP, "epilogue tile does not fit the stage LDS");
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  uint8_t* As = smem;
  uint8_t* Bs = smem + 2 * BM * ROWP;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool consumer = wave < 4;
  int64_t m0, n0;
  tile_origin(g.M, g.N, BM, BN, g.group_m, m0, n0);
  const int64_t k_lo = (int64_t)blockIdx.y * kc;
  const int64_t k_hi = (k_lo + kc) < g.K ? (k_lo + kc) : g.K;
  const int nk = (int)((k_hi - k_lo) / MX_KE);

  // ---- producer state (unused by consumer waves)
  const int pt = tid - 256;
  const int64_t rows_a = (g.M - m0) < BM ? (g.M - m0) : BM;
  const int64_t rows_b = (g.N - n0) < BN ? (g.N - n0) : BN;
  const rsrc_t ad = make_rsrc(g.A + m0 * g.lda, rows_a * g.lda);
  const rsrc_t bd = make_rsrc(g.B + n0 * g.ldb, rows_b * g.ldb);
  const rsrc_t as = make_rsrc(g.a_scale + m0 * g.lds_a, rows_a * g.lds_a);
  const rsrc_t bs = make_rsrc(g.b_scale + n0 * g.lds_b, rows_b * g.lds_b);
  const int ash = __builtin_ctz(g.a_block), bsh = __builtin_ctz(g.b_block);
  int aoff[CA], asrow[CA], ak[CA], boff[CB], bsrow[CB], bk[CB];
#pragma unroll
  for (int i = 0; i < CA; ++i) {
    const int ch = pt + i * NP, r = ch >> 2;
    ak[i] = (int)k_lo + (ch & 3) * 16;
    aoff[i] = r * (int)g.lda + ak[i];
    asrow[i] = r * (int)g.lds_a;
  }
#pragma unroll
  for (int i = 0; i < CB; ++i) {
    const int ch = pt + i * NP, r = ch >> 2;
    bk[i] = (int)k_lo + (ch & 3) * 16;
    boff[i] = r * (int)g.ldb + bk[i];
    bsrow[i] = r * (int)g.lds_b;
  }
  uint4 ra[2][CA], rb[2][CB];
  uint32_t sa[2][CA], sb[2][CB];
  auto fetch = [&](int j, int s) {
    const int kr = (s < nk ? s : nk - 1) * MX_KE;
#pragma unroll
    for (int i = 0; i < CA; ++i) {
      ra[j][i] = bload16(ad, aoff[i] + kr);
      sa[j][i] = bload1(as, asrow[i] + ((ak[i] + kr) >> ash));
    }
#pragma unroll
    for (int i = 0; i < CB; ++i) {
      rb[j][i] = bload16(bd, boff[i] + kr);
      sb[j][i] = bload1(bs, bsrow[i] + ((bk[i] + kr) >> bsh));
    }
  };
  auto stash = [&](int j, int st) {
    uint8_t* a = As + st * BM * ROWP;
    uint8_t* b = Bs + st * BN * ROWP;
#pragma unroll
    for (int i = 0; i < CA; ++i) {
      const int ch = pt + i * NP;
      uint4 lo, hi;
      decode16_mxi8(ra[j][i], (int)sa[j][i] - g.a_bias, lo, hi);
      uint8_t* d = a + (ch >> 2) * ROWP + (ch & 3) * 32;
      *(uint4*)d = lo;
      *(uint4*)(d + 16) = hi;
    }
#pragma unroll
    for (int i = 0; i < CB; ++i) {
      const int ch = pt + i * NP;
      uint4 lo, hi;
      decode16_mxi8(rb[j][i], (int)sb[j][i] - g.b_bias, lo, hi);
      uint8_t* d = b + (ch >> 2) * ROWP + (ch & 3) * 32;
      *(uint4*)d = lo;
      *(uint4*)(d + 16) = hi;
    }
  };

  // ---- consumer state
  const int wm = (wave & 3) / WN, wn = (wave & 3) % WN;
  const int lrow = lane & 31;
  const int lhalf = lane >> 5;
  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
  auto compute = [&](int st) {
    const uint8_t* a = As + st * BM * ROWP + (wm * (BM / WM) + lrow) * ROWP;
    const uint8_t* b = Bs + st * BN * ROWP + (wn * (BN / WN) + lrow) * ROWP;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int off = kk * 32 + lhalf * 16;
      bf16x8 fa[TM], fb[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) fa[i] = *(const bf16x8*)(a + i * 32 * ROWP + off);
#pragma unroll
      for (int j = 0; j < TN; ++j) fb[j] = *(const bf16x8*)(b + j * 32 * ROWP + off);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
    }
  };

  // Iteration k: consumers multiply stage k (buffer k % 2); producers issue
  // stage k + 2's loads into the register set stage k used, then decode
  // stage k + 1 into buffer (k + 1) % 2.  Both buffers are safe: buffer
  // (k + 1) % 2 was last read in iteration k - 1, before its barrier.
  if (!consumer) {
    fetch(0, 0);
    fetch(1, 1);
    stash(0, 0);
  }
  __syncthreads();
  for (int k = 0; k < nk; k += 2) {
    if (consumer) {
      compute(0);
    } else {
      fetch(0, k + 2);
      if (k + 1 < nk) stash(1, 1);
    }
    __syncthreads();
    if (k + 1 >= nk) break;
    if (consumer) {
      compute(1);
    } else {
      fetch(1, k + 3);
      if (k + 2 < nk) stash(0, 0);
    }
    __syncthreads();
  }
  if (!consumer) return;  // no barrier follows: the epilogue syncs within each wave
  if (gridDim.y == 1) {
    store_tile<TM, TN, WM, WN>(g, acc, smem, m0, n0, wave, wm, wn, lane);
  } else {
    GemmArgs p = g;
    p.C = part + (int64_t)blockIdx.y * g.M * g.N;
    p.ldc = g.N;
    p.epi.mode = EPI_PLAIN;
    p.epi.out_dtype = VH_F32;
    p.epi.scale = nullptr;
    p.epi.bias = nullptr;
    store_tile_direct<TM, TN, WM, WN>(p, acc, m0, n0, wm, wn, lane);
  }
}

// C = epilogue(sum over z of part[z]) for split-K partials [S][M][N] (fp32),
// summed in split order; four consecutive elements of a row per thread
// (N % 4 == 0).
// ea / eb (or null): per row of A and column of B, a power of two the sum
// is multiplied by before the epilogue (the exact fp16 operands' rebasing).
__global__ void __launch_bounds__(256) k_split_reduce(const float* __restrict__ part, int S, int64_t M, int64_t N,
                                                      vh_epilogue e, void* __restrict__ C, int64_t ldc,
                                                      const int32_t* __restrict__ ea = nullptr,
                                                      const int32_t* __restrict__ eb = nullptr) {
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  const int64_t MN = M * N;
  if (i >= MN) return;
  float4 v = *(const float4*)(part + i);
  for (int z = 1; z < S; ++z) {
    const float4 t = *(const float4*)(part + z * MN + i);
    v.x += t.x;
    v.y += t.y;
    v.z += t.z;
    v.w += t.w;
  }
  const int64_t row = i / N, col = i % N;
  if (ea) {
    const int r = ea[row];
    v.x = ldexpf(v.x, r + eb[col]);
    v.y = ldexpf(v.y, r + eb[col + 1]);
    v.z = ldexpf(v.z, r + eb[col + 2]);
    v.w = ldexpf(v.w, r + eb[col + 3]);
  }
  const float sc = epi_scale(e);
  const float r0 = epi_value(e, v.x, sc, epi_bias(e, col));
  const float r1 = epi_value(e, v.y, sc, epi_bias(e, col + 1));
  const float r2 = epi_value(e, v.z, sc, epi_bias(e, col + 2));
  const float r3 = epi_value(e, v.w, sc, epi_bias(e, col + 3));
  if (e.out_dtype == VH_BF16) {
    uint16_t* c = (uint16_t*)C + row * ldc + col;
    c[0] = (uint16_t)f2bf(r0);
    c[1] = (uint16_t)f2bf(r1);
    c[2] = (uint16_t)f2bf(r2);
    c[3] = (uint16_t)f2bf(r3);
  } else {
    float* c = (float*)C + row * ldc + col;
    c[0] = r0;
    c[1] = r1;
    c[2] = r2;
    c[3] = r3;
  }
}

// ------------------------------------------------------------ fp8 x fp8
// E4M3 x E4M3 with the stage loads going straight from global memory into
// LDS (buffer_load_dwordx4 ... lds): no staging registers, so NS stages of
// KS K-bytes per row stay in flight in LDS while WM x WN waves (4: one per
// SIMD, accumulators in AGPRs; 8: two per SIMD, so one issues MFMAs while
// the other waits on a load) each run a (BM/WM) x (BN/WN) sub-tile of
// 32x32x64 MFMAs, KS / 64 steps per stage.
//
// Stage layout: A rows then B rows, KS bytes each, the row's 16-byte chunks
// stored at chunk ^ swz(row % 16).  A DMA instruction writes 1 KB of LDS
// contiguously (1024 / KS rows), lane l to byte 16 l, so the swizzle is
// applied by choosing which global chunk each lane fetches; with KS = 128
// every instruction reads whole 128-byte lines.  swz keeps the fragment
// reads (lane l: row l % 32, chunks 4 t + 2 (l / 32) + {0, 1} of step t) on
// distinct 16-byte bank groups for every aligned group of 8 lanes within
// 128 bytes and of 16 lanes within 256 bytes.
//
// Stage s: its fragments for step 0 are in registers; each step runs its
// MFMAs with the next step's fragment reads interleaved.  The DMA of stage
// s + NS - 1 (into the buffer stage s - 1 used) is spread over the MFMAs up
// to the middle of the last step, where the wave waits for its own DMA of
// stage s + 1, waits for its LDS reads, and meets the other waves at a
// barrier; after it, the reads of stage s + 1's first fragments.  Buffer
// reuse is safe: every read of stage s - 1's buffer precedes the barrier of
// stage s - 1 in its wave, and the DMA into it follows that barrier.
template <int KS>
__device__ __forceinline__ int swz(int r) {
  if constexpr (KS == 64) return ((r >> 1) & 3) ^ ((r >> 3) & 1);
  else return (r & 7) ^ ((r >> 3) & 1);
}

typedef __attribute__((address_space(3))) void lds_void;

template <int NST>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(NST >= 0 && NST < 64, "vmcnt range");
  // s_waitcnt vmcnt(NST), expcnt / lgkmcnt left at their maxima
  __builtin_amdgcn_s_waitcnt((NST & 15) | (7 << 4) | (15 << 8) | ((NST >> 4) << 14));
}

// Waits for this wave's outstanding LDS reads, then meets the workgroup.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

typedef int i32x4 __attribute__((ext_vector_type(4)));

// Buffer descriptor words of a raw (unswizzled) resource over [p, p + bytes).
// The words are workgroup-uniform; readfirstlane keeps them in SGPRs, as the
// inline asm that consumes them requires.
__device__ __forceinline__ i32x4 raw_desc(const void* p, int64_t bytes) {
  const uint64_t a = (uint64_t)(uintptr_t)p;
  const int n = bytes > 0x7fffffff ? 0x7fffffff : (int)bytes;
  return i32x4{__builtin_amdgcn_readfirstlane((int)(uint32_t)a),
               __builtin_amdgcn_readfirstlane((int)(uint32_t)((a >> 32) & 0xffffu)),
               __builtin_amdgcn_readfirstlane(n), RSRC_WORD3};
}

// 16 bytes per lane from rsrc + voff straight into LDS at lds + 16 lane.
// Written as inline asm so the compiler adds no wait of its own for it: the
// stage protocol orders these writes (vmcnt waits and barriers).  An offset
// past the resource reads zero.  m0 carries the LDS address (one wait state
// before the load uses it: the s_nop).
__device__ __forceinline__ void dma16(const i32x4& rsrc, uint32_t lds, int voff) {
  asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" : : "v"(voff), "s"(rsrc), "{m0}"(lds) : "memory");
}

// Waves per SIMD the direct-to-LDS kernel asks for: one per four waves of
// its workgroup (at least one).
constexpr int f8dl_wpe(int nw) { return nw >= 4 ? nw / 4 : 1; }

template <int BM, int BN, int NS, int KS, int WM, int WN, int OP, bool BIAS>
__global__ void __launch_bounds__(WM * WN * 64, f8dl_wpe(WM * WN))
    __attribute__((amdgpu_waves_per_eu(f8dl_wpe(WM * WN), f8dl_wpe(WM * WN)))) k_gemm_f8dl(GemmArgs g) {
  constexpr int P = KS / 64;                 // MFMA steps per stage
  constexpr int CPR = KS / 16;               // 16-byte chunks per row
  constexpr int RPI = 64 / CPR;              // rows per DMA instruction
  constexpr int STAGE = (BM + BN) * KS;      // bytes per stage buffer
  constexpr int NW = WM * WN;                // waves
  constexpr int TM = BM / WM / 32, TN = BN / WN / 32;  // 32x32 tiles per wave
  constexpr int LA = BM / RPI / NW, LB = BN / RPI / NW;  // DMA instructions per wave and stage
  constexpr int L = LA + LB;
  static_assert((KS == 64 || KS == 128) && BM % 64 == 0 && BN % 32 == 0 && NS >= 2 && (NS * P) % 2 == 0,
                "bad fp8 tile");
  static_assert(OP == OP_FP8 || OP == OP_BF16 || OP == OP_F16X, "fp8, bf16 or fp16 operands");
  // a 64-byte step is 32 two-byte elements: two 32x32x16 MFMAs
  constexpr bool BF = OP == OP_BF16 || OP == OP_F16X;
  static_assert(BM % (NW * RPI) == 0 && BN % (NW * RPI) == 0 && TM >= 2 && TM % 2 == 0 && TN >= 1,
                "DMA blocks must divide among the waves");
  static_assert((NW * RPI) % 16 == 0, "a wave's DMA blocks share row % 16 (the swizzle)");
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / WN, wn = wave % WN;

  int64_t m0, n0;
  tile_origin(g.M, g.N, BM, BN, g.group_m, m0, n0);
  const int64_t bat = blockIdx.y;
  g.A += bat * g.sa;
  g.B += bat * g.sb;
  g.C = (uint8_t*)g.C + bat * g.sc * (g.epi.out_dtype == VH_F32 ? 4 : 2);
  const int64_t rows_a = (g.M - m0) < BM ? (g.M - m0) : BM;
  const int64_t rows_b = (g.N - n0) < BN ? (g.N - n0) : BN;
  const i32x4 ra = raw_desc(g.A + m0 * g.lda, rows_a * g.lda);
  const i32x4 rb = raw_desc(g.B + n0 * g.ldb, rows_b * g.ldb);
  const int K = (int)g.K * (BF ? 2 : 1);  // bytes of a row
  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_void*)smem;
  // BIAS: the tile's BN biases (at most two per thread, clamped into the
  // row) are read now, ahead of the main loop's DMA; they are older than
  // every stage's loads, so the loop's vmcnt waits only retire them earlier
  constexpr int NBT = BIAS ? (BN + NW * 64 - 1) / (NW * 64) : 1;
  uint32_t braw[NBT];
  if constexpr (BIAS) {
#pragma unroll
    for (int k = 0; k < NBT; ++k) {
      const int64_t c = n0 + threadIdx.x + k * NW * 64;
      const int64_t cc = c < g.N ? c : g.N - 1;
      braw[k] = g.epi.bias_dtype == VH_BF16 ? (uint32_t)((const uint16_t*)g.epi.bias)[cc] << 16
                                            : ((const uint32_t*)g.epi.bias)[cc];
    }
  }

  // DMA: block q of RPI rows (A blocks, then B blocks) is fetched by wave
  // q % NW; lane l takes row q RPI + l / CPR, LDS chunk l % CPR.  Row % 16
  // is the same for all of a wave's blocks (NW RPI is a multiple of 16).
  const int drow = lane / CPR;
  const int dchunk = ((lane % CPR) ^ swz<KS>(((wave * RPI) & 15) + drow)) * 16;
  int voa[LA], vob[LB];
#pragma unroll
  for (int i = 0; i < LA; ++i) voa[i] = ((wave + NW * i) * RPI + drow) * (int)g.lda + dchunk;
#pragma unroll
  for (int i = 0; i < LB; ++i) vob[i] = ((wave + NW * i) * RPI + drow) * (int)g.ldb + dchunk;

  // DMA d of stage ks (0 <= d < L).  Branch-free: a chunk at or past K (the
  // K tail, the stages padded past the end) gets an offset past the
  // resource and reads as zero; rows past M / N are past the resource.
  auto dma = [&](int64_t ks, int d) {
    const int k0 = (int)(ks * KS);
    const bool live = k0 + dchunk < K;
    const uint32_t base = lds0 + (uint32_t)((ks % NS) * STAGE) + wave * 1024;
    if (d < LA) dma16(ra, base + d * NW * 1024, live ? voa[d] + k0 : (int)0x80000000);
    else dma16(rb, base + BM * KS + (d - LA) * NW * 1024, live ? vob[d - LA] + k0 : (int)0x80000000);
  };

  // Fragment read r of step t (0 <= r < 2 (TM + TN)), in the order the
  // MFMAs (i outer, j inner) first need them: A tile 0, the B tiles, A
  // tiles 1 ..; r % 2 is the half.
  const int fsw = swz<KS>(lane & 15);
  const int arow = (wm * (BM / WM) + (lane & 31)) * KS;
  const int brow = BM * KS + (wn * (BN / WN) + (lane & 31)) * KS;
  i32x8 f0a[TM], f0b[TN], f1a[TM], f1b[TN];
  auto read_one = [&](i32x8* fa, i32x8* fb, int buf, int t, int r) {
    const uint8_t* base = smem + buf * STAGE;
    const bool isb = r >= 2 && r < 2 + 2 * TN;
    const int ti = r < 2 ? 0 : isb ? (r - 2) >> 1 : 1 + ((r - 2 - 2 * TN) >> 1);
    const int chunk = (4 * t + 2 * (lane >> 5) + (r & 1)) ^ fsw;
    const uint4 v = *(const uint4*)(base + (isb ? brow : arow) + ti * 32 * KS + chunk * 16);
    i32x8& f = isb ? fb[ti] : fa[ti];
    if (r & 1) f.hi = i32x4{(int)v.x, (int)v.y, (int)v.z, (int)v.w};
    else f.lo = i32x4{(int)v.x, (int)v.y, (int)v.z, (int)v.w};
  };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  constexpr int Q = BF ? 2 * TM * TN : TM * TN;  // MFMAs per step
  // B as the row operand: accumulators come out transposed (store_tile_lds_t).
  // bf16: MFMA q < TM TN takes the first 16 bytes of its fragments, the
  // others the second; both halves of a pair cover distinct K of the step.
  auto mfma = [&](const i32x8* fa, const i32x8* fb, int q) {
    if constexpr (BF) {
      const int p = q % (TM * TN), i = p / TN, j = p % TN;
      const i32x4 a = q < TM * TN ? fa[i].lo : fa[i].hi, b = q < TM * TN ? fb[j].lo : fb[j].hi;
      if constexpr (OP == OP_F16X)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, b), __builtin_bit_cast(f16x8, a),
                                                          acc[i][j], 0, 0, 0);
      else
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, b),
                                                           __builtin_bit_cast(bf16x8, a), acc[i][j], 0, 0, 0);
    } else {
      const int i = q / TN, j = q % TN;
      acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fb[j], fa[i], acc[i][j], 0, 0, 0, 127, 0, 127);
    }
  };

  constexpr int H1 = BF ? TM * TN : TM / 2 * TN;  // MFMAs of the last step before the barrier
  constexpr int NR = 2 * (TM + TN);    // fragment reads per step
  constexpr int PRE = (P - 1) * Q + H1;  // MFMAs of a stage before its barrier

  // The stage count is padded to a multiple of NS (padded stages are zero)
  // so the loop body has no exits between stages.
  const int64_t nk = (((int64_t)K + KS - 1) / KS + NS - 1) / NS * NS;
  // prologue: stages 0 .. NS-2 in flight, stage 0's first fragments read
#pragma unroll
  for (int s = 0; s < NS - 1; ++s)
#pragma unroll
    for (int d = 0; d < L; ++d) dma(s, d);
  wait_vmcnt<(NS - 2) * L>();
  lds_barrier();
#pragma unroll
  for (int r = 0; r < NR; ++r) read_one(f0a, f0b, 0, 0, r);

  // Step t of stage ks on fragments F, reading the next step's into G.
  auto step = [&](int64_t ks, int t, i32x8* fa, i32x8* fb, i32x8* ga, i32x8* gb) {
    const int buf = (int)(ks % NS);
    if (t < P - 1) {
#pragma unroll
      for (int q = 0; q < Q; ++q) {
#pragma unroll
        for (int r = q * NR / Q; r < (q + 1) * NR / Q; ++r) read_one(ga, gb, buf, t + 1, r);
        __builtin_amdgcn_sched_barrier(0);
        mfma(fa, fb, q);
        __builtin_amdgcn_sched_barrier(0);
        const int m = t * Q + q;
#pragma unroll
        for (int d = m * L / PRE; d < (m + 1) * L / PRE; ++d) dma(ks + NS - 1, d);
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
#pragma unroll
      for (int q = 0; q < H1; ++q) {
        mfma(fa, fb, q);
        __builtin_amdgcn_sched_barrier(0);
        const int m = t * Q + q;
#pragma unroll
        for (int d = m * L / PRE; d < (m + 1) * L / PRE; ++d) dma(ks + NS - 1, d);
        __builtin_amdgcn_sched_barrier(0);
      }
      wait_vmcnt<(NS - 2) * L>();
      lds_barrier();
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int q = H1; q < Q; ++q) {
#pragma unroll
        for (int r = (q - H1) * NR / (Q - H1); r < (q - H1 + 1) * NR / (Q - H1); ++r)
          read_one(ga, gb, (buf + 1) % NS, 0, r);
        __builtin_amdgcn_sched_barrier(0);
        mfma(fa, fb, q);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };
  for (int64_t ks = 0; ks < nk; ks += NS) {
#pragma unroll
    for (int u = 0; u < NS * P; u += 2) {
      step(ks + u / P, u % P, f0a, f0b, f1a, f1b);
      step(ks + (u + 1) / P, (u + 1) % P, f1a, f1b, f0a, f0b);
    }
  }
  // every DMA has landed and every wave is done with the stage buffers
  wait_vmcnt<0>();
  if constexpr (OP == OP_F16X) {
    // exact fp16 operands: each sum times 2**(E_row + E_col) (exact in
    // float32), as k_split_reduce applies it to split partials.  Transposed
    // accumulators: lane row m = lane % 32 of tile i, columns
    // 8 q + 4 (lane / 32) + u of tile j for element 4 q + u.
    if (g.ea) {
      const int lrow = lane & 31, lhalf = lane >> 5;
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int64_t row = m0 + wm * (BM / WM) + i * 32 + lrow;
        const int er = g.ea[row < g.M ? row : g.M - 1];
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int64_t col = n0 + wn * (BN / WN) + j * 32 + q * 8 + lhalf * 4;
#pragma unroll
            for (int u = 0; u < 4; ++u) {
              const int ec = g.eb[col + u < g.N ? col + u : g.N - 1];
              acc[i][j][4 * q + u] = ldexpf(acc[i][j][4 * q + u], er + ec);
            }
          }
      }
    }
  }
  __syncthreads();
  float* sb = nullptr;
  if constexpr (BIAS) {
    sb = (float*)(smem + f8dl_epi_bytes<BM, BN, WM, WN>());
#pragma unroll
    for (int k = 0; k < NBT; ++k) {
      const int c = threadIdx.x + k * NW * 64;
      if (c < BN) sb[c] = n0 + c < g.N ? __uint_as_float(braw[k]) : 0.0f;
    }
    __syncthreads();
  }
  if (g.epi.out_dtype == VH_F32) store_tile_t_f32<TM, TN, BIAS>(g, acc, m0, n0, wm, wn, lane, sb);
  else store_tile_lds_t<TM, TN, BIAS>(g, acc, smem, m0, n0, wave, wm, wn, lane, sb);
}

// ------------------------------------------------------------ MX-int8, fp16
// MX-int8 x MX-int8 with 16-element blocks on v_mfma_f32_32x32x16_f16.  A
// code c of a block with exponent e enters as the fp16 value c * 2**(e - E),
// E the largest block exponent of the code's row within the workgroup's K
// range: the byte c ^ 0x80 under the fp16 high byte 0x64 is 1152 + c (one
// v_perm per two codes), and one packed fma by 2**(e - E) and
// -1152 * 2**(e - E) leaves c * 2**(e - E) exactly (e - E >= -24; a block
// further below its row's largest is flushed, a change under 2**-17 of that
// block's magnitude).  Products are exact and accumulate in fp32, as with
// bf16 operands; the epilogue multiplies by 2**(E_row + E_col), exact in
// fp32 -- 1.25 VALU operations per decoded code against 2.5 for bf16.
//
// Block tile 256 x 64, eight waves (two per SIMD, so one's decode overlaps
// the other's MFMAs): wave w owns A rows 32 w .. 32 w + 31 and B rows
// 8 w .. 8 w + 7, and multiplies its A rows by all 64 B columns.  A stage
// is 64 K elements.  Every global load moves data straight into LDS
// (buffer_load ... lds, four lanes per 64-byte row segment), and a wave
// only ever reads raw data it loaded itself, so the raw stages need no
// barrier and the waits are explicit vmcnt counts (the compiler issues no
// global loads in the loop):
// * the split's scale bytes, once, before the loop ([320 rows][nb]);
// * A codes, NS - 1 stages ahead: 1 KB blocks of 16 rows x 64 bytes, chunk
//   c of row r at slot 4 (r % 16) + (c ^ (r / 4 % 4)) (the MFMA-layout
//   read -- 16 rows, one chunk -- hits 16 distinct bank groups), decoded in
//   registers straight into MFMA operands, once per block tile;
// * B codes, likewise (half of each wave's 1 KB DMA is unused), decoded by
//   the loading lanes into a shared fp16 stage (rows padded to MH_PITCH
//   bytes) that every wave reads after the stage's one barrier.
// MFMA step t (of 4) takes, in lane half h, K elements 32 h + 8 t .. + 7 of
// the stage -- a permutation of K both operands share -- so a lane's A codes
// of its row are two whole blocks.  gridDim.y splits K as k_gemm_mxi8 does
// (the splits of a tile share an XCD); partials carry the 2**(E_row +
// E_col) factor, so k_split_reduce adds them as they are.
constexpr int MH_KE = 64;                        // K elements (code bytes) per stage
constexpr int MH_PITCH = 2 * MH_KE + 16;         // LDS pitch of a decoded B row (bytes)
constexpr int MH_BN = 64;
constexpr int MH_NS = 4;                         // raw stages in LDS
constexpr int MH_KQ = 4 * MH_KE;                 // K granule: splits and K are multiples of it
constexpr int MH_KC_MAX = 2048;                  // K elements per split at most (128 scale bytes per row)

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pk_max_u16(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t,
                            __builtin_elementwise_max(__builtin_bit_cast(u16x2, a), __builtin_bit_cast(u16x2, b)));
}

// (2**d, 2**d) and (-1152 * 2**d, ...) as fp16 pairs; both 0 for d < -24.
struct MhMul {
  f16x2 m, o;
};

__device__ __forceinline__ MhMul mh_mul(int d) {
  const _Float16 s = __builtin_amdgcn_ldexph((_Float16)1.0f, d);
  const uint32_t bits = __builtin_bit_cast(unsigned short, s);
  MhMul r;
  r.m = __builtin_bit_cast(f16x2, bits * 0x10001u);
  const f16x2 k = {(_Float16)-1152.0f, (_Float16)-1152.0f};
  r.o = r.m * k;
  return r;
}

// Eight codes (two dwords) of one block -> the fp16 operand c * 2**d.
__device__ __forceinline__ f16x8 mh_decode8(uint32_t w0, uint32_t w1, const MhMul& mu) {
  const uint32_t x0 = w0 ^ 0x80808080u, x1 = w1 ^ 0x80808080u;
  const f16x2 p0 = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, x0, 0x04010400u));
  const f16x2 p1 = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, x0, 0x04030402u));
  const f16x2 p2 = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, x1, 0x04010400u));
  const f16x2 p3 = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, x1, 0x04030402u));
  const f16x2 y0 = __builtin_elementwise_fma(p0, mu.m, mu.o), y1 = __builtin_elementwise_fma(p1, mu.m, mu.o);
  const f16x2 y2 = __builtin_elementwise_fma(p2, mu.m, mu.o), y3 = __builtin_elementwise_fma(p3, mu.m, mu.o);
  return f16x8{y0[0], y0[1], y1[0], y1[1], y2[0], y2[1], y3[0], y3[1]};
}

// The largest byte of 16.
__device__ __forceinline__ uint32_t max_byte16(const uint4& v) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
  uint32_t acc = 0u;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    acc = pk_max_u16(acc, w[q] & 0x00ff00ffu);
    acc = pk_max_u16(acc, (w[q] >> 8) & 0x00ff00ffu);
  }
  const uint32_t a = acc & 0xffffu, b = acc >> 16;
  return a > b ? a : b;
}

// LDS layout (bytes).
struct MhLds {
  static constexpr int STAGE = 256 * MH_KE + 8 * 1024;          // A blocks, then one B DMA block per wave
  static constexpr int FP16 = MH_NS * STAGE;                   // 2 x 64 decoded B rows
  static constexpr int SC = FP16 + 2 * MH_BN * MH_PITCH;       // the split's scale bytes, [256 + 64][nb]
  static constexpr int BYTES = SC + (256 + MH_BN) * (MH_KC_MAX / 16);
};

// explicit vmcnt wait (the DMA loads are invisible to the compiler)
template <int N>
__device__ __forceinline__ void mh_wait() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

__global__ void __launch_bounds__(512, 1) k_gemm_mx8h(GemmArgs g, int64_t kc, float* __restrict__ part) {
  constexpr int BM = 256, BN = MH_BN, TM = 1, TN = 2, NS = MH_NS;
  constexpr int L = 3;  // DMA instructions per wave and stage: two A blocks, one B block
  using Y = MhLds;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  __shared__ uint32_t s_ea[BM], s_eb[BN];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 31, lh = lane >> 5;
  int64_t m0, n0;
  tile_origin(g.M, g.N, BM, BN, g.group_m, m0, n0);
  const int64_t k_lo = (int64_t)blockIdx.y * kc;
  const int64_t k_hi = (k_lo + kc) < g.K ? (k_lo + kc) : g.K;
  const int nk = (int)((k_hi - k_lo) / MH_KE);
  const int nb = nk * (MH_KE / 16);  // scale bytes per row in the split
  const int kb0 = (int)(k_lo / 16);

  const int64_t rows_a = (g.M - m0) < BM ? (g.M - m0) : BM;
  const int64_t rows_b = (g.N - n0) < BN ? (g.N - n0) : BN;
  const i32x4 ra = raw_desc(g.A + m0 * g.lda, rows_a * g.lda);
  const i32x4 rb = raw_desc(g.B + n0 * g.ldb, rows_b * g.ldb);
  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_void*)smem;

  // DMA lanes: row lane / 4 of a 16-row block, chunk (lane % 4) ^ (lane / 16)
  const int drow = lane >> 2, dch = (lane & 3) ^ ((lane >> 4) & 3);
  const int voa0 = (32 * wave + drow) * (int)g.lda + 16 * dch + (int)k_lo;
  const int voa1 = voa0 + 16 * (int)g.lda;
  const bool b_live = lane < 32;  // B rows 8 wave + lane / 4
  const int vob = (8 * wave + drow) * (int)g.ldb + 16 * dch + (int)k_lo;
  auto dma = [&](int s) {
    const bool live = s < nk;  // past the split: zeros, never used
    const uint32_t base = lds0 + (uint32_t)((s % NS) * Y::STAGE);
    const int ko = s * MH_KE;
    dma16(ra, base + (2 * wave) * 1024, live ? voa0 + ko : (int)0x80000000);
    dma16(ra, base + (2 * wave + 1) * 1024, live ? voa1 + ko : (int)0x80000000);
    dma16(rb, base + 256 * MH_KE + wave * 1024, live && b_live ? vob + ko : (int)0x80000000);
  };

  // the split's scale bytes: DMA instruction i (wave i % 8) covers 64 / cpr
  // rows of cpr 16-byte chunks, A rows then B rows; then the first stages
  // (one round trip for both)
  const int cpr = nb / 16;
  const int ninst = (BM + BN) * nb / 1024;
  {
    const i32x4 rsa = raw_desc(g.a_scale + m0 * g.lds_a, rows_a * g.lds_a);
    const i32x4 rsb = raw_desc(g.b_scale + n0 * g.lds_b, rows_b * g.lds_b);
    const uint32_t sc0 = lds0 + Y::SC;
    const int rpi = 64 / cpr, lrow = lane / cpr, lch = lane % cpr;
    for (int i = wave; i < ninst; i += 8) {
      const int row = i * rpi + lrow;
      if (row < BM) dma16(rsa, sc0 + i * 1024, row * (int)g.lds_a + kb0 + 16 * lch);
      else dma16(rsb, sc0 + i * 1024, (row - BM) * (int)g.lds_b + kb0 + 16 * lch);
    }
  }
#pragma unroll
  for (int s = 0; s < NS - 1; ++s) dma(s);
  mh_wait<(NS - 1) * L>();  // this wave's scale DMA (older than the stages) has landed
  __syncthreads();
  // the rows' largest block exponents over this split's K range
  if (tid < BM + BN) {
    uint32_t m = 0u;
    for (int c = 0; c < nb / 16; ++c) {
      const uint32_t v = max_byte16(*(const uint4*)(smem + Y::SC + tid * nb + 16 * c));
      m = v > m ? v : m;
    }
    if (tid < BM) s_ea[tid] = m;
    else s_eb[tid - BM] = m;
  }
  __syncthreads();
  const int ea = (int)s_ea[32 * wave + lr];
  const int brow = 8 * wave + drow;
  const int ebr = (int)s_eb[brow & (BN - 1)];
  const uint8_t* sa_row = smem + Y::SC + (32 * wave + lr) * nb;
  const uint8_t* sb_row = smem + Y::SC + (BM + (brow & (BN - 1))) * nb;

  // this wave's B rows of stage s -> fp16 buffer s % 2 (lanes 0..31)
  auto decode_b = [&](int s) {
    if (b_live) {
      const uint4 c = *(const uint4*)(smem + (s % NS) * Y::STAGE + 256 * MH_KE + wave * 1024 + 16 * lane);
      const MhMul mu = mh_mul((int)sb_row[4 * s + dch] - ebr);
      uint8_t* d = smem + Y::FP16 + (s & 1) * BN * MH_PITCH + brow * MH_PITCH + 32 * dch;
      *(f16x8*)d = mh_decode8(c.x, c.y, mu);
      *(f16x8*)(d + 16) = mh_decode8(c.z, c.w, mu);
    }
  };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int n = 0; n < TN; ++n)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[0][n][r] = 0.0f;

  const int rsw = (lr >> 2) & 3;  // the swizzle of the A row this lane reads
  // every LDS read of the stage goes out first, then the decode / MFMA chain
  auto compute = [&](int s) {
    const uint8_t* blk = smem + (s % NS) * Y::STAGE + (2 * wave + (lr >> 4)) * 1024 + 64 * (lr & 15);
    const uint8_t* bb = smem + Y::FP16 + (s & 1) * BN * MH_PITCH + lr * MH_PITCH + 64 * lh;
    const uint4 c0 = *(const uint4*)(blk + 16 * ((2 * lh) ^ rsw));
    const uint4 c1 = *(const uint4*)(blk + 16 * ((2 * lh + 1) ^ rsw));
    const uint32_t sa = *(const uint32_t*)(sa_row + 4 * s);
    f16x8 fb[4][TN];
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int n = 0; n < TN; ++n) fb[t][n] = *(const f16x8*)(bb + n * 32 * MH_PITCH + 16 * t);
#pragma unroll
    for (int q = 0; q < 2; ++q) {  // block 2 lh + q: steps 2 q, 2 q + 1
      const MhMul mu = mh_mul((int)((sa >> (8 * (2 * lh + q))) & 0xffu) - ea);
      const uint4& c = q ? c1 : c0;
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const f16x8 fa = t ? mh_decode8(c.z, c.w, mu) : mh_decode8(c.x, c.y, mu);
#pragma unroll
        for (int n = 0; n < TN; ++n)
          acc[0][n] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa, fb[2 * q + t][n], acc[0][n], 0, 0, 0);
      }
    }
  };

  // iteration s: stage s + NS - 1 goes out; this wave's DMA of stages s and
  // s + 1 has landed; the wave decodes its B rows of stage s + 1 and
  // multiplies stage s; one barrier publishes the
  // fp16 B stage and retires the buffers stage s used (the wave's LDS reads
  // complete before it).
  mh_wait<(NS - 2) * L>();
  decode_b(0);
  lds_barrier();
  for (int s = 0; s < nk; ++s) {
    dma(s + NS - 1);
    mh_wait<(NS - 2) * L>();
    if (s + 1 < nk) decode_b(s + 1);
    compute(s);
    lds_barrier();
  }
  mh_wait<0>();
  __syncthreads();

  // undo the row / column rebasing: 2**(E_row + E_col), exact in fp32
#pragma unroll
  for (int n = 0; n < TN; ++n) {
    const int eb = (int)s_eb[32 * n + lr] - g.b_bias;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = 32 * wave + (r >> 2) * 8 + lh * 4 + (r & 3);
      acc[0][n][r] = ldexpf(acc[0][n][r], (int)s_ea[row] - g.a_bias + eb);
    }
  }
  if (gridDim.y == 1) {
    store_tile<TM, TN, 8, 1>(g, acc, smem, m0, n0, wave, wave, 0, lane);
  } else {
    GemmArgs p = g;
    p.C = part + (int64_t)blockIdx.y * g.M * g.N;
    p.ldc = g.N;
    p.epi.mode = EPI_PLAIN;
    p.epi.out_dtype = VH_F32;
    p.epi.scale = nullptr;
    p.epi.bias = nullptr;
    store_tile_direct<TM, TN, 8, 1>(p, acc, m0, n0, wave, 0, lane);
  }
}

// Tile-rows per column walk for a BM x BN grid: the group whose per-XCD
// block of tiles (the XCD's share of the grid) streams the fewest operand
// rows, GM BM of A plus (tiles per XCD / GM) BN of B.
int group_rows(int64_t M, int64_t N, int BM, int BN) {
  const int64_t tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  const int64_t per_xcd = (tiles_m * tiles_n + 7) / 8;
  int best = 1;
  int64_t best_rows = -1;
  for (int gm = 1; gm <= 16 && gm <= tiles_m; gm *= 2) {
    const int64_t rows = gm * (int64_t)BM + (per_xcd + gm - 1) / gm * BN;
    if (best_rows < 0 || rows <= best_rows) best = gm, best_rows = rows;
  }
  return best;
}

template <int BM, int BN, int NS, int KS, int WM, int WN, int OP, bool BIAS>
int launch_f8dl_as(GemmArgs g, int64_t batch, hipStream_t stream) {
  g.group_m = group_rows(g.M, g.N, BM, BN);
  constexpr size_t stages = (size_t)NS * (BM + BN) * KS;
  // store_tile_lds_t's bf16 staging, then (BIAS) the tile's float32 biases
  constexpr size_t epi = (size_t)f8dl_epi_bytes<BM, BN, WM, WN>() + (BIAS ? (size_t)BN * 4 : 0);
  constexpr size_t smem = stages > epi ? stages : epi;
  static_assert(smem <= 160 * 1024, "LDS");
  const int64_t tiles = ((g.M + BM - 1) / BM) * ((g.N + BN - 1) / BN);
  static bool attr_set = false;
  if (!attr_set) {
    if (hipFuncSetAttribute((const void*)k_gemm_f8dl<BM, BN, NS, KS, WM, WN, OP, BIAS>,
                            hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)smem) != hipSuccess) {
      vh::set_error("vh_gemm: cannot reserve %zu bytes of LDS", smem);
      return VH_ELAUNCH;
    }
    attr_set = true;
  }
  hipLaunchKernelGGL((k_gemm_f8dl<BM, BN, NS, KS, WM, WN, OP, BIAS>), dim3((unsigned)tiles, (unsigned)batch),
                     dim3(WM * WN * 64), smem, stream, g);
  return vh::check_launch("vh_gemm");
}

// A bias (only the plain epilogue adds one) takes the instantiation that
// loads it; every other epilogue, the one without.
template <int BM, int BN, int NS, int KS, int WM = 2, int WN = 2, int OP = OP_FP8>
int launch_f8dl(GemmArgs g, int64_t batch, hipStream_t stream) {
  if (g.epi.bias && g.epi.mode != EPI_ROUND_SCALE) return launch_f8dl_as<BM, BN, NS, KS, WM, WN, OP, true>(g, batch, stream);
  return launch_f8dl_as<BM, BN, NS, KS, WM, WN, OP, false>(g, batch, stream);
}

template <int BM, int BN, int WM, int WN, int MINB, int PF, int AF, int BF>
int launch_tile(GemmArgs g, int64_t batch, hipStream_t stream) {
  g.group_m = 8;
  constexpr int NT = WM * WN * 64;
  const int64_t tiles = ((g.M + BM - 1) / BM) * ((g.N + BN - 1) / BN);
  const size_t smem = 2 * (BM + BN) * ROWP + 512;
  static bool attr_set = false;
  if (!attr_set) {
    if (hipFuncSetAttribute((const void*)k_gemm<BM, BN, WM, WN, MINB, PF, AF, BF>, hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)smem) != hipSuccess) {
      vh::set_error("vh_gemm: cannot reserve %zu bytes of LDS", smem);
      return VH_ELAUNCH;
    }
    attr_set = true;
  }
  hipLaunchKernelGGL((k_gemm<BM, BN, WM, WN, MINB, PF, AF, BF>), dim3((unsigned)tiles, (unsigned)batch), dim3(NT), smem, stream, g);
  return vh::check_launch("vh_gemm");
}

template <int BM, int BN, int WM, int WN, int P = 2, bool WS = false>
int launch_mxi8(GemmArgs g, int splits, float* part, hipStream_t stream) {
  g.group_m = 8;
  constexpr int NT = WS ? 512 : WM * WN * 64;
  const int64_t tiles = ((g.M + BM - 1) / BM) * ((g.N + BN - 1) / BN);
  const int64_t stages = g.K / MX_KE;
  const int64_t kc = (stages + splits - 1) / splits * MX_KE;
  const int64_t sp = (g.K + kc - 1) / kc;  // every split has at least one stage
  const size_t smem = 2 * (BM + BN) * ROWP;
  static bool attr_set = false;
  if (!attr_set) {
    const void* fn;
    if constexpr (WS) fn = (const void*)k_gemm_mxi8_ws<BM, BN>;
    else fn = (const void*)k_gemm_mxi8<BM, BN, WM, WN, P>;
    if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem) != hipSuccess) {
      vh::set_error("vh_gemm: cannot reserve %zu bytes of LDS", smem);
      return VH_ELAUNCH;
    }
    attr_set = true;
  }
  if constexpr (WS)
    hipLaunchKernelGGL((k_gemm_mxi8_ws<BM, BN>), dim3((unsigned)tiles, (unsigned)sp), dim3(NT), smem, stream, g, kc,
                       sp > 1 ? part : nullptr);
  else
    hipLaunchKernelGGL((k_gemm_mxi8<BM, BN, WM, WN, P>), dim3((unsigned)tiles, (unsigned)sp), dim3(NT), smem, stream,
                       g, kc, sp > 1 ? part : nullptr);
  if (sp > 1) {
    const int64_t quads = g.M * g.N / 4;
    hipLaunchKernelGGL(k_split_reduce, dim3((unsigned)((quads + 255) / 256)), dim3(256), 0, stream, part, (int)sp,
                       g.M, g.N, g.epi, g.C, g.ldc);
  }
  return vh::check_launch("vh_gemm");
}

int launch_mx8h(GemmArgs g, int splits, float* part, hipStream_t stream) {
  g.group_m = group_rows(g.M, g.N, 256, MH_BN);
  const int64_t tiles = ((g.M + 255) / 256) * ((g.N + MH_BN - 1) / MH_BN);
  const int64_t quads = g.K / MH_KQ;
  const int64_t kc = (quads + splits - 1) / splits * MH_KQ;
  const int64_t sp = (g.K + kc - 1) / kc;
  constexpr size_t stages = (size_t)MhLds::BYTES;
  constexpr size_t epi = (size_t)8 * 32 * (MH_BN + 8) * 2;
  constexpr size_t smem = stages > epi ? stages : epi;
  static_assert(smem + 4 * (256 + MH_BN) <= 160 * 1024, "LDS");
  static bool attr_set = false;
  if (!attr_set) {
    if (hipFuncSetAttribute((const void*)k_gemm_mx8h, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem) !=
        hipSuccess) {
      vh::set_error("vh_gemm: cannot reserve %zu bytes of LDS", smem);
      return VH_ELAUNCH;
    }
    attr_set = true;
  }
  hipLaunchKernelGGL(k_gemm_mx8h, dim3((unsigned)tiles, (unsigned)sp), dim3(512), smem, stream, g, kc,
                     sp > 1 ? part : nullptr);
  if (sp > 1) {
    const int64_t q4 = g.M * g.N / 4;
    hipLaunchKernelGGL(k_split_reduce, dim3((unsigned)((q4 + 255) / 256)), dim3(256), 0, stream, part, (int)sp, g.M,
                       g.N, g.epi, g.C, g.ldc);
  }
  return vh::check_launch("vh_gemm");
}

// Whether k_gemm_mx8h takes a descriptor: 16-element blocks, K a whole
// number of stage pairs, 16-byte aligned operand and scale rows.
bool mx8h_fits(const vh_gemm_desc* d) {
  auto al = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
  return d->a_block == 16 && d->b_block == 16 && d->K % MH_KQ == 0 && d->a_scale_ld % 16 == 0 &&
         d->b_scale_ld % 16 == 0 && al(d->A) && al(d->B) && al(d->a_scale) && al(d->b_scale);
}

// The MX-int8 kernel's tile (hint 50..56 bf16 operands, 60 fp16 operands)
// and split count for a descriptor, or cfg 0 when the pair takes k_gemm.
// Splits fill the 256 CUs when the tile grid alone does not; each split
// keeps at least two stages.
void mxi8_plan(const vh_gemm_desc* d, int& cfg, int& splits) {
  cfg = 0;
  splits = 1;
  const bool fits = d->a_fmt == OP_MXI8 && d->b_fmt == OP_MXI8 && d->batch <= 1 && d->K >= MX_KE &&
                    d->K % MX_KE == 0 && d->a_block >= 16 && d->b_block >= 16 && d->N % 4 == 0 &&
                    d->lda % 16 == 0 && d->ldb % 16 == 0 && (d->tile_hint == 0 || d->tile_hint >= 50);
  if (!fits || d->M <= 0 || d->N <= 0) return;
  auto tiles = [&](int64_t bm, int64_t bn) { return ((d->M + bm - 1) / bm) * ((d->N + bn - 1) / bn); };
  cfg = d->tile_hint;
  const bool h = mx8h_fits(d);
  // bf16 operands by default -- measured on MI355X (N = K = 4096): at
  // M = 256, 128 x 128 tiles with 8 waves split 4 ways take 25.8 us (4
  // waves: 30.3 us; 128 x 64 split 4: 28.6 us; producer / consumer waves
  // 27.5 us; split 8 pays twice the partial traffic); at M = 2048, 256 x 128
  // with producer / consumer waves takes 95.1 us.  The fp16-operand kernel
  // (tile 60, k_gemm_mx8h) is taken on request: at M = 256 it ties the
  // bf16 kernels (24 us plus the split reduction), bound by LDS traffic
  // (every wave reads the whole decoded B stage) and the per-stage barrier.
  if (cfg == 60 && !h) cfg = 0;
  if (cfg == 0) cfg = tiles(256, 128) >= 256 ? 56 : 51;
  int64_t bm = 128, bn = 128;
  switch (cfg) {
    case 50: case 51: break;
    case 52: bn = 64; break;
    case 53: bm = 256; break;
    case 54: bm = 64; break;
    case 55: break;
    case 56: bm = 256; break;
    case 60: bm = 256; bn = 64; break;
    default: cfg = 0; return;
  }
  const int64_t t = tiles(bm, bn);
  int64_t sp = d->split_k > 0 ? d->split_k : (t >= 192 ? 1 : (256 + t - 1) / t);
  if (cfg >= 60) {
    const int64_t quads = d->K / MH_KQ;
    if (sp > quads) sp = quads;
    const int64_t min_sp = (d->K + MH_KC_MAX - 1) / MH_KC_MAX;  // the split's scale bytes fit LDS
    if (sp < min_sp) sp = min_sp;
    const int64_t kc = (quads + sp - 1) / sp * MH_KQ;
    splits = (int)((d->K + kc - 1) / kc);
    return;
  }
  const int64_t stages = d->K / MX_KE;
  if (sp > stages / 2) sp = stages / 2 > 1 ? stages / 2 : 1;
  if (d->split_k > 0 && d->split_k <= stages) sp = d->split_k;
  const int64_t kc = (stages + sp - 1) / sp * MX_KE;
  splits = (int)((d->K + kc - 1) / kc);
}

int64_t mxi8_workspace(const vh_gemm_desc* d, int splits) {
  return splits > 1 ? (int64_t)splits * d->M * d->N * 4 : 0;
}

template <int A, int B>
struct Fmts {
  static constexpr int a = A, b = B;
};

// ------------------------------------------------------------ MXNF4 prefill
// linear_mx of codebook operands at any M (ops/quantized.py:651-723 with
// the decode of :574-591): A = the activation's codebook indices, one byte
// each [M, K], with its block scales as codes of their map [M, K / 64]; B =
// the weight as the decode GEMV bakes it (vh_pack_nf4: nibbles in MFMA lane
// order, scale bytes tile-major [N / 16][K / 64][16]), so one baked copy
// serves both.  Every element is decoded while staging to exactly the
// operand the reference multiplies, bf16(level * scale): the index through
// a 16-entry table of level + 128 (lut16: three v_perm per four), an
// unsigned-byte convert, one fma by the block scale that also removes the
// 128 bias ((level + 128) s and 128 s are exact in float32), and the
// hardware round to bf16.  Then v_mfma_f32_32x32x16_bf16 with float32
// accumulation, as the reference's float32 GEMM of the decoded operands:
// the results differ by summation order only.  A stage is one 64-element
// block: per row four 16-element chunks, each one load of 16 index bytes (A)
// or one 8-byte GEMV record (B, lane (r % 16) + 16 c of the row's tile) and
// the row's scale byte; loads run P - 1 stages ahead in registers.
struct Nf4Args {
  uint4 lvb;        // level + 128 of each index, one byte each
  vh_format a_sf;   // the activation's scale map
  vh_format b_sf;   // the weight's scale map
};

// four indices (one per byte, 0..15) -> four bf16 pairs' worth of floats
__device__ __forceinline__ void nf4_levels4(uint32_t biased, float s, float nb, float (&f)[4]) {
  f[0] = fmaf((float)(biased & 0xffu), s, nb);
  f[1] = fmaf((float)((biased >> 8) & 0xffu), s, nb);
  f[2] = fmaf((float)((biased >> 16) & 0xffu), s, nb);
  f[3] = fmaf((float)(biased >> 24), s, nb);
}

// Sixteen biased levels (four dwords, element order) times s -> 16 bf16.
__device__ __forceinline__ void nf4_pack16(const uint32_t (&l)[4], float s, uint4& lo, uint4& hi) {
  const float nb = -128.0f * s;
  uint32_t o[8];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float f[4];
    nf4_levels4(l[j], s, nb, f);
    o[2 * j] = f2bf2_hw(f[0], f[1]);
    o[2 * j + 1] = f2bf2_hw(f[2], f[3]);
  }
  lo = make_uint4(o[0], o[1], o[2], o[3]);
  hi = make_uint4(o[4], o[5], o[6], o[7]);
}

template <int BM, int BN, int WM, int WN, int P>
__global__ void __launch_bounds__(WM * WN * 64) k_gemm_nf4(GemmArgs g, Nf4Args q, int kcs, float* __restrict__ part) {
  constexpr int NT = WM * WN * 64;
  constexpr int CA = BM * 4 / NT, CB = BN * 4 / NT;  // 16-element chunks per thread and stage
  static_assert(CA >= 1 && CB >= 1 && (BM * 4) % NT == 0 && (BN * 4) % NT == 0, "stage chunks must divide");
  constexpr int TM = BM / WM / 32, TN = BN / WN / 32;
  static_assert(TM >= 1 && TN >= 1 && BM % (WM * 32) == 0 && BN % (WN * 32) == 0 && BN % 16 == 0,
                "bad wave layout");
  static_assert(WN * BM * (BN / WN + 8) * 2 <= 2 * (BM + BN) * ROWP, "epilogue tile does not fit the stage LDS");
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  uint8_t* As = smem;                  // [2][BM][ROWP]: 64 bf16 per row
  uint8_t* Bs = smem + 2 * BM * ROWP;  // [2][BN][ROWP]
  float* s_sa = (float*)(smem + 2 * (BM + BN) * ROWP);  // [256] decoded activation scale codes
  float* s_sb = s_sa + 256;                             // [256] decoded weight scale codes

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  int64_t m0, n0;
  tile_origin(g.M, g.N, BM, BN, g.group_m, m0, n0);
  const int nbk = (int)(g.K / 64);  // blocks of a row
  // split blockIdx.y takes blocks [kb0, kb0 + nk)
  const int kb0 = (int)blockIdx.y * kcs;
  const int nk = (nbk - kb0) < kcs ? (nbk - kb0) : kcs;
  const int64_t rows_a = (g.M - m0) < BM ? (g.M - m0) : BM;
  const int64_t rows_b = (g.N - n0) < BN ? (g.N - n0) : BN;  // a multiple of 16
  const rsrc_t ad = make_rsrc(g.A + m0 * g.lda, rows_a * g.lda);
  const rsrc_t as = make_rsrc(g.a_scale + m0 * g.lds_a, rows_a * g.lds_a);
  const rsrc_t bd = make_rsrc(g.B + (n0 / 16) * nbk * 512, rows_b / 16 * nbk * 512);
  const rsrc_t bs = make_rsrc(g.b_scale + (n0 / 16) * nbk * 16, rows_b / 16 * nbk * 16);
  uint32_t base;
  asm volatile("v_mov_b32 %0, 0x3020100" : "=v"(base));

  // chunk i of this thread: row ch / 4, elements 16 (ch % 4) .. + 15 of the stage
  int aoff[CA], asrow[CA], boff[CB], bsoff[CB];
#pragma unroll
  for (int i = 0; i < CA; ++i) {
    const int ch = tid + i * NT, r = ch >> 2;
    aoff[i] = r * (int)g.lda + (ch & 3) * 16;
    asrow[i] = r * (int)g.lds_a;
  }
#pragma unroll
  for (int i = 0; i < CB; ++i) {
    const int ch = tid + i * NT, r = ch >> 2;
    boff[i] = ((r >> 4) * nbk * 64 + (r & 15) + 16 * (ch & 3)) * 8;
    bsoff[i] = (r >> 4) * nbk * 16 + (r & 15);
  }

  static_assert(P >= 2 && P % 2 == 0, "an even number of register sets");
  uint4 ra[P][CA];
  uint2 rb[P][CB];
  uint32_t sa[P][CA], sb[P][CB];
  // Stage s into set j (clamped to the last stage: a prefetch past the end
  // re-reads it and is never stored).
  auto fetch = [&](int j, int s) {
    const int kb = kb0 + (s < nk ? s : nk - 1);
#pragma unroll
    for (int i = 0; i < CA; ++i) {
      ra[j][i] = bload16(ad, aoff[i] + kb * 64);
      sa[j][i] = bload1(as, asrow[i] + kb);
    }
#pragma unroll
    for (int i = 0; i < CB; ++i) {
      rb[j][i] = bload8(bd, boff[i] + kb * 512);
      sb[j][i] = bload1(bs, bsoff[i] + kb * 16);
    }
  };
  auto stash = [&](int j, int st) {
    uint8_t* a = As + st * BM * ROWP;
    uint8_t* b = Bs + st * BN * ROWP;
#pragma unroll
    for (int i = 0; i < CA; ++i) {
      const int ch = tid + i * NT;
      const uint32_t w[4] = {ra[j][i].x, ra[j][i].y, ra[j][i].z, ra[j][i].w};
      uint32_t l[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) l[t] = lut_lo(w[t], base, q.lvb);
      uint4 lo, hi;
      nf4_pack16(l, s_sa[sa[j][i] & 0xffu], lo, hi);
      uint8_t* d = a + (ch >> 2) * ROWP + (ch & 3) * 32;
      *(uint4*)d = lo;
      *(uint4*)(d + 16) = hi;
    }
#pragma unroll
    for (int i = 0; i < CB; ++i) {
      const int ch = tid + i * NT;
      // byte t of the record: element t in its low nibble, t + 8 in its high one
      const uint32_t l[4] = {lut_lo(rb[j][i].x, base, q.lvb), lut_lo(rb[j][i].y, base, q.lvb),
                             lut_hi(rb[j][i].x, base, q.lvb), lut_hi(rb[j][i].y, base, q.lvb)};
      uint4 lo, hi;
      nf4_pack16(l, s_sb[sb[j][i] & 0xffu], lo, hi);
      uint8_t* d = b + (ch >> 2) * ROWP + (ch & 3) * 32;
      *(uint4*)d = lo;
      *(uint4*)(d + 16) = hi;
    }
  };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
  const int lrow = lane & 31;
  const int lhalf = lane >> 5;
  auto compute = [&](int st) {
    const uint8_t* a = As + st * BM * ROWP + (wm * (BM / WM) + lrow) * ROWP;
    const uint8_t* b = Bs + st * BN * ROWP + (wn * (BN / WN) + lrow) * ROWP;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int off = kk * 32 + lhalf * 16;
      bf16x8 fa[TM], fb[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) fa[i] = *(const bf16x8*)(a + i * 32 * ROWP + off);
#pragma unroll
      for (int j = 0; j < TN; ++j) fb[j] = *(const bf16x8*)(b + j * 32 * ROWP + off);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
    }
  };

#pragma unroll
  for (int j = 0; j < P; ++j) fetch(j, j);
  // the scale maps' values, while the first stages load
  for (int c = tid; c < 256; c += NT) {
    s_sa[c] = fmt_decode((uint32_t)c, q.a_sf, nullptr);
    s_sb[c] = fmt_decode((uint32_t)c, q.b_sf, nullptr);
  }
  __syncthreads();
  stash(0, 0);
  __syncthreads();
  for (int ks = 0; ks < nk; ks += P) {
#pragma unroll
    for (int j = 0; j < P; ++j) {
      // stage ks + j is in LDS buffer j % 2; set j is free
      fetch(j, ks + j + P);
      __builtin_amdgcn_sched_barrier(0);
      compute(j & 1);
      __builtin_amdgcn_sched_barrier(0);
      if (ks + j + 1 >= nk) goto done;
      stash((j + 1) % P, (j + 1) & 1);
      __syncthreads();
    }
  }
done:
  __syncthreads();  // the LDS epilogue reuses the stage buffers
  if (gridDim.y == 1) {
    store_tile<TM, TN, WM, WN>(g, acc, smem, m0, n0, wave, wm, wn, lane);
  } else {
    GemmArgs p = g;
    p.C = part + (int64_t)blockIdx.y * g.M * g.N;
    p.ldc = g.N;
    p.epi.mode = EPI_PLAIN;
    p.epi.out_dtype = VH_F32;
    p.epi.scale = nullptr;
    p.epi.bias = nullptr;
    store_tile_direct<TM, TN, WM, WN>(p, acc, m0, n0, wm, wn, lane);
  }
}

// Splits of K (in 64-element blocks) that fill the CUs when the tile grid
// alone does not; each split keeps at least two blocks.
inline int nf4_splits(int64_t tiles, int64_t nbk) {
  if (tiles >= 192) return 1;
  int64_t sp = (256 + tiles - 1) / tiles;
  if (sp > nbk / 2) sp = nbk / 2;
  return sp < 1 ? 1 : (int)sp;
}

template <int BM, int BN, int WM, int WN>
int launch_nf4(GemmArgs g, const Nf4Args& q, int splits, float* part, hipStream_t stream) {
  g.group_m = 8;
  constexpr int NT = WM * WN * 64;
  const int64_t tiles = ((g.M + BM - 1) / BM) * ((g.N + BN - 1) / BN);
  const int nbk = (int)(g.K / 64);
  const int kcs = (nbk + splits - 1) / splits;
  const int sp = (nbk + kcs - 1) / kcs;  // every split has at least one block
  const size_t smem = 2 * (BM + BN) * ROWP + 2 * 256 * 4;
  static_assert(2 * (BM + BN) * ROWP + 2 * 256 * 4 <= 160 * 1024, "LDS");
  static bool attr_set = false;
  if (!attr_set) {
    if (hipFuncSetAttribute((const void*)k_gemm_nf4<BM, BN, WM, WN, 2>, hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)smem) != hipSuccess) {
      vh::set_error("vh_gemm_nf4: cannot reserve %zu bytes of LDS", smem);
      return VH_ELAUNCH;
    }
    attr_set = true;
  }
  hipLaunchKernelGGL((k_gemm_nf4<BM, BN, WM, WN, 2>), dim3((unsigned)tiles, (unsigned)sp), dim3(NT), smem, stream, g,
                     q, kcs, sp > 1 ? part : nullptr);
  if (sp > 1) {
    const int64_t quads = g.M * g.N / 4;
    hipLaunchKernelGGL(k_split_reduce, dim3((unsigned)((quads + 255) / 256)), dim3(256), 0, stream, part, sp, g.M,
                       g.N, g.epi, g.C, g.ldc);
  }
  return vh::check_launch("vh_gemm_nf4");
}

// ------------------------------------------------------------ MXNF4 operands to bf16
// The two-pass form of the prefill: each operand decoded once to exactly
// the bf16(level * scale) k_gemm_nf4 stages (the same lut16 and nf4_pack16
// steps), for the bf16 GEMM.  k_gemm_nf4 decodes a weight block once per
// row tile and an activation block once per column tile; at large M one
// decode plus a write and a read of the bf16 operands costs less.

// Weight as vh_pack_nf4 bakes it, in groups of one 16-row tile and four
// 64-element blocks (256 columns); a workgroup takes NF4_DEC groups.  In a
// group, thread t takes row r = t / 16 and the 16 elements 16 (t % 16) .. +
// 15 of its 256 columns: GEMV record r + 16 c of block t % 16 / 4 (c = t %
// 4; element e in the low nibble of byte e, e + 8 in its high nibble) and
// the row's scale byte.  The 16 threads of a row write its 512 bytes
// contiguously.  Every group's loads go out before the scale table is built.
constexpr int NF4_DEC = 4;

__device__ __forceinline__ void nf4_weight_bf16(int64_t wg, const uint8_t* __restrict__ w, const uint8_t* __restrict__ ws,
                                                const Nf4Args& q, int64_t N, int64_t K, uint16_t* __restrict__ out,
                                                float* s_sc) {
  const int64_t nbk = K / 64, nq = (nbk + 3) / 4, groups = (N / 16) * nq;
  const int r = threadIdx.x >> 4, j = threadIdx.x & 15;
  uint2 rec[NF4_DEC];
  uint32_t sb[NF4_DEC];
  int64_t dst[NF4_DEC];
#pragma unroll
  for (int i = 0; i < NF4_DEC; ++i) {
    const int64_t gi = wg * NF4_DEC + i;
    const int64_t tile = gi / nq, kb = (gi % nq) * 4 + (j >> 2);
    const bool ok = gi < groups && kb < nbk;
    const int64_t u = ok ? tile * nbk + kb : 0;  // (tile, block) record group
    rec[i] = *(const uint2*)(w + (u * 64 + r + 16 * (j & 3)) * 8);
    sb[i] = ws[u * 16 + r];
    dst[i] = ok ? (tile * 16 + r) * K + kb * 64 + (j & 3) * 16 : -1;
  }
  s_sc[threadIdx.x] = fmt_decode(threadIdx.x, q.b_sf, nullptr);
  __syncthreads();
  uint32_t base;
  asm volatile("v_mov_b32 %0, 0x3020100" : "=v"(base));
#pragma unroll
  for (int i = 0; i < NF4_DEC; ++i) {
    if (dst[i] < 0) continue;
    const uint32_t l[4] = {lut_lo(rec[i].x, base, q.lvb), lut_lo(rec[i].y, base, q.lvb),
                           lut_hi(rec[i].x, base, q.lvb), lut_hi(rec[i].y, base, q.lvb)};
    uint4 lo, hi;
    nf4_pack16(l, s_sc[sb[i]], lo, hi);
    *(uint4*)(out + dst[i]) = lo;
    *(uint4*)(out + dst[i] + 8) = hi;
  }
}

// Activation as quantize_mx packs it (index bytes [M, K], scale codes
// [M, K / 64]): each thread takes NF4_DEC runs of 16 indices, 4096
// elements apart, loaded before the scale table is built.
__device__ __forceinline__ void nf4_act_bf16(int64_t wg, const uint8_t* __restrict__ x, const uint8_t* __restrict__ xs,
                                             const Nf4Args& q, int64_t M, int64_t K, uint16_t* __restrict__ out,
                                             float* s_sc) {
  const int64_t chunks = M * K / 16;
  uint4 v[NF4_DEC];
  uint32_t sc[NF4_DEC];
  int64_t e[NF4_DEC];
#pragma unroll
  for (int i = 0; i < NF4_DEC; ++i) {
    const int64_t c = (wg * NF4_DEC + i) * 256 + threadIdx.x;
    const bool ok = c < chunks;
    const int64_t ei = ok ? c * 16 : 0, row = ei / K;
    v[i] = *(const uint4*)(x + ei);
    sc[i] = xs[row * (K / 64) + (ei - row * K) / 64];
    e[i] = ok ? ei : -1;
  }
  s_sc[threadIdx.x] = fmt_decode(threadIdx.x, q.a_sf, nullptr);
  __syncthreads();
  uint32_t base;
  asm volatile("v_mov_b32 %0, 0x3020100" : "=v"(base));
#pragma unroll
  for (int i = 0; i < NF4_DEC; ++i) {
    if (e[i] < 0) continue;
    const uint32_t l[4] = {lut_lo(v[i].x, base, q.lvb), lut_lo(v[i].y, base, q.lvb), lut_lo(v[i].z, base, q.lvb),
                           lut_lo(v[i].w, base, q.lvb)};
    uint4 lo, hi;
    nf4_pack16(l, s_sc[sc[i]], lo, hi);
    *(uint4*)(out + e[i]) = lo;
    *(uint4*)(out + e[i] + 8) = hi;
  }
}

// One launch for both operands: workgroups [0, xw) take the activation,
// the rest the weight.
__global__ void __launch_bounds__(256) k_nf4_decode_bf16(const uint8_t* __restrict__ x, const uint8_t* __restrict__ xs,
                                                         int64_t M, const uint8_t* __restrict__ w,
                                                         const uint8_t* __restrict__ ws, int64_t N, int64_t K, Nf4Args q,
                                                         int64_t xw, uint16_t* __restrict__ x_out,
                                                         uint16_t* __restrict__ w_out) {
  __shared__ float s_sc[256];
  if ((int64_t)blockIdx.x < xw) nf4_act_bf16(blockIdx.x, x, xs, q, M, K, x_out, s_sc);
  else nf4_weight_bf16((int64_t)blockIdx.x - xw, w, ws, q, N, K, w_out, s_sc);
}

}  // namespace

namespace {

// Kernel families a descriptor can be dispatched to (vh_gemm_plan reports
// the family and the tile number within it).
constexpr int FAM_STAGED = 1;       // k_gemm: register-staged, decodes in staging
constexpr int FAM_DIRECT_FP8 = 2;   // k_gemm_f8dl, E4M3 operands
constexpr int FAM_DIRECT_BF16 = 3;  // k_gemm_f8dl, bf16 operands
constexpr int FAM_MXI8 = 4;         // k_gemm_mxi8 / k_gemm_mxi8_ws (+ k_split_reduce)

struct Plan {
  int family, tile, splits;
};

bool is_direct_fp8_tile(int c) {
  switch (c) {
    case 20: case 21: case 23: case 24: case 30: case 31: case 32: case 33: case 34:
    case 35: case 36: case 37: case 40: case 41: case 42: case 43: case 44: case 45: case 46: case 47:
    case 48: return true;
    default: return false;
  }
}

bool is_direct_bf16_tile(int c) { return c == 31 || c == 33 || c == 35 || c == 37 || c == 41; }

int staged_tile(int c) {
  switch (c) {
    case 2: case 3: case 5: case 6: case 7: case 8: case 9: case 10: return c;
    default: return 4;
  }
}

// The one dispatch rule of vh_gemm: which kernel and tile a descriptor runs
// (after validation), from the operand formats, the output's alignment, the
// grid size and tile_hint.
Plan plan_gemm(const vh_gemm_desc* d) {
  const int64_t batch = d->batch < 1 ? 1 : d->batch;
  auto tiles = [&](int bm, int bn) { return ((d->M + bm - 1) / bm) * ((d->N + bn - 1) / bn) * batch; };
  const bool fp8 = d->a_fmt == OP_FP8;
  const bool dl_ok = f8dl_epilogue_ok(d->C, d->epi.out_dtype, d->ldc, d->N);
  // Register-staged kernel (bf16, MX-int8 and posit8 operands; fp8 when the
  // LDS epilogue does not apply).  Measured on MI355X at M = 2048 with fp8
  // data (K in {4096, 14336}, N in {1024, 4096, 14336}): 8-wave blocks (two
  // waves per SIMD) cover the operand loads; the largest tile that still
  // fills the GPU wins (less LDS and L2 traffic per MFMA); a grid too small
  // for 256 CUs takes 128 x 64.
  int staged = d->tile_hint;
  if (staged == 0) {
    if (tiles(256, 256) >= 384) staged = 6;
    else if (tiles(256, 128) >= 256 && d->K >= 8192) staged = 9;
    else if (tiles(128, 128) >= 256) staged = 10;
    else staged = 4;
  }
  staged = staged_tile(staged);
  // The direct-to-LDS kernels move whole aligned 16-byte chunks of each
  // row: rows 16-byte aligned and K a whole number of chunks (a chunk that
  // straddled K would bring the row's padding into the products; fp8 K is
  // validated a multiple of 16 below, where the descriptor is checked).
  const bool chunks_ok = d->lda % 16 == 0 && d->ldb % 16 == 0 && d->K % (fp8 ? 16 : 8) == 0;
  if (fp8 && dl_ok && chunks_ok) {
    // Direct-to-LDS kernels with 128-byte stages.  Measured on MI355X at
    // M = 2048 (K in {4096, 14336}, N in {1024, 4096, 14336}): the largest
    // tile that still gives every CU a block wins, since each CU's operand
    // stream from L2 is the limit; 256 x 256 only pays when the grid covers
    // the GPU well over once; a grid too small even for 128 x 128 takes
    // 64 x 128 (1 x 4 waves).
    // Where 256 x 224 tiles make whole rounds of the 256 CUs and 256 x 256
    // tiles do not (N = 14336 = 64 x 224 at M = 2048: 512 tiles against 448,
    // whose last round is a quarter idle), take 256 x 224 (M = 2048, K =
    // 4096, N = 14336 under sustained load: 106.7 us against 108.7).
    int c = d->tile_hint;
    if (c == 0 && d->N % 224 == 0 && tiles(256, 224) >= 512 && tiles(256, 224) % 256 == 0 &&
        tiles(256, 256) % 256 != 0)
      c = 44;
    if (c == 0) c = tiles(256, 256) >= 384 ? 41 : tiles(256, 128) >= 224 ? 31 : tiles(128, 128) >= 224 ? 33 : 37;
    if (is_direct_fp8_tile(c)) return {FAM_DIRECT_FP8, c, 1};
  }
  if (fp8) return {FAM_STAGED, staged, 1};
  if (d->a_fmt == OP_BF16 && d->b_fmt == OP_BF16 && dl_ok && chunks_ok && (d->tile_hint == 0 || d->tile_hint >= 20)) {
    // As for fp8; a grid under 224 tiles of 128 x 128 takes 128 x 64
    // (M = 256, K = 4096 on MI355X: N = 4096 in 18.5 us against 24.6 us,
    // 21.4 against 30.1 with a float32 result; N = 14336, 224 tiles, stays
    // at 128 x 128: 33.7 us against 46.1).
    int c = d->tile_hint;
    if (c == 0) c = tiles(256, 256) >= 384 ? 41 : tiles(256, 128) >= 224 ? 31 : tiles(128, 128) >= 224 ? 33 : 35;
    if (is_direct_bf16_tile(c)) return {FAM_DIRECT_BF16, c, 1};
  }
  if (d->a_fmt == OP_MXI8 && d->b_fmt == OP_MXI8) {
    int mcfg, splits;
    mxi8_plan(d, mcfg, splits);
    if (mcfg) {
      const int64_t need = mxi8_workspace(d, splits);
      if (splits > 1 && (!d->workspace || d->workspace_bytes < need || (uintptr_t)d->workspace % 16)) splits = 1;
      return {FAM_MXI8, mcfg, splits};
    }
  }
  return {FAM_STAGED, staged, 1};
}

}  // namespace

extern "C" int vh_gemm_plan(const vh_gemm_desc* d, int32_t* family, int32_t* tile, int32_t* splits) {
  VH_REQUIRE(d && family && tile && splits, "vh_gemm_plan: null argument");
  const Plan p = plan_gemm(d);
  *family = p.family;
  *tile = p.tile;
  *splits = p.splits;
  return VH_OK;
}

extern "C" int vh_gemm(const vh_gemm_desc* d, vh_stream_t stream) {
  VH_REQUIRE(d, "vh_gemm: null descriptor");
  VH_REQUIRE(d->A && d->B && d->C, "vh_gemm: null operand");
  VH_REQUIRE(d->M >= 0 && d->N >= 0 && d->K >= 0, "vh_gemm: negative size");
  const bool fp8 = d->a_fmt == OP_FP8;
  VH_REQUIRE(fp8 == (d->b_fmt == OP_FP8), "vh_gemm: fp8 operands must be paired");
  VH_REQUIRE(d->a_fmt >= OP_BF16 && d->a_fmt <= OP_P8 && d->b_fmt >= OP_BF16 && d->b_fmt <= OP_P8,
             "vh_gemm: bad operand format");
  VH_REQUIRE(d->epi.out_dtype == VH_BF16 || d->epi.out_dtype == VH_F32, "vh_gemm: output must be bf16 or f32");
  // the epilogue reads its scalar and bias as bf16 or float32
  VH_REQUIRE(!d->epi.scale || d->epi.scale_dtype == VH_BF16 || d->epi.scale_dtype == VH_F32,
             "vh_gemm: epilogue scale must be bf16 or f32");
  VH_REQUIRE(!d->epi.bias || d->epi.bias_dtype == VH_BF16 || d->epi.bias_dtype == VH_F32,
             "vh_gemm: bias must be bf16 or f32");
  VH_REQUIRE(d->epi.mode == EPI_PLAIN || d->epi.mode == EPI_ROUND_SCALE, "vh_gemm: bad epilogue mode");
  // 16-byte aligned rows (the loads are 16 / 8 bytes wide)
  auto rowbytes_ok = [](int fmt, int64_t ld) { return fmt == OP_BF16 ? (ld % 16 == 0) : (ld % 8 == 0); };
  VH_REQUIRE(rowbytes_ok(d->a_fmt, d->lda) && rowbytes_ok(d->b_fmt, d->ldb), "vh_gemm: row pitch misaligned");
  VH_REQUIRE(((uintptr_t)d->A % 16 == 0) && ((uintptr_t)d->B % 16 == 0), "vh_gemm: operand pointer misaligned");
  const int64_t kmul = fp8 ? 16 : 8;
  VH_REQUIRE(d->K % kmul == 0, "vh_gemm: K must be a multiple of %lld", (long long)kmul);
  for (int s = 0; s < 2; ++s) {
    int fmt = s ? d->b_fmt : d->a_fmt;
    if (fmt == OP_MXI8) {
      const void* sp = s ? d->b_scale : d->a_scale;
      int blk = s ? d->b_block : d->a_block;
      VH_REQUIRE(sp && blk >= 8 && (blk & (blk - 1)) == 0, "vh_gemm: MX int8 operand needs a power-of-two block >= 8");
    }
    if (fmt == OP_P8) VH_REQUIRE(d->lut, "vh_gemm: posit8 operand needs its decode table");
  }
  VH_REQUIRE(d->lda * 256 < (1ll << 31) && d->ldb * 256 < (1ll << 31), "vh_gemm: rows too long for 32-bit offsets");
  if (d->M == 0 || d->N == 0) return VH_OK;
  GemmArgs g;
  memset(&g, 0, sizeof(g));
  g.A = (const uint8_t*)d->A;
  g.B = (const uint8_t*)d->B;
  g.C = d->C;
  g.M = d->M;
  g.N = d->N;
  g.K = d->K;
  g.lda = d->lda;
  g.ldb = d->ldb;
  g.ldc = d->ldc;
  g.a_fmt = d->a_fmt;
  g.b_fmt = d->b_fmt;
  g.a_scale = (const uint8_t*)d->a_scale;
  g.b_scale = (const uint8_t*)d->b_scale;
  g.lds_a = d->a_scale_ld;
  g.lds_b = d->b_scale_ld;
  g.a_block = d->a_block;
  g.b_block = d->b_block;
  g.a_bias = d->a_bias;
  g.b_bias = d->b_bias;
  g.lut = (const uint16_t*)d->lut;
  g.epi = d->epi;
  g.sa = d->batch_stride_a;
  g.sb = d->batch_stride_b;
  g.sc = d->batch_stride_c;
  g.ssa = d->batch_stride_a_scale;
  g.ssb = d->batch_stride_b_scale;
  const int64_t batch = d->batch < 1 ? 1 : d->batch;
  VH_REQUIRE(batch < 65536, "vh_gemm: batch too large");
  hipStream_t st = vh::as_stream(stream);
  const Plan p = plan_gemm(d);
  if (p.family == FAM_DIRECT_FP8) {
    switch (p.tile) {
      case 20: return launch_f8dl<256, 256, 4, 64>(g, batch, st);
      case 21: return launch_f8dl<256, 128, 4, 64>(g, batch, st);
      case 23: return launch_f8dl<128, 128, 8, 64>(g, batch, st);
      case 24: return launch_f8dl<128, 256, 4, 64>(g, batch, st);
      case 30: return launch_f8dl<256, 256, 2, 128>(g, batch, st);
      case 31: return launch_f8dl<256, 128, 3, 128>(g, batch, st);
      case 32: return launch_f8dl<128, 256, 3, 128>(g, batch, st);
      case 33: return launch_f8dl<128, 128, 4, 128>(g, batch, st);
      case 34: return launch_f8dl<256, 128, 2, 128>(g, batch, st);
      case 40: return launch_f8dl<256, 256, 2, 128, 2, 4>(g, batch, st);
      case 41: return launch_f8dl<256, 256, 2, 128, 4, 2>(g, batch, st);
      case 42: return launch_f8dl<256, 128, 3, 128, 2, 4>(g, batch, st);
      case 43: return launch_f8dl<256, 128, 3, 128, 4, 2>(g, batch, st);
      case 44: return launch_f8dl<256, 224, 2, 128, 4, 1>(g, batch, st);
      case 45: return launch_f8dl<128, 448, 2, 128, 2, 2>(g, batch, st);
      case 46: return launch_f8dl<256, 256, 4, 64, 4, 2>(g, batch, st);
      case 47: return launch_f8dl<256, 128, 4, 64, 4, 2>(g, batch, st);
      case 48: return launch_f8dl<256, 256, 4, 64, 2, 4>(g, batch, st);
      case 35: return launch_f8dl<128, 64, 4, 128, 2, 2>(g, batch, st);
      case 36: return launch_f8dl<128, 64, 6, 128, 2, 2>(g, batch, st);
      case 37: return launch_f8dl<64, 128, 4, 128, 1, 4>(g, batch, st);
      default: break;
    }
  } else if (p.family == FAM_DIRECT_BF16) {
    switch (p.tile) {
      case 41: return launch_f8dl<256, 256, 2, 128, 4, 2, OP_BF16>(g, batch, st);
      case 31: return launch_f8dl<256, 128, 3, 128, 2, 2, OP_BF16>(g, batch, st);
      case 33: return launch_f8dl<128, 128, 4, 128, 2, 2, OP_BF16>(g, batch, st);
      case 35: return launch_f8dl<128, 64, 4, 128, 2, 2, OP_BF16>(g, batch, st);
      case 37: return launch_f8dl<64, 128, 4, 128, 1, 4, OP_BF16>(g, batch, st);
      default: break;
    }
  } else if (p.family == FAM_MXI8) {
    float* part = (float*)d->workspace;
    switch (p.tile) {
      case 50: return launch_mxi8<128, 128, 2, 2>(g, p.splits, part, st);
      case 51: return launch_mxi8<128, 128, 4, 2>(g, p.splits, part, st);
      case 52: return launch_mxi8<128, 64, 2, 2>(g, p.splits, part, st);
      case 53: return launch_mxi8<256, 128, 4, 2>(g, p.splits, part, st);
      case 54: return launch_mxi8<64, 128, 1, 4>(g, p.splits, part, st);
      case 55: return launch_mxi8<128, 128, 2, 2, 2, true>(g, p.splits, part, st);
      case 56: return launch_mxi8<256, 128, 2, 2, 2, true>(g, p.splits, part, st);
      case 60: return launch_mx8h(g, p.splits, part, st);
      default: break;
    }
  }
  auto pick = [&](auto tag) -> int {
    constexpr int AF = decltype(tag)::a, BF = decltype(tag)::b;
    switch (p.tile) {
      case 2: return launch_tile<256, 128, 2, 2, 1, 1, AF, BF>(g, batch, st);
      case 3: return launch_tile<128, 128, 2, 2, 2, 2, AF, BF>(g, batch, st);
      case 5: return launch_tile<256, 128, 4, 2, 1, 2, AF, BF>(g, batch, st);
      case 6: return launch_tile<256, 256, 4, 2, 1, 1, AF, BF>(g, batch, st);
      case 7: return launch_tile<128, 256, 2, 4, 1, 2, AF, BF>(g, batch, st);
      case 8: return launch_tile<128, 128, 4, 2, 1, 2, AF, BF>(g, batch, st);
      case 9: return launch_tile<256, 128, 4, 2, 1, 1, AF, BF>(g, batch, st);
      case 10: return launch_tile<128, 128, 4, 2, 1, 1, AF, BF>(g, batch, st);
      default: return launch_tile<128, 64, 2, 2, 2, 2, AF, BF>(g, batch, st);
    }
  };
  if (fp8) return pick(Fmts<OP_FP8, OP_FP8>{});
  if (d->a_fmt == OP_BF16 && d->b_fmt == OP_BF16) return pick(Fmts<OP_BF16, OP_BF16>{});
  if (d->a_fmt == OP_MXI8 && d->b_fmt == OP_MXI8) return pick(Fmts<OP_MXI8, OP_MXI8>{});
  if (d->a_fmt == OP_P8 && d->b_fmt == OP_P8) return pick(Fmts<OP_P8, OP_P8>{});
  if (d->a_fmt == OP_BF16 && d->b_fmt == OP_MXI8) return pick(Fmts<OP_BF16, OP_MXI8>{});
  if (d->a_fmt == OP_BF16 && d->b_fmt == OP_P8) return pick(Fmts<OP_BF16, OP_P8>{});
  vh::set_error("vh_gemm: operand format pair (%d, %d) is not built", d->a_fmt, d->b_fmt);
  return VH_EINVAL;
}

extern "C" int64_t vh_gemm_workspace_bytes(const vh_gemm_desc* d) {
  if (!d) return 0;
  int cfg, splits;
  mxi8_plan(d, cfg, splits);
  return cfg ? mxi8_workspace(d, splits) : 0;
}

// ------------------------------------------------------------ MX-int8 on exact fp16
// linear_mx of MX-int8 operands (ops/quantized.py:651-723) at small M, with
// both operands already decoded to exact fp16 against a power of two per row
// of x and per column of w (vh_quantize_mx8_f16, vh_mx8_bake_f16): a plain
// fp16 direct-to-LDS GEMM over K splits into float32 partials, then the
// split reduction multiplies each sum by 2**(E_row + E_col) and applies the
// epilogue.  The decode is gone from the GEMM's inner loop, which bounds the
// kernels that decode MX-int8 codes in staging at these sizes.
extern "C" int vh_gemm_mx8_f16(const uint16_t* x, const int32_t* ex, const uint16_t* w, const int32_t* ew, int64_t M,
                               int64_t N, int64_t K, const vh_epilogue* epi, void* y, int64_t ldy, float* part,
                               int64_t part_bytes, int32_t splits, int32_t tile, vh_stream_t stream) {
  VH_REQUIRE(x && ex && w && ew && epi && y && (part || splits == 1), "vh_gemm_mx8_f16: null argument");
  VH_REQUIRE(M > 0 && N > 0 && K > 0, "vh_gemm_mx8_f16: empty GEMM");
  VH_REQUIRE(splits >= 1 && K % (8 * (int64_t)splits) == 0,
             "vh_gemm_mx8_f16: K (%lld) must split into %d multiples of 8", (long long)K, splits);
  VH_REQUIRE(N % 4 == 0 && ldy >= N, "vh_gemm_mx8_f16: N must be a multiple of 4 and ldy >= N");
  // one split whose output the kernel's own epilogue can store needs no workspace
  const bool direct = splits == 1 && f8dl_epilogue_ok(y, epi->out_dtype, ldy, N);
  VH_REQUIRE(direct || part_bytes >= (int64_t)splits * M * N * 4,
             "vh_gemm_mx8_f16: workspace of %lld bytes, %lld needed", (long long)part_bytes,
             (long long)((int64_t)splits * M * N * 4));
  VH_REQUIRE((uintptr_t)x % 16 == 0 && (uintptr_t)w % 16 == 0 && (direct || (uintptr_t)part % 16 == 0),
             "vh_gemm_mx8_f16: operands and workspace must be 16-byte aligned");
  VH_REQUIRE(K * 2 < (1ll << 31) && M * K * 2 < (1ll << 31) && N * K * 2 < (1ll << 31),
             "vh_gemm_mx8_f16: operands over 2 GiB");
  VH_REQUIRE(epi->mode == EPI_PLAIN && (epi->out_dtype == VH_BF16 || epi->out_dtype == VH_F32),
             "vh_gemm_mx8_f16: unsupported epilogue");
  VH_REQUIRE(!epi->scale || epi->scale_dtype == VH_BF16 || epi->scale_dtype == VH_F32,
             "vh_gemm_mx8_f16: scale must be bf16 or float32");
  VH_REQUIRE(!epi->bias || epi->bias_dtype == VH_BF16 || epi->bias_dtype == VH_F32,
             "vh_gemm_mx8_f16: bias must be bf16 or float32");
  GemmArgs g;
  memset(&g, 0, sizeof(g));
  g.A = (const uint8_t*)x;
  g.B = (const uint8_t*)w;
  g.C = part;
  g.M = M;
  g.N = N;
  g.K = K / splits;
  g.lda = K * 2;
  g.ldb = K * 2;
  g.ldc = N;
  g.sa = (K / splits) * 2;  // split z reads columns [z K / S, (z + 1) K / S)
  g.sb = (K / splits) * 2;
  g.sc = M * N;             // and writes partial z
  g.epi.mode = EPI_PLAIN;
  g.epi.out_dtype = VH_F32;
  if (direct) {  // the exponents, alpha, bias and the rounding in the GEMM's own epilogue
    g.C = y;
    g.ldc = ldy;
    g.epi = *epi;
    g.ea = ex;
    g.eb = ew;
  }
  hipStream_t st = vh::as_stream(stream);
  int rc;
  switch (tile) {
    case 1: rc = launch_f8dl<64, 128, 4, 128, 1, 4, OP_F16X>(g, splits, st); break;
    case 2: rc = launch_f8dl<128, 64, 4, 128, 2, 2, OP_F16X>(g, splits, st); break;
    case 3: rc = launch_f8dl<256, 128, 3, 128, 2, 2, OP_F16X>(g, splits, st); break;
    case 4: rc = launch_f8dl<64, 64, 8, 128, 1, 2, OP_F16X>(g, splits, st); break;
    default: rc = launch_f8dl<128, 128, 4, 128, 2, 2, OP_F16X>(g, splits, st); break;
  }
  if (rc || direct) return rc;
  const int64_t quads = M * N / 4;
  hipLaunchKernelGGL(k_split_reduce, dim3((unsigned)((quads + 255) / 256)), dim3(256), 0, st, (const float*)part,
                     (int)splits, M, N, *epi, y, ldy, ex, ew);
  return vh::check_launch("vh_gemm_mx8_f16");
}

extern "C" int vh_gemm_nf4(const uint8_t* x_idx, const uint8_t* x_scale, const vh_format* x_scale_fmt, int64_t M,
                           const uint8_t* w_packed, const uint8_t* w_scale, const vh_format* w_scale_fmt,
                           const int8_t* levels16, int64_t N, int64_t K, const vh_epilogue* epi, void* y,
                           int64_t ldy, int32_t tile, int32_t splits, float* part, int64_t part_bytes,
                           vh_stream_t stream) {
  VH_REQUIRE(x_idx && x_scale && x_scale_fmt && w_packed && w_scale && w_scale_fmt && levels16 && epi && y,
             "vh_gemm_nf4: null argument");
  VH_REQUIRE(M >= 1 && N > 0 && K > 0 && N % 16 == 0 && K % 64 == 0,
             "vh_gemm_nf4: needs N %% 16 == 0 and K %% 64 == 0");
  VH_REQUIRE(M * K < (1ll << 31) && (N / 16) * (K / 64) * 512 < (1ll << 31), "vh_gemm_nf4: operands over 2 GiB");
  VH_REQUIRE((uintptr_t)x_idx % 16 == 0 && K % 16 == 0 && (uintptr_t)w_packed % 8 == 0,
             "vh_gemm_nf4: misaligned operand");
  VH_REQUIRE(epi->mode == EPI_PLAIN && (epi->out_dtype == VH_BF16 || epi->out_dtype == VH_F32) && ldy >= N,
             "vh_gemm_nf4: unsupported epilogue");
  VH_REQUIRE(!epi->scale || epi->scale_dtype == VH_BF16 || epi->scale_dtype == VH_F32,
             "vh_gemm_nf4: scale must be bf16 or float32");
  VH_REQUIRE(!epi->bias || epi->bias_dtype == VH_BF16 || epi->bias_dtype == VH_F32,
             "vh_gemm_nf4: bias must be bf16 or float32");
  for (const vh_format* f : {x_scale_fmt, w_scale_fmt})
    VH_REQUIRE(f->kind == VH_FMT_INT || f->kind == VH_FMT_MINIFLOAT || f->kind == VH_FMT_POSIT,
               "vh_gemm_nf4: the scale maps need a closed form with packed codes");
  uint8_t lvb[16];
  for (int v = 0; v < 16; ++v) lvb[v] = (uint8_t)(levels16[v] + 128);
  uint32_t t[4];
  memcpy(t, lvb, 16);
  Nf4Args q;
  q.lvb = make_uint4(t[0], t[1], t[2], t[3]);
  q.a_sf = *x_scale_fmt;
  q.b_sf = *w_scale_fmt;
  GemmArgs g;
  memset(&g, 0, sizeof(g));
  g.A = x_idx;
  g.B = w_packed;
  g.C = y;
  g.M = M;
  g.N = N;
  g.K = K;
  g.lda = K;
  g.ldc = ldy;
  g.a_scale = x_scale;
  g.b_scale = w_scale;
  g.lds_a = K / 64;
  g.epi = *epi;
  hipStream_t st = vh::as_stream(stream);
  int64_t bm = 0;
  VH_REQUIRE(vh_gemm_nf4_plan(M, N, K, &tile, &splits, &bm) == VH_OK, "vh_gemm_nf4: tile must be 0, 1 or 2");
  VH_REQUIRE(splits == 1 || (part && part_bytes >= (int64_t)splits * M * N * 4 && (ldy == N) && N % 4 == 0),
             "vh_gemm_nf4: %d K splits need a workspace of %lld bytes (and ldy == N)", splits,
             (long long)((int64_t)splits * M * N * 4));
  if (tile == 2) return launch_nf4<256, 128, 4, 2>(g, q, splits, part, st);
  return launch_nf4<128, 128, 2, 2>(g, q, splits, part, st);
}

extern "C" int vh_gemm_nf4_plan(int64_t M, int64_t N, int64_t K, int32_t* tile, int32_t* splits, int64_t* bm) {
  VH_REQUIRE(tile && splits && bm && M >= 1 && N > 0 && K >= 64, "vh_gemm_nf4_plan: bad arguments");
  // 256 x 128 tiles (8 waves) while they fill the 256 CUs, else 128 x 128
  // (4 waves) with K split to fill them
  if (*tile == 0) *tile = ((M + 255) / 256) * ((N + 127) / 128) >= 192 ? 2 : 1;
  VH_REQUIRE(*tile == 1 || *tile == 2, "vh_gemm_nf4_plan: tile must be 0, 1 or 2");
  *bm = *tile == 2 ? 256 : 128;
  if (*splits <= 0) *splits = nf4_splits(((M + *bm - 1) / *bm) * ((N + 127) / 128), K / 64);
  const int64_t nbk = K / 64, kcs = (nbk + *splits - 1) / *splits;
  *splits = (int32_t)((nbk + kcs - 1) / kcs);
  return VH_OK;
}

extern "C" int vh_nf4_decode_bf16(const uint8_t* x_idx, const uint8_t* x_scale, const vh_format* x_scale_fmt,
                                  int64_t M, const uint8_t* w_packed, const uint8_t* w_scale,
                                  const vh_format* w_scale_fmt, const int8_t* levels16, int64_t N, int64_t K,
                                  uint16_t* x_out, uint16_t* w_out, vh_stream_t stream) {
  VH_REQUIRE(levels16 && K > 0 && K % 64 == 0, "vh_nf4_decode_bf16: needs the levels and K %% 64 == 0");
  VH_REQUIRE(!x_out || (x_idx && x_scale && x_scale_fmt && M >= 1), "vh_nf4_decode_bf16: activation arguments");
  VH_REQUIRE(!w_out || (w_packed && w_scale && w_scale_fmt && N > 0 && N % 16 == 0),
             "vh_nf4_decode_bf16: weight arguments (N %% 16 == 0)");
  VH_REQUIRE((!x_out || ((uintptr_t)x_idx % 16 == 0 && (uintptr_t)x_out % 16 == 0)) &&
                 (!w_out || ((uintptr_t)w_packed % 8 == 0 && (uintptr_t)w_out % 16 == 0)),
             "vh_nf4_decode_bf16: misaligned operand");
  for (const vh_format* f : {x_out ? x_scale_fmt : nullptr, w_out ? w_scale_fmt : nullptr})
    VH_REQUIRE(!f || f->kind == VH_FMT_INT || f->kind == VH_FMT_MINIFLOAT || f->kind == VH_FMT_POSIT,
               "vh_nf4_decode_bf16: the scale maps need a closed form with packed codes");
  uint8_t lvb[16];
  for (int v = 0; v < 16; ++v) lvb[v] = (uint8_t)(levels16[v] + 128);
  uint32_t t[4];
  memcpy(t, lvb, 16);
  Nf4Args q;
  memset(&q, 0, sizeof(q));
  q.lvb = make_uint4(t[0], t[1], t[2], t[3]);
  if (x_out) q.a_sf = *x_scale_fmt;
  if (w_out) q.b_sf = *w_scale_fmt;
  const int64_t per = 256 * NF4_DEC;
  const int64_t xw = x_out ? (M * K / 16 + per - 1) / per : 0;
  const int64_t groups = w_out ? (N / 16) * ((K / 64 + 3) / 4) : 0;  // (tile, four blocks)
  const int64_t ww = (groups + NF4_DEC - 1) / NF4_DEC;
  VH_REQUIRE(xw + ww < (1ll << 31), "vh_nf4_decode_bf16: operands too large");
  if (xw + ww == 0) return VH_OK;
  hipLaunchKernelGGL(k_nf4_decode_bf16, dim3((unsigned)(xw + ww)), dim3(256), 0, vh::as_stream(stream), x_idx, x_scale,
                     x_out ? M : 0, w_packed, w_scale, w_out ? N : 0, K, q, xw, x_out, w_out);
  return vh::check_launch("vh_nf4_decode_bf16");
}
