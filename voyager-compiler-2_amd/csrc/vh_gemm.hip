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
// The block tile is BM x BN with a 128-byte K stage per row, double buffered
// in LDS (rows padded to 144 bytes so a wave's 16-byte fragment reads hit
// distinct banks); 4 waves (2 x 2), each owning a (BM/2) x (BN/2) sub-tile of
// 32 x 32 MFMA tiles.  Tiles are ordered so that blocks that share operand
// rows run on the same XCD (blocks are dealt to the 8 XCDs round robin).
#include <hip/hip_runtime.h>

#include <cstring>

#include "vh_device.h"
#include "vh_gemm.h"
#include "vh_host.h"

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

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
  vh_epilogue epi;
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

  // ---- tile id with XCD grouping
  const int64_t tiles_m = (g.M + BM - 1) / BM;
  const int64_t tiles_n = (g.N + BN - 1) / BN;
  const int64_t ntiles = tiles_m * tiles_n;
  int64_t pid = blockIdx.x;
  if ((ntiles & 7) == 0) pid = (pid & 7) * (ntiles >> 3) + (pid >> 3);
  // group GM tile-rows so consecutive ids walk down a column band
  constexpr int GM = 8;
  const int64_t group = pid / (GM * tiles_n);
  const int64_t first_m = group * GM;
  const int64_t gsize = (tiles_m - first_m) < GM ? (tiles_m - first_m) : GM;
  const int64_t tm = first_m + (pid % (GM * tiles_n)) % gsize;
  const int64_t tn = (pid % (GM * tiles_n)) / gsize;
  const int64_t m0 = tm * BM, n0 = tn * BN;
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

  // ---- epilogue: lane holds column lrow of each 32x32 tile, rows
  // (r/4)*8 + lhalf*4 + r%4.
  const vh_epilogue& e = g.epi;
  float sc = 1.0f;
  if (e.scale) sc = e.scale_dtype == VH_BF16 ? bf2f(*(const uint16_t*)e.scale) : *(const float*)e.scale;

  // bf16 output through LDS: each wave rounds its sub-tile (hardware
  // converter, round half to even), writes it row-major to LDS (the stage
  // buffers are free after the loop's last barrier), and stores whole
  // 16-byte row chunks.
  constexpr int SUBM = BM / WM, SUBN = BN / WN, PITCH = SUBN + 8;  // bf16 elements
  static_assert(WM * WN * SUBM * PITCH * 2 <= 2 * (BM + BN) * ROWP, "epilogue tile does not fit the stage LDS");
  if (e.out_dtype == VH_BF16 && ((uintptr_t)g.C % 16) == 0 && (g.ldc % 8) == 0 && (g.N % 8) == 0) {
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
    return;
  }
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int64_t col = n0 + wn * (BN / WN) + j * 32 + lrow;
      if (col >= g.N) continue;
      float bias = 0.0f;
      if (e.bias) bias = e.bias_dtype == VH_BF16 ? bf2f(((const uint16_t*)e.bias)[col]) : ((const float*)e.bias)[col];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = m0 + wm * (BM / WM) + i * 32 + (r >> 2) * 8 + lhalf * 4 + (r & 3);
        if (row >= g.M) continue;
        float v = acc[i][j][r];
        if (e.mode == EPI_ROUND_SCALE) {
          // dequantize(linear(xq, wq), s): the GEMM rounds to bf16, then the
          // bf16 product with the scale rounds again.
          v = rbf(rbf(v) * sc);
        } else {
          if (e.scale) v = v * sc;
          if (e.bias) v = v + bias;
        }
        if (e.out_dtype == VH_BF16) ((uint16_t*)g.C)[row * g.ldc + col] = (uint16_t)f2bf(v);
        else ((float*)g.C)[row * g.ldc + col] = v;
      }
    }
  }
}

template <int BM, int BN, int WM, int WN, int MINB, int PF, int AF, int BF>
int launch_tile(const GemmArgs& g, int64_t batch, hipStream_t stream) {
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

template <int A, int B>
struct Fmts {
  static constexpr int a = A, b = B;
};

}  // namespace

extern "C" int vh_gemm(const vh_gemm_desc* d, vh_stream_t stream) {
  VH_REQUIRE(d, "vh_gemm: null descriptor");
  VH_REQUIRE(d->A && d->B && d->C, "vh_gemm: null operand");
  VH_REQUIRE(d->M >= 0 && d->N >= 0 && d->K >= 0, "vh_gemm: negative size");
  const bool fp8 = d->a_fmt == OP_FP8;
  VH_REQUIRE(fp8 == (d->b_fmt == OP_FP8), "vh_gemm: fp8 operands must be paired");
  VH_REQUIRE(d->a_fmt >= OP_BF16 && d->a_fmt <= OP_P8 && d->b_fmt >= OP_BF16 && d->b_fmt <= OP_P8,
             "vh_gemm: bad operand format");
  VH_REQUIRE(d->epi.out_dtype == VH_BF16 || d->epi.out_dtype == VH_F32, "vh_gemm: output must be bf16 or f32");
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
  // Tile choice: enough tiles to fill 256 CUs before growing the tile.
  auto tiles = [&](int bm, int bn) { return ((d->M + bm - 1) / bm) * ((d->N + bn - 1) / bn); };
  int cfg = d->tile_hint;
  if (cfg == 0) {
    // Measured on MI355X at M = 2048 with amax-scaled fp8 data (K in {4096,
    // 14336}, N in {1024, 4096, 14336}): 8-wave blocks (two waves per SIMD)
    // cover the operand loads; the largest tile that still fills the GPU
    // wins (less LDS and L2 traffic per MFMA); a grid too small for 256 CUs
    // takes 128 x 64.
    const int64_t t256 = tiles(256, 256) * batch, t2561 = tiles(256, 128) * batch;
    const int64_t t128 = tiles(128, 128) * batch;
    if (t256 >= 384) cfg = 6;
    else if (t2561 >= 256 && d->K >= 8192) cfg = 9;
    else if (t128 >= 256) cfg = 10;
    else cfg = 4;
  }
  auto pick = [&](auto tag) -> int {
    constexpr int AF = decltype(tag)::a, BF = decltype(tag)::b;
    switch (cfg) {
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
