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
constexpr int NT = 256;     // threads per block

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
// Bytes of one row of a stage that a thread loads with one 16-byte access:
// for fp8/bf16 the stored bytes are the LDS bytes; for decoded formats a
// 16-byte LDS chunk (8 bf16) comes from 8 code bytes.
__device__ __forceinline__ uint4 load16(const uint8_t* p, bool ok) {
  if (!ok) return make_uint4(0, 0, 0, 0);
  return *(const uint4*)p;
}

__device__ __forceinline__ uint2 load8(const uint8_t* p, bool ok) {
  if (!ok) return make_uint2(0, 0);
  return *(const uint2*)p;
}

// bf16 bits of int8 code c times 2**e (exact: |c| < 2**8 and 2**e >= 2**-133
// whenever a code is nonzero in a block that scale could round).
__device__ __forceinline__ uint32_t mxi8_bf16(int c, int e) {
  float v = ldexpf((float)c, e);
  return __float_as_uint(v) >> 16;
}

__device__ __forceinline__ uint4 decode_mxi8(uint2 raw, int e) {
  uint32_t b[8];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    b[j] = (raw.x >> (8 * j)) & 0xffu;
    b[4 + j] = (raw.y >> (8 * j)) & 0xffu;
  }
  uint4 o;
  o.x = mxi8_bf16((int8_t)b[0], e) | (mxi8_bf16((int8_t)b[1], e) << 16);
  o.y = mxi8_bf16((int8_t)b[2], e) | (mxi8_bf16((int8_t)b[3], e) << 16);
  o.z = mxi8_bf16((int8_t)b[4], e) | (mxi8_bf16((int8_t)b[5], e) << 16);
  o.w = mxi8_bf16((int8_t)b[6], e) | (mxi8_bf16((int8_t)b[7], e) << 16);
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

// The 16-byte LDS chunk `c` (0..7) of row `r` of stage starting at element
// k0, for an operand in format fmt.
struct Operand {
  const uint8_t* p;
  int64_t rows, ld, K;
  int fmt;
  const uint8_t* scale;
  int64_t lds;
  int block, bias;
};

__device__ __forceinline__ uint4 fetch_chunk(const Operand& o, int64_t r, int c, int64_t k0, const uint16_t* lut) {
  const bool rok = r < o.rows;
  if (o.fmt == OP_FP8) {
    int64_t k = k0 + c * 16;
    return load16(o.p + r * o.ld + k, rok && k < o.K);
  }
  if (o.fmt == OP_BF16) {
    int64_t k = k0 + c * 8;
    return load16(o.p + r * o.ld + k * 2, rok && k < o.K);
  }
  // decoded formats: 8 elements from 8 code bytes
  int64_t k = k0 + c * 8;
  bool ok = rok && k < o.K;
  uint2 raw = load8(o.p + r * o.ld + k, ok);
  if (o.fmt == OP_MXI8) {
    int e = 0;
    if (ok) e = (int)o.scale[r * o.lds + k / o.block] - o.bias;
    return decode_mxi8(raw, e);
  }
  return decode_p8(raw, lut);
}

template <int BM, int BN, bool FP8>
__global__ void __launch_bounds__(NT, 1) k_gemm(GemmArgs g) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  uint8_t* As = smem;                          // [2][BM][ROWP]
  uint8_t* Bs = smem + 2 * BM * ROWP;          // [2][BN][ROWP]
  uint16_t* lut = (uint16_t*)(smem + 2 * (BM + BN) * ROWP);  // [256] for OP_P8

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  if (g.a_fmt == OP_P8 || g.b_fmt == OP_P8) {
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

  Operand oa{g.A + m0 * g.lda, g.M - m0, g.lda, g.K, g.a_fmt, g.a_scale ? g.a_scale + m0 * g.lds_a : nullptr,
             g.lds_a, g.a_block, g.a_bias};
  Operand ob{g.B + n0 * g.ldb, g.N - n0, g.ldb, g.K, g.b_fmt, g.b_scale ? g.b_scale + n0 * g.lds_b : nullptr,
             g.lds_b, g.b_block, g.b_bias};

  constexpr int KE = FP8 ? 128 : 64;      // K elements per stage
  constexpr int CA = BM * 8 / NT;         // 16-byte chunks per thread (A)
  constexpr int CB = BN * 8 / NT;
  static_assert(CA >= 1 && CB >= 1, "tile too small");

  uint4 ra[CA], rb[CB];
  auto fetch = [&](int64_t k0) {
#pragma unroll
    for (int i = 0; i < CA; ++i) {
      int ch = tid + i * NT;
      ra[i] = fetch_chunk(oa, ch >> 3, ch & 7, k0, lut);
    }
#pragma unroll
    for (int i = 0; i < CB; ++i) {
      int ch = tid + i * NT;
      rb[i] = fetch_chunk(ob, ch >> 3, ch & 7, k0, lut);
    }
  };
  auto stash = [&](int s) {
    uint8_t* a = As + s * BM * ROWP;
    uint8_t* b = Bs + s * BN * ROWP;
#pragma unroll
    for (int i = 0; i < CA; ++i) {
      int ch = tid + i * NT;
      *(uint4*)(a + (ch >> 3) * ROWP + (ch & 7) * 16) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < CB; ++i) {
      int ch = tid + i * NT;
      *(uint4*)(b + (ch >> 3) * ROWP + (ch & 7) * 16) = rb[i];
    }
  };

  constexpr int TM = BM / 64;  // 32-row MFMA tiles per wave
  constexpr int TN = BN / 64;
  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int64_t nk = (g.K + KE - 1) / KE;
  fetch(0);
  stash(0);
  __syncthreads();

  const int lrow = lane & 31;
  const int lhalf = lane >> 5;
  for (int64_t ks = 0; ks < nk; ++ks) {
    const int s = ks & 1;
    if (ks + 1 < nk) fetch((ks + 1) * KE);
    const uint8_t* a = As + s * BM * ROWP + (wm * (BM / 2) + lrow) * ROWP;
    const uint8_t* b = Bs + s * BN * ROWP + (wn * (BN / 2) + lrow) * ROWP;
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
    if (ks + 1 < nk) {
      stash(s ^ 1);
    }
    __syncthreads();
  }

  // ---- epilogue: lane holds column lrow of each 32x32 tile, rows
  // (r/4)*8 + lhalf*4 + r%4.
  const vh_epilogue& e = g.epi;
  float sc = 1.0f;
  if (e.scale) sc = e.scale_dtype == VH_BF16 ? bf2f(*(const uint16_t*)e.scale) : *(const float*)e.scale;
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int64_t col = n0 + wn * (BN / 2) + j * 32 + lrow;
      if (col >= g.N) continue;
      float bias = 0.0f;
      if (e.bias) bias = e.bias_dtype == VH_BF16 ? bf2f(((const uint16_t*)e.bias)[col]) : ((const float*)e.bias)[col];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = m0 + wm * (BM / 2) + i * 32 + (r >> 2) * 8 + lhalf * 4 + (r & 3);
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

template <int BM, int BN, bool FP8>
int launch_tile(const GemmArgs& g, int64_t batch, hipStream_t stream) {
  const int64_t tiles = ((g.M + BM - 1) / BM) * ((g.N + BN - 1) / BN);
  const size_t smem = 2 * (BM + BN) * ROWP + 512;
  static bool attr_set = false;
  if (!attr_set) {
    if (hipFuncSetAttribute((const void*)k_gemm<BM, BN, FP8>, hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)smem) != hipSuccess) {
      vh::set_error("vh_gemm: cannot reserve %zu bytes of LDS", smem);
      return VH_ELAUNCH;
    }
    attr_set = true;
  }
  hipLaunchKernelGGL((k_gemm<BM, BN, FP8>), dim3((unsigned)tiles, (unsigned)batch), dim3(NT), smem, stream, g);
  return vh::check_launch("vh_gemm");
}

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
      VH_REQUIRE(sp && blk >= 8 && blk % 8 == 0, "vh_gemm: MX int8 operand needs scales with block %% 8 == 0");
    }
    if (fmt == OP_P8) VH_REQUIRE(d->lut, "vh_gemm: posit8 operand needs its decode table");
  }
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
    if (tiles(256, 128) * batch >= 256) cfg = 2;
    else if (tiles(128, 128) * batch >= 256) cfg = 3;
    else cfg = 4;
  }
  if (fp8) {
    switch (cfg) {
      case 2: return launch_tile<256, 128, true>(g, batch, st);
      case 3: return launch_tile<128, 128, true>(g, batch, st);
      default: return launch_tile<128, 64, true>(g, batch, st);
    }
  }
  switch (cfg) {
    case 2: return launch_tile<256, 128, false>(g, batch, st);
    case 3: return launch_tile<128, 128, false>(g, batch, st);
    default: return launch_tile<128, 64, false>(g, batch, st);
  }
}
