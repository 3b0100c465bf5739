// MXNF4 decode-shape linear (M <= 16): the weight stream is the roofline.
//
// The reference decodes both operands to bf16 (codebook level x block scale,
// ops/quantized.py:574-591) and runs an fp32 GEMM (ops/quantized.py:651-723).
// Here the weights stay 4-bit: each 64-element block is one
// v_mfma_i32_16x16x64_i8 of int6 levels (exact integer dot products), and the
// two block scales are applied once per block in fp32.  This differs from
// the reference only by its bf16 rounding of each decoded operand (at most
// 2**-9 relative per element), well inside the 1e-2 GEMM tolerance.
//
// Layout: one workgroup per 16 output columns; its WAVES waves split K into
// contiguous ranges, keep 4 or 8 blocks of loads in flight each, and reduce
// through LDS.  WAVES = 4 when there are at least 512 column tiles (long
// per-wave streams, 8+ waves per CU), 16 otherwise (fill the CUs by
// splitting K further).  The tile's activation and weight scales are staged
// in LDS once (decoded to fp32, block-major), so the block loop issues only
// the weight and activation loads.  Weight nibbles are baked in MFMA lane
// order so every lane's 8-byte load is one coalesced 512-byte wave access per
// block; nibbles become int8 levels with three v_perm_b32 per 4 values.
#include <hip/hip_runtime.h>

#include <cstring>

#include "vh_device.h"
#include "vh_host.h"

namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));

constexpr int MAX_BLOCKS = 256;  // K <= 16384 (activation scales staged in LDS)

// Bake: one thread per (tile, block, lane) -> 8 bytes.
__global__ void __launch_bounds__(256) k_pack_nf4(const uint8_t* __restrict__ codes, int64_t N, int64_t K,
                                                  uint8_t* __restrict__ out) {
  const int64_t nb = K / 64;
  const int64_t total = (N / 16) * nb * 64;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= total) return;
  const int lane = (int)(t % 64);
  const int64_t blk = (t / 64) % nb;
  const int64_t tile = t / (64 * nb);
  const int64_t n = tile * 16 + lane % 16;
  const int64_t k0 = blk * 64 + (lane / 16) * 16;
  const uint8_t* src = codes + n * K + k0;
  uint32_t lo = 0, hi = 0;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint32_t byte = (uint32_t)(src[j] & 0xf) | ((uint32_t)(src[j + 8] & 0xf) << 4);
    if (j < 4) lo |= byte << (8 * j);
    else hi |= byte << (8 * (j - 4));
  }
  *(uint2*)(out + t * 8) = make_uint2(lo, hi);
}

// Four byte indices (0..15) -> four int8 levels from a 16-entry table held in
// four dwords (t0 = levels 0..3, ... t3 = levels 12..15).
// The third v_perm picks, per byte i, byte i of the low-half lookup (selector
// i) or of the high-half one (i + 4) by bit 3 of the index: six full-rate
// ops, no per-byte multiply.
__device__ __forceinline__ uint32_t lut16(uint32_t idx, uint32_t t0, uint32_t t1, uint32_t t2, uint32_t t3) {
  const uint32_t sel = idx & 0x07070707u;
  const uint32_t lo = __builtin_amdgcn_perm(t1, t0, sel);
  const uint32_t hi = __builtin_amdgcn_perm(t3, t2, sel);
  const uint32_t pick = ((idx >> 1) & 0x04040404u) | 0x03020100u;
  return __builtin_amdgcn_perm(hi, lo, pick);
}

template <int WAVES>
__global__ void __launch_bounds__(WAVES * 64)
k_gemv_nf4(const int8_t* __restrict__ xl, const float* __restrict__ xs, int M, const uint8_t* __restrict__ wp,
           const uint8_t* __restrict__ ws, vh_format sfmt, uint4 lv, int64_t N, int64_t K, vh_epilogue epi,
           void* __restrict__ y) {
  // activation and weight scales of this tile, block-major: a lane reads
  // its row's / column's scale of block b at [b][.], no bank conflicts
  __shared__ __attribute__((aligned(16))) float s_xs[MAX_BLOCKS][16];
  __shared__ float s_ws[MAX_BLOCKS][16];
  __shared__ float s_red[WAVES][4][64];
  // blocks per round: 16 waves fit 128 VGPRs (and see short K ranges)
  constexpr int UNROLL = WAVES == 16 ? 4 : 8;
  const int tid = threadIdx.x;
  const int nb = (int)(K / 64);
  // wave-uniform block range, kept in scalar registers
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t tile = blockIdx.x;
  const int b0 = wave * nb / WAVES, b1 = (wave + 1) * nb / WAVES;
  const int64_t n = tile * 16 + (lane & 15);
  const int ma = lane & 15;         // activation row this lane feeds to the MFMA
  const int mrow = (lane >> 4) * 4; // output rows this lane accumulates
  const bool a_live = ma < M;

  // Buffer loads: a lane whose row is past M, or a block past this wave's
  // range, reads out of range and gets zeros without a memory access, so
  // it adds nothing to the dot products.  Each wave access is then one
  // 512-byte weight run and at most 64 bytes per live activation row.
  constexpr uint32_t OOB = 0x80000000u;
  const __amdgpu_buffer_rsrc_t wr =
      __builtin_amdgcn_make_buffer_rsrc((void*)(wp + tile * nb * 512), (short)0, nb * 512, 0x00020000);
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc((void*)xl, (short)0, M * (int)K, 0x00020000);
  const uint32_t woff = (uint32_t)lane * 8u;
  const uint32_t xoff = a_live ? (uint32_t)(ma * K + (lane >> 4) * 16) : OOB;
  auto load = [&](int b, vh_u32x2* wv, vh_u32x4* xv) {
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const bool ok = b + u < b1;
      wv[u] = __builtin_amdgcn_raw_buffer_load_b64(wr, ok ? woff + (uint32_t)(b + u) * 512u : OOB, 0, 0);
      xv[u] = __builtin_amdgcn_raw_buffer_load_b128(xr, ok ? xoff + (uint32_t)(b + u) * 64u : OOB, 0, 0);
    }
  };
  // Rounds alternate between two register sets.  With 16 waves (4-block
  // rounds) two rounds are always in flight, the first two loaded before the
  // scales are staged; with 4 waves the second set is loaded once the first
  // is being consumed (two 8-block rounds in flight would not fit 128 VGPRs).
  constexpr bool DEEP = WAVES == 16;
  vh_u32x2 w0[UNROLL], w1[UNROLL];
  vh_u32x4 x0[UNROLL], x1[UNROLL];
  if (b0 < b1) load(b0, w0, x0);
  if (DEEP && b0 + UNROLL < b1) load(b0 + UNROLL, w1, x1);

  const uint8_t* wst = ws + tile * 16 * nb;  // the tile's 16 scale rows are contiguous
  for (int i = tid; i < 16 * nb; i += WAVES * 64) s_ws[i % nb][i / nb] = fmt_decode(wst[i], sfmt, nullptr);
  for (int i = tid; i < nb * 16; i += WAVES * 64) {
    const int bq = i / 16, m = i % 16;
    s_xs[bq][m] = m < M ? xs[(int64_t)m * nb + bq] : 0.0f;
  }
  __syncthreads();

  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  const int blast = b1 > b0 ? b1 - 1 : b0;
  auto round = [&](int b, const vh_u32x2* w, const vh_u32x4* x) {
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const int bb = b + u < b1 ? b + u : blast;  // past the range: zero activations, any finite scale
      i32x4 wl;
      wl[0] = (int)lut16(w[u].x & 0x0f0f0f0fu, lv.x, lv.y, lv.z, lv.w);
      wl[1] = (int)lut16(w[u].y & 0x0f0f0f0fu, lv.x, lv.y, lv.z, lv.w);
      wl[2] = (int)lut16((w[u].x >> 4) & 0x0f0f0f0fu, lv.x, lv.y, lv.z, lv.w);
      wl[3] = (int)lut16((w[u].y >> 4) & 0x0f0f0f0fu, lv.x, lv.y, lv.z, lv.w);
      i32x4 xa = {(int)x[u].x, (int)x[u].y, (int)x[u].z, (int)x[u].w};
      i32x4 d = {0, 0, 0, 0};
      d = __builtin_amdgcn_mfma_i32_16x16x64_i8(xa, wl, d, 0, 0, 0);
      const float swv = s_ws[bb][lane & 15];
      const float4 sx = *(const float4*)&s_xs[bb][mrow];
      acc[0] = fmaf((float)d[0], sx.x * swv, acc[0]);
      acc[1] = fmaf((float)d[1], sx.y * swv, acc[1]);
      acc[2] = fmaf((float)d[2], sx.z * swv, acc[2]);
      acc[3] = fmaf((float)d[3], sx.w * swv, acc[3]);
    }
  };
  if constexpr (DEEP) {
    for (int b = b0; b < b1; b += 2 * UNROLL) {
      round(b, w0, x0);
      if (b + 2 * UNROLL < b1) load(b + 2 * UNROLL, w0, x0);
      if (b + UNROLL >= b1) break;
      round(b + UNROLL, w1, x1);
      if (b + 3 * UNROLL < b1) load(b + 3 * UNROLL, w1, x1);
    }
  } else {
    for (int b = b0; b < b1; b += 2 * UNROLL) {
      if (b + UNROLL < b1) load(b + UNROLL, w1, x1);
      round(b, w0, x0);
      if (b + UNROLL >= b1) break;
      if (b + 2 * UNROLL < b1) load(b + 2 * UNROLL, w0, x0);
      round(b + UNROLL, w1, x1);
    }
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) s_red[wave][r][lane] = acc[r];
  __syncthreads();
  if (wave != 0) return;
  float alpha = 1.0f;
  if (epi.scale) alpha = epi.scale_dtype == VH_BF16 ? bf2f(*(const uint16_t*)epi.scale) : *(const float*)epi.scale;
  float bias = 0.0f;
  if (epi.bias) bias = epi.bias_dtype == VH_BF16 ? bf2f(((const uint16_t*)epi.bias)[n]) : ((const float*)epi.bias)[n];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int m = mrow + r;
    if (m >= M) continue;
    float v = 0.0f;
#pragma unroll
    for (int wv = 0; wv < WAVES; ++wv) v += s_red[wv][r][lane];
    if (epi.scale) v *= alpha;
    if (epi.bias) v += bias;
    if (epi.out_dtype == VH_BF16) ((uint16_t*)y)[m * N + n] = (uint16_t)f2bf(v);
    else ((float*)y)[m * N + n] = v;
  }
}

}  // namespace

extern "C" int vh_pack_nf4(const uint8_t* codes, int64_t N, int64_t K, uint8_t* out, vh_stream_t stream) {
  VH_REQUIRE(codes && out, "vh_pack_nf4: null pointer");
  VH_REQUIRE(N > 0 && K > 0 && N % 16 == 0 && K % 64 == 0, "vh_pack_nf4: needs N %% 16 == 0 and K %% 64 == 0");
  const int64_t total = (N / 16) * (K / 64) * 64;
  const int64_t blocks = (total + 255) / 256;
  hipLaunchKernelGGL(k_pack_nf4, dim3((unsigned)blocks), dim3(256), 0, vh::as_stream(stream), codes, N, K, out);
  return vh::check_launch("vh_pack_nf4");
}

extern "C" int vh_gemv_nf4(const int8_t* x_levels, const float* x_scale, int64_t M, const uint8_t* w_packed,
                           const uint8_t* w_scale, const vh_format* w_scale_fmt, const int8_t* levels16, int64_t N,
                           int64_t K, const vh_epilogue* epi, void* y, vh_stream_t stream) {
  VH_REQUIRE(x_levels && x_scale && w_packed && w_scale && w_scale_fmt && levels16 && epi && y,
             "vh_gemv_nf4: null argument");
  VH_REQUIRE(M >= 1 && M <= 16, "vh_gemv_nf4: M must be in [1, 16] (got %lld)", (long long)M);
  VH_REQUIRE(N > 0 && K > 0 && N % 16 == 0 && K % 64 == 0, "vh_gemv_nf4: needs N %% 16 == 0 and K %% 64 == 0");
  VH_REQUIRE(K / 64 <= MAX_BLOCKS, "vh_gemv_nf4: K must be <= %d", MAX_BLOCKS * 64);
  VH_REQUIRE(((uintptr_t)x_levels % 16 == 0) && ((uintptr_t)w_packed % 8 == 0), "vh_gemv_nf4: misaligned operand");
  VH_REQUIRE(epi->mode == EPI_PLAIN && (epi->out_dtype == VH_BF16 || epi->out_dtype == VH_F32),
             "vh_gemv_nf4: unsupported epilogue");
  VH_REQUIRE(w_scale_fmt->kind != VH_FMT_LUT && w_scale_fmt->kind != VH_FMT_IDENTITY &&
                 w_scale_fmt->kind != VH_FMT_STEPS,
             "vh_gemv_nf4: the weight scale map needs a closed form with packed codes");
  uint32_t t[4];
  memcpy(t, levels16, 16);
  const uint4 lv = make_uint4(t[0], t[1], t[2], t[3]);
  if (N / 16 >= 512)
    hipLaunchKernelGGL(k_gemv_nf4<4>, dim3((unsigned)(N / 16)), dim3(4 * 64), 0, vh::as_stream(stream), x_levels,
                       x_scale, (int)M, w_packed, w_scale, *w_scale_fmt, lv, N, K, *epi, y);
  else
    hipLaunchKernelGGL(k_gemv_nf4<16>, dim3((unsigned)(N / 16)), dim3(16 * 64), 0, vh::as_stream(stream), x_levels,
                       x_scale, (int)M, w_packed, w_scale, *w_scale_fmt, lv, N, K, *epi, y);
  return vh::check_launch("vh_gemv_nf4");
}
