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
// splitting K further).  Activation scales are staged in LDS block-major.  Weight nibbles are baked
// in MFMA lane order so every lane's 8-byte load is one coalesced 512-byte
// wave access per block; nibbles become int8 levels with two v_perm_b32 table
// lookups per 4 values.
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
__device__ __forceinline__ uint32_t lut16(uint32_t idx, uint32_t t0, uint32_t t1, uint32_t t2, uint32_t t3) {
  const uint32_t sel = idx & 0x07070707u;
  const uint32_t lo = __builtin_amdgcn_perm(t1, t0, sel);
  const uint32_t hi = __builtin_amdgcn_perm(t3, t2, sel);
  const uint32_t mask = ((idx >> 3) & 0x01010101u) * 0xffu;
  return (hi & mask) | (lo & ~mask);
}

template <int WAVES>
__global__ void __launch_bounds__(WAVES * 64)
k_gemv_nf4(const int8_t* __restrict__ xl, const float* __restrict__ xs, int M, const uint8_t* __restrict__ wp,
           const uint8_t* __restrict__ ws, vh_format sfmt, uint4 lv, int64_t N, int64_t K, vh_epilogue epi,
           void* __restrict__ y) {
  __shared__ float s_wscale[256];
  __shared__ __attribute__((aligned(16))) float s_xs[MAX_BLOCKS][16];  // activation scales, block-major
  __shared__ float s_red[WAVES][4][64];
  // blocks per round: 16 waves fit 128 VGPRs (and see short K ranges)
  constexpr int UNROLL = WAVES == 16 ? 4 : 8;
  const int tid = threadIdx.x;
  const int64_t nb = K / 64;
  const int lane = tid & 63, wave = tid >> 6;
  const int64_t tile = blockIdx.x;
  const int64_t b0 = wave * nb / WAVES, b1 = (wave + 1) * nb / WAVES;
  const int64_t n = tile * 16 + (lane & 15);
  const int ma = lane & 15;         // activation row this lane feeds to the MFMA
  const int mrow = (lane >> 4) * 4; // output rows this lane accumulates
  const bool a_live = ma < M;
  const int64_t kl = (lane >> 4) * 16;

  const uint8_t* wtile = wp + (tile * nb) * 512 + lane * 8;
  const uint8_t* wsrow = ws + n * nb;
  const int8_t* xrow = xl + (int64_t)(a_live ? ma : 0) * K + kl;

  // One round: UNROLL blocks' weights, activations and weight-scale codes.
  // Every round is loaded one round ahead; the first before the tables are
  // staged, so the memory latency overlaps the set-up.
  uint2 w[UNROLL];
  uint4 x[UNROLL];
  uint32_t sb[UNROLL];
  auto load = [&](int64_t b, uint2* wv, uint4* xv, uint32_t* sv) {
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const int64_t bb = b + u;
      const bool ok = bb < b1;
      wv[u] = ok ? *(const uint2*)(wtile + bb * 512) : make_uint2(0, 0);
      xv[u] = (ok && a_live) ? *(const uint4*)(xrow + bb * 64) : make_uint4(0, 0, 0, 0);
      sv[u] = ok ? wsrow[bb] : 0u;
    }
  };
  load(b0, w, x, sb);

  for (int i = tid; i < 256; i += WAVES * 64) s_wscale[i] = fmt_decode(i, sfmt, nullptr);
  for (int i = tid; i < nb * 16; i += WAVES * 64) {
    const int bq = i / 16, m = i % 16;
    s_xs[bq][m] = m < M ? xs[(int64_t)m * nb + bq] : 0.0f;
  }
  __syncthreads();

  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int64_t b = b0; b < b1; b += UNROLL) {
    uint2 nw[UNROLL];
    uint4 nx[UNROLL];
    uint32_t nsb[UNROLL];
    if (b + UNROLL < b1) load(b + UNROLL, nw, nx, nsb);
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const int64_t bb = b + u;
      if (bb >= b1) break;
      i32x4 wl;
      wl[0] = (int)lut16(w[u].x & 0x0f0f0f0fu, lv.x, lv.y, lv.z, lv.w);
      wl[1] = (int)lut16(w[u].y & 0x0f0f0f0fu, lv.x, lv.y, lv.z, lv.w);
      wl[2] = (int)lut16((w[u].x >> 4) & 0x0f0f0f0fu, lv.x, lv.y, lv.z, lv.w);
      wl[3] = (int)lut16((w[u].y >> 4) & 0x0f0f0f0fu, lv.x, lv.y, lv.z, lv.w);
      i32x4 xa = {(int)x[u].x, (int)x[u].y, (int)x[u].z, (int)x[u].w};
      i32x4 d = {0, 0, 0, 0};
      d = __builtin_amdgcn_mfma_i32_16x16x64_i8(xa, wl, d, 0, 0, 0);
      const float swv = s_wscale[sb[u] & 0xffu];
      const float4 sx = *(const float4*)&s_xs[bb][mrow];
      acc[0] = fmaf((float)d[0], sx.x * swv, acc[0]);
      acc[1] = fmaf((float)d[1], sx.y * swv, acc[1]);
      acc[2] = fmaf((float)d[2], sx.z * swv, acc[2]);
      acc[3] = fmaf((float)d[3], sx.w * swv, acc[3]);
    }
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      w[u] = nw[u];
      x[u] = nx[u];
      sb[u] = nsb[u];
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
