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
// Layout: a workgroup of 8 waves covers T 16-column tiles; the tile's K
// blocks are split into 8 / T contiguous ranges, one per wave, so the T
// waves of a range read the same activation bytes at the same time (they
// hit in L1: the activations are re-read once per T tiles, not per tile).
// Every load is issued per block straight from the baked layouts -- weight
// nibbles in MFMA lane order (one coalesced 512-byte wave access per block),
// the tile's 16 scale bytes of a block contiguous, the activations' scales
// block-major [K/64][16] -- two rounds of UNROLL blocks in flight, with no
// staging prologue; nibbles become int8 levels with three v_perm_b32 per 4
// values.  The K ranges meet through LDS at the end.
#include <hip/hip_runtime.h>

#include <cstring>
#include <type_traits>

#include "vh_device.h"
#include "vh_host.h"

namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));

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

// SK: the weight scale map's kind (fmt_decode_k), fixed at compile time so
// the block loop stays free of branches (a runtime switch there makes the
// compiler drain every outstanding load at each merge).
// NBW: blocks per chunk of a wave's K range (padded with empty blocks); a
// chunk's two rounds are unrolled into straight-line code, where the
// compiler's count of outstanding loads is exact (around a loop, or over
// more rounds, it drains them all or spills).
template <int T, int SK, int NBW, int WAVES>
__global__ void __launch_bounds__(WAVES * 64)
k_gemv_nf4(const int8_t* __restrict__ xl, const float* __restrict__ xs, int M, const uint8_t* __restrict__ wp,
           const uint8_t* __restrict__ ws, vh_format sfmt, uint4 lv, int64_t N, int64_t K, vh_epilogue epi,
           void* __restrict__ y) {
  constexpr int KR = WAVES / T;  // K ranges per tile
  constexpr int UNROLL = NBW < 8 ? NBW : 8;  // blocks per round; two rounds in flight (256 VGPRs)
  constexpr int ROUNDS = NBW / UNROLL;
  __shared__ float s_red[WAVES][4][64];
  const int tid = threadIdx.x;
  const int nb = (int)(K / 64);
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tl = wave % T, kr = wave / T;
  const int64_t tile = (int64_t)blockIdx.x * T + tl;
  const int b0 = kr * nb / KR, b1 = (kr + 1) * nb / KR;
  const int64_t n = tile * 16 + (lane & 15);
  const int ma = lane & 15;          // activation row this lane feeds to the MFMA
  const int mrow = (lane >> 4) * 4;  // output rows this lane accumulates

  // Buffer loads: a lane whose row is past M, or a block past this wave's
  // range, reads out of range and gets zeros without a memory access.
  constexpr uint32_t OOB = 0x80000000u;
  const __amdgpu_buffer_rsrc_t wr =
      __builtin_amdgcn_make_buffer_rsrc((void*)(wp + tile * nb * 512), (short)0, nb * 512, 0x00020000);
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc((void*)xl, (short)0, M * (int)K, 0x00020000);
  const __amdgpu_buffer_rsrc_t wsr =
      __builtin_amdgcn_make_buffer_rsrc((void*)(ws + tile * nb * 16), (short)0, nb * 16, 0x00020000);
  const __amdgpu_buffer_rsrc_t xsr = __builtin_amdgcn_make_buffer_rsrc((void*)xs, (short)0, nb * 64, 0x00020000);
  const uint32_t woff = (uint32_t)lane * 8u;
  const uint32_t xoff = ma < M ? (uint32_t)(ma * K + (lane >> 4) * 16) : OOB;
  const uint32_t wsoff = (uint32_t)(lane & 15), xsoff = (uint32_t)mrow * 4u;
  struct Set {
    vh_u32x2 w[UNROLL];
    vh_u32x4 x[UNROLL];
    vh_u32x4 sx[UNROLL];
    uint32_t sw[UNROLL];
  };
  auto load = [&](int b, Set& st) {
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const bool ok = b + u < b1;
      const uint32_t bb = (uint32_t)(b + u);
      st.w[u] = __builtin_amdgcn_raw_buffer_load_b64(wr, ok ? woff + bb * 512u : OOB, 0, 0);
      st.x[u] = __builtin_amdgcn_raw_buffer_load_b128(xr, ok ? xoff + bb * 64u : OOB, 0, 0);
      st.sw[u] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(wsr, ok ? wsoff + bb * 16u : OOB, 0, 0);
      st.sx[u] = __builtin_amdgcn_raw_buffer_load_b128(xsr, ok ? xsoff + bb * 64u : OOB, 0, 0);
    }
  };
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  auto round = [&](const Set& st) {
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      i32x4 wl;
      wl[0] = (int)lut16(st.w[u].x & 0x0f0f0f0fu, lv.x, lv.y, lv.z, lv.w);
      wl[1] = (int)lut16(st.w[u].y & 0x0f0f0f0fu, lv.x, lv.y, lv.z, lv.w);
      wl[2] = (int)lut16((st.w[u].x >> 4) & 0x0f0f0f0fu, lv.x, lv.y, lv.z, lv.w);
      wl[3] = (int)lut16((st.w[u].y >> 4) & 0x0f0f0f0fu, lv.x, lv.y, lv.z, lv.w);
      const i32x4 xa = {(int)st.x[u].x, (int)st.x[u].y, (int)st.x[u].z, (int)st.x[u].w};
      i32x4 d = {0, 0, 0, 0};
      d = __builtin_amdgcn_mfma_i32_16x16x64_i8(xa, wl, d, 0, 0, 0);
      // past the range: zero dot products (zero activations); the decoded
      // scale of a zero byte is finite
      const float swv = fmt_decode_k<SK>(st.sw[u], sfmt, nullptr);
      acc[0] = fmaf((float)d[0], __uint_as_float(st.sx[u].x) * swv, acc[0]);
      acc[1] = fmaf((float)d[1], __uint_as_float(st.sx[u].y) * swv, acc[1]);
      acc[2] = fmaf((float)d[2], __uint_as_float(st.sx[u].z) * swv, acc[2]);
      acc[3] = fmaf((float)d[3], __uint_as_float(st.sx[u].w) * swv, acc[3]);
    }
  };
  // blocks past the range load zeros without a memory access; a range
  // longer than NBW blocks runs in chunks of NBW
  for (int c0 = b0; c0 < b1; c0 += NBW) {
    Set s[2];
    load(c0, s[0]);
#pragma unroll
    for (int r = 0; r < ROUNDS; ++r) {
      if (r + 1 < ROUNDS) load(c0 + (r + 1) * UNROLL, s[(r + 1) & 1]);
      round(s[r & 1]);
      // keep later rounds' loads in place (two register sets, not ROUNDS):
      // no memory access moves across this point
      asm volatile("" ::: "memory");
    }
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) s_red[wave][r][lane] = acc[r];
  __syncthreads();
  if (kr != 0) return;
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
    for (int q = 0; q < KR; ++q) v += s_red[q * T + tl][r][lane];
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
  VH_REQUIRE(K / 64 <= 8 * 32, "vh_gemv_nf4: K must be <= %d", 8 * 32 * 64);
  VH_REQUIRE(((uintptr_t)x_levels % 16 == 0) && ((uintptr_t)w_packed % 8 == 0), "vh_gemv_nf4: misaligned operand");
  VH_REQUIRE(epi->mode == EPI_PLAIN && (epi->out_dtype == VH_BF16 || epi->out_dtype == VH_F32),
             "vh_gemv_nf4: unsupported epilogue");
  VH_REQUIRE(w_scale_fmt->kind != VH_FMT_LUT && w_scale_fmt->kind != VH_FMT_IDENTITY &&
                 w_scale_fmt->kind != VH_FMT_STEPS,
             "vh_gemv_nf4: the weight scale map needs a closed form with packed codes");
  uint32_t t[4];
  memcpy(t, levels16, 16);
  const uint4 lv = make_uint4(t[0], t[1], t[2], t[3]);
  // tiles per workgroup: one while that leaves the grid under 512
  // workgroups, else 4 (activations re-read once per 4 tiles; 8 waves: two
  // K ranges per tile)
  const int64_t tiles = N / 16;
  hipStream_t st = vh::as_stream(stream);
  const bool four = tiles >= 512 && tiles % 4 == 0 && K / 64 <= 2 * 16;
  // blocks per wave: the tile's K blocks over its K ranges, rounded up to 4,
  // 8 or 16 (longer ranges in chunks of 16)
  const int64_t nb = K / 64;
  const int64_t kr = four ? 2 : 8, bpw = (nb + kr - 1) / kr;
  auto go = [&](auto sk) {
    constexpr int SK = decltype(sk)::value;
    auto launch = [&](auto nbw) {
      constexpr int NBW = decltype(nbw)::value;
      if (four)
        hipLaunchKernelGGL((k_gemv_nf4<4, SK, NBW, 8>), dim3((unsigned)(tiles / 4)), dim3(512), 0, st, x_levels,
                           x_scale, (int)M, w_packed, w_scale, *w_scale_fmt, lv, N, K, *epi, y);
      else
        hipLaunchKernelGGL((k_gemv_nf4<1, SK, NBW, 8>), dim3((unsigned)tiles), dim3(512), 0, st, x_levels, x_scale,
                           (int)M, w_packed, w_scale, *w_scale_fmt, lv, N, K, *epi, y);
    };
    if (bpw <= 4) launch(std::integral_constant<int, 4>{});
    else if (bpw <= 8) launch(std::integral_constant<int, 8>{});
    else launch(std::integral_constant<int, 16>{});
  };
  const vh_format& f = *w_scale_fmt;
  if (f.kind == VH_FMT_INT) go(std::integral_constant<int, K_INT>{});
  else if (f.kind == VH_FMT_MINIFLOAT && (f.flags & VH_FMT_HW_E4M3)) go(std::integral_constant<int, K_E4M3>{});
  else if (f.kind == VH_FMT_MINIFLOAT) go(std::integral_constant<int, K_MINI>{});
  else go(std::integral_constant<int, K_POSIT>{});
  return vh::check_launch("vh_gemv_nf4");
}
