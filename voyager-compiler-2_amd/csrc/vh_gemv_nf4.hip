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
// Layout: a workgroup of 8 waves covers T 16-column tiles (TPW per wave);
// the tile's K blocks are split into 8 / T contiguous ranges, one per wave,
// so the T waves of a range read the same activation bytes at the same time
// (they hit in L1: the activations are re-read once per T tiles, not per
// tile), and a wave with two tiles loads the activation once for both.
// Every load is issued per block straight from the baked layouts -- weight
// nibbles in MFMA lane order (one coalesced 512-byte wave access per block),
// the tile's 16 scale bytes of a block contiguous, the activations' scales
// block-major [K/64][16] (at M > 1 one 16-byte load per lane per round,
// staged through LDS) -- two rounds of UNROLL blocks in flight, with no
// staging prologue; nibbles become int8 levels with three v_perm_b32 per 4
// values, and a weight scale byte becomes its value through a 256-entry
// table in LDS, decoded once per workgroup.  The K ranges meet through LDS
// at the end.
#include <hip/hip_runtime.h>

#include <cstring>
#include <type_traits>

#include "vh_blockscale.h"
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

// A weight scale byte's value, for the kinds the launcher accepts (the ones
// with a closed form: integer, minifloat, posit).
__device__ float scale_value(uint32_t c, const vh_format& f) {
  if (f.kind == VH_FMT_INT) return fmt_decode_k<K_INT>(c, f, nullptr);
  if (f.kind == VH_FMT_MINIFLOAT)
    return (f.flags & VH_FMT_HW_E4M3) ? fmt_decode_k<K_E4M3>(c, f, nullptr) : fmt_decode_k<K_MINI>(c, f, nullptr);
  return fmt_decode_k<K_POSIT>(c, f, nullptr);
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* p, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)(bytes > 0 ? bytes : 0), 0x00020000);
}

// The tile's K-range partial sums (added in range order), alpha, bias and
// the output rounding; run by the waves of range 0.
template <int T, int MR, int WAVES>
__device__ __forceinline__ void finish(float (*s_red)[MR][64], int tl, int lane, int mrow, int M, int64_t n,
                                       int64_t N, const vh_epilogue& epi, void* y) {
  constexpr int KR = WAVES / T;
  float alpha = 1.0f;
  if (epi.scale) alpha = epi.scale_dtype == VH_BF16 ? bf2f(*(const uint16_t*)epi.scale) : *(const float*)epi.scale;
  float bias = 0.0f;
  if (epi.bias) bias = epi.bias_dtype == VH_BF16 ? bf2f(((const uint16_t*)epi.bias)[n]) : ((const float*)epi.bias)[n];
#pragma unroll
  for (int r = 0; r < MR; ++r) {
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

// MR: output rows a lane accumulates -- 4 (rows 4*(lane/16) .. +3 of the
// MFMA's 16x16 result) or 1 when M == 1 (only row 0 is stored, so one
// scale product and one accumulation per block).
// NBW: blocks per chunk of a wave's K range; a chunk's rounds are unrolled
// into straight-line code, where the compiler's count of outstanding loads
// is exact (around a loop, or over more than two register sets, it drains
// them all or spills).
template <int T, int MR, int NBW, int WAVES, int TPW>
__global__ void __launch_bounds__(WAVES * 64)
k_gemv_nf4(const int8_t* __restrict__ xl, const float* __restrict__ xs, int M, const uint8_t* __restrict__ wp,
           const uint8_t* __restrict__ ws, vh_format sfmt, uint4 lv, int64_t N, int64_t K, vh_epilogue epi,
           void* __restrict__ y) {
  static_assert(MR == 1 || MR == 4, "rows per lane");
  static_assert(TPW == 1 || TPW == 2, "tiles per wave");
  constexpr int KR = WAVES / T;  // K ranges per tile
  constexpr int UNROLL = NBW < 8 ? NBW : 8;  // blocks per round; two rounds in flight
  constexpr int ROUNDS = NBW / UNROLL;
  __shared__ float s_red[TPW][WAVES][MR][64];
  __shared__ float s_scale[256];  // the weight scale map, decoded once per workgroup
  // M > 1: a round's activation scales, one 16-byte load per lane, read
  // back per block (rows 4 (lane / 16) .. + 3)
  __shared__ __attribute__((aligned(16))) uint8_t s_sx[MR == 4 ? WAVES : 1][MR == 4 ? 64 * 16 : 16];
  const int tid = threadIdx.x;
  const int nb = (int)(K / 64);
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tl = wave % T, kr = wave / T;
  const int64_t tile0 = ((int64_t)blockIdx.x * T + tl) * TPW;  // this wave's first tile
  const int b0 = kr * nb / KR, b1 = (kr + 1) * nb / KR;
  const int ma = lane & 15;          // activation row this lane feeds to the MFMA
  const int mrow = (lane >> 4) * 4;  // output rows this lane accumulates
  uint32_t base;
  asm volatile("v_mov_b32 %0, 0x3020100" : "=v"(base));

  // Every buffer starts at the round's first block and ends at the wave's
  // range end (the activations: at the end of X), so the per-block offsets
  // are instruction immediates and a block past the range, or a lane whose
  // row is past M, reads zeros without a memory access: its weights and
  // activation scale are zero, so it adds nothing.
  constexpr uint32_t OOB = 0x80000000u;
  const uint32_t woff = (uint32_t)lane * 8u;
  const uint32_t xoff = ma < M ? (uint32_t)(ma * K + (lane >> 4) * 16) : OOB;
  const uint32_t wsoff = (uint32_t)(lane & 15);
  const uint32_t xsoff = lane < UNROLL * 4 ? (uint32_t)lane * 16u : OOB;  // M > 1: the round's scales
  // With one row the activation scale is the same for the whole wave: it
  // is read through the scalar cache at the start of its round, and holds
  // no vector registers while the round's loads are in flight.
  struct Set {
    vh_u32x2 w[TPW][UNROLL];
    vh_u32x4 x[UNROLL];
    vh_u32x4 sx;
    uint32_t sw[TPW][UNROLL];
  };
  auto load = [&](int b, Set& st) __attribute__((always_inline)) {
    // opaque copies of the lane offsets: the per-block constants are then
    // added here, where they become instruction immediates, instead of
    // being hoisted out of the loop into a register each
    uint32_t wo = woff, xo = xoff, wso = wsoff, xso = xsoff;
    asm volatile("" : "+v"(wo), "+v"(xo), "+v"(wso), "+v"(xso));
    const int64_t rem = b1 - b;
    const __amdgpu_buffer_rsrc_t xr = rsrc(xl + (int64_t)b * 64, (int64_t)M * K - (int64_t)b * 64);
    if constexpr (MR == 4) st.sx = __builtin_amdgcn_raw_buffer_load_b128(rsrc(xs + (int64_t)b * 16, rem * 64), xso, 0, 0);
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      const __amdgpu_buffer_rsrc_t wr = rsrc(wp + ((tile0 + t) * nb + b) * 512, rem * 512);
      const __amdgpu_buffer_rsrc_t wsr = rsrc(ws + ((tile0 + t) * nb + b) * 16, rem * 16);
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) {
        st.w[t][u] = __builtin_amdgcn_raw_buffer_load_b64(wr, wo + u * 512u, 0, 0);
        st.sw[t][u] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(wsr, wso + u * 16u, 0, 0);
      }
    }
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) st.x[u] = __builtin_amdgcn_raw_buffer_load_b128(xr, xo + u * 64u, 0, 0);
  };
  float acc[TPW][MR];
#pragma unroll
  for (int t = 0; t < TPW; ++t)
#pragma unroll
    for (int r = 0; r < MR; ++r) acc[t][r] = 0.0f;
  // b: the round's first block
  auto round = [&](Set& st, int b) __attribute__((always_inline)) {
    float sx1[UNROLL];
    if constexpr (MR == 1) {
      typedef const __attribute__((address_space(4))) float cfloat;
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) {
        // row 0's scale of block b + u; zero past the range (block 0 is read
        // there, which always exists)
        sx1[u] = *(const cfloat*)(uintptr_t)(xs + (int64_t)(b + u < b1 ? b + u : 0) * 16);
      }
      // all of them arrive before the round's first LDS read (scalar loads
      // return out of order and share the LDS counter: interleaved, every
      // table read would wait for all outstanding scalar loads)
      static_assert(UNROLL == 4 || UNROLL == 8, "one statement holds the round's scales");
      if constexpr (UNROLL == 8)
        asm volatile("" : "+s"(sx1[0]), "+s"(sx1[1]), "+s"(sx1[2]), "+s"(sx1[3]), "+s"(sx1[4]), "+s"(sx1[5]),
                     "+s"(sx1[6]), "+s"(sx1[7]));
      else
        asm volatile("" : "+s"(sx1[0]), "+s"(sx1[1]), "+s"(sx1[2]), "+s"(sx1[3]));
#pragma unroll
      for (int u = 0; u < UNROLL; ++u)
        if (b + u >= b1) sx1[u] = 0.0f;
    } else {
      // the round's activation scales (zero past the range) into this
      // wave's LDS slot; read back by other lanes of the same wave (LDS
      // keeps a wave's accesses in order)
      asm volatile("" : "+v"(st.sx)::"memory");
      *(vh_u32x4*)&s_sx[wave][lane * 16] = st.sx;
    }
    // Three stages per block, software-pipelined over the round: (a) its
    // registers pass through an empty asm, after every load issued before
    // this round, so its arithmetic cannot rise above them (left alone, the
    // scheduler interleaves loads with arithmetic and a round waits on
    // several memory latencies in turn), and its LDS reads go out; (b) the
    // nibble lookup and the MFMA; (c) the scale products.  (a) runs one
    // block ahead of (b) and (c) one behind, so each block's LDS and MFMA
    // latencies pass while the neighbouring blocks compute; the
    // accumulation order is the block order.
    float swv[TPW][UNROLL];
    vh_u32x4 sxq[UNROLL];
    i32x4 dd[TPW][UNROLL];
    auto stage_a = [&](int u) __attribute__((always_inline)) {
      if constexpr (TPW == 1)
        asm volatile("" : "+v"(st.w[0][u]), "+v"(st.x[u]), "+v"(st.sw[0][u]));
      else
        asm volatile("" : "+v"(st.w[0][u]), "+v"(st.w[1][u]), "+v"(st.x[u]), "+v"(st.sw[0][u]),
                     "+v"(st.sw[1][u]));
      if constexpr (MR == 4) sxq[u] = *(const vh_u32x4*)&s_sx[wave][u * 64 + mrow * 4];
#pragma unroll
      for (int t = 0; t < TPW; ++t) swv[t][u] = s_scale[st.sw[t][u]];
    };
    auto stage_b = [&](int u) __attribute__((always_inline)) {
      const i32x4 xa = {(int)st.x[u].x, (int)st.x[u].y, (int)st.x[u].z, (int)st.x[u].w};
#pragma unroll
      for (int t = 0; t < TPW; ++t) {
        i32x4 wl;
        wl[0] = (int)lut_lo(st.w[t][u].x, base, lv);
        wl[1] = (int)lut_lo(st.w[t][u].y, base, lv);
        wl[2] = (int)lut_hi(st.w[t][u].x, base, lv);
        wl[3] = (int)lut_hi(st.w[t][u].y, base, lv);
        const i32x4 z = {0, 0, 0, 0};
        dd[t][u] = __builtin_amdgcn_mfma_i32_16x16x64_i8(xa, wl, z, 0, 0, 0);
      }
    };
    auto stage_c = [&](int u) __attribute__((always_inline)) {
      // past the range: zero dot products and a zero activation scale; the
      // decoded scale of a zero byte is finite
#pragma unroll
      for (int t = 0; t < TPW; ++t) {
        const i32x4 d = dd[t][u];
        if constexpr (MR == 1) {
          acc[t][0] = fmaf((float)d[0], sx1[u] * swv[t][u], acc[t][0]);
        } else {
          acc[t][0] = fmaf((float)d[0], __uint_as_float(sxq[u].x) * swv[t][u], acc[t][0]);
          acc[t][1] = fmaf((float)d[1], __uint_as_float(sxq[u].y) * swv[t][u], acc[t][1]);
          acc[t][2] = fmaf((float)d[2], __uint_as_float(sxq[u].z) * swv[t][u], acc[t][2]);
          acc[t][3] = fmaf((float)d[3], __uint_as_float(sxq[u].w) * swv[t][u], acc[t][3]);
        }
      }
    };
    stage_a(0);
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      if (u + 1 < UNROLL) stage_a(u + 1);
      stage_b(u);
      if (u > 0) stage_c(u - 1);
    }
    stage_c(UNROLL - 1);
  };
  Set s[2];
  // Two register sets, double-buffered: round r + 2 is loaded into the set
  // round r has just finished with, so a wave always has one round in
  // flight while it computes another.  PRE: the chunk's first two rounds
  // were loaded before it starts.
  auto chunk = [&](int c0, auto pre) __attribute__((always_inline)) {
    if constexpr (!decltype(pre)::value) {
      load(c0, s[0]);
      if constexpr (ROUNDS > 1) load(c0 + UNROLL, s[1]);
    }
#pragma unroll
    for (int r = 0; r < ROUNDS; ++r) {
      round(s[r & 1], c0 + r * UNROLL);
      if (r + 2 < ROUNDS) load(c0 + (r + 2) * UNROLL, s[r & 1]);
      // keep the loads in place: no memory access moves across this point
      asm volatile("" ::: "memory");
    }
  };
  // The first chunk's loads go out before the scale table is built (an
  // empty range loads nothing: every access is past its buffer's end), and
  // the barrier waits for LDS only, so they stay in flight across it.
  load(b0, s[0]);
  if constexpr (ROUNDS > 1) load(b0 + UNROLL, s[1]);
  if (tid < 256) s_scale[tid] = scale_value((uint32_t)tid, sfmt);
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  // a range longer than NBW blocks runs in chunks of NBW
  if (b0 < b1) chunk(b0, std::true_type{});
  for (int c0 = b0 + NBW; c0 < b1; c0 += NBW) chunk(c0, std::false_type{});
#pragma unroll
  for (int t = 0; t < TPW; ++t)
#pragma unroll
    for (int r = 0; r < MR; ++r) s_red[t][wave][r][lane] = acc[t][r];
  __syncthreads();
  if (kr != 0) return;
#pragma unroll
  for (int t = 0; t < TPW; ++t)
    finish<T, MR, WAVES>(s_red[t], tl, lane, mrow, M, (tile0 + t) * 16 + (lane & 15), N, epi, y);
}

// M == 1 with the activation row quantized here: quantize_mx(x, index, [-1],
// 64, quant_max, scale map) (ops/quantized.py:1070-1115) of the blocks this
// wave multiplies, by the arithmetic of the quantize kernels' restatement
// for this case (k_mx_steps_rows8: div_bf16, fmt_value_k and the same
// threshold search, the lane's searches stepping together, with no
// per-element branch), so its levels and scales are those of the two-launch
// path bit for bit.  A round's UNROLL blocks are one contiguous load of
// UNROLL * 64 bfloat16 values, UNROLL consecutive elements per lane (a
// block's amax is a butterfly over its 64 / UNROLL lanes); the int6 levels
// pass through LDS into the MFMA's A operand, whose every row then holds
// row 0 (only row 0 of the product is stored).  The activation is read by
// every tile (it is 2K bytes against the tile's K / 2 of weights).
// TPW: tiles per wave (2: adjacent tiles share the wave's quantized
// activation range, so each range is quantized once per pair of tiles).
template <int T, int NBW, int WAVES, int TPW = 1>
__global__ void __launch_bounds__(WAVES * 64)
k_gemv_nf4_q1(const uint16_t* __restrict__ x, float quant_max, vh_format xsfmt, vh_format xfmt,
              const uint8_t* __restrict__ wp,
              const uint8_t* __restrict__ ws, vh_format sfmt, uint4 lv, int64_t N, int64_t K, vh_epilogue epi,
              void* __restrict__ y) {
  constexpr int KR = WAVES / T;
  constexpr int UNROLL = NBW < 8 ? NBW : 8;
  constexpr int ROUNDS = NBW / UNROLL;
  constexpr int EPL = UNROLL;    // activation elements per lane in a round
  constexpr int LPB = 64 / EPL;  // lanes per block
  static_assert(ROUNDS <= 2 && (UNROLL == 4 || UNROLL == 8), "round shape");
  static_assert(TPW == 1 || TPW == 2, "tiles per wave");
  __shared__ float s_red[TPW][WAVES][1][64];
  __shared__ float s_scale[256];
  __shared__ __attribute__((aligned(4))) uint16_t s_keys[16];  // the element map's thresholds
  __shared__ __attribute__((aligned(16))) uint8_t s_xq[WAVES][UNROLL * 64];
  const int tid = threadIdx.x;
  const int nb = (int)(K / 64);
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tl = wave % T, kr = wave / T;
  const int64_t tile0 = ((int64_t)blockIdx.x * T + tl) * TPW;  // this wave's first tile
  const int b0 = kr * nb / KR, b1 = (kr + 1) * nb / KR;
  uint32_t base;
  asm volatile("v_mov_b32 %0, 0x3020100" : "=v"(base));

  // buffers from the round's first block to the range end (past it: zeros)
  const uint32_t woff = (uint32_t)lane * 8u, wsoff = (uint32_t)(lane & 15), xoff = (uint32_t)lane * (2u * EPL);
  typedef typename std::conditional<EPL == 8, vh_u32x4, vh_u32x2>::type XT;
  struct Set {
    vh_u32x2 w[TPW][UNROLL];
    uint32_t sw[TPW][UNROLL];
    XT x;
  };
  auto load = [&](int b, Set& st) __attribute__((always_inline)) {
    uint32_t wo = woff, wso = wsoff, xo = xoff;
    asm volatile("" : "+v"(wo), "+v"(wso), "+v"(xo));
    const int64_t rem = b1 - b;
    const __amdgpu_buffer_rsrc_t xr = rsrc(x + (int64_t)b * 64, rem * 128);
    // the activation first: waiting for it leaves the weights in flight
    if constexpr (EPL == 8) st.x = __builtin_amdgcn_raw_buffer_load_b128(xr, xo, 0, 0);
    else st.x = __builtin_amdgcn_raw_buffer_load_b64(xr, xo, 0, 0);
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      const __amdgpu_buffer_rsrc_t wr = rsrc(wp + ((tile0 + t) * nb + b) * 512, rem * 512);
      const __amdgpu_buffer_rsrc_t wsr = rsrc(ws + ((tile0 + t) * nb + b) * 16, rem * 16);
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) {
        st.w[t][u] = __builtin_amdgcn_raw_buffer_load_b64(wr, wo + u * 512u, 0, 0);
        st.sw[t][u] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(wsr, wso + u * 16u, 0, 0);
      }
    }
  };
  float acc[TPW];
#pragma unroll
  for (int t = 0; t < TPW; ++t) acc[t] = 0.0f;
  auto round = [&](Set& st, int b) __attribute__((always_inline)) {
    asm volatile("" : "+v"(st.x)::"memory");
    float xv[EPL];
#pragma unroll
    for (int j = 0; j < EPL / 2; ++j) {
      xv[2 * j] = bf2f(st.x[j] & 0xffffu);
      xv[2 * j + 1] = bf2f(st.x[j] >> 16);
    }
    // the block's scale (block_scale, MX_SCALED, bf16, no global scale):
    // the NaN-propagating amax over the block's LPB lanes as one key
    uint32_t mk = 0u;
#pragma unroll
    for (int j = 0; j < EPL; ++j) mk = umax32(mk, amax_key(xv[j]));
    mk = group_umax<LPB>(mk);
    float sc = div_bf16(mk == 0xFFFFFFFFu ? __uint_as_float(0x7fc00000u) : __uint_as_float(mk), quant_max);
    sc = rbf(fmt_value_k<K_MINI>(f2bf(sc), xsfmt, nullptr));
    if (!(sc > 0.0f)) sc = 1.0f;
    // element codes as element_code<K_STEPS> forms them (levels <= 15):
    // q = bf16(x / sc) as div_bf16 forms it, rounded by the hardware
    // converter (a NaN is flagged below, so its payload does not matter)
    uint32_t bq[EPL];
    div_bf16_bits_n(xv, sc, bq);
    uint32_t key[EPL], pos[EPL];
    bool nanv[EPL];
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
      nanv[j] = bf_isnan_bits(bq[j]);
      key[j] = bf_key(bq[j]);
      pos[j] = 0u;
    }
    // the level: steps_level_padded (s_keys is padded with 0xFFFF past
    // nsteps), the lane's searches stepping together
#pragma unroll
    for (int step = 8; step >= 1; step >>= 1) {
#pragma unroll
      for (int j = 0; j < EPL; ++j)
        pos[j] = (uint32_t)s_keys[pos[j] + step - 1] <= key[j] ? pos[j] + step : pos[j];
    }
    uint32_t lvw[EPL / 4];
#pragma unroll
    for (int q = 0; q < EPL / 4; ++q) {
      uint32_t c = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) c |= (nanv[4 * q + j] ? (uint32_t)xfmt.nan_level : pos[4 * q + j]) << (8 * j);
      lvw[q] = lut_lo(c, base, lv);
    }
    if constexpr (EPL == 8) *(vh_u32x2*)&s_xq[wave][8 * lane] = vh_u32x2{lvw[0], lvw[1]};
    else *(uint32_t*)&s_xq[wave][4 * lane] = lvw[0];
    // each block's scale from the first lane of its group; zero past the range
    float sxb[UNROLL];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const float v = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sc), u * LPB));
      sxb[u] = b + u < b1 ? v : 0.0f;
    }
    // the blocks software-pipelined as in k_gemv_nf4: LDS reads one block
    // ahead of the lookup and MFMA, the scale product one block behind
    vh_u32x4 xq[UNROLL];
    float swv[TPW][UNROLL];
    int dd[TPW][UNROLL];
    auto stage_a = [&](int u) __attribute__((always_inline)) {
      if constexpr (TPW == 1)
        asm volatile("" : "+v"(st.w[0][u]), "+v"(st.sw[0][u]));
      else
        asm volatile("" : "+v"(st.w[0][u]), "+v"(st.sw[0][u]), "+v"(st.w[1][u]), "+v"(st.sw[1][u]));
      xq[u] = *(const vh_u32x4*)&s_xq[wave][u * 64 + 16 * (lane >> 4)];
#pragma unroll
      for (int t = 0; t < TPW; ++t) swv[t][u] = s_scale[st.sw[t][u]];
    };
    auto stage_b = [&](int u) __attribute__((always_inline)) {
      const i32x4 xa = {(int)xq[u].x, (int)xq[u].y, (int)xq[u].z, (int)xq[u].w};
#pragma unroll
      for (int t = 0; t < TPW; ++t) {
        i32x4 wl;
        wl[0] = (int)lut_lo(st.w[t][u].x, base, lv);
        wl[1] = (int)lut_lo(st.w[t][u].y, base, lv);
        wl[2] = (int)lut_hi(st.w[t][u].x, base, lv);
        wl[3] = (int)lut_hi(st.w[t][u].y, base, lv);
        const i32x4 z = {0, 0, 0, 0};
        dd[t][u] = __builtin_amdgcn_mfma_i32_16x16x64_i8(xa, wl, z, 0, 0, 0)[0];
      }
    };
    auto stage_c = [&](int u) __attribute__((always_inline)) {
#pragma unroll
      for (int t = 0; t < TPW; ++t) acc[t] = fmaf((float)dd[t][u], sxb[u] * swv[t][u], acc[t]);
    };
    stage_a(0);
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      if (u + 1 < UNROLL) stage_a(u + 1);
      stage_b(u);
      if (u > 0) stage_c(u - 1);
    }
    stage_c(UNROLL - 1);
  };
  Set s[2];
  auto chunk = [&](int c0, auto pre) __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < ROUNDS; ++r) {
      if constexpr (!decltype(pre)::value)
        if (r + 1 < ROUNDS) load(c0 + (r + 1) * UNROLL, s[(r + 1) & 1]);
      round(s[r & 1], c0 + r * UNROLL);
      asm volatile("" ::: "memory");
    }
  };
  load(b0, s[0]);
  if constexpr (ROUNDS == 2) load(b0 + UNROLL, s[1]);
  if (tid < 256) s_scale[tid] = scale_value((uint32_t)tid, sfmt);
  {
    // the first 16 thresholds (all a table of at most 16 levels uses), read
    // through the scalar cache and spread over lanes 0..7 of wave 0 (a
    // per-lane read of the argument would be a vector load, and storing it
    // would wait for every load in flight); 0xFFFF past nsteps
    const uint32_t* kw = (const uint32_t*)xfmt.thr_key;
    uint32_t kv = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) kv = lane == i ? kw[i] : kv;
    const int ns = xfmt.nsteps;
    kv = (2 * lane < ns ? kv & 0xffffu : 0xffffu) | (2 * lane + 1 < ns ? kv & 0xffff0000u : 0xffff0000u);
    if (wave == 0 && lane < 8) *(uint32_t*)&s_keys[2 * lane] = kv;
  }
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  if (b0 < b1) chunk(b0, std::true_type{});
  for (int c0 = b0 + NBW; c0 < b1; c0 += NBW) {
    load(c0, s[0]);
    chunk(c0, std::false_type{});
  }
#pragma unroll
  for (int t = 0; t < TPW; ++t) s_red[t][wave][0][lane] = acc[t];
  __syncthreads();
  if (kr != 0) return;
#pragma unroll
  for (int t = 0; t < TPW; ++t)
    finish<T, 1, WAVES>(s_red[t], tl, lane, (lane >> 4) * 4, 1, (tile0 + t) * 16 + (lane & 15), N, epi, y);
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
  // 8, 16 or 32 (longer ranges in chunks of 32)
  const int64_t nb = K / 64;
  const int64_t kr = four ? 2 : 8, bpw = (nb + kr - 1) / kr;
  // two tiles per wave (the activation loads shared) while that leaves at
  // least 256 workgroups: 896 tiles then run in one round of the CUs
  const bool pair = !four && tiles >= 512 && tiles % 2 == 0;
  auto go = [&](auto mr) {
    constexpr int MR = decltype(mr)::value;
    auto launch = [&](auto nbw) {
      constexpr int NBW = decltype(nbw)::value;
      if (four)
        hipLaunchKernelGGL((k_gemv_nf4<4, MR, NBW, 8, 1>), dim3((unsigned)(tiles / 4)), dim3(512), 0, st, x_levels,
                           x_scale, (int)M, w_packed, w_scale, *w_scale_fmt, lv, N, K, *epi, y);
      else if (pair)
        hipLaunchKernelGGL((k_gemv_nf4<1, MR, NBW, 8, 2>), dim3((unsigned)(tiles / 2)), dim3(512), 0, st, x_levels,
                           x_scale, (int)M, w_packed, w_scale, *w_scale_fmt, lv, N, K, *epi, y);
      else
        hipLaunchKernelGGL((k_gemv_nf4<1, MR, NBW, 8, 1>), dim3((unsigned)tiles), dim3(512), 0, st, x_levels, x_scale,
                           (int)M, w_packed, w_scale, *w_scale_fmt, lv, N, K, *epi, y);
    };
    if (bpw <= 4) launch(std::integral_constant<int, 4>{});
    else if (bpw <= 8) launch(std::integral_constant<int, 8>{});
    else if (bpw <= 16) launch(std::integral_constant<int, 16>{});
    else launch(std::integral_constant<int, 32>{});
  };
  if (M == 1) go(std::integral_constant<int, 1>{});
  else go(std::integral_constant<int, 4>{});
  return vh::check_launch("vh_gemv_nf4");
}

extern "C" int vh_gemv_nf4_m1(const void* x, int32_t x_dtype, float quant_max, const vh_format* x_scale_fmt,
                              const vh_format* x_fmt, const uint8_t* w_packed, const uint8_t* w_scale,
                              const vh_format* w_scale_fmt, const int8_t* levels16, int64_t N, int64_t K,
                              const vh_epilogue* epi, void* y, vh_stream_t stream) {
  VH_REQUIRE(x && x_scale_fmt && x_fmt && w_packed && w_scale && w_scale_fmt && levels16 && epi && y,
             "vh_gemv_nf4_m1: null argument");
  VH_REQUIRE(x_dtype == VH_BF16, "vh_gemv_nf4_m1: the activation must be bfloat16");
  VH_REQUIRE(N > 0 && K > 0 && N % 16 == 0 && K % 64 == 0, "vh_gemv_nf4_m1: needs N %% 16 == 0 and K %% 64 == 0");
  VH_REQUIRE(K / 64 <= 8 * 32, "vh_gemv_nf4_m1: K must be <= %d", 8 * 32 * 64);
  VH_REQUIRE(((uintptr_t)x % 16 == 0) && ((uintptr_t)w_packed % 8 == 0), "vh_gemv_nf4_m1: misaligned operand");
  VH_REQUIRE(kernel_kind(x_scale_fmt) == K_MINI, "vh_gemv_nf4_m1: the activation scale map must be a minifloat");
  VH_REQUIRE(x_fmt->kind == VH_FMT_STEPS && x_fmt->nsteps >= 0 && x_fmt->nsteps <= 15 && x_fmt->nan_level <= 15,
             "vh_gemv_nf4_m1: the activation map must be an index table of at most 16 levels");
  VH_REQUIRE(epi->mode == EPI_PLAIN && (epi->out_dtype == VH_BF16 || epi->out_dtype == VH_F32),
             "vh_gemv_nf4_m1: unsupported epilogue");
  VH_REQUIRE(w_scale_fmt->kind != VH_FMT_LUT && w_scale_fmt->kind != VH_FMT_IDENTITY &&
                 w_scale_fmt->kind != VH_FMT_STEPS,
             "vh_gemv_nf4_m1: the weight scale map needs a closed form with packed codes");
  uint32_t t[4];
  memcpy(t, levels16, 16);
  const uint4 lv = make_uint4(t[0], t[1], t[2], t[3]);
  // the same workgroup shapes as vh_gemv_nf4: two tiles per wave on grids
  // of at least 512 tiles (each K range then quantized once per pair)
  const int64_t tiles = N / 16, nb = K / 64;
  const bool four = tiles >= 512 && tiles % 4 == 0 && nb <= 2 * 16;
  const bool pair = !four && tiles >= 512 && tiles % 2 == 0;
  const int64_t kr = four ? 2 : 8, bpw = (nb + kr - 1) / kr;
  hipStream_t st = vh::as_stream(stream);
  auto launch = [&](auto nbw) {
    constexpr int NBW = decltype(nbw)::value;
    if (four)
      hipLaunchKernelGGL((k_gemv_nf4_q1<4, NBW, 8>), dim3((unsigned)(tiles / 4)), dim3(512), 0, st,
                         (const uint16_t*)x, quant_max, *x_scale_fmt, *x_fmt, w_packed, w_scale, *w_scale_fmt, lv, N,
                         K, *epi, y);
    else if (pair)
      hipLaunchKernelGGL((k_gemv_nf4_q1<1, NBW, 8, 2>), dim3((unsigned)(tiles / 2)), dim3(512), 0, st,
                         (const uint16_t*)x, quant_max, *x_scale_fmt, *x_fmt, w_packed, w_scale, *w_scale_fmt, lv, N,
                         K, *epi, y);
    else
      hipLaunchKernelGGL((k_gemv_nf4_q1<1, NBW, 8>), dim3((unsigned)tiles), dim3(512), 0, st, (const uint16_t*)x,
                         quant_max, *x_scale_fmt, *x_fmt, w_packed, w_scale, *w_scale_fmt, lv, N, K, *epi, y);
  };
  if (bpw <= 4) launch(std::integral_constant<int, 4>{});
  else if (bpw <= 8) launch(std::integral_constant<int, 8>{});
  else launch(std::integral_constant<int, 16>{});
  return vh::check_launch("vh_gemv_nf4_m1");
}
