// Decode step of an MX-int8 / KIVI decoder layer: a batch of single tokens
// through RMSNorm, MX-int8 linears (linear_mx, ops/quantized.py:651-723, with
// the activation quantize_mx of ops/quantized.py:1122-1216 fused into the
// producer of each linear's input) and attention over a KIVI 2-bit cache
// (group-wise affine codes, dequantize of ops/quantized.py:518-571) plus a
// full-precision residual window.
//
// Everything here is weight- or cache-bandwidth bound at a few microseconds
// per launch, so the kernels keep the per-wave instruction stream short:
//
// * MX-int8 GEMV: weights stay one byte.  A weight code c with block
//   exponent e enters an fp16 MFMA as (1024 + (c + 128)) * 2**e, built with
//   one v_perm per two weights from the code bytes and a baked fp16 high byte
//   (25 + e) << 2; a second MFMA against -1152 * 2**e removes the offset.
//   The activations are the fake-quantized values code_x * 2**e_x in fp16, so
//   every product is exact and only the fp32 summation order differs from
//   the reference's fp32 GEMM of the dequantized operands.
// * KIVI attention: flash-decoding over 32-token groups.  Keys are
//   dequantized element by element exactly as the reference's bf16
//   dequantize rounds them ((code - zp) rounded, times scale rounded) and meet
//   the bf16 query on a bf16 MFMA, so each score is the reference's matmul up
//   to summation order, then rounded where eager attention rounds it.  Value
//   codes stay exact fp16 MFMA operands (1024 + c * 4**p, one VALU op per
//   pair); their affine scale moves to the probabilities' operand and the
//   zero-point term is a per-group dot product.  The cache state (main
//   tokens, residual slots) lives in device memory, so a captured step
//   replays across positions, and the fold of a completed residual chunk
//   into the main cache runs on the device.
#include <hip/hip_runtime.h>

#include "vh_device.h"
#include "vh_host.h"

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int MX_SHIFT = 6;  // floor(log2(127)): pot scale 2**(floor(log2(amax)) - 6)
constexpr int GEMV_WAVES = 8;  // two workgroups per CU: one streams while the other reduces
constexpr int HEAD_DIM = 128;
constexpr int GQA = 4;        // query heads per kv head
constexpr int KV_GROUP = 32;  // KIVI group: tokens per key group, channels per value group
constexpr int RES_CAP = VH_KIVI_RES_CAP;

// ------------------------------------------------------- MX-int8 fake quant
// quantize_mx(x, int8, block 16, force_scale_power_of_two=True) followed by
// the code x scale product of linear_mx.  Block scale (mx_utils.py /
// calculate_mx_qparam): 2**(floor(log2(amax)) - 6) in bfloat16, amax == 0
// taking floor(log2) = -126; a scale that underflows to 0 or a NaN amax gives
// scale 1; an infinite amax gives inf.  Codes: clamp(rint(bf16(x / s)),
// -128, 127) with NaN kept.
struct Mx8Scale {
  float s;
  int e;
  bool pow2;
};

VH_DEV Mx8Scale mx8_scale(float amax) {
  Mx8Scale r{1.0f, 0, true};
  if (isnan_f(amax)) return r;
  if (amax == __builtin_inff()) {
    r.s = amax;
    r.pow2 = false;
    return r;
  }
  const int E = amax == 0.0f ? -126 : floor_log2(amax);
  const int e = E - MX_SHIFT;
  const float s = rbf(ldexpf(1.0f, e));
  if (s > 0.0f) {
    r.s = s;
    r.e = e;
  }
  return r;
}

VH_DEV float mx8_fq(float x, const Mx8Scale& sc) {
  float q = rbf(sc.pow2 ? ldexpf(x, -sc.e) : x / sc.s);
  if (!isnan_f(q)) q = fminf(fmaxf(rintf(q), -128.0f), 127.0f);
  return rbf(q * sc.s);
}

// The fp16 operand of a fake-quantized activation; flags values that do not
// fit fp16 (|x| > 65504).
// The same with the overflow noted in `ovf` (one flag update per thread).
VH_DEV _Float16 fq_half_ovf(float v, bool& ovf) {
  const _Float16 h = (_Float16)v;
  ovf |= __builtin_isinf((float)h) && !__builtin_isinf(v);
  return h;
}

VH_DEV _Float16 fq_half(float v, int* flag) {
  const _Float16 h = (_Float16)v;
  if (__builtin_isinf((float)h) && !__builtin_isinf(v)) atomicOr(flag, VH_DECODE_ERR_FP16_RANGE);
  return h;
}

VH_DEV float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// The NaN-propagating maximum of v >= 0 (or NaN) over aligned groups of 16
// lanes, to every lane of the group (NaN comes back as some NaN; every
// caller tests it with isnan).
VH_DEV float max16(float v) { return __uint_as_float(group_umax<16>(amax_key(v))); }

// ------------------------------------------------------------ RMSNorm
// LlamaRMSNorm: h = w * bf16(x * rsqrt(mean(x**2) + eps)) in bfloat16, then
// the MX-int8 fake quantization of h for the next linear.  One workgroup
// per row, one 16-element block per thread and pass.
__global__ void __launch_bounds__(256)
k_rmsnorm_mx8(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w, int64_t H, float eps,
              uint16_t* __restrict__ h_out, _Float16* __restrict__ fq, int* __restrict__ flag) {
  __shared__ float s_sum[4];
  const int64_t row = blockIdx.x;
  const uint16_t* xr = x + row * H;
  const int64_t nb = H / 16;
  float ss = 0.0f;
  for (int64_t b = threadIdx.x; b < nb; b += 256) {
    const uint4* p = (const uint4*)(xr + b * 16);
    const uint4 v0 = p[0], v1 = p[1];
    const uint32_t wv[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float a = bf2f(wv[j] & 0xffffu), c = bf2f(wv[j] >> 16);
      ss = fmaf(a, a, ss);
      ss = fmaf(c, c, ss);
    }
  }
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) s_sum[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float total = s_sum[0] + s_sum[1] + s_sum[2] + s_sum[3];
  const float r = 1.0f / sqrtf(total / (float)H + eps);
  for (int64_t b = threadIdx.x; b < nb; b += 256) {
    const uint4* p = (const uint4*)(xr + b * 16);
    const uint4* q = (const uint4*)(w + b * 16);
    const uint4 v0 = p[0], v1 = p[1], w0 = q[0], w1 = q[1];
    const uint32_t xv[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
    const uint32_t wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
    float h[16];
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      h[2 * j] = rbf(bf2f(wv[j] & 0xffffu) * rbf(bf2f(xv[j] & 0xffffu) * r));
      h[2 * j + 1] = rbf(bf2f(wv[j] >> 16) * rbf(bf2f(xv[j] >> 16) * r));
      amax = nmax(amax, nmax(fabsf(h[2 * j]), fabsf(h[2 * j + 1])));
    }
    if (h_out) {
      uint4* o = (uint4*)(h_out + row * H + b * 16);
      o[0] = make_uint4(f2bf(h[0]) | (f2bf(h[1]) << 16), f2bf(h[2]) | (f2bf(h[3]) << 16),
                        f2bf(h[4]) | (f2bf(h[5]) << 16), f2bf(h[6]) | (f2bf(h[7]) << 16));
      o[1] = make_uint4(f2bf(h[8]) | (f2bf(h[9]) << 16), f2bf(h[10]) | (f2bf(h[11]) << 16),
                        f2bf(h[12]) | (f2bf(h[13]) << 16), f2bf(h[14]) | (f2bf(h[15]) << 16));
    }
    const Mx8Scale sc = mx8_scale(amax);
    f16x8 o0, o1;
    bool ovf = false;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      o0[j] = fq_half_ovf(mx8_fq(h[j], sc), ovf);
      o1[j] = fq_half_ovf(mx8_fq(h[8 + j], sc), ovf);
    }
    if (ovf) atomicOr(flag, VH_DECODE_ERR_FP16_RANGE);
    f16x8* fo = (f16x8*)(fq + row * H + b * 16);
    fo[0] = o0;
    fo[1] = o1;
  }
}

// ------------------------------------------------ MX-int8 as exact fp16 rows
// The operands of vh_gemm_mx8_f16: an MX-int8 row (int8 codes, a power-of-
// two scale 2**e per 16 elements) as code * 2**(e - E) in fp16, E the row's
// largest finite block exponent -- exact, since an 8-bit code at a power of
// two down to 2**-24 is an fp16 value.  Blocks more than 24 binades under E
// are flushed: their products lie below the float32 resolution of the row's
// largest ones.  A block whose scale is not finite writes code * scale, as
// the reference's decode does (infinities and NaN).
constexpr int F16_FLUSH = -24;

VH_DEV _Float16 rebased_f16(float code, int e, bool finite, float s, int E) {
  if (!finite) return (_Float16)(code * s);
  const int d = e - E;
  return (_Float16)(d >= F16_FLUSH ? ldexpf(code, d) : code * 0.0f);
}

// The maximum of v over a 256-thread workgroup (every thread calls it):
// each wave's by DPP moves (signed order as unsigned with the sign bit
// flipped), then the four through LDS.
VH_DEV int block_max_int(int v, int* s_red) {
  v = (int)(group_umax<64>((uint32_t)v ^ 0x80000000u) ^ 0x80000000u);
  if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = v;
  __syncthreads();
  const int r = max(max(s_red[0], s_red[1]), max(s_red[2], s_red[3]));
  __syncthreads();
  return r;
}

// quantize_mx(x, int8, [-1], 16, 127, force_scale_power_of_two=True) of each
// bf16 row (ops/quantized.py:1070-1115; codes and scales as mx8_scale /
// mx8_fq form them), written as the exact fp16 row above with E in ex.  One
// workgroup per row: the blocks' exponents, their maximum, then the codes.
__global__ void __launch_bounds__(256) k_quantize_mx8_f16(const uint16_t* __restrict__ x, int64_t K,
                                                          _Float16* __restrict__ out, int32_t* __restrict__ ex) {
  __shared__ int s_red[4];
  const int64_t row = blockIdx.x;
  const uint16_t* xr = x + row * K;
  const int64_t nb = K / 16;
  int emax = INT_MIN;
  for (int64_t b = threadIdx.x; b < nb; b += 256) {
    const uint4* p = (const uint4*)(xr + b * 16);
    const uint4 v0 = p[0], v1 = p[1];
    const uint32_t wv[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) amax = nmax(amax, nmax(fabsf(bf2f(wv[j] & 0xffffu)), fabsf(bf2f(wv[j] >> 16))));
    const Mx8Scale sc = mx8_scale(amax);
    if (sc.pow2) emax = max(emax, sc.e);
  }
  int E = block_max_int(emax, s_red);
  if (E == INT_MIN) E = 0;
  for (int64_t b = threadIdx.x; b < nb; b += 256) {
    const uint4* p = (const uint4*)(xr + b * 16);
    const uint4 v0 = p[0], v1 = p[1];
    const uint32_t wv[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
    float xv[16];
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      xv[2 * j] = bf2f(wv[j] & 0xffffu);
      xv[2 * j + 1] = bf2f(wv[j] >> 16);
      amax = nmax(amax, nmax(fabsf(xv[2 * j]), fabsf(xv[2 * j + 1])));
    }
    const Mx8Scale sc = mx8_scale(amax);
    f16x8 o[2];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      float q = rbf(sc.pow2 ? ldexpf(xv[j], -sc.e) : xv[j] / sc.s);
      if (!isnan_f(q)) q = fminf(fmaxf(rintf(q), -128.0f), 127.0f);
      o[j >> 3][j & 7] = rebased_f16(q, sc.e, sc.pow2, sc.s, E);
    }
    f16x8* dst = (f16x8*)(out + row * K + b * 16);
    dst[0] = o[0];
    dst[1] = o[1];
  }
  if (threadIdx.x == 0) ex[row] = E;
}

// The same for rows of at most 256 NBT blocks: each thread loads its NBT
// blocks once and keeps them in registers across the row maximum (no second
// read of the row); identical arithmetic, so identical output.
template <int NBT>
__global__ void __launch_bounds__(256) k_quantize_mx8_f16_r(const uint16_t* __restrict__ x, int64_t K,
                                                            _Float16* __restrict__ out, int32_t* __restrict__ ex) {
  __shared__ int s_red[4];
  const int64_t row = blockIdx.x;
  const uint16_t* xr = x + row * K;
  const int nb = (int)(K / 16);
  uint4 raw[NBT][2];
#pragma unroll
  for (int j = 0; j < NBT; ++j) {
    const int b = threadIdx.x + 256 * j;
    if (b < nb) {
      const uint4* p = (const uint4*)(xr + (int64_t)b * 16);
      raw[j][0] = p[0];
      raw[j][1] = p[1];
    } else {
      raw[j][0] = raw[j][1] = make_uint4(0u, 0u, 0u, 0u);
    }
  }
  Mx8Scale sc[NBT];
  int emax = INT_MIN;
#pragma unroll
  for (int j = 0; j < NBT; ++j) {
    const uint32_t wv[8] = {raw[j][0].x, raw[j][0].y, raw[j][0].z, raw[j][0].w,
                            raw[j][1].x, raw[j][1].y, raw[j][1].z, raw[j][1].w};
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = nmax(amax, nmax(fabsf(bf2f(wv[i] & 0xffffu)), fabsf(bf2f(wv[i] >> 16))));
    sc[j] = mx8_scale(amax);
    if (threadIdx.x + 256 * j < nb && sc[j].pow2) emax = max(emax, sc[j].e);
  }
  int E = block_max_int(emax, s_red);
  if (E == INT_MIN) E = 0;
#pragma unroll
  for (int j = 0; j < NBT; ++j) {
    const int b = threadIdx.x + 256 * j;
    if (b >= nb) continue;
    const uint32_t wv[8] = {raw[j][0].x, raw[j][0].y, raw[j][0].z, raw[j][0].w,
                            raw[j][1].x, raw[j][1].y, raw[j][1].z, raw[j][1].w};
    // mx8_fq's division and rebased_f16 with the block's choices made once
    // (a scale that is not a power of two is infinite: x / inf is x * 0)
    const bool p2 = sc[j].pow2;
    const int d = sc[j].e - E;
    const bool keep = d >= F16_FLUSH;
    f16x8 o[2];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float xv = bf2f((i & 1) ? wv[i >> 1] >> 16 : wv[i >> 1] & 0xffffu);
      float q = rbf(p2 ? ldexpf(xv, -sc[j].e) : xv * 0.0f);
      q = isnan_f(q) ? q : fminf(fmaxf(rintf(q), -128.0f), 127.0f);
      o[i >> 3][i & 7] = (_Float16)(p2 ? (keep ? ldexpf(q, d) : q * 0.0f) : q * sc[j].s);
    }
    f16x8* dst = (f16x8*)(out + row * K + (int64_t)b * 16);
    dst[0] = o[0];
    dst[1] = o[1];
  }
  if (threadIdx.x == 0) ex[row] = E;
}

// Packed MX-int8 weights (int8 codes [N, K], scale bytes 2**(byte - bias)
// [N, K / 16], 255 = inf) as exact fp16 rows with their E.  One workgroup
// per row.
__global__ void __launch_bounds__(256) k_mx8_bake_f16(const int8_t* __restrict__ codes, const uint8_t* __restrict__ sb,
                                                      int bias, int64_t K, _Float16* __restrict__ out,
                                                      int32_t* __restrict__ ew) {
  __shared__ int s_red[4];
  const int64_t row = blockIdx.x;
  const int64_t nb = K / 16;
  int emax = INT_MIN;
  for (int64_t b = threadIdx.x; b < nb; b += 256) {
    const int byte = sb[row * nb + b];
    if (byte != 255) emax = max(emax, byte - bias);
  }
  int E = block_max_int(emax, s_red);
  if (E == INT_MIN) E = 0;
  for (int64_t b = threadIdx.x; b < nb; b += 256) {
    const int byte = sb[row * nb + b];
    const bool finite = byte != 255;
    const int4* p = (const int4*)(codes + row * K + b * 16);
    const int4 c = p[0];
    const uint32_t cw[4] = {(uint32_t)c.x, (uint32_t)c.y, (uint32_t)c.z, (uint32_t)c.w};
    f16x8 o[2];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const float code = (float)(int8_t)(cw[j >> 2] >> (8 * (j & 3)));
      o[j >> 3][j & 7] = rebased_f16(code, byte - bias, finite, __builtin_inff(), E);
    }
    f16x8* dst = (f16x8*)(out + row * K + b * 16);
    dst[0] = o[0];
    dst[1] = o[1];
  }
  if (threadIdx.x == 0) ew[row] = E;
}

// The same for rows of at most 256 NBT blocks: each thread loads its NBT
// blocks' codes and scale bytes once, before the row maximum, and keeps
// them in registers; identical arithmetic, so identical output.
template <int NBT>
__global__ void __launch_bounds__(256) k_mx8_bake_f16_r(const int8_t* __restrict__ codes,
                                                        const uint8_t* __restrict__ sb, int bias, int64_t K,
                                                        _Float16* __restrict__ out, int32_t* __restrict__ ew) {
  __shared__ int s_red[4];
  const int64_t row = blockIdx.x;
  const int nb = (int)(K / 16);
  int4 c[NBT];
  int byte[NBT];
#pragma unroll
  for (int j = 0; j < NBT; ++j) {
    const int b = threadIdx.x + 256 * j;
    const bool ok = b < nb;
    c[j] = ok ? *(const int4*)(codes + row * K + (int64_t)b * 16) : make_int4(0, 0, 0, 0);
    byte[j] = ok ? sb[row * nb + b] : 255;
  }
  int emax = INT_MIN;
#pragma unroll
  for (int j = 0; j < NBT; ++j)
    if (byte[j] != 255) emax = max(emax, byte[j] - bias);
  int E = block_max_int(emax, s_red);
  if (E == INT_MIN) E = 0;
#pragma unroll
  for (int j = 0; j < NBT; ++j) {
    const int b = threadIdx.x + 256 * j;
    if (b >= nb) continue;
    const bool finite = byte[j] != 255;
    const uint32_t cw[4] = {(uint32_t)c[j].x, (uint32_t)c[j].y, (uint32_t)c[j].z, (uint32_t)c[j].w};
    f16x8 o[2];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float code = (float)(int8_t)(cw[i >> 2] >> (8 * (i & 3)));
      o[i >> 3][i & 7] = rebased_f16(code, byte[j] - bias, finite, __builtin_inff(), E);
    }
    f16x8* dst = (f16x8*)(out + row * K + (int64_t)b * 16);
    dst[0] = o[0];
    dst[1] = o[1];
  }
  if (threadIdx.x == 0) ew[row] = E;
}

// ------------------------------------------------------------ MX-int8 GEMV
// Baked weight layout, per 16-column tile T (K = 256 G):
//   codes [T][K/64 step pairs][64 lanes][16 B]: bytes 0-7 step 2p, 8-15 step
//         2p + 1; lane l holds column l % 16, k = 32 step + 8 (l / 16) + j, as
//         u = c + 128.
//   hb    [T][G][32 slots][8 B]: slot (l % 16) + 16 (l / 32); byte u is the
//         fp16 high byte (25 + e) << 2 of the scale 2**e of block
//         2 (8 g + u) + l / 32 of that column.
// A workgroup owns NT tiles; its 16 waves split the K groups and reduce
// through LDS.
struct GemvArgs {
  const _Float16* x;  // [M, K] fake-quantized activations
  int32_t M;
  int64_t K;
  const uint8_t* wc;
  const uint8_t* wh;
  int64_t n_out;          // columns of y / fq
  int32_t mode;           // VH_GEMV_*
  const uint16_t* res;    // [M, n_out] bf16 (VH_GEMV_RESIDUAL)
  uint16_t* y;            // [M, n_out] bf16 (may be null for VH_GEMV_SWIGLU)
  _Float16* fq;           // [M, n_out] fp16 (VH_GEMV_SWIGLU)
  int* flag;
  const int32_t* row_exp;  // or null: per row of x, 2**e its sums are multiplied by (rebased activations)
  const int32_t* w_shift;  // or null: per weight row (original order), likewise (rebased weights)
};

template <int NT>
__global__ void __launch_bounds__(GEMV_WAVES * 64, 2) k_gemv_mx8(GemvArgs a) {
  __shared__ float s_red[GEMV_WAVES][NT][4][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t nsp = a.K / 64, ngr = a.K / 256;
  const int64_t tile0 = (int64_t)blockIdx.x * NT;
  const int64_t g0 = wave * ngr / GEMV_WAVES, g1 = (wave + 1) * ngr / GEMV_WAVES;
  const int ma = lane & 15;
  const bool live = ma < a.M;
  const _Float16* xrow = a.x + (int64_t)(live ? ma : 0) * a.K + (lane >> 4) * 8;
  const int slot = (lane & 15) | ((lane >> 5) << 4);

  f32x4 acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = {0.0f, 0.0f, 0.0f, 0.0f};

  for (int64_t g = g0; g < g1; ++g) {
    uint4 c[NT][4];
    uint2 h[NT];
    uint4 xv[8];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const uint8_t* wt = a.wc + ((tile0 + t) * nsp + g * 4) * 1024 + lane * 16;
#pragma unroll
      for (int sp = 0; sp < 4; ++sp) c[t][sp] = *(const uint4*)(wt + sp * 1024);
      h[t] = *(const uint2*)(a.wh + (((tile0 + t) * ngr + g) * 32 + slot) * 8);
    }
#pragma unroll
    for (int s = 0; s < 8; ++s)
      xv[s] = live ? *(const uint4*)(xrow + (g * 8 + s) * 32) : make_uint4(0, 0, 0, 0);

#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const f16x8 av = __builtin_bit_cast(f16x8, xv[s]);
      const uint32_t hs = 4u + (s & 3);
      const uint32_t sel_lo = 0x00u | (hs << 8) | (0x01u << 16) | (hs << 24);
      const uint32_t sel_hi = 0x02u | (hs << 8) | (0x03u << 16) | (hs << 24);
      const uint32_t sel_c = 0x00u | (hs << 8) | (0x00u << 16) | (hs << 24);
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const uint4 cc = c[t][s >> 1];
        const uint32_t w0 = (s & 1) ? cc.z : cc.x, w1 = (s & 1) ? cc.w : cc.y;
        const uint32_t hd = (s < 4) ? h[t].x : h[t].y;
        uint4 b;
        b.x = __builtin_amdgcn_perm(hd, w0, sel_lo);
        b.y = __builtin_amdgcn_perm(hd, w0, sel_hi);
        b.z = __builtin_amdgcn_perm(hd, w1, sel_lo);
        b.w = __builtin_amdgcn_perm(hd, w1, sel_hi);
        const uint32_t cd = __builtin_amdgcn_perm(hd | 0x80808080u, 0x80808080u, sel_c);
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, __builtin_bit_cast(f16x8, b), acc[t], 0, 0, 0);
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, __builtin_bit_cast(f16x8, make_uint4(cd, cd, cd, cd)),
                                                       acc[t], 0, 0, 0);
      }
    }
  }
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) s_red[wave][t][r][lane] = acc[t][r];
  __syncthreads();
  if (threadIdx.x >= 256) return;
  // 4 waves finish: thread (r, l2) owns row 4 (l2 / 16) + r, column l2 % 16;
  // the 16 columns of a row sit in 16 consecutive lanes.
  const int r = threadIdx.x >> 6, l2 = threadIdx.x & 63;
  const int row = (l2 >> 4) * 4 + r, col = l2 & 15;
  const bool row_ok = row < a.M;
  float v[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    float sum = 0.0f;
#pragma unroll
    for (int w = 0; w < GEMV_WAVES; ++w) sum += s_red[w][t][r][l2];
    v[t] = sum;
  }
  if (a.row_exp || a.w_shift) {
    // rebased operands: the sum times 2**(row exponent + column shift), exact
    const int re = a.row_exp && row_ok ? a.row_exp[row] : 0;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      // the weight row of tile t's column: gate / up rows n and n_out + n when paired
      const int64_t n = a.mode == VH_GEMV_SWIGLU ? (t == 0 ? 0 : a.n_out) + (int64_t)blockIdx.x * 16 + col
                                                 : (tile0 + t) * 16 + col;
      v[t] = ldexpf(v[t], re + (a.w_shift ? a.w_shift[n] : 0));
    }
  }
  if (a.mode == VH_GEMV_SWIGLU) {
    // LlamaMLP: act(gate) * up in bfloat16, then the MX-int8 fake
    // quantization of that product for the down projection (tiles 2i / 2i+1
    // are the gate / up rows of output block i).
    const int64_t n = (int64_t)blockIdx.x * 16 + col;
    const float gt = rbf(v[0]), up = rbf(v[NT - 1]);
    const float act = rbf(gt / (1.0f + expf(-gt)));
    const float prod = rbf(act * up);
    const float amax = max16(row_ok ? fabsf(prod) : 0.0f);
    const Mx8Scale sc = mx8_scale(amax);
    if (row_ok) {
      if (a.y) a.y[row * a.n_out + n] = (uint16_t)f2bf(prod);
      a.fq[row * a.n_out + n] = fq_half(mx8_fq(prod, sc), a.flag);
    }
    return;
  }
  if (!row_ok) return;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int64_t n = (tile0 + t) * 16 + col;
    float o = rbf(v[t]);
    if (a.mode == VH_GEMV_RESIDUAL) o = rbf(o + bf2f(a.res[row * a.n_out + n]));
    a.y[row * a.n_out + n] = (uint16_t)f2bf(o);
  }
}

// Bake MX-int8 weights (one code byte per weight, one biased exponent byte per
// 16-weight block, as vh_quantize_mx packs them) into the GEMV layout.
// paired: rows [0, N/2) and [N/2, N) are interleaved tile by tile (gate / up).
// Rebased rows (shift != null): a row whose nonzero blocks' exponents leave
// [-24, 5] (the fp16 exponent field of the operand) is baked against its
// largest, e - (E_row - 5), and its sums multiplied back by 2**(E_row - 5)
// in the GEMV's epilogue (exact); its blocks more than 29 binades under
// E_row are flushed (codes 0).  A row within range keeps shift 0 and bakes
// as without rebasing.  One thread per row.
__global__ void __launch_bounds__(256) k_mx8_row_shift(const uint8_t* __restrict__ codes,
                                                       const uint8_t* __restrict__ scale, int bias, int64_t N,
                                                       int64_t K, int32_t* __restrict__ shift) {
  const int64_t n = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N) return;
  const int64_t nb = K / 16;
  int hi = -1000, lo = 1000;
  for (int64_t b = 0; b < nb; ++b) {
    const uint4 cv = *(const uint4*)(codes + n * K + b * 16);
    const int byte = scale[n * nb + b];
    if ((cv.x | cv.y | cv.z | cv.w) == 0u || byte == 255) continue;
    const int e = byte - bias;
    hi = e > hi ? e : hi;
    lo = e < lo ? e : lo;
  }
  shift[n] = (hi == -1000 || (lo >= -24 && hi <= 5)) ? 0 : hi - 5;
}

__device__ __forceinline__ bool mx8_flushed(const uint8_t* scale, int64_t n, int64_t nb, int64_t blk, int bias,
                                            const int32_t* shift) {
  if (!shift) return false;
  const int byte = scale[n * nb + blk];
  return byte != 255 && byte - bias - shift[n] < -24;
}

__global__ void __launch_bounds__(256) k_bake_mx8_codes(const uint8_t* __restrict__ codes, int64_t N, int64_t K,
                                                        int paired, const uint8_t* __restrict__ scale, int bias,
                                                        const int32_t* __restrict__ shift,
                                                        uint8_t* __restrict__ out) {
  const int64_t nsp = K / 64;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (N / 16) * nsp * 64) return;
  const int lane = (int)(t % 64);
  const int64_t sp = (t / 64) % nsp, tile = t / (64 * nsp);
  const int64_t src_tile = paired ? ((tile & 1) * (N / 32) + (tile >> 1)) : tile;
  const int64_t n = src_tile * 16 + (lane & 15);
  const int64_t k0 = sp * 64 + (lane >> 4) * 8;
  uint2 a = *(const uint2*)(codes + n * K + k0);
  uint2 b = *(const uint2*)(codes + n * K + k0 + 32);
  // a flushed block's codes bake as 0 (the 8 codes of a lane lie in one block)
  if (mx8_flushed(scale, n, K / 16, k0 / 16, bias, shift)) a = make_uint2(0u, 0u);
  if (mx8_flushed(scale, n, K / 16, (k0 + 32) / 16, bias, shift)) b = make_uint2(0u, 0u);
  *(uint4*)(out + t * 16) = make_uint4(a.x ^ 0x80808080u, a.y ^ 0x80808080u, b.x ^ 0x80808080u, b.y ^ 0x80808080u);
}

__global__ void __launch_bounds__(256) k_bake_mx8_scales(const uint8_t* __restrict__ codes,
                                                         const uint8_t* __restrict__ scale, int bias, int64_t N,
                                                         int64_t K, int paired, const int32_t* __restrict__ shift,
                                                         uint8_t* __restrict__ out, int* __restrict__ flag) {
  const int64_t ngr = K / 256, nb = K / 16;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (N / 16) * ngr * 32) return;
  const int sl = (int)(t % 32);
  const int64_t g = (t / 32) % ngr, tile = t / (32 * ngr);
  const int64_t src_tile = paired ? ((tile & 1) * (N / 32) + (tile >> 1)) : tile;
  const int64_t n = src_tile * 16 + (sl & 15);
  uint32_t lo = 0, hi = 0;
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const int64_t blk = 2 * (g * 8 + u) + (sl >> 4);
    const int byte = scale[n * nb + blk];
    const uint4* cp = (const uint4*)(codes + n * K + blk * 16);
    const uint4 cv = *cp;
    const bool zero = (cv.x | cv.y | cv.z | cv.w) == 0u;
    int e = byte - bias - (shift ? shift[n] : 0);
    // an all-zero block contributes nothing at any scale, nor does a flushed one
    if (zero || (shift && byte != 255 && e < -24)) e = 0;
    if (!zero && (byte == 255 || e < -24 || e > 5)) {
      atomicOr(flag, VH_DECODE_ERR_WEIGHT_RANGE);
      e = 0;
    }
    const uint32_t hb = (uint32_t)((25 + e) << 2);
    if (u < 4) lo |= hb << (8 * u);
    else hi |= hb << (8 * (u - 4));
  }
  *(uint2*)(out + t * 8) = make_uint2(lo, hi);
}

// ------------------------------------------------------------ KIVI cache
// Main-cache layout: P = batch x kv heads sequences, each with room for
// group_cap groups of 32 tokens; one 3072-byte block per (P, group).  The
// score kernel reads the key half and the PV kernel the value half, each
// with one 16-byte and one 8-byte load per lane:
//   [0, 1024)     key codes, lane l (kq = l / 16, r = l % 16): dwords
//                 D[2 tile + cs / 2] hold token 16 tile + r, channels
//                 32 kq + 8 cs + j (j < 8): code (cs, j) at bit
//                 16 (cs % 2) + 2 j, so the codes of channels j = 2p, 2p + 1
//                 (one MFMA operand dword) form nibble 4 (cs % 2) + p.
//   [1024, 2048)  value codes, lane l: nibble nb (bits 4 nb .. 4 nb + 3) of
//                 dword w holds channel 16 r8 + r, r8 = 2 w + nb / 4, of
//                 tokens 8 kq + 2 (nb % 4) (bits 4 nb, 4 nb + 1) and the one
//                 after it (bits 4 nb + 2, 4 nb + 3).
//   [2048, 2560)  key scale / zero point, fp16 [128 channels][2]: lane l's
//                 8 bytes are channels 2 l and 2 l + 1.
//   [2560, 3072)  value scale / zero point, fp16: lane l's 8 bytes are the
//                 (scale, zero point) of tokens 2 tp and 2 tp + 1,
//                 tp = 4 (l / 16) + l % 4, in channel group (l / 4) % 4.
// Residual window: keys and values bf16 [P][RES_CAP][128]; slot s holds the
// token at position n_main + s.
// Cache state (device int32[4]): {tokens in the main cache, residual slots
// filled, completion counter of the advance kernel, unused}.
//
// Attention follows the reference's eager chain (transformers'
// eager_attention_forward over the dequantized cache) rounding for rounding:
// scores bf16(bf16(q . k) * scale), probabilities bf16(exp(s - M) * (1 / L))
// from the float32 softmax over every position, values as dequantize rounds
// them (bf16(bf16(code - zero_point) * scale)), and the PV product of those
// bf16 operands accumulated in float32 and rounded once.  Only summation
// orders differ.  That takes two passes over the cache: the score kernel
// (key halves) writes every score and a (max, sum) per split; the PV kernel
// (value halves) reduces those to the softmax's M and L, forms each
// probability and multiplies it into the values; the combine adds the
// splits and the residual window.
// Workspace (float words, in this order): ml [P][splits_cap + 1][GQA][2]
// (max and sum of exp(s - max) over a split's scores; index splits_cap is the
// residual window), po [P][splits_cap][GQA][128] (a split's share of the
// output, already divided by L), sc bf16 [P][GQA][t_stride] (scores: main
// token t at t, residual slot s at group_cap * 32 + s).
constexpr int GROUP_BYTES = 3072;
constexpr int SPLIT_WAVES = 8;
constexpr int GROUPS_PER_WAVE = 2;
constexpr int GROUPS_PER_SPLIT = SPLIT_WAVES * GROUPS_PER_WAVE;
constexpr int GROUPS_PER_CHUNK = RES_CAP / KV_GROUP;  // groups a fold appends
static_assert(RES_CAP == SPLIT_WAVES * 16, "one 16-slot tile of the residual window per wave");

struct KiviArgs {
  const uint16_t* qkv;
  int64_t qkv_ld;
  const uint16_t* rope;  // [2][max_pos][128] bf16 cos / sin
  int64_t max_pos;
  uint8_t* main;
  int64_t group_cap;
  uint16_t* kr;
  uint16_t* vr;
  int32_t* state;  // written by the combine's last workgroup when advancing
  int32_t nkv, nq, splits_cap;
  float scale;  // softmax scale (1 / sqrt(head_dim))
  float* ml;
  float* po;
  uint16_t* sc;
  int64_t t_stride;
  int32_t advance;
  vh_format sf;  // fold: scale / zero-point map
  vh_format cf;  // fold: code map
};

// The device state is what the kernels index with: anything out of range
// (which a caller's corrupted state could hold) stops them before any
// access, and the combine flags it.
VH_DEV bool state_ok(const KiviArgs& a, int n_main, int n_res) {
  return n_main >= 0 && n_main % KV_GROUP == 0 && n_main / KV_GROUP <= a.group_cap && n_res >= 0 &&
         n_res < RES_CAP && (int64_t)n_main + n_res < a.max_pos;
}

// Two scores as eager attention forms them: q . k rounded to bf16 (the bf16
// matmul), times the float32 scale, rounded to bf16 again
// (eager_attention_forward: matmul(q, k^T) * scaling); each rounding done
// for both by one packed conversion.  Returns the bf16 pair (qk0 low).
VH_DEV uint32_t eager_scores_x2(float qk0, float qk1, float scale) {
  const uint32_t t = f2bf2_hw(qk0, qk1);
  return f2bf2_hw(__uint_as_float(t << 16) * scale, __uint_as_float(t & 0xffff0000u) * scale);
}

VH_DEV float lo_bf(uint32_t u) { return __uint_as_float(u << 16); }
VH_DEV float hi_bf(uint32_t u) { return __uint_as_float(u & 0xffff0000u); }

// e**x in float32 to about an ulp, as the softmax's float32 exp: x log2(e)
// is carried as y + ylo (an fma recovers the product's rounding error), then
// 2**y (v_exp_f32) times 1 + ylo ln 2.  With the product rounded to float32
// alone the exponent would be off by up to |x| 2**-24, which moves one
// bf16-rounded probability in a few thousand.
VH_DEV float exp_acc(float x) {
  constexpr float L2E = 1.44269502162933349609375f;   // float32(log2 e)
  constexpr float L2E_LO = 1.925963033500011079e-8f;  // log2 e - L2E
  constexpr float LN2 = 0.693147180559945309f;
  if (x < -104.0f) return 0.0f;  // below the smallest float32 subnormal, and -inf
  const float y = x * L2E;
  const float ylo = fmaf(x, L2E_LO, fmaf(x, L2E, -y));
  const float e = __builtin_amdgcn_exp2f(y);
  return fmaf(e, ylo * LN2, e);
}

VH_DEV float pick4(float v0, float v1, float v2, float v3, int r) {
  return r == 0 ? v0 : (r == 1 ? v1 : (r == 2 ? v2 : v3));
}

// The softmax's maximum M and 1 / L, L = sum of exp(s - M) over every
// position, for head h of sequence P, from the per-split (max, sum) partials
// of the live splits and the residual window.  The PV kernel and the combine
// both reduce them in this one order, so their probabilities agree bit for
// bit.  1 / L is the correctly rounded reciprocal; the probability is then
// e * (1 / L), as the float32 softmax scales its exponentials.
struct SoftmaxTotals {
  float M, rcpL;
};

// The partials of head h: the first ML_PRE splits' and the residual
// window's, loaded (with no predicate: every slot is allocated, a split past
// the capacity re-reads the last) before the kernel reads the state.
constexpr int ML_PRE = 16;
struct MlPre {
  float2 v[ML_PRE];
  float2 r;
};

VH_DEV const float* ml_head(const KiviArgs& a, int P, int h) {
  return a.ml + (int64_t)P * (a.splits_cap + 1) * GQA * 2 + h * 2;
}

VH_DEV MlPre ml_preload(const KiviArgs& a, int P, int h) {
  const float* ml = ml_head(a, P, h);
  MlPre m;
#pragma unroll
  for (int s = 0; s < ML_PRE; ++s)
    m.v[s] = *(const float2*)(ml + (int64_t)(s < a.splits_cap ? s : a.splits_cap - 1) * GQA * 2);
  m.r = *(const float2*)(ml + (int64_t)a.splits_cap * GQA * 2);
  return m;
}

VH_DEV SoftmaxTotals softmax_totals(const KiviArgs& a, const MlPre& pre, int P, int splits, int h) {
  const float* ml = ml_head(a, P, h);
  auto part = [&](int s) { return s < ML_PRE ? pre.v[s] : *(const float2*)(ml + (int64_t)s * GQA * 2); };
  float M = pre.r.x;
#pragma unroll
  for (int s = 0; s < ML_PRE; ++s)
    if (s < splits) M = fmaxf(M, pre.v[s].x);
  for (int s = ML_PRE; s < splits; ++s) M = fmaxf(M, part(s).x);
  float L = 0.0f;
#pragma unroll
  for (int s = 0; s < ML_PRE; ++s)
    if (s < splits) L = fmaf(pre.v[s].y, exp_acc(pre.v[s].x - M), L);
  for (int s = ML_PRE; s < splits; ++s) {
    const float2 p = part(s);
    L = fmaf(p.y, exp_acc(p.x - M), L);
  }
  L = fmaf(pre.r.y, exp_acc(pre.r.x - M), L);
  return {M, 1.0f / L};
}

VH_DEV uint16_t rope1(const uint16_t* base, const uint16_t* cs, const uint16_t* sn, int c) {
  const float x = bf2f(base[c]);
  const float xr = c < HEAD_DIM / 2 ? -bf2f(base[c + HEAD_DIM / 2]) : bf2f(base[c - HEAD_DIM / 2]);
  return (uint16_t)f2bf(rbf(x * bf2f(cs[c])) + rbf(xr * bf2f(sn[c])));
}

// lane l and lane l ^ 16 (l ^ 32)
VH_DEV float sum_x16(float v) { return v + __shfl_xor(v, 16); }
VH_DEV float sum_x32(float v) { return v + __shfl_xor(v, 32); }
VH_DEV float max_x16(float v) { return fmaxf(v, __shfl_xor(v, 16)); }
VH_DEV float max_x32(float v) { return fmaxf(v, __shfl_xor(v, 32)); }

// Pair tables.  Keys and values are both dequantized through LDS tables of
// every MFMA operand dword a group can hold: for a pair of elements that
// share an operand dword (two channels of a token for keys, two tokens of a
// channel for values) and each of the 16 pairs of codes, the bf16 pair of
// dequantized elements -- (code - zero_point) * scale, each bfloat16 op
// rounding its result as the reference's dequantize does
// (ops/quantized.py:518-571).  An operand dword is then one 32-bit LDS read
// at its pair's table + 4 * nibble.  Table (row q, block kq) sits at byte
// 272 q + 64 kq of the wave's 256-byte-aligned tables (16 rows); lane l
// builds table (l % 16, l / 16).  The low address byte before the row
// offset, 64 kq + 4 * nibble, is one byte of a precomputed word
// (KeyNibbles), so an address is one v_perm_b32 of that word and the
// table's base, and the row offset is the read's immediate.  The four blocks
// a read touches fall in distinct LDS banks, and so do the 16 rows a
// quarter-wave writes (the 16-byte skew of the 272-byte rows).
// Keys: row 4 cs + p, block kq holds channels 32 kq + 8 cs + 2p, +1.
// Values: row 4 cg + p, block kq holds tokens 2 tp, 2 tp + 1 (tp = 4 kq + p)
// in channel group cg.
constexpr int PAIR_TAB = 16 * 4;
constexpr int KEY_TAB_ROW = 4 * PAIR_TAB + 16;
constexpr int KEY_TAB_BYTES = 16 * KEY_TAB_ROW;
static_assert(KEY_TAB_BYTES % 256 == 0, "every wave's table 256-byte aligned");

// The two words whose bytes are 64 kq + 4 * nibble for the even (lo) and
// odd (hi) nibbles of a code dword D: nibble 2 b in byte b of lo, 2 b + 1
// in byte b of hi.
struct KeyNibbles {
  uint32_t lo, hi;
};

VH_DEV KeyNibbles key_nibbles(uint32_t D, uint32_t kq_bytes) {
  return {((D << 2) & 0x3c3c3c3cu) | kq_bytes, ((D >> 2) & 0x3c3c3c3cu) | kq_bytes};
}

// LDS address of nibble `nib` (0-7) of D in the table at `base` (256-byte
// aligned); the pair's row offset goes into the read's immediate.
VH_DEV uint32_t key_entry_addr(const KeyNibbles& kn, int nib, uint32_t base) {
  const uint32_t sel = (uint32_t)(nib >> 1) | 0x07060500u;
  return __builtin_amdgcn_perm(base, (nib & 1) ? kn.hi : kn.lo, sel);
}

VH_DEV uint32_t lds_u32(uint32_t addr) {
  return *(const __attribute__((address_space(3))) uint32_t*)(uintptr_t)addr;
}

// One pair of elements from their fp16 (scale, zero point) pairs [s0, z0,
// s1, z1]: the 16 entries (every code pair c0 + 4 c1) at dst, element 0's
// value of c0 in the low half, element 1's of c1 in the high half.
VH_DEV void build_pair_table(const uint2& prm, uint8_t* dst) {
  const f16x2 e0 = __builtin_bit_cast(f16x2, prm.x), e1 = __builtin_bit_cast(f16x2, prm.y);
  uint32_t v01[2], v23[2];  // per element: values of codes 0, 1 and 2, 3 (bf16 pairs)
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const float sc = (float)(q ? e1[0] : e0[0]), zp = (float)(q ? e1[1] : e0[1]);
    const uint32_t t01 = f2bf2_hw(0.0f - zp, 1.0f - zp), t23 = f2bf2_hw(2.0f - zp, 3.0f - zp);
    v01[q] = f2bf2_hw(__uint_as_float(t01 << 16) * sc, __uint_as_float(t01 & 0xffff0000u) * sc);
    v23[q] = f2bf2_hw(__uint_as_float(t23 << 16) * sc, __uint_as_float(t23 & 0xffff0000u) * sc);
  }
  uint32_t ent[16];
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const int c0 = v & 3, c1 = v >> 2;
    // bytes 0-3 of the selection: element 0's value of c0 (low), element 1's of c1 (high)
    const uint32_t lo = c0 < 2 ? v01[0] : v23[0], hi = c1 < 2 ? v01[1] : v23[1];
    const uint32_t sl = (uint32_t)(2 * (c0 & 1)), sh = (uint32_t)(4 + 2 * (c1 & 1));
    ent[v] = __builtin_amdgcn_perm(hi, lo, sl | (sl + 1) << 8 | sh << 16 | (sh + 1) << 24);
  }
#pragma unroll
  for (int k = 0; k < 4; ++k)
    *(uint4*)(dst + 16 * k) = make_uint4(ent[4 * k], ent[4 * k + 1], ent[4 * k + 2], ent[4 * k + 3]);
}

VH_DEV uint8_t* pair_table_slot(uint8_t* tab, int lane) {
  return tab + (lane & 15) * KEY_TAB_ROW + (lane >> 4) * PAIR_TAB;
}

// Orders a wave's LDS table writes before its reads of them by other lanes.
VH_DEV void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// The wave's (max, sum of exp(s - max)) over its scores for the head of its
// lane's column, merged by the workgroup and written as split `slot` of the
// partials.  Lane (kq, n) holds sc[i][j] for token j of its quarter in its
// i-th of ng groups; the four column replicas of a head (n / 4) hold the same
// scores, so replica cg sums only the tokens j % 4 == cg.
template <int NG>
VH_DEV void split_totals(const KiviArgs& a, int P, int slot, const float (&sc)[NG][8], const bool (&live)[NG][8],
                         float (*s_ml)[GQA][2]) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n = lane & 15, cg = n >> 2;
  float m = -__builtin_inff();
#pragma unroll
  for (int i = 0; i < NG; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (live[i][j]) m = fmaxf(m, sc[i][j]);
  m = max_x32(max_x16(m));
  float l = 0.0f;
#pragma unroll
  for (int i = 0; i < NG; ++i)
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const float s = pick4(sc[i][4 * t], sc[i][4 * t + 1], sc[i][4 * t + 2], sc[i][4 * t + 3], cg);
      const bool ok = cg == 0 ? live[i][4 * t] : cg == 1 ? live[i][4 * t + 1] : cg == 2 ? live[i][4 * t + 2]
                                                                                        : live[i][4 * t + 3];
      if (ok) l += exp_acc(s - m);
    }
  l += __shfl_xor(l, 4);
  l += __shfl_xor(l, 8);
  l = sum_x32(sum_x16(l));
  if (lane < GQA) {
    s_ml[wave][lane][0] = m;
    s_ml[wave][lane][1] = l;
  }
  __syncthreads();
  if (tid < GQA) {
    float M = -__builtin_inff();
#pragma unroll
    for (int w = 0; w < SPLIT_WAVES; ++w) M = fmaxf(M, s_ml[w][tid][0]);
    float L = 0.0f;
#pragma unroll
    for (int w = 0; w < SPLIT_WAVES; ++w)
      if (s_ml[w][tid][0] != -__builtin_inff()) L = fmaf(s_ml[w][tid][1], exp_acc(s_ml[w][tid][0] - M), L);
    float* out = a.ml + (((int64_t)P * (a.splits_cap + 1) + slot) * GQA + tid) * 2;
    out[0] = M;
    out[1] = L;
  }
}

// Score pass.  Workgroups (split, P) with split < splits_cap stream the
// main cache's key halves: wave w takes groups GROUPS_PER_SPLIT split +
// SPLIT_WAVES i + w (i < GROUPS_PER_WAVE); splits past the cache's groups
// return at once, so one launch shape serves every cache length up to the
// capacity.  Workgroup split == splits_cap takes the residual window: its
// n_res cached keys and this step's key (RoPE'd from the qkv row), which it
// appends, with this step's value, at residual slot n_res.
// MFMA column n = 4 cg + h repeats query head h in the four columns
// n % 4 == h, so every lane holds its own head's scores: S[tile][r] is the
// score of token 16 tile + 4 kq + r.
__global__ void __launch_bounds__(SPLIT_WAVES * 64) k_kivi_scores(KiviArgs a) {
  static_assert(GQA * HEAD_DIM == SPLIT_WAVES * 64, "one rotated query element per thread");
  __shared__ __attribute__((aligned(256))) uint8_t s_tab[SPLIT_WAVES][KEY_TAB_BYTES];
  __shared__ __attribute__((aligned(16))) uint16_t s_q[GQA][HEAD_DIM];
  __shared__ __attribute__((aligned(16))) uint16_t s_newk[HEAD_DIM];
  __shared__ float s_ml[SPLIT_WAVES][GQA][2];
  const int split = blockIdx.x, P = blockIdx.y;
  const bool residual = split == a.splits_cap;
  const int g_begin = split * GROUPS_PER_SPLIT;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n = lane & 15, kq = lane >> 4, hq = n & 3;
  const uint32_t kq_bytes = (uint32_t)kq * 0x40404040u;  // 64 kq in every byte: the table block
  const int b = P / a.nkv, kvh = P % a.nkv;
  const uint16_t* row = a.qkv + (int64_t)b * a.qkv_ld;
  // The state is read first and used only after every load whose address
  // does not depend on it is out: the query's elements and this wave's key
  // blocks (groups clamped into the capacity: a group past the cache's is
  // read from allocated memory and skipped), or the residual window's rows.
  const int2 st = *(const int2*)a.state;
  const int qh = tid / HEAD_DIM, qc = tid % HEAD_DIM;  // the query element this thread rotates
  const uint16_t* qrow = row + (kvh * GQA + qh) * HEAD_DIM;
  uint32_t qv = qrow[qc], qp = qrow[qc < HEAD_DIM / 2 ? qc + HEAD_DIM / 2 : qc - HEAD_DIM / 2];
  uint4 kc[GROUPS_PER_WAVE];
  uint2 kp[GROUPS_PER_WAVE];
  uint4 k4[4];  // the residual window: slot 16 wave + n, channels 32 kq + 8 cs + [0, 8)
  if (!residual) {
    const uint8_t* seq = a.main + (int64_t)P * a.group_cap * GROUP_BYTES;
#pragma unroll
    for (int i = 0; i < GROUPS_PER_WAVE; ++i) {
      const int g = g_begin + i * SPLIT_WAVES + wave;
      const uint8_t* blk = seq + (int64_t)(g < a.group_cap ? g : a.group_cap - 1) * GROUP_BYTES;
      kp[i] = *(const uint2*)(blk + 2048 + lane * 8);
      kc[i] = *(const uint4*)(blk + lane * 16);
    }
  } else {
    const uint4* src = (const uint4*)(a.kr + ((int64_t)P * RES_CAP + 16 * wave + n) * HEAD_DIM + 32 * kq);
#pragma unroll
    for (int cs = 0; cs < 4; ++cs) k4[cs] = src[cs];
  }
  asm volatile("" ::: "memory");
  const int n_main = st.x, n_res = st.y;
  const int G = n_main / KV_GROUP;
  if (!state_ok(a, n_main, n_res) || (!residual && g_begin >= G)) return;
  int ng = 0;
#pragma unroll
  for (int i = 0; i < GROUPS_PER_WAVE; ++i) ng += g_begin + i * SPLIT_WAVES + wave < G ? 1 : 0;
  const int pos = n_main + n_res;
  const uint16_t* cs_ = a.rope + (int64_t)pos * HEAD_DIM;
  const uint16_t* sn_ = a.rope + (a.max_pos + pos) * HEAD_DIM;
  uint32_t qcs = cs_[qc], qsn = sn_[qc];
  // waits for the query alone; the blocks stay in flight across the barrier
  asm volatile("" : "+v"(qv), "+v"(qp), "+v"(qcs), "+v"(qsn)::"memory");
  {
    const float x = bf2f(qv), xr = qc < HEAD_DIM / 2 ? -bf2f(qp) : bf2f(qp);
    s_q[qh][qc] = (uint16_t)f2bf(rbf(x * bf2f(qcs)) + rbf(xr * bf2f(qsn)));
  }
  if (residual && tid < HEAD_DIM) {
    // this step's key (after RoPE) and value enter residual slot n_res
    const uint16_t kn = rope1(row + (a.nq + kvh) * HEAD_DIM, cs_, sn_, tid);
    const uint16_t vn = row[(a.nq + a.nkv + kvh) * HEAD_DIM + tid];
    s_newk[tid] = kn;
    a.kr[((int64_t)P * RES_CAP + n_res) * HEAD_DIM + tid] = kn;
    a.vr[((int64_t)P * RES_CAP + n_res) * HEAD_DIM + tid] = vn;
  }
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");

  // key B operands: q[head hq][32 kq + 8 cs + j], the same in the four columns of a head
  bf16x8 Bq[4];
#pragma unroll
  for (int cs = 0; cs < 4; ++cs) Bq[cs] = __builtin_bit_cast(bf16x8, *(const uint4*)&s_q[hq][32 * kq + 8 * cs]);
  uint16_t* sc_head = a.sc + ((int64_t)P * GQA + hq) * a.t_stride;

  if (residual) {
    // wave w: residual slots 16 w + r (loaded above); slot n_res is this step's key, from LDS
    const int slot = 16 * wave + n;
    if (slot == n_res) {
#pragma unroll
      for (int cs = 0; cs < 4; ++cs) k4[cs] = *(const uint4*)&s_newk[32 * kq + 8 * cs];
    }
    f32x4 S = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int cs = 0; cs < 4; ++cs) S = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, k4[cs]),
                                                                              Bq[cs], S, 0, 0, 0);
    const uint32_t u0 = eager_scores_x2(S[0], S[1], a.scale), u1 = eager_scores_x2(S[2], S[3], a.scale);
    const int s0 = 16 * wave + 4 * kq;  // slots s0 .. s0 + 3
    if (n < GQA) *(uint2*)(sc_head + a.group_cap * KV_GROUP + s0) = make_uint2(u0, u1);
    float sc[1][8];
    bool live[1][8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      sc[0][j] = j < 4 ? (j & 1 ? hi_bf(j < 2 ? u0 : u1) : lo_bf(j < 2 ? u0 : u1)) : 0.0f;
      live[0][j] = j < 4 && s0 + j <= n_res;
    }
    split_totals<1>(a, P, a.splits_cap, sc, live, s_ml);
    return;
  }

  float sc[GROUPS_PER_WAVE][8];
  bool live[GROUPS_PER_WAVE][8];
  // one group (i constant at each call: the block registers stay unindexed)
  auto group = [&](const int i) __attribute__((always_inline)) {
    const int g = g_begin + i * SPLIT_WAVES + wave;
    // this group's key table, lane l the pair of channels 2 l, 2 l + 1 (the
    // previous group's reads precede these writes in the wave's LDS order)
    build_pair_table(kp[i], pair_table_slot(s_tab[wave], lane));
    wave_lds_sync();
    // scores: S[tile][r] = q[head hq] . k[token 16 tile + 4 kq + r]; operand
    // dword p of channel chunk cs is the table entry of its code nibble
    const uint32_t tab = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t*)s_tab[wave];
    f32x4 S[2] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
    const uint32_t kd[4] = {kc[i].x, kc[i].y, kc[i].z, kc[i].w};
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2) {
        const KeyNibbles kn = key_nibbles(kd[2 * t + h2], kq_bytes);
#pragma unroll
        for (int c2 = 0; c2 < 2; ++c2) {
          const int cs = 2 * h2 + c2;
          uint32_t w[4];
#pragma unroll
          for (int p = 0; p < 4; ++p) w[p] = lds_u32(key_entry_addr(kn, 4 * c2 + p, tab) + (4 * cs + p) * KEY_TAB_ROW);
          S[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              __builtin_bit_cast(bf16x8, make_uint4(w[0], w[1], w[2], w[3])), Bq[cs], S[t], 0, 0, 0);
        }
      }
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const uint32_t u0 = eager_scores_x2(S[t][0], S[t][1], a.scale), u1 = eager_scores_x2(S[t][2], S[t][3], a.scale);
      if (n < GQA) *(uint2*)(sc_head + (int64_t)g * KV_GROUP + 16 * t + 4 * kq) = make_uint2(u0, u1);
      sc[i][4 * t] = lo_bf(u0);
      sc[i][4 * t + 1] = hi_bf(u0);
      sc[i][4 * t + 2] = lo_bf(u1);
      sc[i][4 * t + 3] = hi_bf(u1);
    }
  };
  static_assert(GROUPS_PER_WAVE == 2, "two group calls");
#pragma unroll
  for (int i = 0; i < GROUPS_PER_WAVE; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      sc[i][j] = 0.0f;
      live[i][j] = i < ng;
    }
  if (ng > 0) group(0);
  if (ng > 1) group(1);
  split_totals<GROUPS_PER_WAVE>(a, P, split, sc, live, s_ml);
}

// PV pass.  Workgroups (split, P) as the score pass's main splits, over the
// value halves: each wave's groups, probabilities bf16(exp(s - M) * (1 / L))
// from the scores and the softmax totals, times the values (pair tables),
// on v_mfma_f32_16x16x32_bf16: A = values (row = channel of a 16-channel
// tile, k = token), B = probabilities (column n = head n % 4; the
// replicas are ignored).  The waves add their outputs through LDS and the
// workgroup writes its split's share of the output.
__global__ void __launch_bounds__(SPLIT_WAVES * 64) k_kivi_pv(KiviArgs a) {
  __shared__ __attribute__((aligned(256))) uint8_t s_tab[SPLIT_WAVES][KEY_TAB_BYTES];
  __shared__ __attribute__((aligned(16))) uint16_t s_p[SPLIT_WAVES][GQA][KV_GROUP];
  static_assert(sizeof(float) * SPLIT_WAVES * GQA * HEAD_DIM <= sizeof(s_tab), "outputs reuse the tables");
  const int split = blockIdx.x, P = blockIdx.y;
  const int g_begin = split * GROUPS_PER_SPLIT;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n = lane & 15, kq = lane >> 4;
  const uint32_t kq_bytes = (uint32_t)kq * 0x40404040u;
  const int hp = lane >> 4, tp = lane & 15;  // this lane's probabilities: head hp, tokens 2 tp, 2 tp + 1
  // the state is used only after the value blocks, the scores and the
  // partials are out (groups clamped into the capacity, as the score pass)
  const int2 st = *(const int2*)a.state;
  uint4 vc[GROUPS_PER_WAVE];
  uint2 vp[GROUPS_PER_WAVE];
  uint32_t sp[GROUPS_PER_WAVE];
  const uint8_t* seq = a.main + (int64_t)P * a.group_cap * GROUP_BYTES;
  const uint16_t* sc_head = a.sc + ((int64_t)P * GQA + hp) * a.t_stride;
#pragma unroll
  for (int i = 0; i < GROUPS_PER_WAVE; ++i) {
    const int g = g_begin + i * SPLIT_WAVES + wave;
    const int gl = g < a.group_cap ? g : a.group_cap - 1;
    const uint8_t* blk = seq + (int64_t)gl * GROUP_BYTES;
    vp[i] = *(const uint2*)(blk + 2560 + lane * 8);
    vc[i] = *(const uint4*)(blk + 1024 + lane * 16);
    sp[i] = *(const uint32_t*)(sc_head + (int64_t)gl * KV_GROUP + 2 * tp);
  }
  const MlPre pre = ml_preload(a, P, hp);
  asm volatile("" ::: "memory");
  const int n_main = st.x, n_res = st.y;
  const int G = n_main / KV_GROUP;
  if (!state_ok(a, n_main, n_res) || g_begin >= G) return;
  const int splits = (G + GROUPS_PER_SPLIT - 1) / GROUPS_PER_SPLIT;
  int ng = 0;
#pragma unroll
  for (int i = 0; i < GROUPS_PER_WAVE; ++i) ng += g_begin + i * SPLIT_WAVES + wave < G ? 1 : 0;
  const SoftmaxTotals tot = softmax_totals(a, pre, P, splits, hp);
  f32x4 acc[8];
#pragma unroll
  for (int r8 = 0; r8 < 8; ++r8) acc[r8] = {0.0f, 0.0f, 0.0f, 0.0f};
  auto group = [&](const int i) __attribute__((always_inline)) {
    build_pair_table(vp[i], pair_table_slot(s_tab[wave], lane));
    const float p0 = exp_acc(lo_bf(sp[i]) - tot.M) * tot.rcpL, p1 = exp_acc(hi_bf(sp[i]) - tot.M) * tot.rcpL;
    *(uint32_t*)&s_p[wave][hp][2 * tp] = f2bf2_hw(p0, p1);
    wave_lds_sync();
    const bf16x8 B = __builtin_bit_cast(bf16x8, *(const uint4*)&s_p[wave][n & 3][8 * kq]);
    const uint32_t tab = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t*)s_tab[wave];
    const uint32_t vw[4] = {vc[i].x, vc[i].y, vc[i].z, vc[i].w};
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const KeyNibbles kn = key_nibbles(vw[w], kq_bytes);
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        uint32_t A[4];
#pragma unroll
        for (int p = 0; p < 4; ++p) A[p] = lds_u32(key_entry_addr(kn, 4 * half + p, tab) + (4 * w + p) * KEY_TAB_ROW);
        acc[2 * w + half] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            __builtin_bit_cast(bf16x8, make_uint4(A[0], A[1], A[2], A[3])), B, acc[2 * w + half], 0, 0, 0);
      }
    }
  };
  static_assert(GROUPS_PER_WAVE == 2, "two group calls");
  if (ng > 0) group(0);
  if (ng > 1) group(1);
  __syncthreads();  // every wave is done with its tables
  float(*s_o)[GQA][HEAD_DIM] = reinterpret_cast<float(*)[GQA][HEAD_DIM]>(&s_tab[0][0]);
  // lane (kq, n < 4): head n, channels 16 r8 + 4 kq + r
  if (n < GQA) {
#pragma unroll
    for (int r8 = 0; r8 < 8; ++r8)
      *(f32x4*)&s_o[wave][n][16 * r8 + 4 * kq] = acc[r8];
  }
  __syncthreads();
  const int h = tid >> 7, c = tid & (HEAD_DIM - 1);
  float O = 0.0f;
#pragma unroll
  for (int w = 0; w < SPLIT_WAVES; ++w) O += s_o[w][h][c];
  a.po[(((int64_t)P * a.splits_cap + split) * GQA + h) * HEAD_DIM + c] = O;
}

// Writes one group block from codes (bytes 0..3) and bf16 scale / zero
// point values: keys kcode[t * kstride + ch] (32 tokens), key parameters
// ks / kz [ch]; values vcode[t * vstride + ch], value parameters
// vs / vz[t * 4 + cg].  Thread `lane` writes its 48 bytes.
VH_DEV void write_group(const uint8_t* kcode, int64_t kstride, const uint16_t* ks, const uint16_t* kz,
                        const uint8_t* vcode, int64_t vstride, const uint16_t* vs, const uint16_t* vz, int lane,
                        uint8_t* blk) {
  const int kq = lane >> 4, r = lane & 15;
  uint32_t D[4] = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int cs = 0; cs < 4; ++cs)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint32_t code = kcode[(int64_t)(16 * t + r) * kstride + 32 * kq + 8 * cs + j] & 3u;
        D[2 * t + (cs >> 1)] |= code << (16 * (cs & 1) + 2 * j);
      }
  *(uint4*)(blk + lane * 16) = make_uint4(D[0], D[1], D[2], D[3]);
  uint32_t V[4] = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int w = 0; w < 4; ++w)
#pragma unroll
    for (int nb = 0; nb < 8; ++nb)
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int ch = 16 * (2 * w + (nb >> 2)) + r, tok = 8 * kq + 2 * (nb & 3) + u;
        const uint32_t code = vcode[(int64_t)tok * vstride + ch] & 3u;
        V[w] |= code << (4 * nb + 2 * u);
      }
  *(uint4*)(blk + 1024 + lane * 16) = make_uint4(V[0], V[1], V[2], V[3]);
  // parameters: lanes 0-31 four key channels each, lanes 32-63 the value
  // records of reader lanes 2 i and 2 i + 1
  _Float16 piece[8];
  if (lane < 32) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      piece[2 * k] = (_Float16)bf2f(ks[4 * lane + k]);
      piece[2 * k + 1] = (_Float16)bf2f(kz[4 * lane + k]);
    }
  } else {
    const int i = lane - 32;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int l = 2 * i + e, tp = 4 * (l >> 4) + (l & 3), cg = (l >> 2) & 3;
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int tok = 2 * tp + u;
        piece[4 * e + 2 * u] = (_Float16)bf2f(vs[tok * 4 + cg]);
        piece[4 * e + 2 * u + 1] = (_Float16)bf2f(vz[tok * 4 + cg]);
      }
    }
  }
  *(f16x8*)(blk + 2048 + lane * 16) = *(const f16x8*)piece;
}

// quantize_affine of one 32-element block in bfloat16 with quant range
// [0, 3] and a scale map (ops/quantized.py:1262-1281): scale = (max - min)
// / 3, 1 where not positive, mapped, 1 where not positive; zero point =
// -min / scale + 0, mapped.
struct Affine {
  float s, zp;
};

VH_DEV Affine kivi_affine(float lo, float hi, const vh_format& sf) {
  float s = div_bf16(rbf(hi - lo), 3.0f);
  if (!(s > 0.0f)) s = 1.0f;
  s = fmt_value(f2bf(s), sf, nullptr);
  if (!(s > 0.0f)) s = 1.0f;
  float zp = rbf(div_bf16(-lo, s) + 0.0f);
  zp = fmt_value(f2bf(zp), sf, nullptr);
  return {s, zp};
}

// The code of x in its block: map(bf16(bf16(x / scale) + zero_point)),
// a byte 0..3; a NaN code (not representable in the packed cache) flags.
VH_DEV uint8_t kivi_code(float x, const Affine& af, const vh_format& cf, int* bad) {
  const float q = rbf(div_bf16(x, af.s) + af.zp);
  const float c = fmt_value(f2bf(q), cf, nullptr);
  if (isnan_f(c)) {
    *bad = 1;
    return 0;
  }
  return (uint8_t)(int)c;
}

// The fold of a completed chunk for sequence P: the RES_CAP residual tokens
// quantized with the KIVI specs (quantize_affine: keys grouped along tokens,
// values along channels, group 32) into groups [g0, g0 + GROUPS_PER_CHUNK)
// of the main cache -- what a lowered decode graph stores for a completed
// chunk (codegen/transform/quant_folding.py:1994-2065, 2634-2700).  The
// residual's last slot was written by this step's score pass.  All threads
// of the workgroup; returns with them synchronised.
struct FoldLds {
  uint8_t kc[RES_CAP][HEAD_DIM];
  uint8_t vc[RES_CAP][HEAD_DIM];
  uint16_t ks[GROUPS_PER_CHUNK][HEAD_DIM], kz[GROUPS_PER_CHUNK][HEAD_DIM];
  uint16_t vs[RES_CAP][4], vz[RES_CAP][4];
  int bad;
};

VH_DEV void fold_chunk(const KiviArgs& a, int P, int g0, FoldLds& L, int* flag) {
  const int tid = threadIdx.x, nthreads = blockDim.x;
  if (tid == 0) L.bad = 0;
  __syncthreads();
  int bad = 0;
  const uint16_t* K = a.kr + (int64_t)P * RES_CAP * HEAD_DIM;
  const uint16_t* V = a.vr + (int64_t)P * RES_CAP * HEAD_DIM;
  // keys: one column (group, channel) of 32 tokens per pass
  for (int col = tid; col < GROUPS_PER_CHUNK * HEAD_DIM; col += nthreads) {
    const int g = col / HEAD_DIM, ch = col % HEAD_DIM;
    float lo = bf2f(K[g * KV_GROUP * HEAD_DIM + ch]), hi = lo;
    for (int t = 1; t < KV_GROUP; ++t) {
      const float x = bf2f(K[(g * KV_GROUP + t) * HEAD_DIM + ch]);
      lo = nmin(lo, x);
      hi = nmax(hi, x);
    }
    const Affine af = kivi_affine(lo, hi, a.sf);
    L.ks[g][ch] = (uint16_t)f2bf(af.s);
    L.kz[g][ch] = (uint16_t)f2bf(af.zp);
    for (int t = 0; t < KV_GROUP; ++t)
      L.kc[g * KV_GROUP + t][ch] = kivi_code(bf2f(K[(g * KV_GROUP + t) * HEAD_DIM + ch]), af, a.cf, &bad);
  }
  // values: one row (token, channel group) of 32 channels per pass
  for (int row = tid; row < RES_CAP * 4; row += nthreads) {
    const int t = row / 4, cg = row % 4;
    const uint16_t* vt = V + t * HEAD_DIM + cg * KV_GROUP;
    float lo = bf2f(vt[0]), hi = lo;
    for (int c = 1; c < KV_GROUP; ++c) {
      const float x = bf2f(vt[c]);
      lo = nmin(lo, x);
      hi = nmax(hi, x);
    }
    const Affine af = kivi_affine(lo, hi, a.sf);
    L.vs[t][cg] = (uint16_t)f2bf(af.s);
    L.vz[t][cg] = (uint16_t)f2bf(af.zp);
    for (int c = 0; c < KV_GROUP; ++c) L.vc[t][cg * KV_GROUP + c] = kivi_code(bf2f(vt[c]), af, a.cf, &bad);
  }
  if (bad) L.bad = 1;
  __syncthreads();
  // thread (group, lane) writes its 48 bytes of the group's block
  for (int i = tid; i < GROUPS_PER_CHUNK * 64; i += nthreads) {
    const int g = i >> 6, lane = i & 63;
    uint8_t* blk = a.main + ((int64_t)P * a.group_cap + g0 + g) * GROUP_BYTES;
    write_group(&L.kc[g * KV_GROUP][0], HEAD_DIM, L.ks[g], L.kz[g], &L.vc[g * KV_GROUP][0], HEAD_DIM,
                &L.vs[g * KV_GROUP][0], &L.vz[g * KV_GROUP][0], lane, blk);
  }
  if (tid == 0 && L.bad) atomicOr(flag, VH_DECODE_ERR_KV_CODE);
  __syncthreads();
}

// Per (batch, query head): the residual window's share of the output (its
// n_res cached tokens and this step's, appended by the score pass, with the
// probabilities formed as the PV pass forms them), plus the main splits'
// shares; writes the attention output (bf16, the one rounding) and its
// MX-int8 fake quantization.  256 threads: one probability per residual
// slot, then 16 token subsets x 16 channel octets for the products; the
// first 128 (one per channel) add the splits and write.
constexpr int COMBINE_PRELOAD = 16;  // splits whose shares are loaded up front
constexpr int COMBINE_THREADS = 2 * HEAD_DIM;

__global__ void __launch_bounds__(COMBINE_THREADS) k_kivi_combine(KiviArgs a, uint16_t* __restrict__ attn,
                                                                  _Float16* __restrict__ fq, int* __restrict__ flag) {
  __shared__ float s_p[RES_CAP];
  __shared__ float s_o[16][HEAD_DIM];
  __shared__ FoldLds s_fold;
  // Workgroups go to the 8 XCDs round-robin: XCD x takes the contiguous
  // range x * G / 8 + [0, G / 8) of (batch, head) rows when that keeps the
  // GQA heads of a kv head together (G % 32 == 0), so a residual window is
  // read into one XCD's L2 rather than four.
  const int G = (int)gridDim.x;
  const int bid = (int)blockIdx.x;
  const int bh = G % (8 * GQA) == 0 ? (bid & 7) * (G >> 3) + (bid >> 3) : bid;
  const int b = bh / a.nq, H = bh % a.nq, kvh = H / GQA, h = H % GQA;
  const int P = b * a.nkv + kvh, tid = threadIdx.x;
  // the state is read first, its value used only after the loads below are out
  const int2 st = *(const int2*)a.state;
  const int c = tid & (HEAD_DIM - 1);
  const int co = tid & 15, ts = tid >> 4;  // value octet co, token subset ts (slots ts + 16 u)
  // The residual values, the slot's score and the splits' shares go out
  // before the state is read: their addresses do not depend on it (every
  // slot and split is allocated), and what the state leaves unused is
  // masked once it arrives.
  uint4 vw[RES_CAP / 16];
  const uint4* vp = (const uint4*)(a.vr + (int64_t)P * RES_CAP * HEAD_DIM) + co;
#pragma unroll
  for (int u = 0; u < RES_CAP / 16; ++u) vw[u] = vp[(int64_t)(ts + 16 * u) * (HEAD_DIM / 8)];
  const uint16_t sraw = a.sc[((int64_t)P * GQA + h) * a.t_stride + a.group_cap * KV_GROUP + (tid & (RES_CAP - 1))];
  const MlPre pre = ml_preload(a, P, h);
  const float* base = a.po + ((int64_t)P * a.splits_cap * GQA + h) * HEAD_DIM + c;
  float po[COMBINE_PRELOAD];
#pragma unroll
  for (int s = 0; s < COMBINE_PRELOAD; ++s) {
    // no predicate: a split past the capacity re-reads the last one
    const int se = s < a.splits_cap ? s : a.splits_cap - 1;
    po[s] = base[(int64_t)se * GQA * HEAD_DIM];
  }
  asm volatile("" ::: "memory");  // the loads above are issued before the state is used
  const int n_main = st.x, n_res = st.y;
  const int splits = (n_main / KV_GROUP + GROUPS_PER_SPLIT - 1) / GROUPS_PER_SPLIT;
  if (!state_ok(a, n_main, n_res)) {
    if (tid < HEAD_DIM) {
      const int64_t idx = (int64_t)b * a.nq * HEAD_DIM + H * HEAD_DIM + tid;
      if (attn) attn[idx] = 0;
      fq[idx] = (_Float16)0.0f;
    }
    if (bh == 0 && tid == 0) atomicOr(flag, VH_DECODE_ERR_KV_STATE);
    return;
  }
  const SoftmaxTotals tot = softmax_totals(a, pre, P, splits, h);
  if (tid < RES_CAP) s_p[tid] = tid <= n_res ? rbf(exp_acc(bf2f(sraw) - tot.M) * tot.rcpL) : 0.0f;
  // slots past the window hold stale bytes (a zero weight times a stale
  // infinity would be NaN): cleared
#pragma unroll
  for (int u = 0; u < RES_CAP / 16; ++u)
    if (ts + 16 * u > n_res) vw[u] = make_uint4(0u, 0u, 0u, 0u);
  __syncthreads();
  {
    float o8[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int u = 0; u < RES_CAP / 16; ++u) {
      const float pt = s_p[ts + 16 * u];
      const uint32_t ww[4] = {vw[u].x, vw[u].y, vw[u].z, vw[u].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        o8[2 * j] = fmaf(pt, bf2f(ww[j] & 0xffffu), o8[2 * j]);
        o8[2 * j + 1] = fmaf(pt, bf2f(ww[j] >> 16), o8[2 * j + 1]);
      }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) s_o[ts][co * 8 + j] = o8[j];
  }
  __syncthreads();
  if (tid < HEAD_DIM) {
    float O = 0.0f;
#pragma unroll
    for (int s = 0; s < COMBINE_PRELOAD; ++s)
      if (s < splits) O += po[s];
    for (int s = COMBINE_PRELOAD; s < splits; ++s) O += base[(int64_t)s * GQA * HEAD_DIM];
#pragma unroll
    for (int t16 = 0; t16 < 16; ++t16) O += s_o[t16][c];
    const float o = rbf(O);
    const int64_t idx = (int64_t)b * a.nq * HEAD_DIM + H * HEAD_DIM + c;
    if (attn) attn[idx] = (uint16_t)f2bf(o);
    const Mx8Scale scl = mx8_scale(max16(fabsf(o)));
    fq[idx] = fq_half(mx8_fq(o, scl), flag);
  }
  if (!a.advance) return;
  // The cache bookkeeping after the step: when this step filled the
  // residual's last slot, head 0's workgroup of each sequence folds the
  // sequence's chunk into the main cache (no other workgroup writes it, and
  // this step reads no main group at or past g0); then the last workgroup to
  // finish -- every one has read the state by then -- writes the new state.
  // The counter needs no fence: what it orders is every workgroup's state
  // read (consumed, and past the workgroup barriers above, before its
  // increment is issued) before the last one's state write; everything else
  // this kernel writes is read by later launches only, which the kernel
  // boundary orders.  (An agent-scope fence here writes back the XCD's L2 in
  // every workgroup: it cost 2.3 us per step.)
  const bool fold = n_res + 1 == RES_CAP;
  const int g0 = n_main / KV_GROUP;
  const bool room = g0 + GROUPS_PER_CHUNK <= a.group_cap;
  if (fold && room && h == 0) fold_chunk(a, P, g0, s_fold, flag);
  if (tid == 0) {
    if (fold && !room && bh == 0) atomicOr(flag, VH_DECODE_ERR_KV_FULL);
    const int done = __hip_atomic_fetch_add(&a.state[2], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (done == (int)gridDim.x - 1) {
      if (fold && room) {
        a.state[0] = n_main + RES_CAP;
        a.state[1] = 0;
      } else if (!fold) {
        a.state[1] = n_res + 1;
      }
      a.state[2] = 0;
    }
  }
}

// Bake reference-form quantize_affine outputs (codes as bytes, bf16
// parameters) of T tokens into groups [g0, g0 + T / 32) of each sequence:
// one thread per (P, group, lane).
__global__ void __launch_bounds__(256) k_bake_kivi(const uint8_t* __restrict__ kcode, const uint16_t* __restrict__ ks,
                                                   const uint16_t* __restrict__ kz, const uint8_t* __restrict__ vcode,
                                                   const uint16_t* __restrict__ vs, const uint16_t* __restrict__ vz,
                                                   int64_t P, int64_t T, int64_t group_cap, int64_t g0,
                                                   uint8_t* __restrict__ out) {
  const int64_t G = T / KV_GROUP;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= P * G * 64) return;
  const int lane = (int)(t % 64);
  const int64_t g = (t / 64) % G, p = t / (64 * G);
  uint8_t* blk = out + (p * group_cap + g0 + g) * GROUP_BYTES;
  const int64_t tok0 = p * T + g * KV_GROUP;
  write_group(kcode + tok0 * HEAD_DIM, HEAD_DIM, ks + (p * G + g) * HEAD_DIM, kz + (p * G + g) * HEAD_DIM,
              vcode + tok0 * HEAD_DIM, HEAD_DIM, vs + tok0 * 4, vz + tok0 * 4, lane, blk);
}

__global__ void __launch_bounds__(256) k_bake_kivi_residual(const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
                                                            int64_t P, int64_t n, uint16_t* __restrict__ kr,
                                                            uint16_t* __restrict__ vr) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= P * n * HEAD_DIM) return;
  const int c = (int)(i % HEAD_DIM);
  const int s = (int)((i / HEAD_DIM) % n);
  const int64_t p = i / (HEAD_DIM * n);
  kr[(p * RES_CAP + s) * HEAD_DIM + c] = k[i];
  vr[(p * RES_CAP + s) * HEAD_DIM + c] = v[i];
}

inline unsigned blocks_for(int64_t n, int per) { return (unsigned)((n + per - 1) / per); }

}  // namespace

extern "C" int vh_rmsnorm_mx8(const uint16_t* x, const uint16_t* w, int64_t M, int64_t H, float eps, uint16_t* h_out,
                              uint16_t* fq, int32_t* flag, vh_stream_t stream) {
  VH_REQUIRE(x && w && fq && flag, "vh_rmsnorm_mx8: null argument");
  VH_REQUIRE(M >= 1 && H >= 16 && H % 16 == 0, "vh_rmsnorm_mx8: needs M >= 1 and H %% 16 == 0");
  hipLaunchKernelGGL(k_rmsnorm_mx8, dim3((unsigned)M), dim3(256), 0, vh::as_stream(stream), x, w, H, eps, h_out,
                     (_Float16*)fq, (int*)flag);
  return vh::check_launch("vh_rmsnorm_mx8");
}

extern "C" int vh_mx8_bake(const uint8_t* codes, const uint8_t* scale, int32_t scale_bias, int64_t N, int64_t K,
                           int32_t paired, uint8_t* w_codes, uint8_t* w_hb, int32_t* w_shift, int32_t* flag,
                           vh_stream_t stream) {
  VH_REQUIRE(codes && scale && w_codes && w_hb && flag, "vh_mx8_bake: null argument");
  VH_REQUIRE(N > 0 && K > 0 && N % (paired ? 32 : 16) == 0 && K % 256 == 0,
             "vh_mx8_bake: needs N %% 16 == 0 (32 when paired) and K %% 256 == 0");
  hipStream_t s = vh::as_stream(stream);
  if (w_shift)
    hipLaunchKernelGGL(k_mx8_row_shift, dim3(blocks_for(N, 256)), dim3(256), 0, s, codes, scale, (int)scale_bias, N,
                       K, w_shift);
  const int64_t nc = (N / 16) * (K / 64) * 64, ns = (N / 16) * (K / 256) * 32;
  hipLaunchKernelGGL(k_bake_mx8_codes, dim3(blocks_for(nc, 256)), dim3(256), 0, s, codes, N, K, (int)paired, scale,
                     (int)scale_bias, (const int32_t*)w_shift, w_codes);
  hipLaunchKernelGGL(k_bake_mx8_scales, dim3(blocks_for(ns, 256)), dim3(256), 0, s, codes, scale, (int)scale_bias, N,
                     K, (int)paired, (const int32_t*)w_shift, w_hb, (int*)flag);
  return vh::check_launch("vh_mx8_bake");
}

extern "C" int vh_gemv_mx8(const uint16_t* x_fq, int64_t M, int64_t K, const uint8_t* w_codes, const uint8_t* w_hb,
                           int64_t N, int32_t mode, int32_t tiles_per_block, const uint16_t* residual, uint16_t* y,
                           uint16_t* fq_out, const int32_t* row_exp, const int32_t* w_shift, int32_t* flag,
                           vh_stream_t stream) {
  VH_REQUIRE(x_fq && w_codes && w_hb && flag, "vh_gemv_mx8: null argument");
  VH_REQUIRE(M >= 1 && M <= 16, "vh_gemv_mx8: M must be in [1, 16] (got %lld)", (long long)M);
  VH_REQUIRE(K > 0 && K % 256 == 0 && N > 0 && N % 16 == 0, "vh_gemv_mx8: needs K %% 256 == 0 and N %% 16 == 0");
  VH_REQUIRE(((uintptr_t)x_fq % 16) == 0 && ((uintptr_t)w_codes % 16) == 0 && ((uintptr_t)w_hb % 8) == 0,
             "vh_gemv_mx8: misaligned operand");
  GemvArgs a{(const _Float16*)x_fq, (int32_t)M, K, w_codes, w_hb, N, mode, residual, y, (_Float16*)fq_out, (int*)flag,
             row_exp, w_shift};
  hipStream_t s = vh::as_stream(stream);
  const int64_t tiles = N / 16;
  if (mode == VH_GEMV_SWIGLU) {
    VH_REQUIRE(fq_out, "vh_gemv_mx8: SWIGLU needs fq_out");
    // N output columns from 2N baked columns (gate / up tile pairs)
    hipLaunchKernelGGL(k_gemv_mx8<2>, dim3((unsigned)tiles), dim3(GEMV_WAVES * 64), 0, s, a);
    return vh::check_launch("vh_gemv_mx8");
  }
  VH_REQUIRE(mode == VH_GEMV_STORE || mode == VH_GEMV_RESIDUAL, "vh_gemv_mx8: unknown mode %d", mode);
  VH_REQUIRE(y && (mode != VH_GEMV_RESIDUAL || residual), "vh_gemv_mx8: missing y / residual");
  if (tiles_per_block == 2) {
    VH_REQUIRE(tiles % 2 == 0, "vh_gemv_mx8: two tiles per block need N %% 32 == 0");
    hipLaunchKernelGGL(k_gemv_mx8<2>, dim3((unsigned)(tiles / 2)), dim3(GEMV_WAVES * 64), 0, s, a);
  } else {
    VH_REQUIRE(tiles_per_block == 1, "vh_gemv_mx8: tiles_per_block must be 1 or 2");
    hipLaunchKernelGGL(k_gemv_mx8<1>, dim3((unsigned)tiles), dim3(GEMV_WAVES * 64), 0, s, a);
  }
  return vh::check_launch("vh_gemv_mx8");
}

extern "C" int vh_kivi_bake(const uint8_t* k_codes, const uint16_t* k_scale, const uint16_t* k_zp,
                            const uint8_t* v_codes, const uint16_t* v_scale, const uint16_t* v_zp, int64_t P,
                            int64_t T, int64_t group_cap, int64_t g0, uint8_t* main_out, vh_stream_t stream) {
  VH_REQUIRE(k_codes && k_scale && k_zp && v_codes && v_scale && v_zp && main_out, "vh_kivi_bake: null argument");
  VH_REQUIRE(P > 0 && T > 0 && T % KV_GROUP == 0, "vh_kivi_bake: needs T %% 32 == 0");
  VH_REQUIRE(g0 >= 0 && g0 + T / KV_GROUP <= group_cap, "vh_kivi_bake: groups [%lld, %lld) exceed the capacity %lld",
             (long long)g0, (long long)(g0 + T / KV_GROUP), (long long)group_cap);
  const int64_t G = T / KV_GROUP;
  hipLaunchKernelGGL(k_bake_kivi, dim3(blocks_for(P * G * 64, 256)), dim3(256), 0, vh::as_stream(stream), k_codes,
                     k_scale, k_zp, v_codes, v_scale, v_zp, P, T, group_cap, g0, main_out);
  return vh::check_launch("vh_kivi_bake");
}

extern "C" int vh_kivi_bake_residual(const uint16_t* k, const uint16_t* v, int64_t P, int64_t n, uint16_t* kr,
                                     uint16_t* vr, vh_stream_t stream) {
  VH_REQUIRE(k && v && kr && vr, "vh_kivi_bake_residual: null argument");
  VH_REQUIRE(P > 0 && n >= 0 && n <= RES_CAP, "vh_kivi_bake_residual: n must be in [0, %d]", RES_CAP);
  if (n == 0) return VH_OK;
  hipLaunchKernelGGL(k_bake_kivi_residual, dim3(blocks_for(P * n * HEAD_DIM, 256)), dim3(256), 0,
                     vh::as_stream(stream), k, v, P, n, kr, vr);
  return vh::check_launch("vh_kivi_bake_residual");
}

namespace {

// The attention workspace: the (max, sum) partials, the splits' output
// shares and the bf16 scores, each region a multiple of 4 floats.
int64_t kivi_workspace_floats(int64_t P, int64_t group_cap, int64_t* ml_floats, int64_t* po_floats) {
  const int64_t splits_cap = (group_cap + GROUPS_PER_SPLIT - 1) / GROUPS_PER_SPLIT;
  const int64_t t_stride = group_cap * KV_GROUP + RES_CAP;
  auto up4 = [](int64_t v) { return (v + 3) / 4 * 4; };
  *ml_floats = up4(P * (splits_cap + 1) * GQA * 2);
  *po_floats = up4(P * splits_cap * GQA * HEAD_DIM);
  return *ml_floats + *po_floats + up4(P * GQA * t_stride / 2);
}

int kivi_common(const vh_kivi_desc* d, KiviArgs& a) {
  VH_REQUIRE(d && d->main && d->kr && d->vr && d->state && d->flag, "vh_kivi: null argument");
  VH_REQUIRE(d->batch >= 1 && d->nkv >= 1 && d->nq == GQA * d->nkv, "vh_kivi: needs nq == 4 nkv");
  VH_REQUIRE(d->head_dim == HEAD_DIM, "vh_kivi: head_dim must be %d", HEAD_DIM);
  VH_REQUIRE(d->group_cap >= GROUPS_PER_CHUNK, "vh_kivi: the main cache must hold at least one chunk");
  const int64_t splits_cap = (d->group_cap + GROUPS_PER_SPLIT - 1) / GROUPS_PER_SPLIT;
  VH_REQUIRE(splits_cap < 65535 && d->batch * d->nkv <= 65535, "vh_kivi: cache too large");
  VH_REQUIRE(d->qkv && d->rope && d->attn_fq && d->part, "vh_kivi_attention: null argument");
  VH_REQUIRE(d->max_pos >= 1, "vh_kivi_attention: empty RoPE table");
  VH_REQUIRE(d->qkv_ld >= (int64_t)(d->nq + 2 * d->nkv) * HEAD_DIM, "vh_kivi_attention: qkv_ld too small");
  const int64_t P = d->batch * d->nkv;
  const int64_t t_stride = d->group_cap * KV_GROUP + RES_CAP;
  int64_t ml_floats = 0, po_floats = 0;
  const int64_t need = kivi_workspace_floats(P, d->group_cap, &ml_floats, &po_floats);
  VH_REQUIRE(d->part_floats >= need, "vh_kivi_attention: workspace too small (needs %lld floats)", (long long)need);
  VH_REQUIRE((uintptr_t)d->part % 16 == 0, "vh_kivi_attention: misaligned workspace");
  a = KiviArgs{d->qkv, d->qkv_ld, d->rope, d->max_pos, d->main, d->group_cap, d->kr, d->vr, d->state,
               (int32_t)d->nkv, (int32_t)d->nq, (int32_t)splits_cap, d->softmax_scale, d->part,
               d->part + ml_floats, (uint16_t*)(d->part + ml_floats + po_floats), t_stride,
               d->advance ? 1 : 0, d->scale_fmt, d->code_fmt};
  return VH_OK;
}

}  // namespace

extern "C" int vh_kivi_attention(const vh_kivi_desc* d, vh_stream_t stream) {
  KiviArgs a;
  if (int e = kivi_common(d, a)) return e;
  if (d->advance) {
    VH_REQUIRE(d->scale_fmt.kind == VH_FMT_MINIFLOAT || d->scale_fmt.kind == VH_FMT_INT ||
                   d->scale_fmt.kind == VH_FMT_IDENTITY || d->scale_fmt.kind == VH_FMT_POSIT,
               "vh_kivi_attention: the scale map must be a closed form (minifloat, int, posit or identity)");
    VH_REQUIRE(d->code_fmt.kind == VH_FMT_INT && d->code_fmt.p0 >= 0 && d->code_fmt.p1 <= 3,
               "vh_kivi_attention: the code map must be an integer range within [0, 3]");
  }
  hipStream_t s = vh::as_stream(stream);
  const unsigned P = (unsigned)(d->batch * d->nkv);
  hipLaunchKernelGGL(k_kivi_scores, dim3((unsigned)a.splits_cap + 1, P), dim3(SPLIT_WAVES * 64), 0, s, a);
  hipLaunchKernelGGL(k_kivi_pv, dim3((unsigned)a.splits_cap, P), dim3(SPLIT_WAVES * 64), 0, s, a);
  hipLaunchKernelGGL(k_kivi_combine, dim3((unsigned)(d->batch * d->nq)), dim3(COMBINE_THREADS), 0, s, a, d->attn,
                     (_Float16*)d->attn_fq, (int*)d->flag);
  return vh::check_launch("vh_kivi_attention");
}



extern "C" int vh_quantize_mx8_f16(const uint16_t* x, int64_t M, int64_t K, uint16_t* out, int32_t* ex,
                                   vh_stream_t stream) {
  VH_REQUIRE(x && out && ex, "vh_quantize_mx8_f16: null argument");
  VH_REQUIRE(M > 0 && K > 0 && K % 16 == 0, "vh_quantize_mx8_f16: needs K a multiple of 16");
  VH_REQUIRE((uintptr_t)x % 16 == 0 && (uintptr_t)out % 16 == 0, "vh_quantize_mx8_f16: misaligned tensor");
  const int64_t nb = K / 16;
  hipStream_t s = vh::as_stream(stream);
  if (nb <= 256)
    hipLaunchKernelGGL(k_quantize_mx8_f16_r<1>, dim3((unsigned)M), dim3(256), 0, s, x, K, (_Float16*)out, ex);
  else if (nb <= 512)
    hipLaunchKernelGGL(k_quantize_mx8_f16_r<2>, dim3((unsigned)M), dim3(256), 0, s, x, K, (_Float16*)out, ex);
  else
    hipLaunchKernelGGL(k_quantize_mx8_f16, dim3((unsigned)M), dim3(256), 0, s, x, K, (_Float16*)out, ex);
  return vh::check_launch("vh_quantize_mx8_f16");
}

extern "C" int vh_mx8_bake_f16(const int8_t* codes, const uint8_t* scale, int32_t scale_bias, int64_t N, int64_t K,
                               uint16_t* out, int32_t* ew, vh_stream_t stream) {
  VH_REQUIRE(codes && scale && out && ew, "vh_mx8_bake_f16: null argument");
  VH_REQUIRE(N > 0 && K > 0 && K % 16 == 0, "vh_mx8_bake_f16: needs K a multiple of 16");
  VH_REQUIRE((uintptr_t)codes % 16 == 0 && (uintptr_t)out % 16 == 0, "vh_mx8_bake_f16: misaligned tensor");
  const int64_t nb = K / 16;
  hipStream_t s = vh::as_stream(stream);
  if (nb <= 256)
    hipLaunchKernelGGL(k_mx8_bake_f16_r<1>, dim3((unsigned)N), dim3(256), 0, s, codes, scale, scale_bias, K,
                       (_Float16*)out, ew);
  else if (nb <= 1024)
    hipLaunchKernelGGL(k_mx8_bake_f16_r<4>, dim3((unsigned)N), dim3(256), 0, s, codes, scale, scale_bias, K,
                       (_Float16*)out, ew);
  else
    hipLaunchKernelGGL(k_mx8_bake_f16, dim3((unsigned)N), dim3(256), 0, s, codes, scale, scale_bias, K,
                       (_Float16*)out, ew);
  return vh::check_launch("vh_mx8_bake_f16");
}
