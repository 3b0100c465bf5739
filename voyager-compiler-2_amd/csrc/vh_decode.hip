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
constexpr int PART = HEAD_DIM + 2;  // m, l, o[128]

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

VH_DEV float max16(float v) {
#pragma unroll
  for (int o = 8; o >= 1; o >>= 1) v = nmax(v, __shfl_xor(v, o));
  return v;
}

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
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      o0[j] = fq_half(mx8_fq(h[j], sc), flag);
      o1[j] = fq_half(mx8_fq(h[8 + j], sc), flag);
    }
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

VH_DEV int block_max_int(int v, int* s_red) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = max(v, __shfl_xor(v, o));
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
__global__ void __launch_bounds__(256) k_bake_mx8_codes(const uint8_t* __restrict__ codes, int64_t N, int64_t K,
                                                        int paired, uint8_t* __restrict__ out) {
  const int64_t nsp = K / 64;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (N / 16) * nsp * 64) return;
  const int lane = (int)(t % 64);
  const int64_t sp = (t / 64) % nsp, tile = t / (64 * nsp);
  const int64_t src_tile = paired ? ((tile & 1) * (N / 32) + (tile >> 1)) : tile;
  const int64_t n = src_tile * 16 + (lane & 15);
  const int64_t k0 = sp * 64 + (lane >> 4) * 8;
  const uint2 a = *(const uint2*)(codes + n * K + k0);
  const uint2 b = *(const uint2*)(codes + n * K + k0 + 32);
  *(uint4*)(out + t * 16) = make_uint4(a.x ^ 0x80808080u, a.y ^ 0x80808080u, b.x ^ 0x80808080u, b.y ^ 0x80808080u);
}

__global__ void __launch_bounds__(256) k_bake_mx8_scales(const uint8_t* __restrict__ codes,
                                                         const uint8_t* __restrict__ scale, int bias, int64_t N,
                                                         int64_t K, int paired, uint8_t* __restrict__ out,
                                                         int* __restrict__ flag) {
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
    int e = byte - bias;
    if (zero) e = 0;  // an all-zero block contributes nothing at any scale
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

// ------------------------------------------------------------ KIVI attention
// ------------------------------------------------------------ KIVI cache
// Main-cache layout: P = batch x kv heads sequences, each with room for
// group_cap groups of 32 tokens; one 3072-byte block per (P, group), read by
// one wave with three 16-byte loads per lane:
//   [0, 1024)     key codes, lane l (kq = l / 16, r = l % 16): dwords
//                 D[2 tile + cs / 2] hold token 16 tile + r, channels
//                 32 kq + 8 cs + j (j < 8): code (cs, j) at bit
//                 16 (cs % 2) + 2 j, so the codes of channels j = 2p, 2p + 1
//                 (one MFMA operand dword) form nibble 4 (cs % 2) + p.
//   [1024, 2048)  value codes, lane l: dword w holds row tiles r8 = 2 w and
//                 2 w + 1 (channel 16 r8 + r) at tokens tok(kq, j): code at
//                 bit 8 (r8 % 2) + 16 (j % 2) + 2 (j / 2).
//   [2048, 2560)  key scale / zero point, fp16 [128 channels][2].
//   [2560, 3072)  value scale / zero point, fp16 [4 kq][8 j][4 channel
//                 groups][2] of token tok(kq, j).
// tok(kq, j) = 16 (j / 4) + 4 kq + j % 4: the token the score MFMA leaves in
// lane quarter kq, register j % 4 of tile j / 4.
// Residual window: keys and values bf16 [P][RES_CAP][128]; slot s holds the
// token at position n_main + s.
// Cache state (device int32[4]): {tokens in the main cache, residual slots
// filled, completion counter of the advance kernel, unused}.
constexpr int GROUP_BYTES = 3072;
constexpr int SPLIT_WAVES = 8;
constexpr int GROUPS_PER_WAVE = 2;
constexpr int GROUPS_PER_SPLIT = SPLIT_WAVES * GROUPS_PER_WAVE;
constexpr int GROUPS_PER_CHUNK = RES_CAP / KV_GROUP;  // groups a fold appends
constexpr float LOG2E = 1.4426950408889634f;
// value operands are p * s * 2**(V_EXP - e), e = floor(log2) of the largest
// value scale the wave reads: at most 2**(V_EXP + 1), far above fp16
// subnormals for any term that matters
constexpr int V_EXP = 14;

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
  float* part;  // [P][splits_cap][GQA][PART]
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

// A score as eager attention forms it, in log2 units for exp2: q . k rounded
// to bf16 (the bf16 matmul), times the scale rounded to bf16 again
// (transformers' eager_attention_forward: matmul(q, k^T) * scaling).
VH_DEV float eager_score_log2(float qk, float scale) {
  return __uint_as_float(f2bf2_hw(__uint_as_float(f2bf2_hw(qk, 0.0f) << 16) * scale, 0.0f) << 16) * LOG2E;
}

// Two scores through the same chain, each bf16 rounding done for both by
// one packed conversion (the same rounding as one at a time).
VH_DEV float2 eager_score_log2_x2(float qk0, float qk1, float scale) {
  const uint32_t t = f2bf2_hw(qk0, qk1);
  const uint32_t u = f2bf2_hw(__uint_as_float(t << 16) * scale, __uint_as_float(t & 0xffff0000u) * scale);
  return make_float2(__uint_as_float(u << 16) * LOG2E, __uint_as_float(u & 0xffff0000u) * LOG2E);
}

VH_DEV uint16_t rope1(const uint16_t* base, const uint16_t* cs, const uint16_t* sn, int c) {
  const float x = bf2f(base[c]);
  const float xr = c < HEAD_DIM / 2 ? -bf2f(base[c + HEAD_DIM / 2]) : bf2f(base[c - HEAD_DIM / 2]);
  return (uint16_t)f2bf(rbf(x * bf2f(cs[c])) + rbf(xr * bf2f(sn[c])));
}

VH_DEV uint32_t pack_h2(float a, float b) {
  const f16x2 h = {(_Float16)a, (_Float16)b};
  return __builtin_bit_cast(uint32_t, h);
}

// lane l and lane l ^ 16 (l ^ 32)
VH_DEV float sum_x16(float v) { return v + __shfl_xor(v, 16); }
VH_DEV float sum_x32(float v) { return v + __shfl_xor(v, 32); }
VH_DEV float max_x16(float v) { return fmaxf(v, __shfl_xor(v, 16)); }
VH_DEV float max_x32(float v) { return fmaxf(v, __shfl_xor(v, 32)); }

// Value code operands: the pair of 2-bit fields at bits 2p and 16 + 2p of W
// becomes the fp16 pair (1024 + c * 4**p), one v_and_or_b32 with a mask
// held in a VGPR; the 4**-p goes into the other operand and the 1024 offset
// is removed by one MFMA against -1024.  mk[p] = 0x00030003 << 2p.
struct CodeMasks {
  uint32_t mk[4];
};

VH_DEV CodeMasks code_masks() {
  CodeMasks m;
#pragma unroll
  for (int p = 0; p < 4; ++p) asm volatile("v_mov_b32 %0, %1" : "=v"(m.mk[p]) : "i"(0x00030003u << (2 * p)));
  return m;
}

// The four operand dwords of the codes at bits 8 half + [0, 8) and
// 16 + 8 half + [0, 8) of W.
VH_DEV f16x8 code_operand(uint32_t W, int half, const CodeMasks& m) {
  const uint32_t w = half ? (W >> 8) : W;
  return __builtin_bit_cast(f16x8, make_uint4((w & m.mk[0]) | 0x64006400u, (w & m.mk[1]) | 0x64006400u,
                                              (w & m.mk[2]) | 0x64006400u, (w & m.mk[3]) | 0x64006400u));
}

// Per wave and group, a table of every key operand the group can hold: for
// each pair of channels (2p, 2p + 1 of 8 cs + [0, 8) in block kq) and each of
// the 16 pairs of codes, the bf16 pair of dequantized keys -- (code -
// zero_point) * scale, each bfloat16 op rounding its result as the
// reference's dequantize does (ops/quantized.py:518-571).  An MFMA operand
// dword is then one 32-bit LDS read at its pair's table + 4 * nibble.
// Pair 4 cs + p of block kq sits at byte 272 (4 cs + p) + 64 kq of the
// wave's 256-byte-aligned table.  The low address byte before the row
// offset, 64 kq + 4 * nibble, is one byte of a precomputed word
// (KeyNibbles), so an address is one v_perm_b32 of that word and the table's
// base, and the row offset is the read's immediate.  The four blocks a read
// touches fall in distinct LDS banks, and so do the 16 rows a quarter-wave
// writes (the 16-byte skew of the 272-byte rows).
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

// One pair of channels from its fp16 (scale, zero point) pairs [s0, z0, s1,
// z1]: the 16 entries (every code pair) at dst.
VH_DEV void build_key_pair(const uint2& prm, uint8_t* dst) {
  const f16x2 e0 = __builtin_bit_cast(f16x2, prm.x), e1 = __builtin_bit_cast(f16x2, prm.y);
  uint32_t v01[2], v23[2];  // per channel: keys of codes 0, 1 and 2, 3 (bf16 pairs)
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
    // bytes 0-3 of the selection: channel 0's key of c0 (low), channel 1's of c1 (high)
    const uint32_t lo = c0 < 2 ? v01[0] : v23[0], hi = c1 < 2 ? v01[1] : v23[1];
    const uint32_t sl = (uint32_t)(2 * (c0 & 1)), sh = (uint32_t)(4 + 2 * (c1 & 1));
    ent[v] = __builtin_amdgcn_perm(hi, lo, sl | (sl + 1) << 8 | sh << 16 | (sh + 1) << 24);
  }
#pragma unroll
  for (int k = 0; k < 4; ++k)
    *(uint4*)(dst + 16 * k) = make_uint4(ent[4 * k], ent[4 * k + 1], ent[4 * k + 2], ent[4 * k + 3]);
}

// Workgroups (split, P) stream the main cache: wave w takes groups
// GROUPS_PER_SPLIT split + SPLIT_WAVES i + w (i < GROUPS_PER_WAVE) with one
// online softmax, the waves merge through LDS and the workgroup leaves one
// (max, sum, output) partial per query head.  Splits past the cache's groups
// return at once (the combine merges only the live ones), so one launch
// shape serves every cache length up to the capacity.
// MFMA column n = 4 cg + h: the score MFMA repeats query head h in the four
// columns n % 4 == h, so every lane holds its own head's scores, and the
// value MFMA's column n carries p * s for value channel group cg of head h.
// Of a 16-channel output tile only the columns of its own channel group are
// kept, so each lane builds one column of value operands (one scale per
// token) instead of four.  Only the query waits for memory before the
// workgroup barrier: a wave's second group is still loading while its first
// is computed.
__global__ void __launch_bounds__(SPLIT_WAVES * 64) k_kivi_split(KiviArgs a) {
  static_assert(GQA * HEAD_DIM == SPLIT_WAVES * 64, "one rotated query element per thread");
  __shared__ __attribute__((aligned(256))) uint8_t s_tab[SPLIT_WAVES][KEY_TAB_BYTES];
  __shared__ __attribute__((aligned(16))) uint4 s_prm[SPLIT_WAVES][GROUPS_PER_WAVE][64];
  __shared__ __attribute__((aligned(16))) uint16_t s_q[GQA][HEAD_DIM];
  __shared__ float s_part[SPLIT_WAVES][GQA][PART];
  const int n_main = a.state[0], n_res = a.state[1];
  const int G = n_main / KV_GROUP;
  const int split = blockIdx.x, P = blockIdx.y;
  const int g_begin = split * GROUPS_PER_SPLIT;
  if (!state_ok(a, n_main, n_res) || g_begin >= G) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n = lane & 15, kq = lane >> 4;
  const int cg = n >> 2, hq = n & 3;  // this lane's column: value channel group cg of query head hq
  const uint32_t kq_bytes = (uint32_t)kq * 0x40404040u;  // 64 kq in every byte: the key table block
  const int b = P / a.nkv, kvh = P % a.nkv;
  const int pos = n_main + n_res;

  // the query element this thread rotates (head tid / 128, channel tid % 128) goes out first
  const int qh = tid / HEAD_DIM, qc = tid % HEAD_DIM;
  const uint16_t* qrow = a.qkv + (int64_t)b * a.qkv_ld + (kvh * GQA + qh) * HEAD_DIM;
  uint32_t qv = qrow[qc], qp = qrow[qc < HEAD_DIM / 2 ? qc + HEAD_DIM / 2 : qc - HEAD_DIM / 2];
  uint32_t qcs = a.rope[(int64_t)pos * HEAD_DIM + qc], qsn = a.rope[(a.max_pos + pos) * HEAD_DIM + qc];
  asm volatile("" ::: "memory");
  // then this wave's blocks, group by group (an absent group re-reads a live one; it is skipped)
  uint4 kc[GROUPS_PER_WAVE], vc[GROUPS_PER_WAVE], pr[GROUPS_PER_WAVE];
  int ng = 0;
  const uint8_t* seq = a.main + (int64_t)P * a.group_cap * GROUP_BYTES;
#pragma unroll
  for (int i = 0; i < GROUPS_PER_WAVE; ++i) {
    const int g = g_begin + i * SPLIT_WAVES + wave;
    ng += g < G ? 1 : 0;
    const uint8_t* blk = seq + (int64_t)(g < G ? g : G - 1) * GROUP_BYTES;
    pr[i] = *(const uint4*)(blk + 2048 + lane * 16);
    kc[i] = *(const uint4*)(blk + lane * 16);
    vc[i] = *(const uint4*)(blk + 1024 + lane * 16);
  }
  // waits for the query alone; the blocks stay in flight across the barrier
  asm volatile("" : "+v"(qv), "+v"(qp), "+v"(qcs), "+v"(qsn)::"memory");
  {
    const float x = bf2f(qv), xr = qc < HEAD_DIM / 2 ? -bf2f(qp) : bf2f(qp);
    s_q[qh][qc] = (uint16_t)f2bf(rbf(x * bf2f(qcs)) + rbf(xr * bf2f(qsn)));
  }
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");

  // key B operands: q[head hq][32 kq + 8 cs + j], the same in the four columns of a head
  bf16x8 Bq[4];
#pragma unroll
  for (int cs = 0; cs < 4; ++cs) Bq[cs] = __builtin_bit_cast(bf16x8, *(const uint4*)&s_q[hq][32 * kq + 8 * cs]);
  const CodeMasks cm = code_masks();
  const f16x8 NEG = __builtin_bit_cast(f16x8, make_uint4(0xE400E400u, 0xE400E400u, 0xE400E400u, 0xE400E400u));
  float m = -__builtin_inff(), lsum = 0.0f, zt = 0.0f, vmax = 0.0f;
  int ve = 0;
  f32x4 acc[8];
#pragma unroll
  for (int r8 = 0; r8 < 8; ++r8) acc[r8] = {0.0f, 0.0f, 0.0f, 0.0f};

  // one group (i constant at each call: the block registers stay unindexed)
  auto group = [&](const int i) __attribute__((always_inline)) {
    // the group's parameters (keys: lanes 0-31, values: lanes 32-63) to LDS;
    // the largest value scale of the wave's groups so far sets the value
    // operands' exponent
    s_prm[wave][i][lane] = pr[i];
    if (lane >= 32) {
      const f16x8 e = __builtin_bit_cast(f16x8, pr[i]);
      vmax = fmaxf(vmax, fmaxf(fmaxf((float)e[0], (float)e[2]), fmaxf((float)e[4], (float)e[6])));
    }
    vmax = max_x32(max_x16(vmax));
    vmax = fmaxf(vmax, __shfl_xor(vmax, 8));
    vmax = fmaxf(vmax, __shfl_xor(vmax, 4));
    vmax = fmaxf(vmax, __shfl_xor(vmax, 2));
    vmax = fmaxf(vmax, __shfl_xor(vmax, 1));
    const int ve_new = (vmax > 0.0f && vmax < __builtin_inff()) ? floor_log2(vmax) : 0;
    // this group's key table, lane l the pair of channels 2 l, 2 l + 1 (the
    // wave's LDS accesses stay in order: the parameters above land first, and
    // the previous group's reads precede these writes)
    build_key_pair(*(const uint2*)((const uint8_t*)s_prm[wave][i] + 8 * lane),
                   s_tab[wave] + (lane & 15) * KEY_TAB_ROW + (lane >> 4) * PAIR_TAB);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
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
          for (int p = 0; p < 4; ++p) {
            const uint32_t addr = key_entry_addr(kn, 4 * c2 + p, tab);
            w[p] = *(const __attribute__((address_space(3))) uint32_t*)(uintptr_t)(addr + (4 * cs + p) * KEY_TAB_ROW);
          }
          S[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              __builtin_bit_cast(bf16x8, make_uint4(w[0], w[1], w[2], w[3])), Bq[cs], S[t], 0, 0, 0);
        }
      }
    // online softmax (every lane of a head holds its running max)
    float sc[8];
    float mg = -__builtin_inff();
#pragma unroll
    for (int j = 0; j < 8; j += 2) {
      const float2 s2 = eager_score_log2_x2(S[j >> 2][j & 3], S[j >> 2][(j & 3) + 1], a.scale);
      sc[j] = s2.x;
      sc[j + 1] = s2.y;
      mg = fmaxf(mg, fmaxf(s2.x, s2.y));
    }
    mg = max_x32(max_x16(mg));
    const float m_new = fmaxf(m, mg);
    const float alpha = __builtin_amdgcn_exp2f(m - m_new);
    m = m_new;
    float p[8];
    float ps = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      p[j] = __builtin_amdgcn_exp2f(sc[j] - m_new);
      ps += p[j];
    }
    lsum = lsum * alpha + ps;
    if (i > 0) {  // the first group starts from zero; a new exponent rescales by a power of two (exact)
      const float f = alpha * ldexpf(1.0f, ve - ve_new);
      zt *= f;
#pragma unroll
      for (int r8 = 0; r8 < 8; ++r8) acc[r8] *= f;
    }
    ve = ve_new;
    // value B operands of column (cg, hq): p * s * 2**(V_EXP - ve) * 4**-(j / 2)
    // at the lane's tokens; the zero-point term accumulates p * s * zp in the
    // same 2**(V_EXP - ve) units
    const float bscale = ldexpf(1.0f, V_EXP - ve);
    const uint8_t* vprm = (const uint8_t*)&s_prm[wave][i][32] + cg * 4;
    uint32_t bv[4];
#pragma unroll
    for (int pp = 0; pp < 4; ++pp) {
      const f16x2 e0 = *(const f16x2*)(vprm + (kq * 8 + 2 * pp) * 16);
      const f16x2 e1 = *(const f16x2*)(vprm + (kq * 8 + 2 * pp + 1) * 16);
      const float f = bscale * (1.0f / (float)(1 << (2 * pp)));
      const float p0 = p[2 * pp] * f, p1 = p[2 * pp + 1] * f;
      const float b0 = fmaf(p0, (float)e0[0], 0.0f), b1 = fmaf(p1, (float)e1[0], 0.0f);
      const float z = fmaf(b1, (float)e1[1], b0 * (float)e0[1]);
      zt = fmaf(z, (float)(1 << (2 * pp)), zt);
      bv[pp] = pack_h2(b0, b1);
    }
    const f16x8 B = __builtin_bit_cast(f16x8, make_uint4(bv[0], bv[1], bv[2], bv[3]));
    const uint32_t vw[4] = {vc[i].x, vc[i].y, vc[i].z, vc[i].w};
#pragma unroll
    for (int r8 = 0; r8 < 8; ++r8) {
      acc[r8] = __builtin_amdgcn_mfma_f32_16x16x32_f16(code_operand(vw[r8 >> 1], r8 & 1, cm), B, acc[r8], 0, 0, 0);
      acc[r8] = __builtin_amdgcn_mfma_f32_16x16x32_f16(NEG, B, acc[r8], 0, 0, 0);
    }
  };
  static_assert(GROUPS_PER_WAVE == 2, "two group calls");
  if (ng > 0) group(0);
  if (ng > 1) group(1);
  // wave totals: sums over the lane quarters; column (cg, hq) keeps the
  // channel tiles of its group, o[head hq][16 r8 + 4 kq + r] for r8 / 2 == cg
  lsum = sum_x32(sum_x16(lsum));
  zt = sum_x32(sum_x16(zt));
  const float oscale = ldexpf(1.0f, ve - V_EXP);
#pragma unroll
  for (int r8 = 0; r8 < 8; ++r8)
    if ((r8 >> 1) == cg) {
#pragma unroll
      for (int r = 0; r < 4; ++r) s_part[wave][hq][2 + 16 * r8 + 4 * kq + r] = (acc[r8][r] - zt) * oscale;
    }
  if (n < GQA && kq == 0) {
    s_part[wave][hq][0] = m;
    s_part[wave][hq][1] = lsum;
  }
  __syncthreads();
  // merge the waves: thread (head, channel)
  const int h = tid >> 7, c = tid & (HEAD_DIM - 1);
  float M = -__builtin_inff();
#pragma unroll
  for (int w = 0; w < SPLIT_WAVES; ++w) M = fmaxf(M, s_part[w][h][0]);
  float L = 0.0f, O = 0.0f;
#pragma unroll
  for (int w = 0; w < SPLIT_WAVES; ++w) {
    const float mw = s_part[w][h][0];
    const float f = mw == -__builtin_inff() ? 0.0f : __builtin_amdgcn_exp2f(mw - M);
    L = fmaf(f, s_part[w][h][1], L);
    O = fmaf(f, s_part[w][h][2 + c], O);
  }
  float* out = a.part + (((int64_t)P * a.splits_cap + split) * GQA + h) * PART;
  if (c == 0) {
    out[0] = M;
    out[1] = L;
  }
  out[2 + c] = O;
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
  for (int r8 = 0; r8 < 8; ++r8)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int tok = 16 * (j >> 2) + 4 * kq + (j & 3);
      const uint32_t code = vcode[(int64_t)tok * vstride + 16 * r8 + r] & 3u;
      V[r8 >> 1] |= code << (8 * (r8 & 1) + 16 * (j & 1) + 2 * (j >> 1));
    }
  *(uint4*)(blk + 1024 + lane * 16) = make_uint4(V[0], V[1], V[2], V[3]);
  // parameters: lanes 0-31 four key channels each, lanes 32-63 one value token each
  _Float16 piece[8];
  if (lane < 32) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      piece[2 * k] = (_Float16)bf2f(ks[4 * lane + k]);
      piece[2 * k + 1] = (_Float16)bf2f(kz[4 * lane + k]);
    }
  } else {
    const int i = lane - 32, qq = i >> 3, j = i & 7;
    const int tok = 16 * (j >> 2) + 4 * qq + (j & 3);
#pragma unroll
    for (int cg = 0; cg < 4; ++cg) {
      piece[2 * cg] = (_Float16)bf2f(vs[tok * 4 + cg]);
      piece[2 * cg + 1] = (_Float16)bf2f(vz[tok * 4 + cg]);
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
// last token (slot RES_CAP - 1, written by this step) comes from LDS.  All
// threads of the workgroup; returns with them synchronised.
struct FoldLds {
  uint8_t kc[RES_CAP][HEAD_DIM];
  uint8_t vc[RES_CAP][HEAD_DIM];
  uint16_t ks[GROUPS_PER_CHUNK][HEAD_DIM], kz[GROUPS_PER_CHUNK][HEAD_DIM];
  uint16_t vs[RES_CAP][4], vz[RES_CAP][4];
  int bad;
};

VH_DEV float res_at(const uint16_t* R, const uint16_t* last, int t, int ch) {
  return bf2f(t == RES_CAP - 1 ? last[ch] : R[t * HEAD_DIM + ch]);
}

VH_DEV void fold_chunk(const KiviArgs& a, int P, int g0, const uint16_t* newk, const uint16_t* newv, FoldLds& L,
                       int* flag) {
  const int tid = threadIdx.x, nthreads = blockDim.x;
  if (tid == 0) L.bad = 0;
  __syncthreads();
  int bad = 0;
  const uint16_t* K = a.kr + (int64_t)P * RES_CAP * HEAD_DIM;
  const uint16_t* V = a.vr + (int64_t)P * RES_CAP * HEAD_DIM;
  // keys: one column (group, channel) of 32 tokens per pass
  for (int col = tid; col < GROUPS_PER_CHUNK * HEAD_DIM; col += nthreads) {
    const int g = col / HEAD_DIM, ch = col % HEAD_DIM;
    float lo = res_at(K, newk, g * KV_GROUP, ch), hi = lo;
    for (int t = 1; t < KV_GROUP; ++t) {
      const float x = res_at(K, newk, g * KV_GROUP + t, ch);
      lo = nmin(lo, x);
      hi = nmax(hi, x);
    }
    const Affine af = kivi_affine(lo, hi, a.sf);
    L.ks[g][ch] = (uint16_t)f2bf(af.s);
    L.kz[g][ch] = (uint16_t)f2bf(af.zp);
    for (int t = 0; t < KV_GROUP; ++t)
      L.kc[g * KV_GROUP + t][ch] = kivi_code(res_at(K, newk, g * KV_GROUP + t, ch), af, a.cf, &bad);
  }
  // values: one row (token, channel group) of 32 channels per pass
  for (int row = tid; row < RES_CAP * 4; row += nthreads) {
    const int t = row / 4, cg = row % 4;
    float lo = res_at(V, newv, t, cg * KV_GROUP), hi = lo;
    for (int c = 1; c < KV_GROUP; ++c) {
      const float x = res_at(V, newv, t, cg * KV_GROUP + c);
      lo = nmin(lo, x);
      hi = nmax(hi, x);
    }
    const Affine af = kivi_affine(lo, hi, a.sf);
    L.vs[t][cg] = (uint16_t)f2bf(af.s);
    L.vz[t][cg] = (uint16_t)f2bf(af.zp);
    for (int c = 0; c < KV_GROUP; ++c)
      L.vc[t][cg * KV_GROUP + c] = kivi_code(res_at(V, newv, t, cg * KV_GROUP + c), af, a.cf, &bad);
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

// Per (batch, query head): attention over the residual window (its n_res
// cached tokens and this step's key / value, taken from the qkv row), merged
// with the main-cache splits; writes the attention output (bf16) and its
// MX-int8 fake quantization.  The workgroup of head 0 of each kv head
// appends this step's key (after RoPE) and value at residual slot n_res.
// 256 threads: two per residual key row, 16 token subsets for the values;
// the first 128 (one per channel) merge and write.
constexpr int COMBINE_PRELOAD = 16;  // splits whose partials are loaded up front
constexpr int COMBINE_THREADS = 2 * HEAD_DIM;

VH_DEV float block_max256(float v, float* s_red) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = v;
  __syncthreads();
  const float r = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
  __syncthreads();
  return r;
}

VH_DEV float block_sum256(float v, float* s_red) {
  v = wave_sum(v);
  if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = v;
  __syncthreads();
  const float r = (s_red[0] + s_red[1]) + (s_red[2] + s_red[3]);
  __syncthreads();
  return r;
}

__global__ void __launch_bounds__(COMBINE_THREADS) k_kivi_combine(KiviArgs a, uint16_t* __restrict__ attn,
                                                                  _Float16* __restrict__ fq, int* __restrict__ flag) {
  __shared__ __attribute__((aligned(16))) float s_q[HEAD_DIM];
  __shared__ float s_p[RES_CAP];
  __shared__ float s_o[16][HEAD_DIM];
  __shared__ float s_red[4];
  __shared__ uint16_t s_newk[HEAD_DIM], s_newv[HEAD_DIM];
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
  const int c = tid & (HEAD_DIM - 1);              // channel (first half of the block: merge / output)
  const int tk = tid >> 1, kh = tid & 1;           // key row tk, channel half kh
  const int co = tid & 15, ts = tid >> 4;          // value octet co, token subset ts (slots ts + 16u)
  const bool merger = tid < HEAD_DIM;
  // The residual window and the split partials go out before the state is
  // read: their addresses do not depend on it (every slot of the window and
  // every split of the partials is allocated), and what the state leaves
  // unused is masked once it arrives.
  uint4 kw[HEAD_DIM / 16], vw[RES_CAP / 16];
  const uint4* kp = (const uint4*)(a.kr + ((int64_t)P * RES_CAP + tk) * HEAD_DIM + kh * (HEAD_DIM / 2));
  const uint4* vp = (const uint4*)(a.vr + (int64_t)P * RES_CAP * HEAD_DIM) + co;
#pragma unroll
  for (int i = 0; i < HEAD_DIM / 16; ++i) kw[i] = kp[i];
#pragma unroll
  for (int u = 0; u < RES_CAP / 16; ++u) vw[u] = vp[(int64_t)(ts + 16 * u) * (HEAD_DIM / 8)];
  const float* base = a.part + ((int64_t)P * a.splits_cap * GQA + h) * PART;
  float pm[COMBINE_PRELOAD], pl[COMBINE_PRELOAD], po[COMBINE_PRELOAD];
#pragma unroll
  for (int s = 0; s < COMBINE_PRELOAD; ++s) {
    // no predicate: a split past the capacity re-reads the last one
    const int se = s < a.splits_cap ? s : a.splits_cap - 1;
    const float* ps = base + (int64_t)se * GQA * PART;
    pm[s] = ps[0];
    pl[s] = ps[1];
    po[s] = ps[2 + c];
  }
  asm volatile("" ::: "memory");  // the loads above are issued before the state is used
  const int n_main = st.x, n_res = st.y;
  const int pos = n_main + n_res;
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
  // slots past the window and splits past the cache hold stale bytes (a
  // zero weight times a stale infinity would be NaN): cleared
#pragma unroll
  for (int u = 0; u < RES_CAP / 16; ++u)
    if (ts + 16 * u >= n_res) vw[u] = make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
  for (int s = 0; s < COMBINE_PRELOAD; ++s)
    if (s >= splits) {
      pm[s] = -__builtin_inff();
      pl[s] = 0.0f;
      po[s] = 0.0f;
    }
  const uint16_t* qrow = a.qkv + (int64_t)b * a.qkv_ld;
  const uint16_t* cs_ = a.rope + (int64_t)pos * HEAD_DIM;
  const uint16_t* sn_ = a.rope + (a.max_pos + pos) * HEAD_DIM;
  // RoPE of this step's query / key (channel c; the second half of the block duplicates)
  const float qc = bf2f(rope1(qrow + H * HEAD_DIM, cs_, sn_, c));
  const uint16_t kn = rope1(qrow + (a.nq + kvh) * HEAD_DIM, cs_, sn_, c);
  const uint16_t vn = qrow[(a.nq + a.nkv + kvh) * HEAD_DIM + c];
  if (merger) s_q[c] = qc;
  // this step's own score, q . k_new
  const float s_new = eager_score_log2(block_sum256(merger ? qc * bf2f(kn) : 0.0f, s_red), a.scale);
  if (h == 0 && merger) {
    // this step's key (after RoPE) and value enter residual slot n_res (read
    // by later steps only: this step takes them from the qkv row)
    a.kr[((int64_t)P * RES_CAP + n_res) * HEAD_DIM + c] = kn;
    a.vr[((int64_t)P * RES_CAP + n_res) * HEAD_DIM + c] = vn;
    s_newk[c] = kn;
    s_newv[c] = vn;
  }
  // score of residual slot tk: two threads, 64 channels each
  float acc = 0.0f;
  {
    const float4* q4 = (const float4*)(s_q + kh * (HEAD_DIM / 2));
#pragma unroll
    for (int i = 0; i < HEAD_DIM / 16; ++i) {
      const float4 qa = q4[2 * i], qb = q4[2 * i + 1];
      const uint32_t ww[4] = {kw[i].x, kw[i].y, kw[i].z, kw[i].w};
      acc = fmaf(qa.x, bf2f(ww[0] & 0xffffu), acc);
      acc = fmaf(qa.y, bf2f(ww[0] >> 16), acc);
      acc = fmaf(qa.z, bf2f(ww[1] & 0xffffu), acc);
      acc = fmaf(qa.w, bf2f(ww[1] >> 16), acc);
      acc = fmaf(qb.x, bf2f(ww[2] & 0xffffu), acc);
      acc = fmaf(qb.y, bf2f(ww[2] >> 16), acc);
      acc = fmaf(qb.z, bf2f(ww[3] & 0xffffu), acc);
      acc = fmaf(qb.w, bf2f(ww[3] >> 16), acc);
    }
  }
  acc += __shfl_xor(acc, 1);
  float sc = -__builtin_inff();
  if (tk < n_res) sc = eager_score_log2(acc, a.scale);
  else if (tk == n_res) sc = s_new;
  const float mr = block_max256(kh == 0 ? sc : -__builtin_inff(), s_red);
  const float p = tk <= n_res ? exp2f(sc - mr) : 0.0f;
  if (kh == 0) s_p[tk] = p;
  const float lr = block_sum256(kh == 0 ? p : 0.0f, s_red);
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
  if (merger) {
    float orr = s_p[n_res] * bf2f(vn);
#pragma unroll
    for (int t16 = 0; t16 < 16; ++t16) orr += s_o[t16][c];
    // merge with the main-cache splits
    float M = mr;
#pragma unroll
    for (int s = 0; s < COMBINE_PRELOAD; ++s) M = fmaxf(M, pm[s]);
    for (int s = COMBINE_PRELOAD; s < splits; ++s) M = fmaxf(M, base[(int64_t)s * GQA * PART]);
    const float fr = exp2f(mr - M);
    float L = lr * fr, O = orr * fr;
#pragma unroll
    for (int s = 0; s < COMBINE_PRELOAD; ++s) {
      const float f = pm[s] == -__builtin_inff() ? 0.0f : exp2f(pm[s] - M);
      L = fmaf(f, pl[s], L);
      O = fmaf(f, po[s], O);
    }
    for (int s = COMBINE_PRELOAD; s < splits; ++s) {
      const float* ps = base + (int64_t)s * GQA * PART;
      const float f = ps[0] == -__builtin_inff() ? 0.0f : exp2f(ps[0] - M);
      L = fmaf(f, ps[1], L);
      O = fmaf(f, ps[2 + c], O);
    }
    const float o = rbf(O / L);
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
  if (fold && room && h == 0) fold_chunk(a, P, g0, s_newk, s_newv, s_fold, flag);
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
                           int32_t paired, uint8_t* w_codes, uint8_t* w_hb, int32_t* flag, vh_stream_t stream) {
  VH_REQUIRE(codes && scale && w_codes && w_hb && flag, "vh_mx8_bake: null argument");
  VH_REQUIRE(N > 0 && K > 0 && N % (paired ? 32 : 16) == 0 && K % 256 == 0,
             "vh_mx8_bake: needs N %% 16 == 0 (32 when paired) and K %% 256 == 0");
  hipStream_t s = vh::as_stream(stream);
  const int64_t nc = (N / 16) * (K / 64) * 64, ns = (N / 16) * (K / 256) * 32;
  hipLaunchKernelGGL(k_bake_mx8_codes, dim3(blocks_for(nc, 256)), dim3(256), 0, s, codes, N, K, (int)paired, w_codes);
  hipLaunchKernelGGL(k_bake_mx8_scales, dim3(blocks_for(ns, 256)), dim3(256), 0, s, codes, scale, (int)scale_bias, N,
                     K, (int)paired, w_hb, (int*)flag);
  return vh::check_launch("vh_mx8_bake");
}

extern "C" int vh_gemv_mx8(const uint16_t* x_fq, int64_t M, int64_t K, const uint8_t* w_codes, const uint8_t* w_hb,
                           int64_t N, int32_t mode, int32_t tiles_per_block, const uint16_t* residual, uint16_t* y,
                           uint16_t* fq_out, int32_t* flag, vh_stream_t stream) {
  VH_REQUIRE(x_fq && w_codes && w_hb && flag, "vh_gemv_mx8: null argument");
  VH_REQUIRE(M >= 1 && M <= 16, "vh_gemv_mx8: M must be in [1, 16] (got %lld)", (long long)M);
  VH_REQUIRE(K > 0 && K % 256 == 0 && N > 0 && N % 16 == 0, "vh_gemv_mx8: needs K %% 256 == 0 and N %% 16 == 0");
  VH_REQUIRE(((uintptr_t)x_fq % 16) == 0 && ((uintptr_t)w_codes % 16) == 0 && ((uintptr_t)w_hb % 8) == 0,
             "vh_gemv_mx8: misaligned operand");
  GemvArgs a{(const _Float16*)x_fq, (int32_t)M, K, w_codes, w_hb, N, mode, residual, y, (_Float16*)fq_out, (int*)flag};
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

int kivi_common(const vh_kivi_desc* d, KiviArgs& a) {
  VH_REQUIRE(d && d->main && d->kr && d->vr && d->state && d->flag, "vh_kivi: null argument");
  VH_REQUIRE(d->batch >= 1 && d->nkv >= 1 && d->nq == GQA * d->nkv, "vh_kivi: needs nq == 4 nkv");
  VH_REQUIRE(d->head_dim == HEAD_DIM, "vh_kivi: head_dim must be %d", HEAD_DIM);
  VH_REQUIRE(d->group_cap >= GROUPS_PER_CHUNK, "vh_kivi: the main cache must hold at least one chunk");
  const int64_t splits_cap = (d->group_cap + GROUPS_PER_SPLIT - 1) / GROUPS_PER_SPLIT;
  VH_REQUIRE(splits_cap <= 65535 && d->batch * d->nkv <= 65535, "vh_kivi: cache too large");
  VH_REQUIRE(d->qkv && d->rope && d->attn_fq && d->part, "vh_kivi_attention: null argument");
  VH_REQUIRE(d->max_pos >= 1, "vh_kivi_attention: empty RoPE table");
  VH_REQUIRE(d->qkv_ld >= (int64_t)(d->nq + 2 * d->nkv) * HEAD_DIM, "vh_kivi_attention: qkv_ld too small");
  VH_REQUIRE(d->part_floats >= d->batch * d->nkv * splits_cap * GQA * PART,
             "vh_kivi_attention: workspace too small (needs %lld floats)",
             (long long)(d->batch * d->nkv * splits_cap * GQA * PART));
  a = KiviArgs{d->qkv, d->qkv_ld, d->rope, d->max_pos, d->main, d->group_cap, d->kr, d->vr, d->state,
               (int32_t)d->nkv, (int32_t)d->nq, (int32_t)splits_cap, d->softmax_scale, d->part,
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
  hipLaunchKernelGGL(k_kivi_split, dim3((unsigned)a.splits_cap, P), dim3(SPLIT_WAVES * 64), 0, s, a);
  hipLaunchKernelGGL(k_kivi_combine, dim3((unsigned)(d->batch * d->nq)), dim3(COMBINE_THREADS), 0, s, a, d->attn,
                     (_Float16*)d->attn_fq, (int*)d->flag);
  return vh::check_launch("vh_kivi_attention");
}



extern "C" int vh_quantize_mx8_f16(const uint16_t* x, int64_t M, int64_t K, uint16_t* out, int32_t* ex,
                                   vh_stream_t stream) {
  VH_REQUIRE(x && out && ex, "vh_quantize_mx8_f16: null argument");
  VH_REQUIRE(M > 0 && K > 0 && K % 16 == 0, "vh_quantize_mx8_f16: needs K a multiple of 16");
  VH_REQUIRE((uintptr_t)x % 16 == 0 && (uintptr_t)out % 16 == 0, "vh_quantize_mx8_f16: misaligned tensor");
  hipLaunchKernelGGL(k_quantize_mx8_f16, dim3((unsigned)M), dim3(256), 0, vh::as_stream(stream), x, K,
                     (_Float16*)out, ex);
  return vh::check_launch("vh_quantize_mx8_f16");
}

extern "C" int vh_mx8_bake_f16(const int8_t* codes, const uint8_t* scale, int32_t scale_bias, int64_t N, int64_t K,
                               uint16_t* out, int32_t* ew, vh_stream_t stream) {
  VH_REQUIRE(codes && scale && out && ew, "vh_mx8_bake_f16: null argument");
  VH_REQUIRE(N > 0 && K > 0 && K % 16 == 0, "vh_mx8_bake_f16: needs K a multiple of 16");
  VH_REQUIRE((uintptr_t)codes % 16 == 0 && (uintptr_t)out % 16 == 0, "vh_mx8_bake_f16: misaligned tensor");
  hipLaunchKernelGGL(k_mx8_bake_f16, dim3((unsigned)N), dim3(256), 0, vh::as_stream(stream), codes, scale, scale_bias,
                     K, (_Float16*)out, ew);
  return vh::check_launch("vh_mx8_bake_f16");
}
