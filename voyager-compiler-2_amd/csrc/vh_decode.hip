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
// * KIVI attention: flash-decoding over 32-token steps.  Codes (0..3) become
//   exact fp16 MFMA operands with two or three VALU ops per pair; the affine
//   scale moves to the other operand (q * s for keys, p * s for values) and
//   the zero-point term is a per-group dot product, so the cache is never
//   dequantized element by element.
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
constexpr int ATT_WAVES = 4;
constexpr int GROUPS_PER_WAVE = 4;  // one super-step of 128 tokens per wave
constexpr int STEPS_PER_SPLIT = ATT_WAVES * GROUPS_PER_WAVE;
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
// Main-cache layout (P = batch x kv heads, G = groups of 32 tokens): one
// 3 KB block per (P, g), read by one wave with three 16-byte loads per lane
// and staged through LDS:
//   [0, 1024)     key codes [2 tiles][64 lanes][8 B]: lane l of tile t holds
//                 token 32 g + 16 t + l % 16, channels 32 cs + 8 (l / 16) + j
//                 as 2-bit fields (dword cs / 2; pair (cs % 2) 4 + p at bits
//                 2k and 16 + 2k for j = 2p, 2p + 1).
//   [1024, 2048)  value codes [64 lanes][16 B]: lane l dword d holds tiles
//                 2d, 2d + 1 (channel 16 r8 + l % 16) at tokens tok(l / 16, j),
//                 pair hh 4 + p for j = 2p, 2p + 1.
//   [2048, 2560)  key scale / zero point fp16 [4 cs][4 q][8 scale, 8 zp] for
//                 channels 32 cs + 8 q + j (the group's per-channel affine).
//   [2560, 3072)  value scale / zero point fp16 [4 q][8 j][4 groups][2] of
//                 token tok(q, j) (per-token affine of each 32 channels).
// tok(q, j) = 16 (j / 4) + 4 q + j % 4 is the token the score MFMA leaves in
// lane group q, register j % 4 of tile j / 4.
// Residual window: keys and values bf16 [P][RES_CAP][128].
constexpr int GROUP_BYTES = 3072;

struct KiviArgs {
  const uint16_t* qkv;
  int64_t qkv_ld;
  const uint16_t* cos;
  const uint16_t* sin;
  const uint8_t* main;
  uint16_t* kr;
  uint16_t* vr;
  int32_t n_groups, n_res, nkv, nq, splits;
  float scale_log2;
  float* part;
};


VH_DEV uint16_t rope1(const uint16_t* base, const uint16_t* cs, const uint16_t* sn, int c) {
  const float x = bf2f(base[c]);
  const float xr = c < HEAD_DIM / 2 ? -bf2f(base[c + HEAD_DIM / 2]) : bf2f(base[c - HEAD_DIM / 2]);
  return (uint16_t)f2bf(rbf(x * bf2f(cs[c])) + rbf(xr * bf2f(sn[c])));
}

VH_DEV uint32_t pack_h2(float a, float b) {
  const f16x2 h = {(_Float16)a, (_Float16)b};
  return __builtin_bit_cast(uint32_t, h);
}

// Cross-lane reductions: DPP row rotations (row_ror:4 / :8, lane i reads
// lane (i - 4) / (i - 8) mod 16 of its row) combine the four group columns of
// a head (lanes n, n + 4, n + 8, n + 12 of a 16-lane row).
VH_DEV float ror4(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x124, 0xf, 0xf, false));
}
VH_DEV float ror8(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x128, 0xf, 0xf, false));
}
// lane l and lane l ^ 16 (l ^ 32)
VH_DEV float sum_x16(float v) { return v + __shfl_xor(v, 16); }
VH_DEV float sum_x32(float v) { return v + __shfl_xor(v, 32); }
VH_DEV float max_x16(float v) { return fmaxf(v, __shfl_xor(v, 16)); }
VH_DEV float max_x32(float v) { return fmaxf(v, __shfl_xor(v, 32)); }

// Code operands: the pair of 2-bit fields at bits 2p and 16 + 2p of W
// becomes the fp16 pair (1024 + c * 4**p), one v_and_or_b32 with a mask
// held in a VGPR; the 4**-p goes into the other operand.  mk[p] =
// 0x00030003 << 2p.
struct CodeMasks {
  uint32_t mk[4];
};

VH_DEV CodeMasks code_masks() {
  CodeMasks m;
#pragma unroll
  for (int p = 0; p < 4; ++p) asm volatile("v_mov_b32 %0, %1" : "=v"(m.mk[p]) : "i"(0x00030003u << (2 * p)));
  return m;
}

// The four operand dwords of pairs kb .. kb + 3 (kb = 0 or 4) of W.
VH_DEV f16x8 code_operand(uint32_t W, int kb, const CodeMasks& m) {
  const uint32_t w = kb ? (W >> 8) : W;
  return __builtin_bit_cast(f16x8, make_uint4((w & m.mk[0]) | 0x64006400u, (w & m.mk[1]) | 0x64006400u,
                                              (w & m.mk[2]) | 0x64006400u, (w & m.mk[3]) | 0x64006400u));
}

VH_DEV uint4 sel4(bool c, const uint4& v) { return c ? v : make_uint4(0u, 0u, 0u, 0u); }

constexpr float V_SCALE = 256.0f;  // value operands carry 2**8 (kept clear of fp16 subnormals)

// One super-step (ng of 4 consecutive 32-token groups staged at blk0) for one
// wave, from a fresh softmax state.  MFMA column n = lane % 16 is (group
// gq = n / 4, head h = n % 4): the lane's B operands (q * s for keys, p * s
// for values) are built once, for its own group.  Scores come from per-group
// accumulators (each column reads its own group's); the value MFMAs take the
// operand masked to the group.  The +1024 offset of the code operands is one
// MFMA against a constant operand.  Outputs: the head's max m (all lanes of
// the head), the lane's partial sum, acc (o^T, scaled by V_SCALE, column n)
// and zt (the zero-point and offset terms of column n, per channel group,
// partial over the lane group q).
VH_DEV void main_superstep(const uint8_t* blk0, int ng, const uint4 (&qh)[4], int lane, float scale_log2, float& m,
                           float& lsum, f32x4 (&acc)[8], float (&zt)[4]) {
  const int n = lane & 15, q = lane >> 4, gq = n >> 2;
  const bool own_live = gq < ng;
  const uint8_t* own = blk0 + gq * GROUP_BYTES;
  const CodeMasks cm = code_masks();
  const f16x8 ONE = __builtin_bit_cast(f16x8, make_uint4(0x64006400u, 0x64006400u, 0x64006400u, 0x64006400u));
  // keys: (q * s) * 4**-p of the own group (fp16) and the zero-point term
  f16x8 Bk[4];
  float bias = 0.0f;
#pragma unroll
  for (int cs = 0; cs < 4; ++cs) {
    const f16x8 sv = *(const f16x8*)(own + 2048 + (cs * 4 + q) * 32);
    const f16x8 zv = *(const f16x8*)(own + 2048 + (cs * 4 + q) * 32 + 16);
    const uint32_t qw[4] = {qh[cs].x, qh[cs].y, qh[cs].z, qh[cs].w};
    uint32_t bq[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const float q0 = bf2f(qw[p] & 0xffffu) * (float)sv[2 * p];
      const float q1 = bf2f(qw[p] >> 16) * (float)sv[2 * p + 1];
      bias = fmaf(q0, (float)zv[2 * p], bias);
      bias = fmaf(q1, (float)zv[2 * p + 1], bias);
      const float f = 1.0f / (float)(1 << (2 * p));
      bq[p] = pack_h2(q0 * f, q1 * f);
    }
    Bk[cs] = __builtin_bit_cast(f16x8, make_uint4(bq[0], bq[1], bq[2], bq[3]));
  }
  f32x4 Sc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int cs = 0; cs < 4; ++cs) Sc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ONE, Bk[cs], Sc, 0, 0, 0);
  f32x4 S[4][2];
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    S[g][0] = {0.0f, 0.0f, 0.0f, 0.0f};
    S[g][1] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (g >= ng) continue;
    const uint8_t* blk = blk0 + g * GROUP_BYTES;
    const uint2 kc0 = *(const uint2*)(blk + lane * 8);
    const uint2 kc1 = *(const uint2*)(blk + 512 + lane * 8);
#pragma unroll
    for (int cs = 0; cs < 4; ++cs) {
      const int kb = (cs & 1) * 4;
      S[g][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(code_operand(cs < 2 ? kc0.x : kc0.y, kb, cm), Bk[cs], S[g][0],
                                                      0, 0, 0);
      S[g][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(code_operand(cs < 2 ? kc1.x : kc1.y, kb, cm), Bk[cs], S[g][1],
                                                      0, 0, 0);
    }
  }
  bias = sum_x32(sum_x16(bias));
  const float off = Sc[0] + bias;
  float sc[2][4];
  float mloc = -__builtin_inff();
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float v = gq == 0 ? S[0][t][r] : gq == 1 ? S[1][t][r] : gq == 2 ? S[2][t][r] : S[3][t][r];
      sc[t][r] = own_live ? (v - off) * scale_log2 : -__builtin_inff();
      mloc = fmaxf(mloc, sc[t][r]);
    }
  mloc = fmaxf(mloc, ror4(mloc));
  mloc = fmaxf(mloc, ror8(mloc));
  m = max_x32(max_x16(mloc));
  float p[8];
  lsum = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    p[j] = exp2f(sc[j >> 2][j & 3] - m);
    lsum += p[j];
  }
  // values: (p * s) * 2**8 * 4**-pp of the own group per channel group
  f16x8 Bv[4];
#pragma unroll
  for (int gc = 0; gc < 4; ++gc) {
    uint32_t pw[4];
    zt[gc] = 0.0f;
#pragma unroll
    for (int pp = 0; pp < 4; ++pp) {
      const f16x8 e0 = *(const f16x8*)(own + 2560 + (q * 8 + 2 * pp) * 16);
      const f16x8 e1 = *(const f16x8*)(own + 2560 + (q * 8 + 2 * pp + 1) * 16);
      // (an absent group's block is a staged copy of a present one: finite, and its p are 0)
      const float p0 = p[2 * pp] * (float)e0[2 * gc], p1 = p[2 * pp + 1] * (float)e1[2 * gc];
      zt[gc] = fmaf(p0, (float)e0[2 * gc + 1], zt[gc]);
      zt[gc] = fmaf(p1, (float)e1[2 * gc + 1], zt[gc]);
      const float f = V_SCALE / (float)(1 << (2 * pp));
      pw[pp] = pack_h2(p0 * f, p1 * f);
    }
    Bv[gc] = __builtin_bit_cast(f16x8, make_uint4(pw[0], pw[1], pw[2], pw[3]));
    // the +1024 offset of the value codes, for this column (lane group 0 only)
    f32x4 vc = {0.0f, 0.0f, 0.0f, 0.0f};
    vc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ONE, Bv[gc], vc, 0, 0, 0);
    if (q == 0) zt[gc] += vc[0] * (1.0f / V_SCALE);
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    if (g >= ng) break;
    const uint4 vcode = *(const uint4*)(blk0 + g * GROUP_BYTES + 1024 + lane * 16);
    const uint32_t vw[4] = {vcode.x, vcode.y, vcode.z, vcode.w};
    f16x8 Bm[4];
#pragma unroll
    for (int gc = 0; gc < 4; ++gc) Bm[gc] = __builtin_bit_cast(f16x8, sel4(gq == g, __builtin_bit_cast(uint4, Bv[gc])));
#pragma unroll
    for (int r8 = 0; r8 < 8; ++r8)
      acc[r8] = __builtin_amdgcn_mfma_f32_16x16x32_f16(code_operand(vw[r8 >> 1], (r8 & 1) * 4, cm), Bm[r8 >> 1],
                                                      acc[r8], 0, 0, 0);
  }
}

// Workgroups (split, P) stream the main cache: each wave stages one
// super-step (GROUPS_PER_WAVE groups, 12 KB) in LDS and computes it.
__global__ void __launch_bounds__(ATT_WAVES * 64) k_kivi_split(KiviArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t s_q[GQA][HEAD_DIM];
  __shared__ __attribute__((aligned(16))) uint4 s_stage[ATT_WAVES][GROUPS_PER_WAVE * GROUP_BYTES / 16];
  float (*s_part)[GQA][PART] = (float (*)[GQA][PART])&s_stage[0][0];  // reused once the waves are done
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int P = blockIdx.y, split = blockIdx.x;
  const int b = P / a.nkv, kvh = P % a.nkv;
  const int n = lane & 15, q = lane >> 4;
  const uint16_t* qrow = a.qkv + (int64_t)b * a.qkv_ld;

  // this wave's blocks go out before anything else
  // (a partial super-step re-reads its last group for the absent ones; they are masked)
  const int g0 = split * STEPS_PER_SPLIT + wave * GROUPS_PER_WAVE;
  const int ng = max(0, min(GROUPS_PER_WAVE, a.n_groups - g0));
  static_assert(GROUPS_PER_WAVE == 4, "the prefetch registers below are spelled out for 4 groups");
  uint4 pa0, pa1, pa2, pb0, pb1, pb2, pc0, pc1, pc2, pd0, pd1, pd2;  // [group][third of the block]
  const uint4* gsrc = (const uint4*)(a.main + ((int64_t)P * a.n_groups + g0) * GROUP_BYTES) + lane;
  if (ng > 0) {
    const uint4* ga = gsrc;
    const uint4* gb = gsrc + min(1, ng - 1) * (GROUP_BYTES / 16);
    const uint4* gc = gsrc + min(2, ng - 1) * (GROUP_BYTES / 16);
    const uint4* gd = gsrc + min(3, ng - 1) * (GROUP_BYTES / 16);
    pa0 = ga[0]; pa1 = ga[64]; pa2 = ga[128];
    pb0 = gb[0]; pb1 = gb[64]; pb2 = gb[128];
    pc0 = gc[0]; pc1 = gc[64]; pc2 = gc[128];
    pd0 = gd[0]; pd1 = gd[64]; pd2 = gd[128];
  }
  for (int i = tid; i < GQA * HEAD_DIM; i += ATT_WAVES * 64) {
    const int h = i / HEAD_DIM, c = i % HEAD_DIM;
    s_q[h][c] = rope1(qrow + (kvh * GQA + h) * HEAD_DIM, a.cos, a.sin, c);
  }
  if (ng > 0) {
    uint4* sa = s_stage[wave] + lane;
    uint4* sb = sa + GROUP_BYTES / 16;
    uint4* sc = sb + GROUP_BYTES / 16;
    uint4* sd = sc + GROUP_BYTES / 16;
    sa[0] = pa0; sa[64] = pa1; sa[128] = pa2;
    sb[0] = pb0; sb[64] = pb1; sb[128] = pb2;
    sc[0] = pc0; sc[64] = pc1; sc[128] = pc2;
    sd[0] = pd0; sd[64] = pd1; sd[128] = pd2;
  }
  __syncthreads();

  float m = -__builtin_inff(), lsum = 0.0f;
  f32x4 acc[8];
  float zt[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (ng > 0) {
    uint4 qh[4];
#pragma unroll
    for (int cs = 0; cs < 4; ++cs) qh[cs] = *(const uint4*)&s_q[n & 3][cs * 32 + q * 8];
    main_superstep((const uint8_t*)s_stage[wave], ng, qh, lane, a.scale_log2, m, lsum, acc, zt);
  }
  // columns -> heads: o = acc / V_SCALE - zt summed over the four group
  // columns of the head (and zt over the lane groups)
#pragma unroll
  for (int gc = 0; gc < 4; ++gc) zt[gc] = sum_x32(sum_x16(zt[gc]));
#pragma unroll
  for (int r8 = 0; r8 < 8; ++r8)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float v = acc[r8][r] * (1.0f / V_SCALE) - zt[r8 >> 1];
      v += ror4(v);
      v += ror8(v);
      acc[r8][r] = v;
    }
  lsum += ror4(lsum);
  lsum += ror8(lsum);
  lsum = sum_x32(sum_x16(lsum));
  __syncthreads();  // the stage area becomes s_part
  // wave result in lanes n < 4 (head n): o[ch] for ch = 16 r8 + 4 q + r
  if (n < GQA) {
#pragma unroll
    for (int r8 = 0; r8 < 8; ++r8)
#pragma unroll
      for (int r = 0; r < 4; ++r) s_part[wave][n][2 + r8 * 16 + q * 4 + r] = acc[r8][r];
    if (q == 0) {
      s_part[wave][n][0] = m;
      s_part[wave][n][1] = lsum;
    }
  }
  __syncthreads();
  // merge the waves: thread (h, pair of channels)
  const int h = tid >> 6, c2 = (tid & 63) * 2;
  float M = -__builtin_inff();
#pragma unroll
  for (int w = 0; w < ATT_WAVES; ++w) M = fmaxf(M, s_part[w][h][0]);
  float L = 0.0f, o0 = 0.0f, o1 = 0.0f;
#pragma unroll
  for (int w = 0; w < ATT_WAVES; ++w) {
    const float mw = s_part[w][h][0];
    const float f = mw == -__builtin_inff() ? 0.0f : exp2f(mw - M);
    L = fmaf(f, s_part[w][h][1], L);
    o0 = fmaf(f, s_part[w][h][2 + c2], o0);
    o1 = fmaf(f, s_part[w][h][3 + c2], o1);
  }
  float* out = a.part + (((int64_t)P * a.splits + split) * GQA + h) * PART;
  if ((tid & 63) == 0) {
    out[0] = M;
    out[1] = L;
  }
  out[2 + c2] = o0;
  out[3 + c2] = o1;
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
  const int bh = blockIdx.x, b = bh / a.nq, H = bh % a.nq, kvh = H / GQA, h = H % GQA;
  const int P = b * a.nkv + kvh, tid = threadIdx.x;
  const int c = tid & (HEAD_DIM - 1);              // channel (first half of the block: merge / output)
  const int tk = tid >> 1, kh = tid & 1;           // key row tk, channel half kh
  const int co = tid & 15, ts = tid >> 4;          // value octet co, token subset ts (slots ts + 16u)
  const uint16_t* qrow = a.qkv + (int64_t)b * a.qkv_ld;
  // every independent load goes out first (one round trip)
  uint4 kw[HEAD_DIM / 16], vw[RES_CAP / 16];
  const uint4* kp = (const uint4*)(a.kr + ((int64_t)P * RES_CAP + tk) * HEAD_DIM + kh * (HEAD_DIM / 2));
  const uint4* vp = (const uint4*)(a.vr + (int64_t)P * RES_CAP * HEAD_DIM) + co;
#pragma unroll
  for (int i = 0; i < HEAD_DIM / 16; ++i) kw[i] = tk < a.n_res ? kp[i] : make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
  for (int u = 0; u < RES_CAP / 16; ++u)
    vw[u] = ts + 16 * u < a.n_res ? vp[(int64_t)(ts + 16 * u) * (HEAD_DIM / 8)] : make_uint4(0u, 0u, 0u, 0u);
  const float* base = a.part + ((int64_t)P * a.splits * GQA + h) * PART;
  float pm[COMBINE_PRELOAD], pl[COMBINE_PRELOAD], po[COMBINE_PRELOAD];
  const bool merger = tid < HEAD_DIM;
#pragma unroll
  for (int s = 0; s < COMBINE_PRELOAD; ++s) {
    const bool ok = merger && s < a.splits;
    const float* ps = base + (int64_t)s * GQA * PART;
    pm[s] = ok ? ps[0] : -__builtin_inff();
    pl[s] = ok ? ps[1] : 0.0f;
    po[s] = ok ? ps[2 + c] : 0.0f;
  }
  // RoPE of this step's query / key (channel c; the second half of the block duplicates)
  const float qc = bf2f(rope1(qrow + H * HEAD_DIM, a.cos, a.sin, c));
  const uint16_t kn = rope1(qrow + (a.nq + kvh) * HEAD_DIM, a.cos, a.sin, c);
  const uint16_t vn = qrow[(a.nq + a.nkv + kvh) * HEAD_DIM + c];
  if (merger) s_q[c] = qc;
  // this step's own score, q . k_new
  const float s_new = block_sum256(merger ? qc * bf2f(kn) : 0.0f, s_red) * a.scale_log2;
  if (h == 0 && merger) {
    // this step's key (after RoPE) and value enter residual slot n_res (read
    // by later steps only: this step takes them from the qkv row)
    a.kr[((int64_t)P * RES_CAP + a.n_res) * HEAD_DIM + c] = kn;
    a.vr[((int64_t)P * RES_CAP + a.n_res) * HEAD_DIM + c] = vn;
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
  if (tk < a.n_res) sc = acc * a.scale_log2;
  else if (tk == a.n_res) sc = s_new;
  const float mr = block_max256(kh == 0 ? sc : -__builtin_inff(), s_red);
  const float p = tk <= a.n_res ? exp2f(sc - mr) : 0.0f;
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
  if (!merger) return;
  float orr = s_p[a.n_res] * bf2f(vn);
#pragma unroll
  for (int t16 = 0; t16 < 16; ++t16) orr += s_o[t16][c];
  // merge with the main-cache splits
  float M = mr;
#pragma unroll
  for (int s = 0; s < COMBINE_PRELOAD; ++s) M = fmaxf(M, pm[s]);
  for (int s = COMBINE_PRELOAD; s < a.splits; ++s) M = fmaxf(M, base[(int64_t)s * GQA * PART]);
  const float fr = exp2f(mr - M);
  float L = lr * fr, O = orr * fr;
#pragma unroll
  for (int s = 0; s < COMBINE_PRELOAD; ++s) {
    const float f = pm[s] == -__builtin_inff() ? 0.0f : exp2f(pm[s] - M);
    L = fmaf(f, pl[s], L);
    O = fmaf(f, po[s], O);
  }
  for (int s = COMBINE_PRELOAD; s < a.splits; ++s) {
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

// Bake the main cache: one thread per (P, g, lane) writes its key codes
// (2 x 8 B), value codes (16 B) and one 16-byte piece of the scale / zero
// point quarter (lanes 0-31 keys, 32-63 values).
__global__ void __launch_bounds__(256) k_bake_kivi(const uint8_t* __restrict__ kcode, const uint16_t* __restrict__ ks,
                                                   const uint16_t* __restrict__ kz, const uint8_t* __restrict__ vcode,
                                                   const uint16_t* __restrict__ vs, const uint16_t* __restrict__ vz,
                                                   int64_t P, int64_t T, uint8_t* __restrict__ out) {
  const int64_t G = T / KV_GROUP;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= P * G * 64) return;
  const int lane = (int)(t % 64), q = lane >> 4;
  const int64_t g = (t / 64) % G, p = t / (64 * G);
  uint8_t* blk = out + (p * G + g) * GROUP_BYTES;
  // keys: tile tt, token 32 g + 16 tt + lane % 16
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) {
    const uint8_t* src = kcode + (p * T + g * KV_GROUP + tt * 16 + (lane & 15)) * HEAD_DIM;
    uint32_t w[2] = {0u, 0u};
#pragma unroll
    for (int cs = 0; cs < 4; ++cs)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint32_t c = src[cs * 32 + q * 8 + j] & 3u;
        const int k = (cs & 1) * 4 + j / 2;
        w[cs >> 1] |= c << ((j & 1) * 16 + 2 * k);
      }
    *(uint2*)(blk + tt * 512 + lane * 8) = make_uint2(w[0], w[1]);
  }
  // values: tile r8 (channel 16 r8 + lane % 16), tokens tok(q, j)
  uint32_t v[4] = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int r8 = 0; r8 < 8; ++r8)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t tok = g * KV_GROUP + 16 * (j / 4) + 4 * q + (j % 4);
      const uint32_t c = vcode[(p * T + tok) * HEAD_DIM + r8 * 16 + (lane & 15)] & 3u;
      const int k = (r8 & 1) * 4 + j / 2;
      v[r8 >> 1] |= c << ((j & 1) * 16 + 2 * k);
    }
  *(uint4*)(blk + 1024 + lane * 16) = make_uint4(v[0], v[1], v[2], v[3]);
  _Float16 piece[8];
  if (lane < 32) {
    // key piece: slot (cs, qq) = lane / 2, half 0 scale / 1 zp
    const int slot = lane >> 1, cs = slot >> 2, qq = slot & 3;
    const uint16_t* src = ((lane & 1) ? kz : ks) + (p * G + g) * HEAD_DIM + cs * 32 + qq * 8;
#pragma unroll
    for (int j = 0; j < 8; ++j) piece[j] = (_Float16)bf2f(src[j]);
    *(f16x8*)(blk + 2048 + lane * 16) = *(const f16x8*)piece;
  } else {
    // value piece: (qq, j) = (lane - 32) / 8, % 8 -> 4 groups x (scale, zp)
    const int i = lane - 32, qq = i >> 3, j = i & 7;
    const int64_t tok = g * KV_GROUP + 16 * (j / 4) + 4 * qq + (j % 4);
#pragma unroll
    for (int gc = 0; gc < 4; ++gc) {
      piece[2 * gc] = (_Float16)bf2f(vs[(p * T + tok) * 4 + gc]);
      piece[2 * gc + 1] = (_Float16)bf2f(vz[(p * T + tok) * 4 + gc]);
    }
    *(f16x8*)(blk + 2560 + i * 16) = *(const f16x8*)piece;
  }
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
                            int64_t T, uint8_t* main_out, vh_stream_t stream) {
  VH_REQUIRE(k_codes && k_scale && k_zp && v_codes && v_scale && v_zp && main_out, "vh_kivi_bake: null argument");
  VH_REQUIRE(P > 0 && T > 0 && T % KV_GROUP == 0, "vh_kivi_bake: needs T %% 32 == 0");
  const int64_t G = T / KV_GROUP;
  hipLaunchKernelGGL(k_bake_kivi, dim3(blocks_for(P * G * 64, 256)), dim3(256), 0, vh::as_stream(stream), k_codes,
                     k_scale, k_zp, v_codes, v_scale, v_zp, P, T, main_out);
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

extern "C" int vh_kivi_attention(const vh_kivi_desc* d, vh_stream_t stream) {
  VH_REQUIRE(d && d->qkv && d->cos && d->sin && d->kr && d->vr && d->attn_fq && d->flag,
             "vh_kivi_attention: null argument");
  VH_REQUIRE(d->batch >= 1 && d->nkv >= 1 && d->nq == GQA * d->nkv, "vh_kivi_attention: needs nq == 4 nkv");
  VH_REQUIRE(d->head_dim == HEAD_DIM, "vh_kivi_attention: head_dim must be %d", HEAD_DIM);
  VH_REQUIRE(d->n_main >= 0 && d->n_main % KV_GROUP == 0, "vh_kivi_attention: n_main must be a multiple of 32");
  VH_REQUIRE(d->n_main == 0 || d->main, "vh_kivi_attention: missing main cache");
  VH_REQUIRE(d->n_res >= 0 && d->n_res < RES_CAP, "vh_kivi_attention: n_res must be in [0, %d)", RES_CAP);
  VH_REQUIRE(d->qkv_ld >= (int64_t)(d->nq + 2 * d->nkv) * HEAD_DIM, "vh_kivi_attention: qkv_ld too small");
  const int G = (int)(d->n_main / KV_GROUP);
  const int splits = (G + STEPS_PER_SPLIT - 1) / STEPS_PER_SPLIT;
  VH_REQUIRE(d->part_floats >= (int64_t)d->batch * d->nkv * splits * GQA * PART,
             "vh_kivi_attention: workspace too small (needs %lld floats)",
             (long long)d->batch * d->nkv * splits * GQA * PART);
  VH_REQUIRE(splits == 0 || d->part, "vh_kivi_attention: missing workspace");
  KiviArgs a{d->qkv, d->qkv_ld, d->cos, d->sin, d->main, d->kr, d->vr, G, (int32_t)d->n_res, (int32_t)d->nkv,
             (int32_t)d->nq, splits, d->softmax_scale * 1.4426950408889634f, d->part};
  hipStream_t s = vh::as_stream(stream);
  const unsigned P = (unsigned)(d->batch * d->nkv);
  if (splits > 0) hipLaunchKernelGGL(k_kivi_split, dim3((unsigned)splits, P), dim3(ATT_WAVES * 64), 0, s, a);
  hipLaunchKernelGGL(k_kivi_combine, dim3((unsigned)(d->batch * d->nq)), dim3(COMBINE_THREADS), 0, s, a, d->attn,
                     (_Float16*)d->attn_fq, (int*)d->flag);
  return vh::check_launch("vh_kivi_attention");
}
