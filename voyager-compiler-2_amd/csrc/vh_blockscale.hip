// Block-scaled quantization: quantize_mx / calculate_mx_qparam
// (ops/quantized.py:958-1115) and quantize_affine (ops/quantized.py:1218-1283).
//
// A tensor is seen as contiguous [outer, L, inner] with blocks of `block`
// elements along L (the reference's _reshape_to_blocks, mx_utils.py:66-125:
// a partial last block is zero-padded for the reduction).
//
// Row path (inner == 1, L % 8 == 0, block % 8 == 0, block <= 512): each
// thread holds 8 consecutive elements (one 16-byte bf16 load); the block's
// reduction is a butterfly over block/8 lanes of the wavefront (no LDS), so
// every element is read from HBM exactly once and codes + scales are written
// once.  Up to 2**18 elements with blocks of at most 64, one element per
// lane instead (the block's butterfly spans block lanes).  Column path
// (everything else): one thread per (outer, block, inner) column,
// consecutive threads on consecutive `inner` for coalescing.
#include <hip/hip_runtime.h>

#include <cstring>

#include "vh_blockscale.h"
#include "vh_device.h"
#include "vh_host.h"

namespace {

// Stage the code remap table in LDS (256 bytes); every thread must call it.
VH_DEV void stage_code_lut(const Params& P, uint8_t* clut) {
  if (P.code_lut) {
    for (int i = threadIdx.x; i < 256; i += blockDim.x) clut[i] = P.code_lut[i];
    __syncthreads();
  }
}

// LEAN >= 0: the instance for bf16 input, packed codes and scale bytes, no
// code remap, global scale or block-major scales, in mode LEAN -- the
// runtime fields are replaced by those constants in a local copy of the
// parameters, so the compiler drops every branch they decide (the same
// arithmetic: the same output).
template <int VEC, int KIND, int SKIND, int LEAN = -1>
__global__ void __launch_bounds__(256)
k_rows(const void* __restrict__ x, int64_t rows, int64_t L, int64_t nblk, int g, Params Pin,
       void* __restrict__ scale_out, void* __restrict__ zp_out, void* __restrict__ codes_out) {
  Params P = Pin;
  if constexpr (LEAN >= 0) {
    P.mode = LEAN;
    P.cdt = VH_BF16;
    P.codes_dtype = VH_U8;
    P.scale_dtype = VH_U8;
    P.code_lut = nullptr;
    P.gs = nullptr;
    P.scale_t16 = 0;
  }
  __shared__ uint16_t lds[2 * VH_MAX_STEPS];
  __shared__ uint16_t slds[2 * VH_MAX_STEPS];
  __shared__ uint8_t clut[256];
  const int64_t tpr = nblk * g;  // threads per row
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t row = t / tpr;
  const int64_t v = t % tpr;
  const bool live = row < rows && v * VEC < L;
  const int64_t base = row * L + v * VEC;
  // the element loads go out first; the table staging runs under their latency
  float xv[VEC];
  if (live) {
    if (VEC == 8 && P.cdt == VH_BF16) {
      uint4 raw = *(const uint4*)((const uint16_t*)x + base);
      uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        xv[2 * j] = bf2f(w[j] & 0xffffu);
        xv[2 * j + 1] = bf2f(w[j] >> 16);
      }
    } else {
#pragma unroll
      for (int j = 0; j < VEC; ++j) xv[j] = load_x(x, P.cdt, base + j);
    }
  } else {
#pragma unroll
    for (int j = 0; j < VEC; ++j) xv[j] = 0.0f;  // zero padding of a partial block
  }
  // (the tables are read from the kernel argument: indexing the local copy
  // by thread would keep it in memory)
  if constexpr (KIND == K_STEPS) stage_steps(Pin.fmt, lds);
  if constexpr (SKIND == K_STEPS || SKIND == K_RUNTIME) stage_steps(Pin.sfmt, slds);
  stage_code_lut(P, clut);
  float hi, lo;
  if (P.mode == AFFINE) {
    hi = xv[0];
    lo = xv[0];
#pragma unroll
    for (int j = 1; j < VEC; ++j) {
      hi = nmax(hi, xv[j]);
      lo = nmin(lo, xv[j]);
    }
  } else {
    hi = fabsf(xv[0]);
#pragma unroll
    for (int j = 1; j < VEC; ++j) hi = nmax(hi, fabsf(xv[j]));
  }
  // butterfly over the g lanes of this block (g is a power of two <= 64)
  for (int off = 1; off < g; off <<= 1) {
    hi = nmax(hi, __shfl_xor(hi, off));
    if (P.mode == AFFINE) lo = nmin(lo, __shfl_xor(lo, off));
  }
  if (row >= rows) return;
  BlockScale bs = block_scale<SKIND>(hi, lo, P, slds);
  const int64_t blk = v / g;
  if ((v % g) == 0 && blk < nblk) {
    const int64_t si = P.scale_t16 ? blk * 16 + row : row * nblk + blk;
    if (P.scale_dtype == VH_U8) ((uint8_t*)scale_out)[si] = (uint8_t)bs.packed;
    else store_f(scale_out, P.scale_dtype, si, bs.scale);
    if (P.mode == AFFINE) store_f(zp_out, P.cdt, si, bs.zp);
  }
  if constexpr (KIND == K_NONE) return;
  if (!live || !codes_out) return;
  if constexpr (VEC == 8 && KIND == K_STEPS) {
    // Packed indices of a codebook of at most 16 levels (element_code's
    // steps for this case, no reference-form values): the eight searches
    // step together, so their LDS reads overlap.
    if (P.mode != AFFINE && P.cdt == VH_BF16 && P.codes_dtype == VH_U8 && !P.code_lut && P.fmt.nsteps <= 15) {
      const int ns = P.fmt.nsteps;
      uint32_t key[8], pos[8];
      bool nanv[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float q = div_bf16(xv[j], bs.el_scale);
        const uint32_t b = !isnan_f(q) ? (__float_as_uint(q) >> 16) : f2bf(q);
        nanv[j] = bf_isnan_bits(b);
        key[j] = bf_key(b);
        pos[j] = 0;
      }
#pragma unroll
      for (int step = 8; step >= 1; step >>= 1) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int nxt = (int)pos[j] + step;
          const bool ok = nxt <= ns && (uint32_t)lds[nxt <= ns ? nxt - 1 : 0] <= key[j];
          pos[j] = ok ? (uint32_t)nxt : pos[j];
        }
      }
      uint32_t c8[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) c8[j] = nanv[j] ? (uint32_t)P.fmt.nan_level : pos[j];
      uint2 pk;
      pk.x = c8[0] | (c8[1] << 8) | (c8[2] << 16) | (c8[3] << 24);
      pk.y = c8[4] | (c8[5] << 8) | (c8[6] << 16) | (c8[7] << 24);
      *(uint2*)((uint8_t*)codes_out + base) = pk;
      return;
    }
  }
  float cv[VEC];
  uint32_t cc[VEC];
#pragma unroll
  for (int j = 0; j < VEC; ++j) element_code<KIND>(xv[j], bs, P, lds, clut, &cv[j], &cc[j]);
  if (P.codes_dtype == VH_U8) {
    if constexpr (VEC == 8) {
      uint2 pk;
      pk.x = cc[0] | (cc[1] << 8) | (cc[2] << 16) | (cc[3] << 24);
      pk.y = cc[4] | (cc[5] << 8) | (cc[6] << 16) | (cc[7] << 24);
      *(uint2*)((uint8_t*)codes_out + base) = pk;
    } else {
#pragma unroll
      for (int j = 0; j < VEC; ++j) ((uint8_t*)codes_out)[base + j] = (uint8_t)cc[j];
    }
  } else if (VEC == 8 && P.cdt == VH_BF16) {
    uint4 pk;
    pk.x = f2bf(cv[0]) | (f2bf(cv[1]) << 16);
    pk.y = f2bf(cv[2]) | (f2bf(cv[3]) << 16);
    pk.z = f2bf(cv[4]) | (f2bf(cv[5]) << 16);
    pk.w = f2bf(cv[6]) | (f2bf(cv[7]) << 16);
    *(uint4*)((uint16_t*)codes_out + base) = pk;
  } else {
#pragma unroll
    for (int j = 0; j < VEC; ++j) store_f(codes_out, P.cdt, base + j, cv[j]);
  }
}

// quantize_mx with power-of-two scales to packed integer codes and scale
// bytes, bf16 rows (the MX-int8 form of configs 1 and 5 and the lowered
// graphs): block_scale (MX_POT) and element_code (K_INT) for that case
// restated without their runtime switches, NaN-propagating maxima as a
// plain max and a NaN flag -- the same values, codes and bytes.  Thread
// layout as k_rows<8>: eight consecutive elements, g = block / 8 lanes per
// block.
// IDX: the index type (32-bit when every thread index fits).  REF: the
// reference form instead of packed bytes -- codes as bf16 values (NaN kept,
// -0 kept) and the scales as bf16 values, as quantized_ops.quantize_mx
// returns them.
template <typename IDX, bool REF>
__global__ void __launch_bounds__(256)
k_mx_pot_int_rows8(const uint16_t* __restrict__ x, int64_t rows, int64_t L, int64_t nblk, int g, int shift,
                   int pot_bias, float lo, float hi, void* __restrict__ scale_out, void* __restrict__ codes_out) {
  const IDX tpr = (IDX)(nblk * g);
  const IDX t = (IDX)blockIdx.x * (IDX)blockDim.x + (IDX)threadIdx.x;
  const int64_t row = (int64_t)(t / tpr);
  const int64_t v = (int64_t)(t - (IDX)row * tpr);
  const bool live = row < rows && v * 8 < L;
  const int64_t base = row * L + v * 8;
  uint4 raw = make_uint4(0u, 0u, 0u, 0u);  // zero padding of a partial block
  if (live) raw = *(const uint4*)(x + base);
  const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
  float xv[8];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    xv[2 * j] = __uint_as_float(w[j] << 16);
    xv[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
  }
  // the block's amax over its g lanes (NaN-propagating, as one key)
  uint32_t mk = 0u;
#pragma unroll
  for (int j = 0; j < 8; ++j) mk = umax32(mk, amax_key(xv[j]));
  mk = group_umax_rt(mk, g);
  const uint32_t nan = mk == 0xFFFFFFFFu;
  const float m = __uint_as_float(mk);
  if (row >= rows) return;
  // the block's scale (block_scale, MX_POT, bf16)
  float s;
  int e = 0;
  bool inf = false;
  if (nan) {
    s = 1.0f;
  } else if (m == __builtin_inff()) {
    s = __builtin_inff();
    inf = true;
  } else {
    e = (m == 0.0f ? -126 : floor_log2(m)) - shift;
    s = rbf(ldexpf(1.0f, e));
    if (s == __builtin_inff()) inf = true;
    if (!(s > 0.0f)) {
      s = 1.0f;
      e = 0;
    }
  }
  const int64_t blk = v / g;
  if (v - blk * g == 0 && blk < nblk) {
    const int byte = inf ? 255 : e + pot_bias;
    if constexpr (REF) ((uint16_t*)scale_out)[row * nblk + blk] = (uint16_t)f2bf(s);
    else ((uint8_t*)scale_out)[row * nblk + blk] = (uint8_t)(byte < 0 ? 0 : (byte > 254 && !inf ? 254 : byte));
  }
  if (!live) return;
  // 1 / s exactly when s is a normal power of two: x * (1 / s) is x / s
  const uint32_t sb = __float_as_uint(s);
  const bool exact = s >= 0x1p-126f && s <= 0x1p126f && (sb & 0x7fffffu) == 0u;
  const float inv = __uint_as_float((uint32_t)(254 - (int)(sb >> 23)) << 23);
  float q[8];
  if (exact) {
#pragma unroll
    for (int j = 0; j < 8; ++j) q[j] = rbf(xv[j] * inv);
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) q[j] = div_bf16(xv[j], s);
  }
  uint32_t c[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float r = fminf(fmaxf(rintf(q[j]), lo), hi);
    if constexpr (REF) c[j] = q[j] != q[j] ? 0x7FC0u : f2bf(r);  // an integer: exact in bf16
    else c[j] = q[j] != q[j] ? 0u : ((uint32_t)(int32_t)r & 0xffu);
  }
  if constexpr (REF) {
    *(uint4*)((uint16_t*)codes_out + base) =
        make_uint4(c[0] | (c[1] << 16), c[2] | (c[3] << 16), c[4] | (c[5] << 16), c[6] | (c[7] << 16));
  } else {
    uint2 pk;
    pk.x = c[0] | (c[1] << 8) | (c[2] << 16) | (c[3] << 24);
    pk.y = c[4] | (c[5] << 8) | (c[6] << 16) | (c[7] << 24);
    *(uint2*)((uint8_t*)codes_out + base) = pk;
  }
}

// quantize_mx with a minifloat scale map to packed codebook indices (a
// table of at most 15 thresholds: the 16-level codebooks), bf16 rows:
// block_scale (MX_SCALED, no global scale) and element_code (K_STEPS) for
// that case restated without their runtime switches -- the same scale
// codes and indices.  Thread layout as k_rows<8>.
template <typename IDX>
__global__ void __launch_bounds__(256)
k_mx_steps_rows8(const uint16_t* __restrict__ x, int64_t rows, int64_t L, int64_t nblk, int g, float quant_max,
                 vh_format sfmt, vh_format fmt, uint8_t* __restrict__ scale_out, uint8_t* __restrict__ codes_out) {
  __shared__ uint16_t keys[16];
  const IDX tpr = (IDX)(nblk * g);
  const IDX t = (IDX)blockIdx.x * (IDX)blockDim.x + (IDX)threadIdx.x;
  const int64_t row = (int64_t)(t / tpr);
  const int64_t v = (int64_t)(t - (IDX)row * tpr);
  const bool live = row < rows && v * 8 < L;
  const int64_t base = row * L + v * 8;
  uint4 raw = make_uint4(0u, 0u, 0u, 0u);  // zero padding of a partial block
  if (live) raw = *(const uint4*)(x + base);
  // the thresholds, padded with 0xFFFF (steps_level_padded)
  if (threadIdx.x < 16) keys[threadIdx.x] = threadIdx.x < fmt.nsteps ? fmt.thr_key[threadIdx.x] : 0xFFFFu;
  __syncthreads();
  const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
  float xv[8];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    xv[2 * j] = __uint_as_float(w[j] << 16);
    xv[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
  }
  // the block's amax over its g lanes (NaN-propagating, as one key)
  uint32_t mk = 0u;
#pragma unroll
  for (int j = 0; j < 8; ++j) mk = umax32(mk, amax_key(xv[j]));
  mk = group_umax_rt(mk, g);
  const uint32_t nan = mk == 0xFFFFFFFFu;
  const float m = __uint_as_float(mk);
  if (row >= rows) return;
  const float hi = nan ? __uint_as_float(0x7fc00000u) : m;
  float s = div_bf16(hi, quant_max);
  s = rbf(fmt_value_k<K_MINI>(f2bf(s), sfmt, nullptr));
  if (!(s > 0.0f)) s = 1.0f;
  const int64_t blk = v / g;
  if (v - blk * g == 0 && blk < nblk) {
    const uint32_t b = f2bf(s);
    scale_out[row * nblk + blk] = (uint8_t)fmt_code_k<K_MINI>(b, bf2f(b), sfmt, nullptr);
  }
  if (!live) return;
  uint32_t key[8], pos[8];
  bool nanv[8];
  uint32_t bq[8];
  div_bf16_bits_n(xv, s, bq);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    nanv[j] = bf_isnan_bits(bq[j]);
    key[j] = bf_key(bq[j]);
    pos[j] = 0;
  }
  // steps_level_padded for the eight elements, stepping together
#pragma unroll
  for (int step = 8; step >= 1; step >>= 1) {
#pragma unroll
    for (int j = 0; j < 8; ++j) pos[j] = (uint32_t)keys[pos[j] + step - 1] <= key[j] ? pos[j] + step : pos[j];
  }
  uint32_t c[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) c[j] = nanv[j] ? (uint32_t)fmt.nan_level : pos[j];
  uint2 pk;
  pk.x = c[0] | (c[1] << 8) | (c[2] << 16) | (c[3] << 24);
  pk.y = c[4] | (c[5] << 8) | (c[6] << 16) | (c[7] << 24);
  *(uint2*)(codes_out + base) = pk;
}

// The same at decode sizes, one element per lane (a block's g lanes reduce
// it): the activation quantize ahead of the MXNF4 GEMV -- indices remapped
// through `clut` to the GEMV's levels when given, scales as float32 values
// (block-major [nblk][16] with t16) or packed codes.
__global__ void __launch_bounds__(256)
k_mx_steps_lanes(const uint16_t* __restrict__ x, int64_t rows, int64_t L, int64_t nblk, int g, float quant_max,
                 vh_format sfmt, vh_format fmt, int t16, int scale_f32, void* __restrict__ scale_out,
                 uint8_t* __restrict__ codes_out, const uint8_t* __restrict__ code_lut) {
  __shared__ __attribute__((aligned(4))) uint16_t keys[16];
  __shared__ uint8_t clut[256];
  // rows * L <= 2**18 (the launcher's bound): 32-bit indices; g divides L
  // and is a power of two, so the blocks are aligned groups of g lanes
  const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
  const uint32_t Lu = (uint32_t)L;
  const bool live = t < (uint32_t)(rows * L);
  const uint32_t row = t / Lu, v = t - row * Lu;
  // The loads go out together, before any wait: the element (index 0 past
  // the end), the thresholds through the scalar cache (spread over lanes
  // 0..7, padded with 0xFFFF for steps_level_padded) and the code map.
  const uint32_t xb = x[live ? t : 0u];
  const uint32_t* kw = (const uint32_t*)fmt.thr_key;
  const int lane = (int)(threadIdx.x & 63u);
  uint32_t kv = 0u;
#pragma unroll
  for (int i = 0; i < 8; ++i) kv = lane == i ? kw[i] : kv;
  const int ns = fmt.nsteps;
  kv = (2 * lane < ns ? kv & 0xffffu : 0xffffu) | (2 * lane + 1 < ns ? kv & 0xffff0000u : 0xffff0000u);
  uint32_t cl = 0u;
  if (code_lut) cl = code_lut[threadIdx.x];
  if (threadIdx.x < 8) *(uint32_t*)&keys[2 * threadIdx.x] = kv;
  if (code_lut) clut[threadIdx.x] = (uint8_t)cl;
  const float xv = live ? __uint_as_float(xb << 16) : 0.0f;
  // the block's amax (NaN-propagating) across its g lanes
  const uint32_t mk = group_umax_rt(amax_key(xv), g);
  __syncthreads();
  if (!live) return;
  const float hi = mk == 0xFFFFFFFFu ? __uint_as_float(0x7fc00000u) : __uint_as_float(mk);
  float s = div_bf16(hi, quant_max);
  s = rbf(fmt_value_k<K_MINI>(f2bf(s), sfmt, nullptr));
  if (!(s > 0.0f)) s = 1.0f;
  const uint32_t blk = v >> __builtin_ctz((unsigned)g);
  if ((v & ((uint32_t)g - 1u)) == 0u) {
    const uint32_t si = t16 ? blk * 16u + row : row * (uint32_t)nblk + blk;
    if (scale_f32) {
      ((float*)scale_out)[si] = s;
    } else {
      const uint32_t b = f2bf(s);
      ((uint8_t*)scale_out)[si] = (uint8_t)fmt_code_k<K_MINI>(b, bf2f(b), sfmt, nullptr);
    }
  }
  const float q = div_bf16(xv, s);
  const uint32_t b = !isnan_f(q) ? (__float_as_uint(q) >> 16) : f2bf(q);
  uint32_t c;
  if (bf_isnan_bits(b)) c = (uint32_t)fmt.nan_level;
  else c = steps_level_padded<8>(bf_key(b), keys);
  if (code_lut) c = clut[c & 0xffu];
  codes_out[t] = (uint8_t)c;
}

// One thread per (outer, block, inner) column.
template <int KIND, int SKIND>
__global__ void __launch_bounds__(256)
k_cols(const void* __restrict__ x, int64_t outer, int64_t L, int64_t inner, int64_t block, int64_t nblk, Params P,
       void* __restrict__ scale_out, void* __restrict__ zp_out, void* __restrict__ codes_out) {
  __shared__ uint16_t lds[2 * VH_MAX_STEPS];
  __shared__ uint16_t slds[2 * VH_MAX_STEPS];
  __shared__ uint8_t clut[256];
  if constexpr (KIND == K_STEPS) stage_steps(P.fmt, lds);
  if constexpr (SKIND == K_STEPS || SKIND == K_RUNTIME) stage_steps(P.sfmt, slds);
  stage_code_lut(P, clut);
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = outer * nblk * inner;
  if (t >= total) return;
  const int64_t in = t % inner;
  const int64_t blk = (t / inner) % nblk;
  const int64_t o = t / (inner * nblk);
  const int64_t l0 = blk * block;
  const int64_t l1 = l0 + block < L ? l0 + block : L;
  const int64_t base = o * L * inner + in;
  float hi, lo;
  if (P.mode == AFFINE) {
    hi = load_x(x, P.cdt, base + l0 * inner);
    lo = hi;
  } else {
    hi = 0.0f;
    lo = 0.0f;
  }
  for (int64_t l = l0; l < l1; ++l) {
    float xv = load_x(x, P.cdt, base + l * inner);
    if (P.mode == AFFINE) {
      hi = nmax(hi, xv);
      lo = nmin(lo, xv);
    } else {
      hi = nmax(hi, fabsf(xv));
    }
  }
  if (P.mode == AFFINE && l1 - l0 < block) {  // zero padding joins min and max
    hi = nmax(hi, 0.0f);
    lo = nmin(lo, 0.0f);
  }
  BlockScale bs = block_scale<SKIND>(hi, lo, P, slds);
  const int64_t si = (o * nblk + blk) * inner + in;
  if (P.scale_dtype == VH_U8) ((uint8_t*)scale_out)[si] = (uint8_t)bs.packed;
  else store_f(scale_out, P.scale_dtype, si, bs.scale);
  if (P.mode == AFFINE) store_f(zp_out, P.cdt, si, bs.zp);
  if constexpr (KIND == K_NONE) return;
  if (!codes_out) return;
  for (int64_t l = l0; l < l1; ++l) {
    int64_t i = base + l * inner;
    float cv;
    uint32_t cc;
    element_code<KIND>(load_x(x, P.cdt, i), bs, P, lds, clut, &cv, &cc);
    if (P.codes_dtype == VH_U8) ((uint8_t*)codes_out)[i] = (uint8_t)cc;
    else store_f(codes_out, P.cdt, i, cv);
  }
}

// Scale maps the configs use get their own kernels; any other map runs the
// runtime switch.
template <typename F>
int dispatch_scale(const Params& P, F&& fn) {
  if (!P.has_sfmt) return fn(std::integral_constant<int, K_NONE>{});
  const int k = kernel_kind(&P.sfmt);
  if (k == K_MINI) return fn(std::integral_constant<int, K_MINI>{});
  return fn(std::integral_constant<int, K_RUNTIME>{});
}

int launch(const void* x, int64_t outer, int64_t L, int64_t inner, int64_t block, const Params& P,
           void* scale_out, void* zp_out, void* codes_out, hipStream_t stream, const char* what) {
  const int64_t nblk = (L + block - 1) / block;
  const bool rows_ok = inner == 1 && L % 8 == 0 && block % 8 == 0 && block <= 512 &&
                       ((block / 8) & (block / 8 - 1)) == 0;
  // Small tensors (decode-size activations): one element per lane, so each
  // lane's dependent chain (scale map, element map) is an eighth as long and
  // there are eight times as many waves.
  const bool lanes_ok = inner == 1 && block <= 64 && (block & (block - 1)) == 0 && L % block == 0 &&
                        outer * L <= (1 << 18);
  // the decode-size activation quantize of the MXNF4 GEMV (and any small
  // tensor of that form) takes its own kernel
  const bool steps_lanes = lanes_ok && P.mode == MX_SCALED && P.cdt == VH_BF16 && P.codes_dtype == VH_U8 &&
                           (P.scale_dtype == VH_F32 || P.scale_dtype == VH_U8) && !P.gs && codes_out &&
                           P.has_fmt && kernel_kind(&P.fmt) == K_STEPS && P.fmt.nsteps <= 15 && P.has_sfmt &&
                           kernel_kind(&P.sfmt) == K_MINI;
  if (steps_lanes) {
    const int64_t threads = outer * L;
    hipLaunchKernelGGL(k_mx_steps_lanes, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream,
                       (const uint16_t*)x, outer, L, nblk, (int)block, P.quant_max, P.sfmt, P.fmt, P.scale_t16,
                       P.scale_dtype == VH_F32 ? 1 : 0, scale_out, (uint8_t*)codes_out, P.code_lut);
  } else if (lanes_ok) {
    const int g = (int)block;
    const int64_t threads = outer * nblk * g;
    const int64_t blocks = (threads + 255) / 256;
    dispatch_kind(P.has_fmt ? kernel_kind(&P.fmt) : (int)K_NONE, [&](auto kind) {
      constexpr int K = decltype(kind)::value;
      return dispatch_scale(P, [&](auto skind) {
        constexpr int S = decltype(skind)::value;
        hipLaunchKernelGGL((k_rows<1, K, S>), dim3((unsigned)blocks), dim3(256), 0, stream, x, outer, L, nblk, g, P,
                           scale_out, zp_out, codes_out);
        return 0;
      });
    });
  } else if (rows_ok) {
    const int g = (int)(block / 8);
    const int64_t threads = outer * nblk * g;
    const int64_t blocks = (threads + 255) / 256;
    VH_REQUIRE(blocks < (1ll << 31), "%s: tensor too large", what);
    // the packed forms the configs and lowered graphs run take a lean instance
    const bool lean = P.mode != AFFINE && P.cdt == VH_BF16 && P.codes_dtype == VH_U8 && P.scale_dtype == VH_U8 &&
                      !P.code_lut && !P.gs && !P.scale_t16 && codes_out && P.has_fmt;
    const int k0 = P.has_fmt ? kernel_kind(&P.fmt) : (int)K_NONE;
    // the same with reference-form outputs (bf16 codes and scales)
    const bool lean_ref = P.mode == MX_POT && P.cdt == VH_BF16 && P.codes_dtype == VH_BF16 &&
                          P.scale_dtype == VH_BF16 && !P.code_lut && !P.gs && !P.scale_t16 && codes_out &&
                          P.has_fmt && !P.has_sfmt && k0 == K_INT;
    if ((lean && P.mode == MX_POT && k0 == K_INT && !P.has_sfmt) || lean_ref) {
      const bool i32 = blocks * 256 < (1ll << 31);
      auto go = [&](auto kern) {
        hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(256), 0, stream, (const uint16_t*)x, outer, L, nblk, g,
                           P.shift, P.pot_bias, (float)P.fmt.p0, (float)P.fmt.p1, scale_out, codes_out);
      };
      if (lean_ref) {
        if (i32) go(k_mx_pot_int_rows8<uint32_t, true>);
        else go(k_mx_pot_int_rows8<int64_t, true>);
      } else {
        if (i32) go(k_mx_pot_int_rows8<uint32_t, false>);
        else go(k_mx_pot_int_rows8<int64_t, false>);
      }
    } else if (lean && P.mode == MX_SCALED && k0 == K_STEPS && P.has_sfmt && kernel_kind(&P.sfmt) == K_MINI) {
      if (P.fmt.nsteps <= 15) {
        if (blocks * 256 < (1ll << 31))
          hipLaunchKernelGGL(k_mx_steps_rows8<uint32_t>, dim3((unsigned)blocks), dim3(256), 0, stream,
                             (const uint16_t*)x, outer, L, nblk, g, P.quant_max, P.sfmt, P.fmt, (uint8_t*)scale_out,
                             (uint8_t*)codes_out);
        else
          hipLaunchKernelGGL(k_mx_steps_rows8<int64_t>, dim3((unsigned)blocks), dim3(256), 0, stream,
                             (const uint16_t*)x, outer, L, nblk, g, P.quant_max, P.sfmt, P.fmt, (uint8_t*)scale_out,
                             (uint8_t*)codes_out);
      } else {
        hipLaunchKernelGGL((k_rows<8, K_STEPS, K_MINI, MX_SCALED>), dim3((unsigned)blocks), dim3(256), 0, stream, x,
                           outer, L, nblk, g, P, scale_out, zp_out, codes_out);
      }
    } else {
      dispatch_kind(k0, [&](auto kind) {
        constexpr int K = decltype(kind)::value;
        return dispatch_scale(P, [&](auto skind) {
          constexpr int S = decltype(skind)::value;
          hipLaunchKernelGGL((k_rows<8, K, S>), dim3((unsigned)blocks), dim3(256), 0, stream, x, outer, L, nblk, g, P,
                             scale_out, zp_out, codes_out);
          return 0;
        });
      });
    }
  } else {
    const int64_t threads = outer * nblk * inner;
    const int64_t blocks = (threads + 255) / 256;
    VH_REQUIRE(blocks < (1ll << 31), "%s: tensor too large", what);
    dispatch_kind(P.has_fmt ? kernel_kind(&P.fmt) : (int)K_NONE, [&](auto kind) {
      constexpr int K = decltype(kind)::value;
      return dispatch_scale(P, [&](auto skind) {
        constexpr int S = decltype(skind)::value;
        hipLaunchKernelGGL((k_cols<K, S>), dim3((unsigned)blocks), dim3(256), 0, stream, x, outer, L, inner, block,
                           nblk, P, scale_out, zp_out, codes_out);
        return 0;
      });
    });
  }
  return vh::check_launch(what);
}

int check_common(const void* x, int32_t x_dtype, int64_t outer, int64_t L, int64_t inner, int64_t block,
                 const char* what) {
  VH_REQUIRE(x, "%s: null input", what);
  VH_REQUIRE(vh::is_float_dtype(x_dtype), "%s: input dtype %d unsupported", what, x_dtype);
  VH_REQUIRE(outer >= 0 && L >= 0 && inner >= 0, "%s: negative size", what);
  VH_REQUIRE(block > 0, "%s: block_size must be > 0", what);
  return VH_OK;
}

bool packable(const vh_format& f) {
  switch (f.kind) {
    case VH_FMT_INT: return (f.p0 >= -128 && f.p1 <= 127) || (f.p0 >= 0 && f.p1 <= 255);
    case VH_FMT_MINIFLOAT: return f.p0 + f.p1 + ((f.flags & VH_FMT_SIGNED) ? 1 : 0) <= 8;
    case VH_FMT_POSIT: return f.p0 <= 8;
    case VH_FMT_STEPS: return true;
    default: return false;
  }
}

int quantize_mx_impl(const void* x, int32_t x_dtype, int64_t outer, int64_t L, int64_t inner, int64_t block,
                     float quant_max, int32_t pot, const vh_format* scale_fmt, const void* global_scale,
                     int32_t gs_dtype, const vh_format* fmt, void* scale_out, int32_t scale_dtype, int32_t pot_bias,
                     void* codes_out, int32_t codes_dtype, const uint8_t* code_lut, int scale_t16,
                     vh_stream_t stream) {
  int rc;
  if ((rc = check_common(x, x_dtype, outer, L, inner, block, "vh_quantize_mx"))) return rc;
  VH_REQUIRE(scale_out, "vh_quantize_mx: null scale output");
  VH_REQUIRE(!codes_out || fmt, "vh_quantize_mx: codes need an element map");
  VH_REQUIRE(scale_dtype == x_dtype || scale_dtype == VH_U8 || scale_dtype == VH_F32,
             "vh_quantize_mx: scale dtype must be the input's, f32 or u8");
  VH_REQUIRE(!code_lut || codes_dtype == VH_U8, "vh_quantize_mx: a code remap needs packed codes");
  VH_REQUIRE(!codes_out || codes_dtype == x_dtype || codes_dtype == VH_U8,
             "vh_quantize_mx: codes dtype must be the input's or u8");
  VH_REQUIRE(!(codes_out && codes_dtype == VH_U8) || packable(*fmt), "vh_quantize_mx: element map has no packed form");
  VH_REQUIRE(!(scale_dtype == VH_U8 && !pot) || (scale_fmt && packable(*scale_fmt)),
             "vh_quantize_mx: packed scales need pot or a packable scale map");
  VH_REQUIRE(pot || quant_max != 0.0f, "vh_quantize_mx: quant_max must be nonzero");
  Params P;
  memset(&P, 0, sizeof(P));
  P.mode = pot ? MX_POT : MX_SCALED;
  P.cdt = x_dtype;
  P.quant_max = quant_max;
  if (pot) {
    VH_REQUIRE(quant_max > 0.0f, "vh_quantize_mx: quant_max must be positive for power-of-two scales");
    P.shift = (int)floorf(log2f(quant_max));
  }
  if (scale_fmt) {
    P.has_sfmt = 1;
    P.sfmt = *scale_fmt;
  }
  if (global_scale) {
    VH_REQUIRE(!pot, "vh_quantize_mx: a global scale needs non-power-of-two scales");
    VH_REQUIRE(vh::is_float_dtype(gs_dtype), "vh_quantize_mx: global scale dtype unsupported");
    P.gs = global_scale;
    P.gs_dtype = gs_dtype;
  }
  if (fmt) {
    P.has_fmt = 1;
    P.fmt = *fmt;
  }
  P.scale_dtype = scale_dtype;
  P.pot_bias = pot_bias;
  P.codes_dtype = codes_dtype;
  P.code_lut = code_lut;
  P.scale_t16 = scale_t16;
  if (outer * L * inner == 0) return VH_OK;
  return launch(x, outer, L, inner, block, P, scale_out, nullptr, codes_out, vh::as_stream(stream),
                "vh_quantize_mx");
}

}  // namespace

extern "C" int vh_quantize_mx(const void* x, int32_t x_dtype, int64_t outer, int64_t L, int64_t inner,
                              int64_t block, float quant_max, int32_t pot, const vh_format* scale_fmt,
                              const void* global_scale, int32_t gs_dtype, const vh_format* fmt, void* scale_out,
                              int32_t scale_dtype, int32_t pot_bias, void* codes_out, int32_t codes_dtype,
                              const uint8_t* code_lut, vh_stream_t stream) {
  return quantize_mx_impl(x, x_dtype, outer, L, inner, block, quant_max, pot, scale_fmt, global_scale, gs_dtype, fmt,
                          scale_out, scale_dtype, pot_bias, codes_out, codes_dtype, code_lut, 0, stream);
}

extern "C" int vh_quantize_mx_rows16(const void* x, int32_t x_dtype, int64_t rows, int64_t L, int64_t block,
                                     float quant_max, const vh_format* scale_fmt, const vh_format* fmt,
                                     float* scale_out, uint8_t* codes_out, const uint8_t* code_lut,
                                     vh_stream_t stream) {
  VH_REQUIRE(rows >= 1 && rows <= 16, "vh_quantize_mx_rows16: rows must be in [1, 16] (got %lld)", (long long)rows);
  VH_REQUIRE(L % block == 0, "vh_quantize_mx_rows16: L must be a multiple of block");
  return quantize_mx_impl(x, x_dtype, rows, L, 1, block, quant_max, 0, scale_fmt, nullptr, 0, fmt, scale_out, VH_F32,
                          0, codes_out, VH_U8, code_lut, 1, stream);
}

extern "C" int vh_quantize_affine(const void* x, int32_t x_dtype, int64_t outer, int64_t L, int64_t inner,
                                  int64_t block, float quant_min, float quant_max, const vh_format* scale_fmt,
                                  const vh_format* fmt, void* scale_out, void* zp_out, void* codes_out,
                                  int32_t codes_dtype, vh_stream_t stream) {
  int rc;
  if ((rc = check_common(x, x_dtype, outer, L, inner, block, "vh_quantize_affine"))) return rc;
  VH_REQUIRE(scale_out && zp_out, "vh_quantize_affine: null output");
  VH_REQUIRE(!codes_out || fmt, "vh_quantize_affine: codes need an element map");
  VH_REQUIRE(!codes_out || codes_dtype == x_dtype || codes_dtype == VH_U8, "vh_quantize_affine: bad codes dtype");
  VH_REQUIRE(!(codes_out && codes_dtype == VH_U8) || packable(*fmt),
             "vh_quantize_affine: element map has no packed form");
  Params P;
  memset(&P, 0, sizeof(P));
  P.mode = AFFINE;
  P.cdt = x_dtype;
  P.quant_max = quant_max;
  P.quant_min = quant_min;
  if (scale_fmt) {
    P.has_sfmt = 1;
    P.sfmt = *scale_fmt;
  }
  if (fmt) {
    P.has_fmt = 1;
    P.fmt = *fmt;
  }
  P.scale_dtype = x_dtype;
  P.codes_dtype = codes_dtype;
  if (outer * L * inner == 0) return VH_OK;
  return launch(x, outer, L, inner, block, P, scale_out, zp_out, codes_out, vh::as_stream(stream),
                "vh_quantize_affine");
}
