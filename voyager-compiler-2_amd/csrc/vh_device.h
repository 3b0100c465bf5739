// Device-side numeric formats of the quantized-operator path (gfx950).
//
// Every quantization map of the reference is a 65,536-entry table indexed by
// a bfloat16 bit pattern (ops/quantized.py:147-190, fake_quantize.py:68-122).
// Here each table family is a closed form evaluated in registers; the host
// only selects a closed form after a device kernel has rebuilt the caller's
// table from it and found every entry equal, so "closed form == table" holds
// by construction.  Unrecognised tables are gathered from memory (VH_FMT_LUT).
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "../../include/voyager_hip.h"

#define VH_DEV static __device__ __forceinline__

// ---------------------------------------------------------------- bf16 bits
VH_DEV float bf2f(uint32_t b) { return __uint_as_float(b << 16); }

// Round-to-nearest-even float32 -> bfloat16 bits; NaN -> canonical 0x7FC0.
VH_DEV uint32_t f2bf(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7FC0u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

// Two float32 values to packed bfloat16 bits (lo, hi) with the gfx950
// converter (v_cvt_pk_bf16_f32: round half to even, denormals kept).
typedef __bf16 vh_bf16x2 __attribute__((ext_vector_type(2)));
typedef float vh_f32x2 __attribute__((ext_vector_type(2)));
VH_DEV uint32_t f2bf2_hw(float lo, float hi) {
  vh_f32x2 v = {lo, hi};
  vh_bf16x2 h = __builtin_convertvector(v, vh_bf16x2);
  return __builtin_bit_cast(uint32_t, h);
}

// Streaming accesses that bypass cache residency (the nt bit): each element
// of a large elementwise op is touched once, so its lines should not evict
// data that is reused.  Measured from HBM (inputs rotated through more than
// the 256 MB Infinity Cache), the hint makes 8M-64M-element quantize streams
// 5-10% faster than plain accesses; with cache-resident inputs it is the
// other way round.  8- and 16-byte loads and stores.
typedef unsigned int vh_u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int vh_u32x2 __attribute__((ext_vector_type(2)));
VH_DEV uint4 ld_stream16(const void* p) {
  const vh_u32x4 v = __builtin_nontemporal_load((const vh_u32x4*)p);
  return make_uint4(v.x, v.y, v.z, v.w);
}
VH_DEV uint2 ld_stream8(const void* p) {
  const vh_u32x2 v = __builtin_nontemporal_load((const vh_u32x2*)p);
  return make_uint2(v.x, v.y);
}
VH_DEV void st_stream8(void* p, uint2 v) { __builtin_nontemporal_store(vh_u32x2{v.x, v.y}, (vh_u32x2*)p); }
VH_DEV void st_stream16(void* p, uint4 v) { __builtin_nontemporal_store(vh_u32x4{v.x, v.y, v.z, v.w}, (vh_u32x4*)p); }

// The float32 value rounded to bfloat16 and back (an eager bf16 op result).
VH_DEV float rbf(float f) { return bf2f(f2bf(f)); }

// float32 -> float16 -> float32 with round-to-nearest-even (an fp16 op result).
VH_DEV float rhf(float f) { return __half2float(__float2half_rn(f)); }

// Round a float32 value to the storage dtype of an eager op's result.
VH_DEV float round_to(float f, int dtype) {
  if (dtype == VH_BF16) return rbf(f);
  if (dtype == VH_F16) return rhf(f);
  return f;
}

VH_DEV bool isnan_f(float f) { return f != f; }

// NaN-propagating max/min, as torch.amax / torch.amin.
// (written as selects: the nested conditional compiled to branches)
VH_DEV float nmax(float a, float b) {
  const bool na = isnan_f(a), nb = isnan_f(b);
  const float m = fmaxf(a, b);
  const float n = na ? a : b;
  return (na | nb) ? n : m;
}
VH_DEV float nmin(float a, float b) {
  const bool na = isnan_f(a), nb = isnan_f(b);
  const float m = fminf(a, b);
  const float n = na ? a : b;
  return (na | nb) ? n : m;
}

// RNE_bf16(RN_f32(x / s)), the result of an eager bfloat16 division.
// x * rcp(s) is within 3 float32 ulps of RN_f32(x / s) when s and 1/s are
// normal (rcp is accurate to 1 ulp), so unless that product lies within 4
// ulps of a bfloat16 rounding midpoint (low 16 bits near 0x8000) both round
// to the same bfloat16; the rare remainder takes the correctly rounded
// division.  Zeros, infinities and NaNs take the fast path and agree.
VH_DEV float div_bf16(float x, float s) {
  const float as = fabsf(s);
  if (as >= 0x1p-126f && as <= 0x1p126f) {
    const float q = x * __builtin_amdgcn_rcpf(s);
    const uint32_t u = __float_as_uint(q);
    if (((u - 0x7FFCu) & 0xFFFFu) > 8u) return bf2f(f2bf(q));
  }
  return bf2f(f2bf(x / s));
}

// The bfloat16 bits of div_bf16(x[j], s) for N (even) values, rounded by the
// hardware converter (v_cvt_pk_bf16_f32: half to even, denormals kept):
// f2bf(div_bf16(x[j], s)) for every non-NaN result; a NaN result is some NaN
// pattern, which callers test with bf_isnan_bits.
template <int N>
VH_DEV void div_bf16_bits_n(const float (&x)[N], float s, uint32_t (&b)[N]) {
  static_assert(N % 2 == 0, "pairs");
  const float as = fabsf(s);
  const bool normal = as >= 0x1p-126f && as <= 0x1p126f;
  const float r = __builtin_amdgcn_rcpf(s);
  uint32_t slow = 0u;
#pragma unroll
  for (int j = 0; j < N; j += 2) {
    const float p0 = x[j] * r, p1 = x[j + 1] * r;
    const uint32_t pk = f2bf2_hw(p0, p1);
    b[j] = pk & 0xffffu;
    b[j + 1] = pk >> 16;
    slow |= (uint32_t)(!normal || ((__float_as_uint(p0) - 0x7FFCu) & 0xFFFFu) <= 8u) << j;
    slow |= (uint32_t)(!normal || ((__float_as_uint(p1) - 0x7FFCu) & 0xFFFFu) <= 8u) << (j + 1);
  }
  if (slow) {
#pragma unroll
    for (int j = 0; j < N; ++j)
      if ((slow >> j) & 1u) b[j] = f2bf(x[j] / s);
  }
}

// The unsigned maximum over aligned groups of G consecutive lanes (G a power
// of two up to 64), delivered to every lane of the group: DPP moves inside
// rows of 16 lanes (quad_perm [1,0,3,2] and [2,3,0,1], row_half_mirror,
// row_mirror: each step pairs every lane with one of the other half of its
// 2^k group), then across rows a lane exchange (G = 32) or the four row
// maxima through scalar registers (G = 64).  Register moves only, with no
// LDS round trip; every lane of the wave must be active.
VH_DEV uint32_t umax32(uint32_t a, uint32_t b) { return a > b ? a : b; }
template <int G>
VH_DEV uint32_t group_umax(uint32_t v) {
  static_assert(G >= 1 && G <= 64 && (G & (G - 1)) == 0, "group size");
  if constexpr (G >= 2) v = umax32(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false));
  if constexpr (G >= 4) v = umax32(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false));
  if constexpr (G >= 8) v = umax32(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xF, 0xF, false));
  if constexpr (G >= 16) v = umax32(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xF, 0xF, false));
  if constexpr (G == 32) v = umax32(v, (uint32_t)__shfl_xor((int)v, 16));
  if constexpr (G == 64) {
    const uint32_t r0 = (uint32_t)__builtin_amdgcn_readlane((int)v, 0);
    const uint32_t r1 = (uint32_t)__builtin_amdgcn_readlane((int)v, 16);
    const uint32_t r2 = (uint32_t)__builtin_amdgcn_readlane((int)v, 32);
    const uint32_t r3 = (uint32_t)__builtin_amdgcn_readlane((int)v, 48);
    v = umax32(umax32(r0, r1), umax32(r2, r3));
  }
  return v;
}

// group_umax for a group size known only at run time (a power of two <= 64).
VH_DEV uint32_t group_umax_rt(uint32_t v, int g) {
  switch (g) {
    case 64: return group_umax<64>(v);
    case 32: return group_umax<32>(v);
    case 16: return group_umax<16>(v);
    case 8: return group_umax<8>(v);
    case 4: return group_umax<4>(v);
    case 2: return group_umax<2>(v);
    default: return v;
  }
}

// A block maximum of |x| with torch.amax's NaN propagation, as one unsigned
// key: the bits of |x| (ordered as the values, +inf included), NaN above
// them all.
VH_DEV uint32_t amax_key(float a) { return a != a ? 0xFFFFFFFFu : __float_as_uint(fabsf(a)); }

// The eager result dtype's rounding of x / s.
VH_DEV float div_round(float x, float s, int dtype) {
  if (dtype == VH_BF16) return div_bf16(x, s);
  return round_to(x / s, dtype);
}

// floor(log2(|a|)) of a finite nonzero float32, subnormals included.
VH_DEV int floor_log2(float a) {
  uint32_t u = __float_as_uint(a) & 0x7fffffffu;
  int ef = (int)(u >> 23);
  if (ef) return ef - 127;
  uint32_t m = u & 0x7fffffu;
  return (31 - (int)__clz(m)) - 149;
}

// Order-preserving key of a bfloat16 pattern: -NaN < -inf < ... < -0 < +0 <
// ... < +inf < +NaN as unsigned 16-bit integers.
VH_DEV uint32_t bf_key(uint32_t b) {
  return (b & 0x8000u) ? (~b & 0xffffu) : (b | 0x8000u);
}

// ---------------------------------------------------------------- formats
// INT: clamp(round_half_even(v), lo, hi); NaN stays NaN; -0 is kept
// (fake_quantize.py:95-96).
VH_DEV float fmt_int(float x, const vh_format& f) {
  float r = rintf(x);
  float lo = (float)f.p0, hi = (float)f.p1;
  return r < lo ? lo : (r > hi ? hi : r);
}

// MINIFLOAT: saturate to the bfloat16-rounded max, then round half-even to a
// grid of p1 mantissa bits with subnormals below exponent emin, then clamp to
// max_norm (fake_quantize.py:98-111 with dtypes/fp8.py:69-135).  A zero
// input gives +0; a nonzero input that rounds to zero keeps its sign.
// OCP E4M3 (max 448) on the hardware converter, which rounds half to even
// with subnormals; zero maps to +0 like the table.  Returns the fp8 byte.
VH_DEV uint32_t e4m3_hw_code(float x) {
  if (x == 0.0f) return 0u;
  const float c = isnan_f(x) ? x : fminf(fmaxf(x, -448.0f), 448.0f);
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(c, c, 0, false) & 0xffu;
}

VH_DEV float e4m3_hw_value(float x) {
  if (isnan_f(x)) return x;
  return __builtin_amdgcn_cvt_f32_fp8((int)e4m3_hw_code(x), 0);
}

// The E4M3 byte of a value already on the grid (a table entry): exact, with
// the sign of zero kept.
VH_DEV uint32_t e4m3_encode(float v) {
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(v, v, 0, false) & 0xffu;
}

VH_DEV float fmt_minifloat(float x, const vh_format& f) {
  if (isnan_f(x)) return x;
  if (f.flags & VH_FMT_HW_E4M3) return e4m3_hw_value(x);
  if (!(f.flags & VH_FMT_SIGNED)) x = fabsf(x);
  float cm = f.clamp_bf16;
  x = x < -cm ? -cm : (x > cm ? cm : x);
  if (x == 0.0f) return 0.0f;
  float a = fabsf(x);
  int e = floor_log2(a);
  if (e < f.emin) e = f.emin;
  float r = rintf(ldexpf(a, f.p1 - e));
  float out = ldexpf(r, e - f.p1);
  if (out > f.max_norm) out = f.max_norm;
  return copysignf(out, x);
}

// POSIT<p0, es=p1>: rounding by manipulation of the float32 encoding, the
// same steps as dtypes/posit.py:8-73 (round_to_even=True): regime/exponent/
// fraction assembled into one bit string, rounded at the posit's last bit
// with guard and sticky bits, saturating at maxpos, and with magnitudes below
// 2**floor(-(n-1)*2**es + 2**(es-1)) flushed to zero.  Inf/NaN -> NaN.
VH_DEV float fmt_posit(float x, const vh_format& f) {
  const int nbits = f.p0, es = f.p1;
  if (!(fabsf(x) <= 3.4028235e38f)) return __uint_as_float(0x7fc00000u);
  if (x == 0.0f) return 0.0f;
  int32_t raw = (int32_t)__float_as_uint(x);
  int32_t scale = ((raw & 0x7F800000) >> 23) - 127;
  int32_t frac = raw & 0x7FFFFF;
  const int32_t max_scale = (nbits - 2) * (1 << es);
  bool pos = scale >= 0;
  bool dominated = pos ? (scale > max_scale) : (scale < -max_scale);
  bool up = false;
  int32_t ecut = es, fcut = 23;
  if (!dominated) {
    // Here |scale| <= max_scale, so every shift below stays within 64 bits.
    int32_t run = pos ? 1 + (scale >> es) : -(scale >> es);
    int64_t regime = (pos ? (int64_t)((1ull << (run + 1)) - 1ull) : 0) ^ 1;
    int64_t expo = scale & ((1 << es) - 1);
    int64_t pbits = (regime << (23 + es)) | (expo << 23) | frac;
    int32_t len = 2 + run + es + 23;
    int64_t last = (int64_t)1 << (len - nbits);
    int64_t guard = last >> 1;
    int64_t sticky = guard - 1;
    bool lb = (pbits & last) != 0;
    bool gb = (pbits & guard) != 0;
    bool sb = (pbits & sticky) != 0;
    up = (lb && gb) || (gb && sb);
    ecut = 2 + run + es - nbits;
    ecut = ecut < 0 ? 0 : (ecut > es ? es : ecut);
    fcut = len - nbits;
    fcut = fcut < 0 ? 0 : (fcut > 23 ? 23 : fcut);
  }
  // A dominated regime truncates every exponent and fraction bit and never
  // rounds up: 2 + run + es - nbits >= es + 1 and len - nbits >= 24 there.
  scale &= (int32_t)(0xffffffffu << ecut);
  scale = scale < -max_scale ? -max_scale : (scale > max_scale ? max_scale : scale);
  frac &= (int32_t)(0xffffffffu << fcut);
  int32_t out = ((scale + 127) << 23) | frac;
  if (up) out += 1 << (fcut + ecut);
  float v = __int_as_float(out);
  v = x < 0.0f ? -v : v;
  if (fabsf(x) < f.thresh) v = 0.0f;
  return v;
}

// STEPS: a table that is a non-decreasing step function of the value.  The
// level is the number of thresholds whose key is <= the input's key (keys are
// staged in LDS by the kernel: `keys` holds f.thr_key).  NaN inputs are
// handled by the caller (they take nan_out / nan_level).
// TOP: the first halving's step (32 covers up to 63 thresholds; a table
// known to hold at most 2 * TOP - 1 may start lower).  `keys` must hold
// 2 * TOP - 1 readable entries (those past nsteps are read and ignored).
template <int TOP = 32>
VH_DEV uint32_t steps_level(uint32_t b, int nsteps, const uint16_t* keys) {
  // Branch-free search: six halvings cover up to 63 thresholds, so the
  // lookups of a thread's elements can overlap.  The key is read before the
  // bound is tested (nxt - 1 <= 2 * TOP - 2): with the test first, each read
  // became a branch of its own, waited on alone.
  const uint32_t k = bf_key(b);
  int pos = 0;
#pragma unroll
  for (int step = TOP; step >= 1; step >>= 1) {
    const int nxt = pos + step;
    const bool ok = (nxt <= nsteps) & ((uint32_t)keys[nxt - 1] <= k);
    pos = ok ? nxt : pos;
  }
  return (uint32_t)pos;
}

// steps_level over a key table padded with 0xFFFF from nsteps on (at least
// 2 * TOP - 1 entries): the same level for every non-NaN input, whose key is
// below 0xFF81 (only a NaN's key reaches a padded entry), with no bound test.
template <int TOP>
VH_DEV uint32_t steps_level_padded(uint32_t k, const uint16_t* keys) {
  uint32_t pos = 0;
#pragma unroll
  for (int step = TOP; step >= 1; step >>= 1) pos = (uint32_t)keys[pos + step - 1] <= k ? pos + step : pos;
  return pos;
}

// Stage a STEPS format's keys and entries in LDS (2 * VH_MAX_STEPS halves).
// Every thread of the block must call it.
VH_DEV void stage_steps(const vh_format& f, uint16_t* lds) {
  if (f.kind == VH_FMT_STEPS) {
    for (int i = threadIdx.x; i < VH_MAX_STEPS; i += blockDim.x) {
      lds[i] = f.thr_key[i];
      lds[VH_MAX_STEPS + i] = f.val[i];
    }
  }
  __syncthreads();
}

VH_DEV bool bf_isnan_bits(uint32_t b) { return (b & 0x7fffu) > 0x7f80u; }

// Four 4-bit indices -> four int8 levels from a 16-entry table held in four
// dwords (t0 = levels 0..3, ... t3 = levels 12..15).  `sel` holds the low
// three bits of each index (one per byte), `hib` its bit 3 at bit 2 of the
// byte; the third v_perm picks, per byte i, byte i of the low-half lookup
// (selector i) or of the high-half one (i + 4).  `base` is 0x03020100 in a
// VGPR: with a register operand the merge selector is one v_and_or_b32 (a
// VOP3 encoding takes no second literal here).
VH_DEV uint32_t lut16(uint32_t sel, uint32_t hib, uint32_t base, uint32_t t0, uint32_t t1,
                        uint32_t t2, uint32_t t3) {
  const uint32_t lo = __builtin_amdgcn_perm(t1, t0, sel);
  const uint32_t hi = __builtin_amdgcn_perm(t3, t2, sel);
  return __builtin_amdgcn_perm(hi, lo, (hib & 0x04040404u) | base);
}

// The low / high nibbles of a dword of packed indices.
VH_DEV uint32_t lut_lo(uint32_t w, uint32_t base, const uint4& lv) {
  return lut16(w & 0x07070707u, w >> 1, base, lv.x, lv.y, lv.z, lv.w);
}
VH_DEV uint32_t lut_hi(uint32_t w, uint32_t base, const uint4& lv) {
  return lut16((w >> 4) & 0x07070707u, w >> 5, base, lv.x, lv.y, lv.z, lv.w);
}

// Kernels are specialised on the format kind (K_* below) so each instance
// holds only its own closed form; the runtime-dispatch versions serve the
// per-block scale maps.
enum {
  K_IDENTITY = VH_FMT_IDENTITY,
  K_INT = VH_FMT_INT,
  K_MINI = VH_FMT_MINIFLOAT,
  K_POSIT = VH_FMT_POSIT,
  K_STEPS = VH_FMT_STEPS,
  K_LUT = VH_FMT_LUT,
  K_E4M3 = 6,  // VH_FMT_MINIFLOAT with VH_FMT_HW_E4M3
  K_NONE = 7,  // no map
};

static inline int kernel_kind(const vh_format* f) {
  if (!f) return K_NONE;
  if (f->kind == VH_FMT_MINIFLOAT && (f->flags & VH_FMT_HW_E4M3)) return K_E4M3;
  return f->kind;
}

// Apply a format to a bfloat16 input; returns the table entry's value as
// float32 (bfloat16 entries are exact in float32; index tables are small
// integers).  K_LUT tables are gathered from device memory.
template <int KIND>
VH_DEV float fmt_value_k(uint32_t b, const vh_format& f, const uint16_t* lds) {
  const float x = bf2f(b);
  if constexpr (KIND == K_IDENTITY || KIND == K_NONE) {
    return x;
  } else if constexpr (KIND == K_INT) {
    return fmt_int(x, f);
  } else if constexpr (KIND == K_E4M3) {
    return e4m3_hw_value(x);
  } else if constexpr (KIND == K_MINI) {
    return rbf(fmt_minifloat(x, f));
  } else if constexpr (KIND == K_POSIT) {
    return rbf(fmt_posit(x, f));
  } else if constexpr (KIND == K_STEPS) {
    if (bf_isnan_bits(b)) return bf2f(f.nan_out);
    return bf2f(lds[VH_MAX_STEPS + steps_level(b, f.nsteps, lds)]);
  } else {
    return bf2f(((const uint16_t*)f.lut)[b & 0xffffu]);
  }
}

VH_DEV float fmt_value(uint32_t b, const vh_format& f, const uint16_t* lds) {
  switch (f.kind) {
    case VH_FMT_IDENTITY: return fmt_value_k<K_IDENTITY>(b, f, lds);
    case VH_FMT_INT: return fmt_value_k<K_INT>(b, f, lds);
    case VH_FMT_MINIFLOAT: return fmt_value_k<K_MINI>(b, f, lds);
    case VH_FMT_POSIT: return fmt_value_k<K_POSIT>(b, f, lds);
    case VH_FMT_STEPS: return fmt_value_k<K_STEPS>(b, f, lds);
    default: return fmt_value_k<K_LUT>(b, f, lds);
  }
}

// ------------------------------------------------------------ packed codes
// One byte per element: INT two's complement; MINIFLOAT sign|exponent|
// mantissa fields (fp8_e4m3 is the OCP E4M3 byte the fp8 MFMA reads);
// POSIT the posit bit string; STEPS the level index.  Packed int8 holds
// neither NaN nor -0: a NaN element packs as 0 and -0 as +0.

VH_DEV uint32_t mini_code(float v, const vh_format& f) {
  if (f.flags & VH_FMT_HW_E4M3) return e4m3_encode(v);
  const int mb = f.p1;
  uint32_t sign = 0;
  if ((f.flags & VH_FMT_SIGNED) && (__float_as_uint(v) >> 31)) sign = 1u << (f.p0 + mb);
  if (isnan_f(v)) return sign | (((1u << f.p0) - 1u) << mb) | ((1u << mb) - 1u);
  float a = fabsf(v);
  if (a == 0.0f) return sign;
  int e = floor_log2(a);
  uint32_t ef, m;
  if (e < f.emin) {  // subnormal
    ef = 0;
    m = (uint32_t)ldexpf(a, mb - f.emin);
  } else {
    ef = (uint32_t)(e - f.emin + 1);
    m = (uint32_t)ldexpf(a, mb - e) - (1u << mb);
  }
  return sign | (ef << mb) | m;
}

VH_DEV float mini_decode(uint32_t c, const vh_format& f) {
  const int mb = f.p1;
  uint32_t m = c & ((1u << mb) - 1u);
  uint32_t ef = (c >> mb) & ((1u << f.p0) - 1u);
  float a = ef ? ldexpf((float)(m + (1u << mb)), (int)ef - 1 + f.emin - mb)
               : ldexpf((float)m, f.emin - mb);
  if ((f.flags & VH_FMT_SIGNED) && ((c >> (f.p0 + mb)) & 1u)) a = -a;
  return a;
}

// Posit bit string of an exactly representable posit value.
VH_DEV uint32_t posit_code(float v, const vh_format& f) {
  const int n = f.p0, es = f.p1;
  if (isnan_f(v)) return 1u << (n - 1);  // NaR
  if (v == 0.0f) return 0;
  float a = fabsf(v);
  int s = floor_log2(a);
  int k = s >> es;               // regime value (floor)
  int ex = s - (k << es);        // exponent bits
  uint32_t fr = __float_as_uint(a) & 0x7fffffu;  // fraction (23 bits)
  // Assemble regime | exponent | fraction into a long bit string.
  uint64_t body;
  int blen;
  if (k >= 0) {
    body = ((1ull << (k + 1)) - 1ull) << 1;  // k+1 ones then a zero
    blen = k + 2;
  } else {
    body = 1ull;                              // -k zeros then a one
    blen = -k + 1;
  }
  body = (body << es) | (uint64_t)ex;
  blen += es;
  body = (body << 23) | fr;
  blen += 23;
  int avail = n - 1;
  uint32_t bits = blen > avail ? (uint32_t)(body >> (blen - avail))
                               : (uint32_t)(body << (avail - blen));
  bits &= (1u << avail) - 1u;
  if (v < 0.0f) bits = ((~bits) + 1u) & ((1u << n) - 1u);
  return bits;
}

VH_DEV float posit_decode(uint32_t c, const vh_format& f) {
  const int n = f.p0, es = f.p1;
  c &= (1u << n) - 1u;
  if (c == 0) return 0.0f;
  if (c == (1u << (n - 1))) return __uint_as_float(0x7fc00000u);
  bool neg = (c >> (n - 1)) & 1u;
  if (neg) c = ((~c) + 1u) & ((1u << n) - 1u);
  int i = n - 2;
  uint32_t first = (c >> i) & 1u;
  int run = 0;
  while (i >= 0 && ((c >> i) & 1u) == first) { run++; i--; }
  i--;  // skip the terminating bit
  int k = first ? run - 1 : -run;
  int ex = 0, ebits = 0;
  while (ebits < es) {
    ex <<= 1;
    if (i >= 0) { ex |= (c >> i) & 1u; i--; }
    ebits++;
  }
  int fbits = i + 1;
  uint32_t fr = fbits > 0 ? (c & ((1u << fbits) - 1u)) : 0u;
  float val = ldexpf(1.0f + ldexpf((float)fr, -fbits), k * (1 << es) + ex);
  return neg ? -val : val;
}

// Packed code of an element whose table value is v (bits b of the input).
template <int KIND>
VH_DEV uint32_t fmt_code_k(uint32_t b, float v, const vh_format& f, const uint16_t* lds) {
  if constexpr (KIND == K_INT) {
    return isnan_f(v) ? 0u : ((uint32_t)(int32_t)v & 0xffu);
  } else if constexpr (KIND == K_E4M3) {
    return e4m3_encode(v);
  } else if constexpr (KIND == K_MINI) {
    return mini_code(v, f) & 0xffu;
  } else if constexpr (KIND == K_POSIT) {
    return posit_code(v, f) & 0xffu;
  } else if constexpr (KIND == K_STEPS) {
    if (bf_isnan_bits(b)) return (uint32_t)f.nan_level;
    return steps_level(b, f.nsteps, lds);
  } else {
    return 0u;
  }
}

VH_DEV uint32_t fmt_code(uint32_t b, float v, const vh_format& f, const uint16_t* lds) {
  switch (f.kind) {
    case VH_FMT_INT: return fmt_code_k<K_INT>(b, v, f, lds);
    case VH_FMT_MINIFLOAT: return fmt_code_k<K_MINI>(b, v, f, lds);
    case VH_FMT_POSIT: return fmt_code_k<K_POSIT>(b, v, f, lds);
    case VH_FMT_STEPS: return fmt_code_k<K_STEPS>(b, v, f, lds);
    default: return 0u;
  }
}

// The reference-form value of a packed code (the table entry, as float32).
template <int KIND>
VH_DEV float fmt_decode_k(uint32_t c, const vh_format& f, const uint16_t* lds) {
  if constexpr (KIND == K_INT) {
    return (f.p0 < 0) ? (float)(int8_t)(uint8_t)c : (float)(uint8_t)c;
  } else if constexpr (KIND == K_E4M3) {
    return rbf(__builtin_amdgcn_cvt_f32_fp8((int)c, 0));
  } else if constexpr (KIND == K_MINI) {
    // Codes beyond max_norm are the format's NaN (the map never emits
    // them for a finite input).
    float v = mini_decode(c, f);
    return fabsf(v) > f.max_norm ? __uint_as_float(0x7fc00000u) : rbf(v);
  } else if constexpr (KIND == K_POSIT) {
    return rbf(posit_decode(c, f));
  } else if constexpr (KIND == K_STEPS) {
    return bf2f(lds[VH_MAX_STEPS + (c < VH_MAX_STEPS ? c : VH_MAX_STEPS - 1)]);
  } else {
    return 0.0f;
  }
}

VH_DEV float fmt_decode(uint32_t c, const vh_format& f, const uint16_t* lds) {
  switch (f.kind) {
    case VH_FMT_INT: return fmt_decode_k<K_INT>(c, f, lds);
    case VH_FMT_MINIFLOAT:
      if (f.flags & VH_FMT_HW_E4M3) return fmt_decode_k<K_E4M3>(c, f, lds);
      return fmt_decode_k<K_MINI>(c, f, lds);
    case VH_FMT_POSIT: return fmt_decode_k<K_POSIT>(c, f, lds);
    case VH_FMT_STEPS: return fmt_decode_k<K_STEPS>(c, f, lds);
    default: return 0.0f;
  }
}

// Dispatch a kernel template on a format's kind: F is called with an
// integral-constant kind.
template <typename F>
static inline int dispatch_kind(int kind, F&& fn) {
  switch (kind) {
    case K_IDENTITY: return fn(std::integral_constant<int, K_IDENTITY>{});
    case K_INT: return fn(std::integral_constant<int, K_INT>{});
    case K_MINI: return fn(std::integral_constant<int, K_MINI>{});
    case K_POSIT: return fn(std::integral_constant<int, K_POSIT>{});
    case K_STEPS: return fn(std::integral_constant<int, K_STEPS>{});
    case K_LUT: return fn(std::integral_constant<int, K_LUT>{});
    case K_E4M3: return fn(std::integral_constant<int, K_E4M3>{});
    default: return fn(std::integral_constant<int, K_NONE>{});
  }
}
