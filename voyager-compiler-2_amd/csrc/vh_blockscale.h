// Per-block scale and per-element code of block-scaled quantization
// (quantize_mx / calculate_mx_qparam, ops/quantized.py:958-1115, and
// quantize_affine, ops/quantized.py:1218-1283), shared by the quantize
// kernels and the kernels that quantize their activations in place.
#pragma once

#include "vh_device.h"

namespace {

enum Mode { MX_POT = 0, MX_SCALED = 1, AFFINE = 2 };

struct Params {
  int mode;
  int cdt;            // compute dtype: the input's
  float quant_max;    // MX: element max; AFFINE: quant_max
  float quant_min;    // AFFINE
  int shift;          // MX_POT: floor(log2(quant_max))
  int has_sfmt;       // scale map present
  vh_format sfmt;     // scale map
  const void* gs;     // MX_SCALED: 0-d global scale (device), or null
  int gs_dtype;
  int has_fmt;        // element map present (calculate_mx_qparam has none)
  vh_format fmt;      // element map
  int scale_dtype;    // cdt or VH_U8
  int pot_bias;       // packed pot scale byte = e + pot_bias
  int codes_dtype;    // cdt or VH_U8
  const uint8_t* code_lut;  // packed codes are remapped through this (or null)
  int scale_t16;            // scales written block-major [nblk][16] (rows <= 16)
};

VH_DEV float load_x(const void* p, int dt, int64_t i) {
  if (dt == VH_BF16) return bf2f(((const uint16_t*)p)[i]);
  if (dt == VH_F16) return __half2float(((const __half*)p)[i]);
  return ((const float*)p)[i];
}

VH_DEV void store_f(void* p, int dt, int64_t i, float v) {
  if (dt == VH_BF16) ((uint16_t*)p)[i] = (uint16_t)f2bf(v);
  else if (dt == VH_F16) ((__half*)p)[i] = __float2half_rn(v);
  else ((float*)p)[i] = v;
}

// vmap of a value in the compute dtype through a map, result in cdt.
VH_DEV float vmap1(float v, const vh_format& f, const uint16_t* lds, int cdt) {
  uint32_t b = f2bf(v);
  return round_to(fmt_value(b, f, lds), cdt);
}

struct BlockScale {
  float scale;      // the returned scale (cdt value)
  float el_scale;   // what the elements are divided by
  float inv;        // MX_POT: 1 / el_scale when that is exact and normal, else 0
  float zp;         // AFFINE zero point
  uint32_t packed;  // packed scale byte
};

// The scale map applied to a value (SKIND = K_NONE: no map; a specialised
// kind, or K_LUT + 1 for the runtime switch).
constexpr int K_RUNTIME = 8;

template <int SKIND>
VH_DEV float smap_value(uint32_t b, const vh_format& f, const uint16_t* slds) {
  if constexpr (SKIND == K_RUNTIME) return fmt_value(b, f, slds);
  else return fmt_value_k<SKIND>(b, f, slds);
}

template <int SKIND>
VH_DEV uint32_t smap_code(uint32_t b, float v, const vh_format& f, const uint16_t* slds) {
  if constexpr (SKIND == K_RUNTIME) return fmt_code(b, v, f, slds);
  else return fmt_code_k<SKIND>(b, v, f, slds);
}

// Scale of one block from its reductions (hi = amax for MX, max for AFFINE;
// lo = min for AFFINE).
template <int SKIND>
VH_DEV BlockScale block_scale(float hi, float lo, const Params& P, const uint16_t* slds) {
  BlockScale r;
  r.zp = 0.0f;
  r.inv = 0.0f;
  r.packed = 0;
  const int cdt = P.cdt;
  if (P.mode == MX_POT) {
    // floor(log2(fp32(amax) + 2**-126 * (amax == 0))), mx_utils.py:47-51;
    // then 2**(e - shift) in the compute dtype (ops/quantized.py:995-1015).
    float s;
    int e = 0;
    bool inf = false;
    if (isnan_f(hi)) {
      s = 1.0f;  // NaN > 0 is false
    } else if (hi == __builtin_inff()) {
      s = __builtin_inff();
      inf = true;
    } else {
      int E = hi == 0.0f ? -126 : floor_log2(hi);
      e = E - P.shift;
      s = round_to(ldexpf(1.0f, e), cdt);
      if (s == __builtin_inff()) inf = true;
      if (!(s > 0.0f)) { s = 1.0f; e = 0; }
    }
    r.scale = s;
    r.el_scale = s;
    // a power of two in [2**-126, 2**126]: x / s and x * (1 / s) are the
    // same exact quotient, rounded alike
    const uint32_t sb = __float_as_uint(s);
    if (s >= 0x1p-126f && s <= 0x1p126f && (sb & 0x7fffffu) == 0u)
      r.inv = __uint_as_float((uint32_t)(254 - (int)(sb >> 23)) << 23);
    int byte = inf ? 255 : e + P.pot_bias;
    r.packed = (uint32_t)(byte < 0 ? 0 : (byte > 254 && !inf ? 254 : byte));
    return r;
  }
  if (P.mode == MX_SCALED) {
    float s = div_round(hi, P.quant_max, cdt);
    // A 0-d global scale enters the bf16 ops at its own precision: eager
    // bf16 / fp32-scalar divides (and multiplies) in float32, then rounds.
    const float gs = P.gs ? load_x(P.gs, P.gs_dtype, 0) : 1.0f;
    if (P.gs) s = div_round(s, gs, cdt);
    if constexpr (SKIND != K_NONE) {
      const uint32_t sb = f2bf(s);
      s = round_to(smap_value<SKIND>(sb, P.sfmt, slds), cdt);
    }
    if (!(s > 0.0f)) s = 1.0f;
    r.scale = s;
    r.el_scale = P.gs ? round_to(s * gs, cdt) : s;
    if constexpr (SKIND != K_NONE) {
      uint32_t b = f2bf(s);
      r.packed = smap_code<SKIND>(b, bf2f(b), P.sfmt, slds);
    }
    return r;
  }
  // AFFINE (ops/quantized.py:1262-1281)
  float s = div_round(round_to(hi - lo, cdt), P.quant_max - P.quant_min, cdt);
  if (!(s > 0.0f)) s = 1.0f;
  if constexpr (SKIND != K_NONE) {
    s = round_to(smap_value<SKIND>(f2bf(s), P.sfmt, slds), cdt);
    if (!(s > 0.0f)) s = 1.0f;
  }
  float zp = round_to(div_round(-lo, s, cdt) + P.quant_min, cdt);
  if constexpr (SKIND != K_NONE) zp = round_to(smap_value<SKIND>(f2bf(zp), P.sfmt, slds), cdt);
  r.scale = s;
  r.el_scale = s;
  r.zp = zp;
  return r;
}

// One element's reference-form code value and packed byte.
template <int KIND>
VH_DEV void element_code(float x, const BlockScale& bs, const Params& P, const uint16_t* lds, const uint8_t* clut,
                         float* v, uint32_t* code) {
  float q = (P.mode == MX_POT && bs.inv != 0.0f) ? round_to(x * bs.inv, P.cdt) : div_round(x, bs.el_scale, P.cdt);
  if (P.mode == AFFINE) q = round_to(q + bs.zp, P.cdt);
  const uint32_t b = (P.cdt == VH_BF16 && !isnan_f(q)) ? (__float_as_uint(q) >> 16) : f2bf(q);
  if constexpr (KIND == K_STEPS) {
    const bool nan = bf_isnan_bits(b);
    // (a wave-uniform branch: a table of at most 15 thresholds, as the
    // 16-entry codebooks, needs four halvings rather than six)
    const uint32_t lvl = nan ? (uint32_t)P.fmt.nan_level
                             : P.fmt.nsteps <= 15 ? steps_level<8>(b, P.fmt.nsteps, lds)
                                                  : steps_level(b, P.fmt.nsteps, lds);
    *v = round_to(nan ? bf2f(P.fmt.nan_out) : bf2f(lds[VH_MAX_STEPS + lvl]), P.cdt);
    *code = lvl;
  } else {
    const float val = fmt_value_k<KIND>(b, P.fmt, lds);
    *v = round_to(val, P.cdt);
    *code = fmt_code_k<KIND>(b, val, P.fmt, lds);
  }
  if (P.code_lut) *code = clut[*code & 0xffu];
}

}  // namespace
