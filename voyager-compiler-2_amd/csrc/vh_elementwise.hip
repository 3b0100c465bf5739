// Elementwise quantized ops: table rebuild, quantize (+ vmap) and dequantize.
//
// quantize   (ops/quantized.py:449-515):  out = F(rc(rc(x / s) + zp))
// dequantize (ops/quantized.py:518-571):  out = G(rc((Fin(x) - zp) * s))
// vmap       (ops/quantized.py:147-184):  out = F(x)
// where rc rounds to the compute dtype (each eager op's result dtype) and the
// maps F, Fin, G are closed forms of the caller's 65,536-entry tables.
//
// HBM-bound: every thread moves 8 consecutive elements with 16-byte loads
// (bf16) and stores, so a wavefront touches 1 KiB contiguous per access.
#include <hip/hip_runtime.h>

#include <cmath>

#include <cstring>
#include <string>

#include "vh_device.h"
#include "vh_host.h"

namespace vh {

static thread_local std::string g_error;

void set_error(const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_error = buf;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return VH_ELAUNCH;
  }
  return VH_OK;
}

}  // namespace vh

extern "C" const char* vh_last_error(void) { return vh::g_error.c_str(); }
extern "C" int vh_abi_version(void) { return VH_ABI_VERSION; }

// ------------------------------------------------------------ table rebuild
// Rebuilds a table with the same specialised closed form the quantize
// kernels run, so a table that passes verification is what they compute.
template <int KIND>
__global__ void __launch_bounds__(256) k_build_table(vh_format f, uint16_t* out) {
  __shared__ uint16_t lds[2 * VH_MAX_STEPS];
  stage_steps(f, lds);
  uint32_t b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= 65536u) return;
  if constexpr (KIND == K_IDENTITY) {
    out[b] = (uint16_t)b;  // bit for bit, NaN payloads included
  } else if constexpr (KIND == K_LUT) {
    out[b] = ((const uint16_t*)f.lut)[b];
  } else {
    out[b] = (uint16_t)f2bf(fmt_value_k<KIND>(b, f, lds));
  }
}

extern "C" int vh_build_table(const vh_format* fmt, uint16_t* out, vh_stream_t stream) {
  VH_REQUIRE(fmt && out, "vh_build_table: null argument");
  VH_REQUIRE(fmt->kind >= VH_FMT_IDENTITY && fmt->kind <= VH_FMT_LUT, "vh_build_table: bad kind %d", fmt->kind);
  VH_REQUIRE(fmt->kind != VH_FMT_STEPS || (fmt->nsteps >= 0 && fmt->nsteps < VH_MAX_STEPS),
             "vh_build_table: nsteps %d out of range", fmt->nsteps);
  hipStream_t st = vh::as_stream(stream);
  return dispatch_kind(kernel_kind(fmt), [&](auto kind) {
    constexpr int K = decltype(kind)::value;
    if constexpr (K == K_NONE) {
      return (int)VH_EINVAL;
    } else {
      hipLaunchKernelGGL(k_build_table<K>, dim3(256), dim3(256), 0, st, *fmt, out);
      return vh::check_launch("vh_build_table");
    }
  });
}

// ------------------------------------------------------------ param access
struct Shape {
  int64_t dim[VH_MAX_DIMS];  // sizes, innermost last
  int32_t ndim;
};

VH_DEV float load_any(const void* p, int dtype, int64_t i) {
  switch (dtype) {
    case VH_BF16: return bf2f(((const uint16_t*)p)[i]);
    case VH_F16: return __half2float(((const __half*)p)[i]);
    case VH_F32: return ((const float*)p)[i];
    default: return 0.0f;
  }
}

VH_DEV void store_any(void* p, int dtype, int64_t i, float v) {
  switch (dtype) {
    case VH_BF16: ((uint16_t*)p)[i] = (uint16_t)f2bf(v); break;
    case VH_F16: ((__half*)p)[i] = __float2half_rn(v); break;
    case VH_F32: ((float*)p)[i] = v; break;
    default: break;
  }
}

// Offset of element `flat`'s parameter.  `narrow`: the tensor has fewer than
// 2^31 elements, so every index and dim fits 32-bit unsigned division (a
// block wider than 2^32 - 1 acts as 2^32 - 1 on such indices).
VH_DEV int64_t param_offset(const vh_param& p, const Shape& s, int64_t flat, bool narrow) {
  int64_t off = 0;
  if (narrow) {
    uint32_t f = (uint32_t)flat;
    for (int d = s.ndim - 1; d >= 0; --d) {
      const uint32_t n = (uint32_t)s.dim[d];
      const uint32_t i = f % n;
      f /= n;
      const uint32_t dv = p.div[d] > 0xffffffffll ? 0xffffffffu : (uint32_t)p.div[d];
      off += (int64_t)(i / dv) * p.stride[d];
    }
    return off;
  }
  for (int d = s.ndim - 1; d >= 0; --d) {
    int64_t n = s.dim[d];
    int64_t i = flat % n;
    flat /= n;
    off += (i / p.div[d]) * p.stride[d];
  }
  return off;
}

// Value of bfloat16 pattern `b` under format f as the compute dtype sees it.
// vmap casts a non-bf16 input to bfloat16 for the index and its result back.

// ------------------------------------------------------------ quantize
// One thread: VEC consecutive elements.
constexpr int VEC = 8;

// Parameter values of elements base .. base + VEC - 1 (those below n).  The
// index is decomposed once per group; within a row of the innermost dim the
// offsets step by the innermost block, and a group whose elements share one
// offset (a block of >= 8 along the innermost dim) loads it once.
VH_DEV void param_values(const vh_param& p, const Shape& s, int64_t base, int64_t n, float* v) {
  const int last = s.ndim - 1;
  const int64_t L = last >= 0 ? s.dim[last] : 1;
  const bool narrow = n < (1ll << 31);
  const int64_t c0 = narrow ? (int64_t)((uint32_t)base % (uint32_t)L) : base % L;
  if (last >= 0 && c0 + VEC <= L && base + VEC <= n && L < (1ll << 31)) {
    const int64_t o0 = param_offset(p, s, base, narrow);
    const int32_t dv = (int32_t)p.div[last], q0 = (int32_t)c0 / dv;
    const int32_t q7 = ((int32_t)c0 + VEC - 1) / dv;
    if (q7 == q0 || p.stride[last] == 0) {
      const float v0 = load_any(p.ptr, p.dtype, o0);
#pragma unroll
      for (int j = 0; j < VEC; ++j) v[j] = v0;
    } else {
#pragma unroll
      for (int j = 0; j < VEC; ++j)
        v[j] = load_any(p.ptr, p.dtype, o0 + (int64_t)(((int32_t)c0 + j) / dv - q0) * p.stride[last]);
    }
    return;
  }
  for (int j = 0; j < VEC; ++j)
    if (base + j < n) v[j] = load_any(p.ptr, p.dtype, param_offset(p, s, base + j, narrow));
}

template <int KIND>
__global__ void __launch_bounds__(256)
k_quantize(const void* __restrict__ x, int x_dtype, int64_t n, Shape shape, vh_param sp, vh_param zp,
           int cdt, vh_format f, void* __restrict__ out, int out_dtype) {
  __shared__ uint16_t lds[2 * VH_MAX_STEPS];
  if constexpr (KIND == K_STEPS) stage_steps(f, lds);
  int64_t base = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * VEC;
  if (base >= n) return;
  const bool full = base + VEC <= n;
  float xv[VEC];
  if (x_dtype == VH_BF16 && full) {
    uint4 raw = ld_stream16((const uint16_t*)x + base);
    uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      xv[2 * j] = bf2f(w[j] & 0xffffu);
      xv[2 * j + 1] = bf2f(w[j] >> 16);
    }
  } else {
    for (int j = 0; j < VEC; ++j) xv[j] = (base + j < n) ? load_any(x, x_dtype, base + j) : 0.0f;
  }
  // Per-element parameters: one value, or indexed (a loop, kept out of the
  // unrolled element code).
  float sv[VEC], zv[VEC];
  const float s0 = (sp.ptr && sp.scalar) ? load_any(sp.ptr, sp.dtype, 0) : 1.0f;
  const float z0 = (zp.ptr && zp.scalar) ? load_any(zp.ptr, zp.dtype, 0) : 0.0f;
#pragma unroll
  for (int j = 0; j < VEC; ++j) {
    sv[j] = s0;
    zv[j] = z0;
  }
  if (sp.ptr && !sp.scalar) param_values(sp, shape, base, n, sv);
  if (zp.ptr && !zp.scalar) param_values(zp, shape, base, n, zv);
  const bool has_s = sp.ptr != nullptr, has_z = zp.ptr != nullptr;
  uint32_t res[VEC];
  float outv[VEC];
#pragma unroll
  for (int j = 0; j < VEC; ++j) {
    float q = xv[j];
    if (has_s) q = div_round(q, sv[j], cdt);
    if (has_z) q = round_to(q + zv[j], cdt);
    if constexpr (KIND != K_NONE) {
      // vmap indexes by the bfloat16 pattern (exact when cdt is bf16)
      const uint32_t b = (cdt == VH_BF16 && !isnan_f(q)) ? (__float_as_uint(q) >> 16) : f2bf(q);
      const float v = fmt_value_k<KIND>(b, f, lds);
      res[j] = fmt_code_k<KIND>(b, v, f, lds);
      outv[j] = v;
    } else {
      res[j] = 0;
      outv[j] = q;
    }
  }
  if (out_dtype == VH_U8) {
    uint8_t* o = (uint8_t*)out;
    if (full) {
      uint2 pk;
      pk.x = res[0] | (res[1] << 8) | (res[2] << 16) | (res[3] << 24);
      pk.y = res[4] | (res[5] << 8) | (res[6] << 16) | (res[7] << 24);
      st_stream8(o + base, pk);
    } else {
      for (int j = 0; j < VEC; ++j)
        if (base + j < n) o[base + j] = (uint8_t)res[j];
    }
  } else if (out_dtype == VH_BF16 && full) {
    uint4 pk;
    pk.x = f2bf(outv[0]) | (f2bf(outv[1]) << 16);
    pk.y = f2bf(outv[2]) | (f2bf(outv[3]) << 16);
    pk.z = f2bf(outv[4]) | (f2bf(outv[5]) << 16);
    pk.w = f2bf(outv[6]) | (f2bf(outv[7]) << 16);
    st_stream16((uint16_t*)out + base, pk);
  } else {
    for (int j = 0; j < VEC; ++j)
      if (base + j < n) store_any(out, out_dtype, base + j, outv[j]);
  }
}

// Per-tensor fast path: contiguous bfloat16 input, one scale, no zero point,
// bfloat16 compute.  Each thread keeps UNROLL 16-byte loads in flight; the
// reciprocal of the scale is taken once; the bf16 rounding of x/s uses the
// same midpoint test as div_bf16 with the hardware bf16 converter.
constexpr int UNROLL = 4;

typedef unsigned short vh_u16x2 __attribute__((ext_vector_type(2)));

VH_DEV uint32_t pk_sub_u16(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t, __builtin_bit_cast(vh_u16x2, a) - __builtin_bit_cast(vh_u16x2, b));
}
VH_DEV uint32_t pk_min_u16(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t,
                            __builtin_elementwise_min(__builtin_bit_cast(vh_u16x2, a), __builtin_bit_cast(vh_u16x2, b)));
}
VH_DEV uint32_t pk_max_u16(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t,
                            __builtin_elementwise_max(__builtin_bit_cast(vh_u16x2, a), __builtin_bit_cast(vh_u16x2, b)));
}

// Per-tensor quantize to packed OCP E4M3 bytes (the FP8 GEMM operand):
// code = E4M3(bf16(x / s)) with saturation at 448, as the table does.  Per
// pair of elements: x * rcp(s), the hardware bf16 rounding, the 448 clamp as
// a packed integer min on the bf16 magnitude, the hardware fp8 converter
// (+0.0 first: an exact zero takes code 0 whatever its sign).  Two running
// packed 16-bit extremes flag the rare cases this shortcut cannot decide --
// a product within 4 fp32 ulps of a bf16 rounding midpoint, a NaN -- and the
// thread then redoes its elements with the correctly rounded division.
// Workgroup b converts the U * 256 consecutive 16-byte groups from
// b * U * 256 (one contiguous run of memory per workgroup, every load issued
// before the first use): on MI355X this streams 2048 x 4096 bf16 at 4.8 TB/s
// with no arithmetic, against 4.1 TB/s for a grid-stride loop.
template <int U>
__global__ void __launch_bounds__(256)
k_quantize_e4m3_pt(const uint16_t* __restrict__ x, int64_t nvec, const void* sp, int sdt, uint8_t* __restrict__ out) {
  constexpr int64_t stride = 256;
  {
    const int64_t v0 = (int64_t)blockIdx.x * (U * 256) + threadIdx.x;
    constexpr int UNROLL = U;
    // the element loads go out first and unconditionally (a group past the
    // end reloads the last one and is not stored); the scale is read after
    // them through the scalar cache (a bfloat16 scale as the aligned 4-byte
    // word that holds it, which lies in the same mapped allocation), so its
    // latency overlaps theirs and no wait for it holds them back
    uint4 raw[UNROLL];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const int64_t v = v0 + u * stride;
      raw[u] = ld_stream16(x + (v < nvec ? v : nvec - 1) * 8);
    }
    asm volatile("" ::: "memory");
    typedef const __attribute__((address_space(4))) uint32_t cword;  // constant space: a scalar load
    const uintptr_t a = (uintptr_t)sp;
    const uint32_t w = *(cword*)(a & ~(uintptr_t)3);
    const uint32_t h = (a & 2) ? (w >> 16) : (w & 0xffffu);
    const float s = sdt == VH_F32 ? __uint_as_float(w) : sdt == VH_F16 ? __half2float(__ushort_as_half((unsigned short)h))
                                                                     : bf2f(h);
    const float as = fabsf(s);
    const bool fast_scale = as >= 0x1p-126f && as <= 0x1p126f;
    const float r = __builtin_amdgcn_rcpf(s);
    uint2 res[UNROLL];
    uint32_t mn = 0xffffffffu, mx = 0u;
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const uint32_t w[4] = {raw[u].x, raw[u].y, raw[u].z, raw[u].w};
      uint32_t o[2] = {0u, 0u};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float q0 = __uint_as_float(w[j] << 16) * r;
        const float q1 = __uint_as_float(w[j] & 0xffff0000u) * r;
        const uint32_t lo = __builtin_amdgcn_perm(__float_as_uint(q1), __float_as_uint(q0), 0x05040100u);
        mn = pk_min_u16(mn, pk_sub_u16(lo, 0x7ffc7ffcu));
        uint32_t b = f2bf2_hw(q0, q1);
        const uint32_t m = b & 0x7fff7fffu;
        mx = pk_max_u16(mx, m);
        b = pk_min_u16(m, 0x43e043e0u) | (b & 0x80008000u);
        const float f0 = __uint_as_float(b << 16) + 0.0f;
        const float f1 = __uint_as_float(b & 0xffff0000u) + 0.0f;
        if (j & 1) o[j >> 1] = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(f0, f1, (int)o[j >> 1], true);
        else o[j >> 1] = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(f0, f1, (int)o[j >> 1], false);
      }
      res[u] = make_uint2(o[0], o[1]);
    }
    const bool exact_needed = !fast_scale || (mn & 0xffffu) <= 8u || (mn >> 16) <= 8u || (mx & 0xffffu) > 0x7f80u ||
                              (mx >> 16) > 0x7f80u;
    if (exact_needed) {
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) {
        const uint32_t w[4] = {raw[u].x, raw[u].y, raw[u].z, raw[u].w};
        uint32_t o[2] = {0u, 0u};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float xv = bf2f(j & 1 ? w[j >> 1] >> 16 : w[j >> 1] & 0xffffu);
          const uint32_t c = e4m3_hw_code(bf2f(f2bf(xv / s)));
          o[j >> 2] |= c << (8 * (j & 3));
        }
        res[u] = make_uint2(o[0], o[1]);
      }
    }
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const int64_t v = v0 + u * stride;
      if (v < nvec) st_stream8(out + v * 8, res[u]);
    }
  }
}

// Measurement aid: the per-tensor quantize's memory access with no
// arithmetic -- workgroup b reads the U * 256 consecutive 16-byte groups
// from b * U * 256 (non-temporal), every load before the first store, and
// writes 8 bytes per group (half of each one's bytes) -- so a quantize's
// bandwidth can be read against what its own access pattern reaches.
template <int U>
__global__ void __launch_bounds__(256) k_stream_2to1(const uint16_t* __restrict__ x, int64_t nvec,
                                                     uint8_t* __restrict__ out) {
  const int64_t v0 = (int64_t)blockIdx.x * (U * 256) + threadIdx.x;
  uint4 raw[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t v = v0 + u * 256;
    raw[u] = ld_stream16(x + (v < nvec ? v : nvec - 1) * 8);
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t v = v0 + u * 256;
    if (v < nvec)
      st_stream8(out + v * 8, make_uint2(__builtin_amdgcn_perm(raw[u].y, raw[u].x, 0x07050301u),
                                         __builtin_amdgcn_perm(raw[u].w, raw[u].z, 0x07050301u)));
  }
}

// ------------------------------------------------------------ posit tables
// A posit's code (or reference-form value) as a function of the bfloat16
// pattern q = bf16(x / s) only changes for magnitudes between the flush
// threshold and maxpos.  Each workgroup builds an LDS table indexed by
//   key(q) = min(max(q & 0x7fff, lo1), hi1) - lo1 + (q & 0x8000 ? PLANE : 0)
// with lo1 = lo - 1 below the flush threshold (every smaller magnitude, zero
// included, shares its entry) and hi1 = hi + 1 above maxpos (every larger
// finite magnitude saturates there); lo .. hi (host-chosen, one binade
// beyond both ends) get the closed form.  Non-finite q, which the clamp
// would send to the saturated entry, are caught per batch and take NaR.  The
// closed form runs once per positive magnitude; its negative twin is the
// posit negation (two's complement of the code; the value with its sign
// flipped, zero staying +0).  Two keys cost six packed 16-bit ops.
constexpr int TAB_THREADS = 1024;
constexpr int TAB_UNROLL = 4;
constexpr uint32_t TAB_PLANE = 0x2000;  // entries per sign plane (max)

template <bool PACKED>
__device__ __forceinline__ uint32_t posit_entry(uint32_t b, const vh_format& f) {
  const float v = fmt_value_k<K_POSIT>(b, f, nullptr);
  return PACKED ? fmt_code_k<K_POSIT>(b, v, f, nullptr) : f2bf(v);
}

template <bool PACKED>
__device__ __forceinline__ uint32_t posit_negate(uint32_t c, const vh_format& f) {
  if constexpr (PACKED) return (0u - c) & ((1u << f.p0) - 1u);
  else return (c & 0x7fffu) ? (c ^ 0x8000u) : c;
}

template <bool PACKED>
__device__ __forceinline__ void build_posit_table(const vh_format& f, int lo1, int hi1, void* tab) {
  uint8_t* tb = (uint8_t*)tab;
  uint16_t* th = (uint16_t*)tab;
  for (int m = lo1 + (int)threadIdx.x; m <= hi1; m += blockDim.x) {
    const uint32_t b = m == lo1 ? 1u : m == hi1 ? 0x7f7fu : (uint32_t)m;
    const uint32_t c = posit_entry<PACKED>(b, f);
    const uint32_t n = posit_negate<PACKED>(c, f);
    const int i = m - lo1;
    if constexpr (PACKED) {
      tb[i] = (uint8_t)c;
      tb[i + TAB_PLANE] = (uint8_t)n;
    } else {
      th[i] = (uint16_t)c;
      th[i + TAB_PLANE] = (uint16_t)n;
    }
  }
  __syncthreads();
}

// Table offsets of the two bf16 patterns in q, one per half.
VH_DEV uint32_t posit_keys(uint32_t q, uint32_t lo1x2, uint32_t hi1x2) {
  const uint32_t c = pk_min_u16(pk_max_u16(q & 0x7fff7fffu, lo1x2), hi1x2);
  return pk_sub_u16(c, lo1x2) | ((q >> 2) & 0x20002000u);
}

// quantize(x, s, qmap=posit) per tensor: q = bf16(x / s) as in k_quantize_pt,
// then the table.  One 1024-thread workgroup per CU builds the table once;
// its first loads are issued before the build and each later batch is
// loaded while the previous one converts.  q is formed from x * rcp(s) with the hardware
// bf16 converter; a thread whose batch holds a product within 4 fp32 ulps of
// a bf16 rounding midpoint (or a scale outside the normal range) redoes the
// batch with the correctly rounded division, and a batch holding a
// non-finite q looks each element's NaR case up separately.
template <bool PACKED>
__global__ void __launch_bounds__(TAB_THREADS)
k_quantize_posit_tab(const uint16_t* __restrict__ x, int64_t nvec, const void* sp, int sdt, vh_format f, int lo, int hi,
                     void* __restrict__ out) {
  extern __shared__ uint32_t tab[];
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t step = stride * TAB_UNROLL;
  auto load = [&](uint4* raw, int64_t v0) {
#pragma unroll
    for (int u = 0; u < TAB_UNROLL; ++u) {
      const int64_t v = v0 + u * stride;
      raw[u] = v < nvec ? ld_stream16(x + v * 8) : make_uint4(0, 0, 0, 0);
    }
  };
  int64_t v0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  uint4 r0[TAB_UNROLL], r1[TAB_UNROLL];
  load(r0, v0);
  const int lo1 = lo - 1, hi1 = hi + 1;
  build_posit_table<PACKED>(f, lo1, hi1, tab);
  const uint32_t nar[2] = {posit_entry<PACKED>(0x7fc0u, f), posit_entry<PACKED>(0xffc0u, f)};
  const uint32_t lo1x2 = (uint32_t)lo1 | ((uint32_t)lo1 << 16);
  const uint32_t hi1x2 = (uint32_t)hi1 | ((uint32_t)hi1 << 16);
  const uint8_t* tb = (const uint8_t*)tab;
  const uint16_t* th = (const uint16_t*)tab;
  const float s = load_any(sp, sdt, 0);
  const float as = fabsf(s);
  const bool fast = as >= 0x1p-126f && as <= 0x1p126f;
  const float r = __builtin_amdgcn_rcpf(s);
  // both entries of q, packed; with `special` a non-finite half takes NaR
  auto lookup = [&](uint32_t q, bool special) -> uint32_t {
    const uint32_t k = posit_keys(q, lo1x2, hi1x2);
    uint32_t c0 = PACKED ? (uint32_t)tb[k & 0xffffu] : (uint32_t)th[k & 0xffffu];
    uint32_t c1 = PACKED ? (uint32_t)tb[k >> 16] : (uint32_t)th[k >> 16];
    if (special) {
      if ((q & 0x7fffu) >= 0x7f80u) c0 = nar[(q >> 15) & 1u];
      if (((q >> 16) & 0x7fffu) >= 0x7f80u) c1 = nar[q >> 31];
    }
    return PACKED ? (c0 | (c1 << 8)) : (c0 | (c1 << 16));
  };
  auto convert = [&](const uint4* raw, int64_t vb) {
    uint32_t qb[TAB_UNROLL][4];
    uint32_t mn = 0xffffffffu, mx = 0u;
#pragma unroll
    for (int u = 0; u < TAB_UNROLL; ++u) {
      const uint32_t w[4] = {raw[u].x, raw[u].y, raw[u].z, raw[u].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float q0 = __uint_as_float(w[j] << 16) * r;
        const float q1 = __uint_as_float(w[j] & 0xffff0000u) * r;
        const uint32_t low = __builtin_amdgcn_perm(__float_as_uint(q1), __float_as_uint(q0), 0x05040100u);
        mn = pk_min_u16(mn, pk_sub_u16(low, 0x7ffc7ffcu));
        qb[u][j] = f2bf2_hw(q0, q1);
        mx = pk_max_u16(mx, qb[u][j] & 0x7fff7fffu);
      }
    }
    const bool exact = !fast || (mn & 0xffffu) <= 8u || (mn >> 16) <= 8u;
    if (exact) {  // rare: correctly rounded division
#pragma unroll
      for (int u = 0; u < TAB_UNROLL; ++u) {
        const uint32_t w[4] = {raw[u].x, raw[u].y, raw[u].z, raw[u].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) qb[u][j] = f2bf(bf2f(w[j] & 0xffffu) / s) | (f2bf(bf2f(w[j] >> 16) / s) << 16);
      }
    }
    const bool special = exact || (mx & 0xffffu) >= 0x7f80u || (mx >> 16) >= 0x7f80u;
#pragma unroll
    for (int u = 0; u < TAB_UNROLL; ++u) {
      const int64_t v = vb + u * stride;
      uint32_t o[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] = lookup(qb[u][j], special);
      if (v < nvec) {
        if constexpr (PACKED) st_stream8((uint8_t*)out + v * 8, make_uint2(o[0] | (o[1] << 16), o[2] | (o[3] << 16)));
        else st_stream16((uint16_t*)out + v * 8, make_uint4(o[0], o[1], o[2], o[3]));
      }
    }
  };
  for (;;) {
    if (v0 >= nvec) break;
    load(r1, v0 + step);
    convert(r0, v0);
    v0 += step;
    if (v0 >= nvec) break;
    load(r0, v0 + step);
    convert(r1, v0);
    v0 += step;
  }
}

// Host: the table's magnitude range for a posit map and its LDS bytes, or
// false for a map it does not cover.  Below 2**(floor(-(n-1) 2**es +
// 2**(es-1)) - 1) every magnitude flushes to zero; above 2**((n-2) 2**es +
// 1) every finite one saturates at maxpos.
bool posit_table_range(const vh_format& f, bool packed, int* lo, int* hi, size_t* lds_bytes) {
  const int n = f.p0, es = f.p1;
  if (f.kind != VH_FMT_POSIT || n < 2 || es < 0 || es > 4) return false;
  const double e_lo = std::floor(-(n - 1) * std::ldexp(1.0, es) + std::ldexp(1.0, es - 1)) - 1.0;
  const double e_hi = (n - 2) * std::ldexp(1.0, es) + 1.0;
  if (e_lo < -126 || e_hi > 127) return false;
  *lo = (int)(e_lo + 127) << 7;
  *hi = (int)(e_hi + 127) << 7;
  if (*lo < 1 || *hi + 1 >= 0x7f80 || *hi - *lo + 3 > (int)TAB_PLANE) return false;
  *lds_bytes = (size_t)2 * TAB_PLANE * (packed ? 1 : 2);
  return true;
}

// out[i] = tab[x[i]] (low 16 bits) for i < 16 n16.  A wave takes 1024-code
// units: lane l converts codes 8 l .. 8 l + 7 of each half, so both of its
// 16-byte stores belong to one contiguous 1 KB wave store; GATHER_UNROLL
// units are in flight per wave.  The last n16 % 64 groups of 16 codes go one
// per thread.
constexpr int GATHER_UNROLL = 4;

__device__ __forceinline__ uint4 gather8(uint2 c, const uint32_t* tab) {
  return make_uint4(tab[c.x & 0xffu] | (tab[(c.x >> 8) & 0xffu] << 16),
                    tab[(c.x >> 16) & 0xffu] | (tab[c.x >> 24] << 16),
                    tab[c.y & 0xffu] | (tab[(c.y >> 8) & 0xffu] << 16),
                    tab[(c.y >> 16) & 0xffu] | (tab[c.y >> 24] << 16));
}

__device__ __forceinline__ void gather16(const uint8_t* __restrict__ x, int64_t n16, const uint32_t* tab,
                                         uint16_t* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int64_t units = n16 / 64;
  const int64_t nwaves = ((int64_t)gridDim.x * blockDim.x) >> 6;
  for (int64_t u0 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6; u0 < units; u0 += nwaves * GATHER_UNROLL) {
    uint2 c[GATHER_UNROLL][2];
#pragma unroll
    for (int u = 0; u < GATHER_UNROLL; ++u) {
      const int64_t unit = u0 + u * nwaves;
#pragma unroll
      for (int h = 0; h < 2; ++h)
        c[u][h] = unit < units ? ld_stream8(x + unit * 1024 + h * 512 + lane * 8) : make_uint2(0, 0);
    }
#pragma unroll
    for (int u = 0; u < GATHER_UNROLL; ++u) {
      const int64_t unit = u0 + u * nwaves;
      if (unit < units) {
#pragma unroll
        for (int h = 0; h < 2; ++h) st_stream16(out + unit * 1024 + h * 512 + lane * 8, gather8(c[u][h], tab));
      }
    }
  }
  const int64_t i = units * 64 + (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n16) {
    const uint4 c = ld_stream16(x + i * 16);
    st_stream16(out + i * 16, gather8(make_uint2(c.x, c.y), tab));
    st_stream16(out + i * 16 + 8, gather8(make_uint2(c.z, c.w), tab));
  }
}

// dequantize of packed codes to bfloat16 (optionally times a scalar scale,
// rounded to bf16 as the reference's eager product): a 256-entry table of
// the reference-form values, built per workgroup; 16 codes per thread.
template <int KIN>
__global__ void __launch_bounds__(256)
k_dequantize_tab(const uint8_t* __restrict__ x, int64_t n16, const void* sp, int sdt, vh_format fin,
                 uint16_t* __restrict__ out) {
  __shared__ uint16_t lds_in[2 * VH_MAX_STEPS];
  __shared__ uint32_t tab[256];
  if constexpr (KIN == K_STEPS) stage_steps(fin, lds_in);
  const bool has_s = sp != nullptr;
  const float s = has_s ? load_any(sp, sdt, 0) : 1.0f;
  for (int c = threadIdx.x; c < 256; c += blockDim.x) {
    float v = fmt_decode_k<KIN>((uint32_t)c, fin, lds_in);
    if (has_s) v = rbf(v * s);
    tab[c] = f2bf(v);
  }
  __syncthreads();
  gather16(x, n16, tab, out);
}

// Packed bytes -> bf16 through a 256-entry table held in device memory.
__global__ void __launch_bounds__(256)
k_decode_bytes(const uint8_t* __restrict__ x, int64_t n, const uint16_t* __restrict__ lut, uint16_t* __restrict__ out) {
  __shared__ uint32_t tab[256];
  for (int c = threadIdx.x; c < 256; c += blockDim.x) tab[c] = lut[c];
  __syncthreads();
  const int64_t n16 = n / 16;
  gather16(x, n16, tab, out);
  // the last n % 16 bytes, one per thread of the first workgroup
  if (blockIdx.x == 0 && threadIdx.x < (int)(n - n16 * 16)) {
    const int64_t i = n16 * 16 + threadIdx.x;
    out[i] = (uint16_t)tab[x[i]];
  }
}

template <int KIND, bool PACKED>
__global__ void __launch_bounds__(256)
k_quantize_pt(const uint16_t* __restrict__ x, int64_t nvec, const void* sp, int sdt, vh_format f,
              void* __restrict__ out) {
  __shared__ uint16_t lds[2 * VH_MAX_STEPS];
  if constexpr (KIND == K_STEPS) stage_steps(f, lds);
  const float s = load_any(sp, sdt, 0);
  const float as = fabsf(s);
  const bool fast = as >= 0x1p-126f && as <= 0x1p126f;
  const float r = __builtin_amdgcn_rcpf(s);
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t v0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; v0 < nvec; v0 += stride * UNROLL) {
    uint4 raw[UNROLL];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const int64_t v = v0 + u * stride;
      raw[u] = v < nvec ? ld_stream16(x + v * 8) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const int64_t v = v0 + u * stride;
      if (v >= nvec) break;
      const uint32_t w[4] = {raw[u].x, raw[u].y, raw[u].z, raw[u].w};
      float q[8];
      bool slow = !fast;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float xv = bf2f(j & 1 ? w[j >> 1] >> 16 : w[j >> 1] & 0xffffu);
        q[j] = xv * r;
        const uint32_t ub = __float_as_uint(q[j]);
        slow |= ((ub - 0x7FFCu) & 0xFFFFu) <= 8u;
      }
      uint32_t qb[4];
      if (!slow) {
#pragma unroll
        for (int j = 0; j < 4; ++j) qb[j] = f2bf2_hw(q[2 * j], q[2 * j + 1]);
      } else {  // near a bf16 midpoint: correctly rounded division
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float x0 = bf2f(w[j] & 0xffffu), x1 = bf2f(w[j] >> 16);
          qb[j] = f2bf(x0 / s) | (f2bf(x1 / s) << 16);
        }
      }
      uint32_t o[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uint32_t c[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const uint32_t b = (qb[j] >> (16 * h)) & 0xffffu;
          if constexpr (KIND == K_E4M3) {
            c[h] = e4m3_hw_code(bf2f(b));
            if constexpr (!PACKED) c[h] = f2bf(__builtin_amdgcn_cvt_f32_fp8((int)c[h], 0));
          } else if constexpr (KIND == K_NONE) {
            c[h] = b;
          } else {
            const float val = fmt_value_k<KIND>(b, f, lds);
            c[h] = PACKED ? fmt_code_k<KIND>(b, val, f, lds) : f2bf(val);
          }
        }
        o[j] = PACKED ? (c[0] | (c[1] << 8)) : (c[0] | (c[1] << 16));
      }
      if constexpr (PACKED) {
        st_stream8((uint8_t*)out + v * 8, make_uint2(o[0] | (o[1] << 16), o[2] | (o[3] << 16)));
      } else {
        st_stream16((uint16_t*)out + v * 8, make_uint4(o[0], o[1], o[2], o[3]));
      }
    }
  }
}

static int check_shape(const int64_t* shape, int32_t ndim, Shape* s, int64_t* n) {
  VH_REQUIRE(ndim >= 0 && ndim <= VH_MAX_DIMS, "tensor rank %d exceeds %d", ndim, VH_MAX_DIMS);
  int64_t total = 1;
  s->ndim = ndim > 0 ? ndim : 1;
  for (int d = 0; d < VH_MAX_DIMS; ++d) s->dim[d] = 1;
  for (int d = 0; d < ndim; ++d) {
    VH_REQUIRE(shape[d] >= 0, "negative size");
    s->dim[d] = shape[d];
    total *= shape[d];
  }
  *n = total;
  return VH_OK;
}

static int check_param(const vh_param* p, const Shape& s, const char* name) {
  if (!p || !p->ptr) return VH_OK;
  VH_REQUIRE(vh::is_float_dtype(p->dtype), "%s: dtype %d is not a float dtype", name, p->dtype);
  if (p->scalar) return VH_OK;
  for (int d = 0; d < s.ndim; ++d) {
    VH_REQUIRE(p->div[d] >= 1, "%s: divisor of dim %d must be >= 1", name, d);
    VH_REQUIRE(p->stride[d] >= 0, "%s: negative stride", name);
  }
  return VH_OK;
}

static int check_fmt(const vh_format* f, const char* name) {
  if (!f) return VH_OK;
  VH_REQUIRE(f->kind >= VH_FMT_IDENTITY && f->kind <= VH_FMT_LUT, "%s: bad format kind %d", name, f->kind);
  VH_REQUIRE(f->kind != VH_FMT_STEPS || (f->nsteps >= 0 && f->nsteps < VH_MAX_STEPS),
             "%s: nsteps out of range", name);
  VH_REQUIRE(f->kind != VH_FMT_LUT || f->lut, "%s: LUT format without a table", name);
  return VH_OK;
}

static vh_param null_param() {
  vh_param p;
  memset(&p, 0, sizeof(p));
  return p;
}

static bool packable(const vh_format* f) {
  if (!f) return false;
  switch (f->kind) {
    case VH_FMT_INT: return (f->p0 >= -128 && f->p1 <= 127) || (f->p0 >= 0 && f->p1 <= 255);
    case VH_FMT_MINIFLOAT: return f->p0 + f->p1 + ((f->flags & VH_FMT_SIGNED) ? 1 : 0) <= 8;
    case VH_FMT_POSIT: return f->p0 <= 8;
    case VH_FMT_STEPS: return true;
    default: return false;
  }
}

extern "C" int vh_stream_2to1(const void* x, int64_t nvec, void* out, vh_stream_t stream) {
  VH_REQUIRE(x && out && nvec > 0, "vh_stream_2to1: null argument or empty");
  VH_REQUIRE(((uintptr_t)x % 16) == 0 && ((uintptr_t)out % 8) == 0, "vh_stream_2to1: misaligned operand");
  VH_REQUIRE(nvec / 1024 < (1ll << 31), "vh_stream_2to1: too large");
  hipStream_t st = vh::as_stream(stream);
  // the E4M3 quantize's choice: 4 groups per thread up to 2^21 groups, 8 beyond
  if (nvec <= (1ll << 21))
    hipLaunchKernelGGL(k_stream_2to1<4>, dim3((unsigned)((nvec + 1023) / 1024)), dim3(256), 0, st,
                       (const uint16_t*)x, nvec, (uint8_t*)out);
  else
    hipLaunchKernelGGL(k_stream_2to1<8>, dim3((unsigned)((nvec + 2047) / 2048)), dim3(256), 0, st,
                       (const uint16_t*)x, nvec, (uint8_t*)out);
  return vh::check_launch("vh_stream_2to1");
}

extern "C" int vh_quantize(const void* x, int32_t x_dtype, const int64_t* shape, int32_t ndim,
                           const vh_param* scale, const vh_param* zero_point, int32_t compute_dtype,
                           const vh_format* fmt, void* out, int32_t out_dtype, vh_stream_t stream) {
  Shape s;
  int64_t n;
  int rc;
  if ((rc = check_shape(shape, ndim, &s, &n))) return rc;
  VH_REQUIRE(x && out, "vh_quantize: null tensor");
  VH_REQUIRE(vh::is_float_dtype(x_dtype), "vh_quantize: input dtype %d unsupported", x_dtype);
  VH_REQUIRE(vh::is_float_dtype(compute_dtype), "vh_quantize: compute dtype %d unsupported", compute_dtype);
  if ((rc = check_param(scale, s, "scale"))) return rc;
  if ((rc = check_param(zero_point, s, "zero_point"))) return rc;
  if ((rc = check_fmt(fmt, "qmap"))) return rc;
  VH_REQUIRE(out_dtype != VH_U8 || packable(fmt), "vh_quantize: this map has no packed form");
  VH_REQUIRE(out_dtype == VH_U8 || vh::is_float_dtype(out_dtype), "vh_quantize: bad output dtype");
  if (n == 0) return VH_OK;
  vh_param sp = scale ? *scale : null_param();
  vh_param zp = zero_point ? *zero_point : null_param();
  vh_format f;
  memset(&f, 0, sizeof(f));
  if (fmt) f = *fmt;
  hipStream_t st = vh::as_stream(stream);
  const bool aligned = ((uintptr_t)x % 16 == 0) && ((uintptr_t)out % 16 == 0);
  if (x_dtype == VH_BF16 && compute_dtype == VH_BF16 && sp.ptr && sp.scalar && !zp.ptr && n % 8 == 0 && aligned &&
      (out_dtype == VH_U8 || out_dtype == VH_BF16)) {
    const int64_t nvec = n / 8;
    VH_REQUIRE(nvec / 1024 < (1ll << 31), "vh_quantize: tensor too large");
    int64_t blocks = (nvec + 256 * UNROLL - 1) / (256 * UNROLL);
    if (blocks > 8192) blocks = 8192;
    int lo = 0, hi = 0;
    size_t tab_bytes = 0;
    // the posit table costs a few thousand closed-form evaluations per
    // workgroup: one 1024-thread workgroup per CU, each over a long range
    int64_t tab_blocks = (nvec + TAB_THREADS * TAB_UNROLL - 1) / (TAB_THREADS * TAB_UNROLL);
    if (tab_blocks > 256) tab_blocks = 256;
    return dispatch_kind(kernel_kind(fmt), [&](auto kind) {
      constexpr int K = decltype(kind)::value;
      if (out_dtype == VH_U8) {
        if constexpr (K == K_NONE || K == K_IDENTITY || K == K_LUT) {
          return (int)VH_EINVAL;  // unreachable: checked by packable()
        } else if constexpr (K == K_E4M3) {
          // 4 groups per thread up to 2^21 groups, 8 beyond (measured best for
          // the 16.8 MB and 58.7 MB inputs)
          if (nvec <= (1ll << 21)) {
            hipLaunchKernelGGL(k_quantize_e4m3_pt<4>, dim3((unsigned)((nvec + 1023) / 1024)), dim3(256), 0, st,
                               (const uint16_t*)x, nvec, sp.ptr, sp.dtype, (uint8_t*)out);
          } else {
            hipLaunchKernelGGL(k_quantize_e4m3_pt<8>, dim3((unsigned)((nvec + 2047) / 2048)), dim3(256), 0, st,
                               (const uint16_t*)x, nvec, sp.ptr, sp.dtype, (uint8_t*)out);
          }
        } else if (K == K_POSIT && posit_table_range(f, true, &lo, &hi, &tab_bytes)) {
          hipLaunchKernelGGL(k_quantize_posit_tab<true>, dim3((unsigned)tab_blocks), dim3(TAB_THREADS), tab_bytes, st,
                             (const uint16_t*)x, nvec, sp.ptr, sp.dtype, f, lo, hi, out);
        } else {
          hipLaunchKernelGGL((k_quantize_pt<K, true>), dim3((unsigned)blocks), dim3(256), 0, st,
                             (const uint16_t*)x, nvec, sp.ptr, sp.dtype, f, out);
        }
      } else if (K == K_POSIT && posit_table_range(f, false, &lo, &hi, &tab_bytes)) {
        hipLaunchKernelGGL(k_quantize_posit_tab<false>, dim3((unsigned)tab_blocks), dim3(TAB_THREADS), tab_bytes, st,
                           (const uint16_t*)x, nvec, sp.ptr, sp.dtype, f, lo, hi, out);
      } else {
        hipLaunchKernelGGL((k_quantize_pt<K, false>), dim3((unsigned)blocks), dim3(256), 0, st,
                           (const uint16_t*)x, nvec, sp.ptr, sp.dtype, f, out);
      }
      return vh::check_launch("vh_quantize");
    });
  }
  int64_t threads = (n + VEC - 1) / VEC;
  int64_t blocks = (threads + 255) / 256;
  VH_REQUIRE(blocks < (1ll << 31), "vh_quantize: tensor too large");
  return dispatch_kind(kernel_kind(fmt), [&](auto kind) {
    constexpr int K = decltype(kind)::value;
    hipLaunchKernelGGL(k_quantize<K>, dim3((unsigned)blocks), dim3(256), 0, st, x, x_dtype, n, s, sp, zp,
                       compute_dtype, f, out, out_dtype);
    return vh::check_launch("vh_quantize");
  });
}

// ------------------------------------------------------------ stochastic rounding
// quantize with a seed (ops/quantized.py:318-446, 449-515): x / scale (+ zp)
// as quantize computes it, then rounded to one of the two levels around it.
// Element i (logical row-major order) takes byte i % 4 of word i % 16 / 4 of
// the Philox4x32-10 draw (Salmon et al., SC'11) of counter i / 16 keyed by
// the 64-bit seed; it rounds to the level farther from zero when
// |v| + byte / 256 * (high - low) >= |far| in float32.  One thread: the 16
// elements of one draw.  Levels in LDS, searched as torch.searchsorted
// (first level >= v; NaN past the end).
constexpr int SR_ELEMS = 16;

VH_DEV void philox4x32_10(uint32_t c[4], uint32_t k0, uint32_t k1) {
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    const uint32_t hi0 = __umulhi(c[0], 0xD2511F53u), lo0 = c[0] * 0xD2511F53u;
    const uint32_t hi1 = __umulhi(c[2], 0xCD9E8D57u), lo1 = c[2] * 0xCD9E8D57u;
    const uint32_t n0 = hi1 ^ c[1] ^ k0, n2 = hi0 ^ c[3] ^ k1;
    c[0] = n0, c[1] = lo1, c[2] = n2, c[3] = lo0;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
}

// The rounding rule on one value: no contraction, each float32 operation
// rounded as torch's eager ops round it.
VH_DEV float sr_round(float v, const float* lv, int nlev, uint32_t byte) {
#pragma clang fp contract(off)
  if (!isnan_f(v)) v = fminf(fmaxf(v, lv[0]), lv[nlev - 1]);
  int lo = 0, hi = nlev;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (!(lv[mid] >= v)) lo = mid + 1;
    else hi = mid;
  }
  const int upper = lo < nlev - 1 ? lo : nlev - 1;
  const float high = lv[upper];
  const float low = high == v ? high : lv[upper > 0 ? upper - 1 : 0];
  const bool neg = v < 0.0f;
  const float near = neg ? high : low, far = neg ? low : high;
  const float noise = (float)byte / 256.0f;
  const float gap = high - low;
  const float step = noise * gap;
  const float lhs = fabsf(v) + step;
  return lhs >= fabsf(far) ? far : near;
}

__global__ void __launch_bounds__(256)
k_quantize_sr(const void* __restrict__ x, int x_dtype, int64_t n, Shape shape, vh_param sp, vh_param zp, int cdt,
              const void* __restrict__ levels, int lv_dtype, int nlev, const int64_t* __restrict__ seed,
              void* __restrict__ out, int out_dtype) {
  extern __shared__ float s_lv[];
  for (int i = threadIdx.x; i < nlev; i += blockDim.x) s_lv[i] = load_any(levels, lv_dtype, i);
  __syncthreads();
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t base = t * SR_ELEMS;
  if (base >= n) return;
  const uint64_t sd = (uint64_t)seed[0];
  uint32_t w[4] = {(uint32_t)t, (uint32_t)((uint64_t)t >> 32), 0u, 0u};
  philox4x32_10(w, (uint32_t)sd, (uint32_t)(sd >> 32));
  const float s0 = (sp.ptr && sp.scalar) ? load_any(sp.ptr, sp.dtype, 0) : 1.0f;
  const float z0 = (zp.ptr && zp.scalar) ? load_any(zp.ptr, zp.dtype, 0) : 0.0f;
#pragma unroll
  for (int h = 0; h < SR_ELEMS / VEC; ++h) {
    const int64_t b8 = base + h * VEC;
    if (b8 >= n) break;
    float sv[VEC], zv[VEC];
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
      sv[j] = s0;
      zv[j] = z0;
    }
    if (sp.ptr && !sp.scalar) param_values(sp, shape, b8, n, sv);
    if (zp.ptr && !zp.scalar) param_values(zp, shape, b8, n, zv);
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
      const int64_t i = b8 + j;
      if (i >= n) break;
      float q = load_any(x, x_dtype, i);
      if (sp.ptr) q = div_round(q, sv[j], cdt);
      if (zp.ptr) q = round_to(q + zv[j], cdt);
      const int e = h * VEC + j;
      const uint32_t byte = (w[e >> 2] >> (8 * (e & 3))) & 0xFFu;
      store_any(out, out_dtype, i, sr_round(q, s_lv, nlev, byte));
    }
  }
}

extern "C" int vh_quantize_sr(const void* x, int32_t x_dtype, const int64_t* shape, int32_t ndim,
                              const vh_param* scale, const vh_param* zero_point, int32_t compute_dtype,
                              const void* levels, int32_t levels_dtype, int32_t nlevels, const int64_t* seed,
                              void* out, int32_t out_dtype, vh_stream_t stream) {
  Shape s;
  int64_t n;
  int rc;
  if ((rc = check_shape(shape, ndim, &s, &n))) return rc;
  VH_REQUIRE(x && out && levels && seed, "vh_quantize_sr: null pointer");
  VH_REQUIRE(vh::is_float_dtype(x_dtype) && vh::is_float_dtype(compute_dtype) && vh::is_float_dtype(out_dtype) &&
                 vh::is_float_dtype(levels_dtype),
             "vh_quantize_sr: dtypes must be bf16, fp16 or fp32");
  VH_REQUIRE(nlevels >= 1 && nlevels <= VH_SR_MAX_LEVELS, "vh_quantize_sr: %d levels (1 .. %d supported)", nlevels,
             VH_SR_MAX_LEVELS);
  if ((rc = check_param(scale, s, "scale"))) return rc;
  if ((rc = check_param(zero_point, s, "zero_point"))) return rc;
  if (n == 0) return VH_OK;
  const vh_param sp = scale ? *scale : null_param();
  const vh_param zp = zero_point ? *zero_point : null_param();
  const int64_t threads = (n + SR_ELEMS - 1) / SR_ELEMS;
  const int64_t blocks = (threads + 255) / 256;
  VH_REQUIRE(blocks < (1ll << 31), "vh_quantize_sr: tensor too large");
  hipLaunchKernelGGL(k_quantize_sr, dim3((unsigned)blocks), dim3(256), (size_t)nlevels * sizeof(float),
                     vh::as_stream(stream), x, x_dtype, n, s, sp, zp, compute_dtype, levels, levels_dtype, nlevels,
                     seed, out, out_dtype);
  return vh::check_launch("vh_quantize_sr");
}

// ------------------------------------------------------------ codebooks
// encode (ops/quantized.py:232-287) and decode (:290-315) against codebook
// tables under a region grid (_region_view, :193-229): element e uses table
// region(e) = sum_d (i_d / div[d]) * stride[d].  encode rounds its value to
// bfloat16 and counts the leading edges with !(edge >= v), which is
// torch.searchsorted's left bisection (a NaN lands past the last edge), then
// writes that index or its entry.  The edges are staged in LDS when all the
// tables fit in CB_LDS_FLOATS; otherwise the search reads them through the
// cache.
constexpr int CB_LDS_FLOATS = 12288;

struct CbDev {
  const float* edges;
  const void* entries;
  int edt;
  int nedges, k;
  int top;  // the largest power of two <= nedges (0: no edges)
  int64_t regions;
  vh_param region;
};

VH_DEV int cb_search(const float* E, int nedges, int top, float v) {
  int lo = 0;
  for (int step = top; step > 0; step >>= 1) {
    const int j = lo + step;
    if (j <= nedges && !(E[j - 1] >= v)) lo = j;
  }
  return lo;
}

template <bool STAGE>
__global__ void __launch_bounds__(256)
k_encode(const void* __restrict__ x, int x_dtype, int64_t n, Shape shape, vh_param sp, vh_param zp, int cdt,
         CbDev cb, void* __restrict__ out) {
  extern __shared__ float s_edges[];
  const float* E = cb.edges;
  if constexpr (STAGE) {
    const int total = (int)(cb.regions * cb.nedges);
    for (int i = threadIdx.x; i < total; i += blockDim.x) s_edges[i] = cb.edges[i];
    __syncthreads();
    E = s_edges;
  }
  const int64_t base = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * VEC;
  if (base >= n) return;
  const bool narrow = n < (1ll << 31);
  float sv[VEC], zv[VEC];
  const float s0 = (sp.ptr && sp.scalar) ? load_any(sp.ptr, sp.dtype, 0) : 1.0f;
  const float z0 = (zp.ptr && zp.scalar) ? load_any(zp.ptr, zp.dtype, 0) : 0.0f;
#pragma unroll
  for (int j = 0; j < VEC; ++j) {
    sv[j] = s0;
    zv[j] = z0;
  }
  if (sp.ptr && !sp.scalar) param_values(sp, shape, base, n, sv);
  if (zp.ptr && !zp.scalar) param_values(zp, shape, base, n, zv);
  for (int j = 0; j < VEC; ++j) {
    const int64_t i = base + j;
    if (i >= n) break;
    float q = load_any(x, x_dtype, i);
    if (sp.ptr) q = div_round(q, sv[j], cdt);
    if (zp.ptr) q = round_to(q + zv[j], cdt);
    const int64_t r = cb.region.scalar ? 0 : param_offset(cb.region, shape, i, narrow);
    const int idx = cb_search(E + r * cb.nedges, cb.nedges, cb.top, rbf(q));
    const float val = cb.entries ? load_any(cb.entries, cb.edt, r * cb.k + idx) : (float)idx;
    store_any(out, cdt, i, round_to(val, cdt));
  }
}

// decode: entry long(x) of the element's table (negative indices count from
// the end when `wrap`), rounded to the codes' dtype, NaN where torch's
// indexing would raise; then, with a scale, times the element's scale,
// rounded to out_dtype.
__global__ void __launch_bounds__(256)
k_decode_cb(const void* __restrict__ x, int x_dtype, int64_t n, Shape shape, CbDev cb, int wrap, vh_param sp,
            void* __restrict__ out, int out_dtype) {
  const int64_t base = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * VEC;
  if (base >= n) return;
  const bool narrow = n < (1ll << 31);
  float sv[VEC];
  const float s0 = (sp.ptr && sp.scalar) ? load_any(sp.ptr, sp.dtype, 0) : 1.0f;
#pragma unroll
  for (int j = 0; j < VEC; ++j) sv[j] = s0;
  if (sp.ptr && !sp.scalar) param_values(sp, shape, base, n, sv);
  for (int j = 0; j < VEC; ++j) {
    const int64_t i = base + j;
    if (i >= n) break;
    const float c = load_any(x, x_dtype, i);
    float val = __builtin_nanf("");
    if (fabsf(c) < 0x1p62f) {
      int64_t t = (int64_t)c;
      if (t < 0 && wrap) t += cb.k;
      if (t >= 0 && t < cb.k) {
        const int64_t r = cb.region.scalar ? 0 : param_offset(cb.region, shape, i, narrow);
        val = round_to(load_any(cb.entries, cb.edt, r * cb.k + t), x_dtype);
      }
    }
    if (sp.ptr) val = round_to(val * sv[j], out_dtype);
    store_any(out, out_dtype, i, val);
  }
}

static int check_codebook(const vh_codebook* cb, const Shape& s, bool encode, CbDev* d) {
  VH_REQUIRE(cb, "codebook: null descriptor");
  VH_REQUIRE(cb->k >= 1 && cb->k <= 65536, "codebook: %d entries per table (1 .. 65536 supported)", cb->k);
  VH_REQUIRE(cb->regions >= 1, "codebook: %lld regions", (long long)cb->regions);
  if (encode) {
    VH_REQUIRE(cb->nedges >= 0 && cb->nedges < 65536, "codebook: %d edges per table", cb->nedges);
    VH_REQUIRE(cb->nedges == 0 || cb->edges, "codebook: edges missing");
    VH_REQUIRE(!cb->entries || cb->nedges == cb->k - 1, "codebook: %d edges for %d entries", cb->nedges, cb->k);
  } else {
    VH_REQUIRE(cb->entries, "codebook: entries missing");
  }
  VH_REQUIRE(!cb->entries || vh::is_float_dtype(cb->entries_dtype), "codebook: entry dtype %d unsupported",
             cb->entries_dtype);
  if (!cb->region.scalar) {
    for (int dd = 0; dd < s.ndim; ++dd) {
      VH_REQUIRE(cb->region.div[dd] >= 1 && cb->region.stride[dd] >= 0, "codebook: bad region grid on dim %d", dd);
    }
  }
  d->edges = cb->edges;
  d->entries = cb->entries;
  d->edt = cb->entries_dtype;
  d->nedges = cb->nedges;
  d->k = cb->k;
  int top = 0;
  if (cb->nedges > 0) {
    top = 1;
    while (top * 2 <= cb->nedges) top *= 2;
  }
  d->top = top;
  d->regions = cb->regions;
  d->region = cb->region;
  return VH_OK;
}

extern "C" int vh_quantize_codebook(const void* x, int32_t x_dtype, const int64_t* shape, int32_t ndim,
                                    const vh_param* scale, const vh_param* zero_point, int32_t compute_dtype,
                                    const vh_codebook* cb, void* out, vh_stream_t stream) {
  Shape s;
  int64_t n;
  int rc;
  if ((rc = check_shape(shape, ndim, &s, &n))) return rc;
  VH_REQUIRE(x && out, "vh_quantize_codebook: null tensor");
  VH_REQUIRE(vh::is_float_dtype(x_dtype) && vh::is_float_dtype(compute_dtype),
             "vh_quantize_codebook: dtypes must be bf16, fp16 or fp32");
  if ((rc = check_param(scale, s, "scale"))) return rc;
  if ((rc = check_param(zero_point, s, "zero_point"))) return rc;
  CbDev d;
  if ((rc = check_codebook(cb, s, true, &d))) return rc;
  if (n == 0) return VH_OK;
  const vh_param sp = scale ? *scale : null_param();
  const vh_param zp = zero_point ? *zero_point : null_param();
  const int64_t blocks = ((n + VEC - 1) / VEC + 255) / 256;
  VH_REQUIRE(blocks < (1ll << 31), "vh_quantize_codebook: tensor too large");
  const int64_t total = d.regions * d.nedges;
  if (total <= CB_LDS_FLOATS) {
    hipLaunchKernelGGL(k_encode<true>, dim3((unsigned)blocks), dim3(256), (size_t)(total ? total : 1) * sizeof(float),
                       vh::as_stream(stream), x, x_dtype, n, s, sp, zp, compute_dtype, d, out);
  } else {
    hipLaunchKernelGGL(k_encode<false>, dim3((unsigned)blocks), dim3(256), 0, vh::as_stream(stream), x, x_dtype, n, s,
                       sp, zp, compute_dtype, d, out);
  }
  return vh::check_launch("vh_quantize_codebook");
}

extern "C" int vh_decode_codebook(const void* x, int32_t x_dtype, const int64_t* shape, int32_t ndim,
                                  const vh_codebook* cb, int32_t wrap_negative, const vh_param* scale, void* out,
                                  int32_t out_dtype, vh_stream_t stream) {
  Shape s;
  int64_t n;
  int rc;
  if ((rc = check_shape(shape, ndim, &s, &n))) return rc;
  VH_REQUIRE(x && out, "vh_decode_codebook: null tensor");
  VH_REQUIRE(vh::is_float_dtype(x_dtype) && vh::is_float_dtype(out_dtype),
             "vh_decode_codebook: dtypes must be bf16, fp16 or fp32");
  if ((rc = check_param(scale, s, "scale"))) return rc;
  CbDev d;
  if ((rc = check_codebook(cb, s, false, &d))) return rc;
  if (n == 0) return VH_OK;
  const vh_param sp = scale ? *scale : null_param();
  const int64_t blocks = ((n + VEC - 1) / VEC + 255) / 256;
  VH_REQUIRE(blocks < (1ll << 31), "vh_decode_codebook: tensor too large");
  hipLaunchKernelGGL(k_decode_cb, dim3((unsigned)blocks), dim3(256), 0, vh::as_stream(stream), x, x_dtype, n, s, d,
                     wrap_negative ? 1 : 0, sp, out, out_dtype);
  return vh::check_launch("vh_decode_codebook");
}

// ------------------------------------------------------------ block amax
// max |x| over blocks of `block` along L of contiguous [outer, L, inner]
// (zero padding past L, NaN propagating as torch.amax): one stage of
// _shared_exponents' / calculate_mx_qparam's reduction over several axes
// (quantization/mx_utils.py:16-63, ops/quantized.py:958-1031).  One thread
// per output element; consecutive threads take consecutive `inner`.
__global__ void __launch_bounds__(256)
k_block_amax(const void* __restrict__ x, int dt, int64_t outer, int64_t L, int64_t inner, int64_t block, int64_t nb,
             void* __restrict__ out) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= outer * nb * inner) return;
  const int64_t i = t % inner, b = (t / inner) % nb, o = t / (inner * nb);
  const int64_t l0 = b * block, l1 = l0 + block < L ? l0 + block : L;
  float m = 0.0f;
  for (int64_t l = l0; l < l1; ++l) m = nmax(m, fabsf(load_any(x, dt, (o * L + l) * inner + i)));
  store_any(out, dt, t, m);
}

extern "C" int vh_block_amax(const void* x, int32_t x_dtype, int64_t outer, int64_t L, int64_t inner, int64_t block,
                             void* out, vh_stream_t stream) {
  VH_REQUIRE(x && out, "vh_block_amax: null tensor");
  VH_REQUIRE(vh::is_float_dtype(x_dtype), "vh_block_amax: dtype %d unsupported", x_dtype);
  VH_REQUIRE(outer >= 0 && L >= 0 && inner >= 0 && block >= 1, "vh_block_amax: bad view");
  const int64_t nb = (L + block - 1) / block, total = outer * nb * inner;
  if (total == 0) return VH_OK;
  const int64_t blocks = (total + 255) / 256;
  VH_REQUIRE(blocks < (1ll << 31), "vh_block_amax: tensor too large");
  hipLaunchKernelGGL(k_block_amax, dim3((unsigned)blocks), dim3(256), 0, vh::as_stream(stream), x, x_dtype, outer, L,
                     inner, block, nb, out);
  return vh::check_launch("vh_block_amax");
}

// ------------------------------------------------------------ dequantize
template <int KIN>
__global__ void __launch_bounds__(256)
k_dequantize(const void* __restrict__ x, int x_dtype, int64_t n, Shape shape, vh_param sp, vh_param zp, int cdt,
             vh_format fin, int has_out, vh_format fout, void* __restrict__ out, int out_dtype) {
  __shared__ uint16_t lds_in[2 * VH_MAX_STEPS];
  __shared__ uint16_t lds_out[2 * VH_MAX_STEPS];
  if constexpr (KIN == K_STEPS) stage_steps(fin, lds_in);
  if (has_out) stage_steps(fout, lds_out);
  int64_t base = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * VEC;
  if (base >= n) return;
  const bool full = base + VEC <= n;
  float sv[VEC], zv[VEC];
  const float s0 = (sp.ptr && sp.scalar) ? load_any(sp.ptr, sp.dtype, 0) : 1.0f;
  const float z0 = (zp.ptr && zp.scalar) ? load_any(zp.ptr, zp.dtype, 0) : 0.0f;
#pragma unroll
  for (int j = 0; j < VEC; ++j) {
    sv[j] = s0;
    zv[j] = z0;
  }
  if (sp.ptr && !sp.scalar) param_values(sp, shape, base, n, sv);
  if (zp.ptr && !zp.scalar) param_values(zp, shape, base, n, zv);
  // inputs: bf16 patterns (16-byte loads when the group is whole)
  uint32_t xb[VEC];
  if (x_dtype == VH_BF16 && full) {
    const uint4 raw = ld_stream16((const uint16_t*)x + base);
    const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      xb[2 * j] = w[j] & 0xffffu;
      xb[2 * j + 1] = w[j] >> 16;
    }
  }
  float outv[VEC];
#pragma unroll
  for (int j = 0; j < VEC; ++j) {
    const int64_t i = base + j;
    float v = 0.0f;
    if (full || i < n) {
      if (x_dtype == VH_U8) {
        v = fmt_decode_k<KIN>(((const uint8_t*)x)[i], fin, lds_in);
      } else {
        const bool vec = x_dtype == VH_BF16 && full;
        v = vec ? bf2f(xb[j]) : load_any(x, x_dtype, i);
        if constexpr (KIN != K_NONE) {
          const uint32_t b = vec ? xb[j] : x_dtype == VH_BF16 ? (uint32_t)((const uint16_t*)x)[i] : f2bf(v);
          v = round_to(fmt_value_k<KIN>(b, fin, lds_in), x_dtype);
        }
      }
      if (zp.ptr) v = round_to(v - zv[j], cdt);
      if (sp.ptr) v = round_to(v * sv[j], cdt);
      if (has_out) v = round_to(fmt_value(f2bf(v), fout, lds_out), cdt);
    }
    outv[j] = v;
  }
  if (out_dtype == VH_BF16 && full) {
    uint4 pk;
    pk.x = f2bf(outv[0]) | (f2bf(outv[1]) << 16);
    pk.y = f2bf(outv[2]) | (f2bf(outv[3]) << 16);
    pk.z = f2bf(outv[4]) | (f2bf(outv[5]) << 16);
    pk.w = f2bf(outv[6]) | (f2bf(outv[7]) << 16);
    st_stream16((uint16_t*)out + base, pk);
  } else {
    for (int j = 0; j < VEC; ++j)
      if (base + j < n) store_any(out, out_dtype, base + j, outv[j]);
  }
}

extern "C" int vh_dequantize(const void* x, int32_t x_dtype, const int64_t* shape, int32_t ndim,
                             const vh_param* scale, const vh_param* zero_point, int32_t compute_dtype,
                             const vh_format* fmt_in, const vh_format* fmt_out, void* out, int32_t out_dtype,
                             vh_stream_t stream) {
  Shape s;
  int64_t n;
  int rc;
  if ((rc = check_shape(shape, ndim, &s, &n))) return rc;
  VH_REQUIRE(x && out, "vh_dequantize: null tensor");
  VH_REQUIRE(vh::is_float_dtype(x_dtype) || x_dtype == VH_U8, "vh_dequantize: input dtype %d unsupported",
             x_dtype);
  VH_REQUIRE(x_dtype != VH_U8 || packable(fmt_in), "vh_dequantize: packed input needs a packable input map");
  VH_REQUIRE(vh::is_float_dtype(compute_dtype) && vh::is_float_dtype(out_dtype), "vh_dequantize: bad dtype");
  if ((rc = check_param(scale, s, "scale"))) return rc;
  if ((rc = check_param(zero_point, s, "zero_point"))) return rc;
  if ((rc = check_fmt(fmt_in, "input_qmap"))) return rc;
  if ((rc = check_fmt(fmt_out, "output_qmap"))) return rc;
  if (n == 0) return VH_OK;
  vh_param sp = scale ? *scale : null_param();
  vh_param zp = zero_point ? *zero_point : null_param();
  vh_format fi, fo;
  memset(&fi, 0, sizeof(fi));
  memset(&fo, 0, sizeof(fo));
  if (fmt_in) fi = *fmt_in;
  if (fmt_out) fo = *fmt_out;
  hipStream_t st = vh::as_stream(stream);
  if (x_dtype == VH_U8 && out_dtype == VH_BF16 && compute_dtype == VH_BF16 && !fmt_out && !zp.ptr &&
      (!sp.ptr || sp.scalar) && n % 16 == 0 && ((uintptr_t)x % 16) == 0 && ((uintptr_t)out % 16) == 0) {
    // packed codes -> bf16: a 256-entry table per workgroup
    const int64_t n16 = n / 16;
    int64_t blocks = (n16 + 1023) / 1024;
    if (blocks > 4096) blocks = 4096;
    return dispatch_kind(kernel_kind(fmt_in), [&](auto kind) {
      constexpr int K = decltype(kind)::value;
      if constexpr (K == K_NONE || K == K_IDENTITY || K == K_LUT) {
        return (int)VH_EINVAL;  // unreachable: checked by packable()
      } else {
        hipLaunchKernelGGL(k_dequantize_tab<K>, dim3((unsigned)blocks), dim3(256), 0, st, (const uint8_t*)x, n16,
                           sp.ptr, sp.dtype, fi, (uint16_t*)out);
        return vh::check_launch("vh_dequantize");
      }
    });
  }
  int64_t threads = (n + VEC - 1) / VEC;
  int64_t blocks = (threads + 255) / 256;
  VH_REQUIRE(blocks < (1ll << 31), "vh_dequantize: tensor too large");
  return dispatch_kind(kernel_kind(fmt_in), [&](auto kind) {
    constexpr int K = decltype(kind)::value;
    hipLaunchKernelGGL(k_dequantize<K>, dim3((unsigned)blocks), dim3(256), 0, st, x, x_dtype, n, s, sp, zp,
                       compute_dtype, fi, fmt_out ? 1 : 0, fo, out, out_dtype);
    return vh::check_launch("vh_dequantize");
  });
}

extern "C" int vh_decode_bytes(const void* codes, int64_t n, const void* lut, void* out, vh_stream_t stream) {
  VH_REQUIRE(codes && lut && out, "vh_decode_bytes: null pointer");
  VH_REQUIRE(n >= 0, "vh_decode_bytes: negative size");
  VH_REQUIRE(((uintptr_t)codes % 16) == 0 && ((uintptr_t)out % 16) == 0, "vh_decode_bytes: pointers must be 16-byte aligned");
  if (n == 0) return VH_OK;
  int64_t blocks = (n / 16 + 1023) / 1024;
  if (blocks < 1) blocks = 1;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(k_decode_bytes, dim3((unsigned)blocks), dim3(256), 0, vh::as_stream(stream), (const uint8_t*)codes, n,
                     (const uint16_t*)lut, (uint16_t*)out);
  return vh::check_launch("vh_decode_bytes");
}
