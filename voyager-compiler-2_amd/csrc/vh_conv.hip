// conv2d of the quantized-operator path (quantized_ops.conv2d,
// ops/layout.py:170-215, and conv2d_mx, ops/quantized.py:596-643) as an
// explicit-im2col GEMM on the bf16 MFMA GEMM of vh_gemm.hip: per group, the
// input patches become the rows of A [N*OH*OW, KP] (columns (c, kh, kw),
// zero-padded to KP, a multiple of 8, for the GEMM's 16-byte rows), the
// weights the rows of B [K/groups, KP], and the GEMM writes the output
// channels of the group into an NHWC result (bias in its float32
// epilogue); an NCHW result is transposed through LDS tiles.  Convolutions
// are off the measured path; these kernels are plain index maps.
#include <hip/hip_runtime.h>

#include "vh_device.h"
#include "vh_host.h"

namespace {

__global__ void __launch_bounds__(256) k_im2col(const uint16_t* __restrict__ x, vh_conv_geom g, int nhwc, int grp,
                                                int64_t kp, uint16_t* __restrict__ a) {
  const int64_t M = g.N * g.OH * g.OW, total = M * kp;
  const int64_t Cg = g.C / g.groups, KK = g.KH * g.KW, J = Cg * KK;
  const int64_t step = (int64_t)gridDim.x * blockDim.x;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += step) {
    const int64_t m = e / kp, j = e - m * kp;
    uint16_t v = 0;
    if (j < J) {
      const int64_t c = j / KK, r = j - c * KK, kh = r / g.KW, kw = r - kh * g.KW;
      const int64_t ow = m % g.OW, t = m / g.OW, oh = t % g.OH, n = t / g.OH;
      const int64_t ih = oh * g.stride[0] - g.padding[0] + kh * g.dilation[0];
      const int64_t iw = ow * g.stride[1] - g.padding[1] + kw * g.dilation[1];
      if (ih >= 0 && ih < g.H && iw >= 0 && iw < g.W) {
        const int64_t ca = grp * Cg + c;
        v = x[nhwc ? ((n * g.H + ih) * g.W + iw) * g.C + ca : ((n * g.C + ca) * g.H + ih) * g.W + iw];
      }
    }
    a[e] = v;
  }
}

__global__ void __launch_bounds__(256) k_conv_wpack(const uint16_t* __restrict__ w, vh_conv_geom g, int hwio,
                                                    int grp, int64_t kp, uint16_t* __restrict__ out) {
  const int64_t Kg = g.K / g.groups, Cg = g.C / g.groups, KK = g.KH * g.KW, J = Cg * KK;
  const int64_t total = Kg * kp;
  const int64_t step = (int64_t)gridDim.x * blockDim.x;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += step) {
    const int64_t k = e / kp, j = e - k * kp;
    uint16_t v = 0;
    if (j < J) {
      const int64_t c = j / KK, r = j - c * KK, kh = r / g.KW, kw = r - kh * g.KW;
      const int64_t ka = grp * Kg + k;
      v = w[hwio ? ((kh * g.KW + kw) * g.C + c) * g.K + ka : ((ka * Cg + c) * g.KH + kh) * g.KW + kw];
    }
    out[e] = v;
  }
}

// dst[n, c, p] = src[n, p, c] in 32 x 32 tiles (reads and writes coalesced).
template <typename T>
__global__ void __launch_bounds__(256) k_nhwc_to_nchw(const T* __restrict__ src, int64_t P, int64_t C,
                                                      T* __restrict__ dst) {
  __shared__ T tile[32][33];
  const int64_t n = blockIdx.z, p0 = (int64_t)blockIdx.x * 32, c0 = (int64_t)blockIdx.y * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
  for (int i = ty; i < 32; i += 8) {
    const int64_t p = p0 + i, c = c0 + tx;
    if (p < P && c < C) tile[i][tx] = src[(n * P + p) * C + c];
  }
  __syncthreads();
  for (int i = ty; i < 32; i += 8) {
    const int64_t c = c0 + i, p = p0 + tx;
    if (c < C && p < P) dst[(n * C + c) * P + p] = tile[tx][i];
  }
}

unsigned grid_for(int64_t total) {
  int64_t b = (total + 255) / 256;
  return (unsigned)(b < 1 ? 1 : b > 65536 ? 65536 : b);
}

int check_geom(const vh_conv_geom* g, const char* what) {
  VH_REQUIRE(g != nullptr, "%s: null geometry", what);
  VH_REQUIRE(g->N > 0 && g->C > 0 && g->H > 0 && g->W > 0 && g->K > 0 && g->KH > 0 && g->KW > 0 && g->OH > 0 &&
                 g->OW > 0 && g->groups > 0 && g->C % g->groups == 0 && g->K % g->groups == 0,
             "%s: bad convolution geometry", what);
  VH_REQUIRE(g->stride[0] > 0 && g->stride[1] > 0 && g->dilation[0] > 0 && g->dilation[1] > 0 && g->padding[0] >= 0 &&
                 g->padding[1] >= 0,
             "%s: stride and dilation must be positive, padding non-negative", what);
  // the output size the geometry claims is the one aten computes
  const int64_t oh = (g->H + 2 * g->padding[0] - g->dilation[0] * (g->KH - 1) - 1) / g->stride[0] + 1;
  const int64_t ow = (g->W + 2 * g->padding[1] - g->dilation[1] * (g->KW - 1) - 1) / g->stride[1] + 1;
  VH_REQUIRE(oh == g->OH && ow == g->OW, "%s: output size %lld x %lld does not follow from the geometry", what,
             (long long)g->OH, (long long)g->OW);
  return VH_OK;
}

}  // namespace

extern "C" int vh_conv_im2col(const void* x, int32_t dtype, const vh_conv_geom* g, int32_t nhwc, int32_t group,
                              int64_t kp, void* a, vh_stream_t stream) {
  if (int rc = check_geom(g, "vh_conv_im2col")) return rc;
  VH_REQUIRE(dtype == VH_BF16, "vh_conv_im2col: bf16 feature maps only");
  VH_REQUIRE(x && a && group >= 0 && group < g->groups && kp >= (g->C / g->groups) * g->KH * g->KW,
             "vh_conv_im2col: bad arguments");
  hipLaunchKernelGGL(k_im2col, dim3(grid_for(g->N * g->OH * g->OW * kp)), dim3(256), 0, vh::as_stream(stream),
                     (const uint16_t*)x, *g, (int)nhwc, (int)group, kp, (uint16_t*)a);
  return vh::check_launch("vh_conv_im2col");
}

extern "C" int vh_conv_pack_weight(const void* w, int32_t dtype, const vh_conv_geom* g, int32_t hwio, int32_t group,
                                   int64_t kp, void* out, vh_stream_t stream) {
  if (int rc = check_geom(g, "vh_conv_pack_weight")) return rc;
  VH_REQUIRE(dtype == VH_BF16, "vh_conv_pack_weight: bf16 weights only");
  VH_REQUIRE(!hwio || g->groups == 1, "vh_conv_pack_weight: HWIO weights are dense (groups == 1)");
  VH_REQUIRE(w && out && group >= 0 && group < g->groups && kp >= (g->C / g->groups) * g->KH * g->KW,
             "vh_conv_pack_weight: bad arguments");
  hipLaunchKernelGGL(k_conv_wpack, dim3(grid_for(g->K / g->groups * kp)), dim3(256), 0, vh::as_stream(stream),
                     (const uint16_t*)w, *g, (int)hwio, (int)group, kp, (uint16_t*)out);
  return vh::check_launch("vh_conv_pack_weight");
}

extern "C" int vh_nhwc_to_nchw(const void* src, int32_t dtype, int64_t n, int64_t p, int64_t c, void* dst,
                               vh_stream_t stream) {
  VH_REQUIRE(src && dst && n > 0 && n <= 65535 && p > 0 && c > 0 && (c + 31) / 32 <= 65535,
             "vh_nhwc_to_nchw: bad arguments");
  const dim3 grid((unsigned)((p + 31) / 32), (unsigned)((c + 31) / 32), (unsigned)n);
  if (dtype == VH_F32)
    hipLaunchKernelGGL(k_nhwc_to_nchw<uint32_t>, grid, dim3(256), 0, vh::as_stream(stream), (const uint32_t*)src, p,
                       c, (uint32_t*)dst);
  else if (dtype == VH_BF16 || dtype == VH_F16)
    hipLaunchKernelGGL(k_nhwc_to_nchw<uint16_t>, grid, dim3(256), 0, vh::as_stream(stream), (const uint16_t*)src, p,
                       c, (uint16_t*)dst);
  else
    VH_REQUIRE(false, "vh_nhwc_to_nchw: dtype %d unsupported", dtype);
  return vh::check_launch("vh_nhwc_to_nchw");
}
