"""``quantized_ops.conv2d`` and ``conv2d_mx`` on the GPU.

``conv2d`` (``ops/layout.py:170-215``) is aten's convolution on feature maps
stored NCHW or NHWC (a dense NHWC convolution's weight HWIO); ``conv2d_mx``
(``ops/quantized.py:596-643``) decodes both operands first (code, then
block scale, as ``linear_mx`` does) and runs it.  Here the convolution is
im2col + the bf16 MFMA GEMM with float32 accumulation, per group:
``vh_conv_im2col`` lays each output pixel's patch out as a row,
``vh_conv_pack_weight`` the group's filters in the same column order,
``vh_gemm`` writes the group's channels of an NHWC result with the bias in
its float32 epilogue and one rounding to the output dtype, and
``vh_nhwc_to_nchw`` transposes an NCHW result.  Operands must be bfloat16
(the decoded operands of ``conv2d_mx`` are); results are bfloat16 or, with
``out_dtype``, float32.
"""

import ctypes

import torch

from . import _lib
from ._lib import VH_BF16, dtype_code, load, ptr, stream_of
from .gemm import EPI_PLAIN, OP_BF16, GemmDesc, _decode, _epilogue, run
from .ops import _require_gpu
from .registry import cuda_kernel, fake_kernel

TENSOR_LAYOUTS = ("nchw", "nhwc")


class ConvGeom(ctypes.Structure):
    """``vh_conv_geom``."""

    _fields_ = [
        ("N", ctypes.c_int64), ("C", ctypes.c_int64), ("H", ctypes.c_int64), ("W", ctypes.c_int64),
        ("K", ctypes.c_int64), ("KH", ctypes.c_int64), ("KW", ctypes.c_int64),
        ("OH", ctypes.c_int64), ("OW", ctypes.c_int64),
        ("stride", ctypes.c_int32 * 2), ("padding", ctypes.c_int32 * 2), ("dilation", ctypes.c_int32 * 2),
        ("groups", ctypes.c_int32),
    ]


def _pair(v):
    return tuple(v) if isinstance(v, (list, tuple)) else (v, v)


def _conv2d_cuda(input, weight, bias=None, stride=(1, 1), padding=(0, 0), dilation=(1, 1), groups=1, *,
                 layout="nchw", out_dtype=None):
    _require_gpu(input, weight, bias)
    assert layout in TENSOR_LAYOUTS, layout
    if input.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise NotImplementedError(f"quantized_ops.conv2d: bfloat16 operands on the GPU (got {input.dtype}, "
                                  f"{weight.dtype})")
    if input.dim() != 4 or weight.dim() != 4:
        raise NotImplementedError("quantized_ops.conv2d: batched 4-D feature maps on the GPU")
    dtype = input.dtype if out_dtype is None else out_dtype
    if dtype not in (torch.bfloat16, torch.float32):
        raise NotImplementedError(f"quantized_ops.conv2d: {dtype} results are not supported on the GPU")
    nhwc = layout == "nhwc"
    hwio = nhwc and groups == 1
    x = input.contiguous()
    w = weight.contiguous()
    if nhwc:
        N, H, W, C = x.shape
    else:
        N, C, H, W = x.shape
    if hwio:
        KH, KW, Cw, K = w.shape
    else:
        K, Cw, KH, KW = w.shape
    if C % groups or K % groups or Cw != C // groups:
        raise RuntimeError(f"conv2d: weight {list(weight.shape)} does not fit {C} input channels in {groups} "
                           "groups")
    (sh, sw), (ph, pw), (dh, dw) = _pair(stride), _pair(padding), _pair(dilation)
    OH = (H + 2 * ph - dh * (KH - 1) - 1) // sh + 1
    OW = (W + 2 * pw - dw * (KW - 1) - 1) // sw + 1
    if OH <= 0 or OW <= 0:
        raise RuntimeError("conv2d: the kernel does not fit the padded input")
    g = ConvGeom(N, C, H, W, K, KH, KW, OH, OW)
    g.stride[:], g.padding[:], g.dilation[:] = (sh, sw), (ph, pw), (dh, dw)
    g.groups = groups
    Kg, J = K // groups, (C // groups) * KH * KW
    kp = (J + 7) // 8 * 8
    M = N * OH * OW
    dev = input.device
    out_nhwc = torch.empty(N, OH, OW, K, dtype=dtype, device=dev)
    a = torch.empty(M, kp, dtype=torch.bfloat16, device=dev)
    wp = torch.empty(Kg, kp, dtype=torch.bfloat16, device=dev)
    b32 = None if bias is None else bias.to(torch.float32).contiguous()
    lib_ = load()
    st_ = ctypes.c_void_p(stream_of(x))
    esize = out_nhwc.element_size()
    for grp in range(groups):
        _lib.check(lib_.vh_conv_im2col(ptr(x), VH_BF16, ctypes.byref(g), 1 if nhwc else 0, grp, kp, ptr(a), st_),
                   "vh_conv_im2col")
        _lib.check(lib_.vh_conv_pack_weight(ptr(w), VH_BF16, ctypes.byref(g), 1 if hwio else 0, grp, kp, ptr(wp),
                                            st_), "vh_conv_pack_weight")
        d = GemmDesc()
        d.A, d.B = a.data_ptr(), wp.data_ptr()
        d.C = out_nhwc.data_ptr() + grp * Kg * esize
        d.M, d.N, d.K = M, Kg, kp
        d.lda = d.ldb = kp * 2
        d.ldc = K
        d.a_fmt = d.b_fmt = OP_BF16
        bg = None if b32 is None else b32[grp * Kg:(grp + 1) * Kg]
        d.epi = _epilogue(EPI_PLAIN, dtype, None, bg)
        run(d, dev)
    if nhwc:
        return out_nhwc
    out = torch.empty(N, K, OH, OW, dtype=dtype, device=dev)
    _lib.check(lib_.vh_nhwc_to_nchw(ptr(out_nhwc), dtype_code(dtype), N, OH * OW, K, ptr(out), st_),
               "vh_nhwc_to_nchw")
    return out


def _conv2d_mx_cuda(input, weight, bias=None, stride=1, padding=0, dilation=1, groups=1, *, input_scale=None,
                    weight_scale=None, block_size=None, input_code=None, weight_code=None, layout="nchw",
                    out_dtype=None):
    """``ops/quantized.py:606-643``: decode, then ``conv2d``."""
    _require_gpu(input, weight, bias, input_scale, weight_scale, input_code, weight_code)
    x = _decode(input, input_scale, input_code, block_size)
    w = _decode(weight, weight_scale, weight_code, block_size)
    return _conv2d_cuda(x, w, bias, _pair(stride), _pair(padding), _pair(dilation), groups, layout=layout,
                        out_dtype=out_dtype)


cuda_kernel("conv2d")(_conv2d_cuda)
cuda_kernel("conv2d_mx")(_conv2d_mx_cuda)


def _conv_shape(input, weight, stride, padding, dilation, groups, layout):
    (sh, sw), (ph, pw), (dh, dw) = _pair(stride), _pair(padding), _pair(dilation)
    nhwc = layout == "nhwc"
    N, H, W = (input.shape[0], input.shape[1], input.shape[2]) if nhwc else (input.shape[0], input.shape[2],
                                                                            input.shape[3])
    if nhwc and groups == 1:
        KH, KW, K = weight.shape[0], weight.shape[1], weight.shape[3]
    else:
        K, KH, KW = weight.shape[0], weight.shape[2], weight.shape[3]
    OH = (H + 2 * ph - dh * (KH - 1) - 1) // sh + 1
    OW = (W + 2 * pw - dw * (KW - 1) - 1) // sw + 1
    return (N, OH, OW, K) if nhwc else (N, K, OH, OW)


@fake_kernel("conv2d")
def _conv2d_fake(input, weight, bias=None, stride=(1, 1), padding=(0, 0), dilation=(1, 1), groups=1, *,
                 layout="nchw", out_dtype=None):
    shape = _conv_shape(input, weight, stride, padding, dilation, groups, layout)
    return input.new_empty(shape, dtype=input.dtype if out_dtype is None else out_dtype)


@fake_kernel("conv2d_mx")
def _conv2d_mx_fake(input, weight, bias=None, stride=1, padding=0, dilation=1, groups=1, *,
                    input_scale=None, weight_scale=None, block_size=None, input_code=None, weight_code=None,
                    layout="nchw", out_dtype=None):
    shape = _conv_shape(input, weight, stride, padding, dilation, groups, layout)
    return input.new_empty(shape, dtype=input.dtype if out_dtype is None else out_dtype)

