"""Packed (one byte per code) forms of the quantize ops.

The reference's schemas return codes and scales as floating tensors ("ref
form").  A GEMM reads 1-byte codes at half the HBM traffic of bfloat16 ones,
so the GPU path can also emit packed codes:

* element codes: int two's complement, minifloat sign|exponent|mantissa
  fields (``fp8_e4m3`` is the OCP E4M3 byte the fp8 MFMA consumes), posit
  bit strings, or codebook level indices;
* power-of-two block scales as biased exponent bytes, ``2**(byte - bias)``
  with ``bias = 127 + floor(log2(quant_max))`` (255 = inf), which covers every
  scale an int8 / fp8 block can get, the bfloat16 subnormal ones included;
* other block scales as codes of their scale map (``fp8_e5m3`` bytes).

These are the lowered-graph forms; ``unpack_*`` turn them back into the
reference form bit for bit.
"""

import ctypes
import math
from typing import NamedTuple, Optional

import torch

from . import _lib, formats
from ._lib import VH_U8, dtype_code, load, ptr, stream_of
from .ops import _block_view, _elementwise, _scale_shape


def pot_bias(quant_max: float) -> int:
    return 127 + int(math.floor(math.log2(quant_max)))


class PackedMX(NamedTuple):
    codes: torch.Tensor     # uint8, the input's shape
    scale: torch.Tensor     # uint8, one per block
    fmt: formats.Classified
    scale_fmt: Optional[formats.Classified]
    pot: bool
    bias: int
    block_size: int
    axis: int


def quantize_packed(x: torch.Tensor, scale: torch.Tensor, qmap: torch.Tensor) -> torch.Tensor:
    """``quantize(x, scale, qmap=qmap)`` with one-byte codes."""
    c = formats.classify(qmap)
    cdt = torch.result_type(x, scale)
    return _elementwise("quantize", x, scale, None, None, cdt, c.fmt, None, torch.uint8)


def unpack_codes(codes: torch.Tensor, qmap: torch.Tensor, dtype=torch.bfloat16) -> torch.Tensor:
    """Reference-form codes (the map's entries) of packed codes."""
    c = formats.classify(qmap)
    return _elementwise("dequantize", codes, None, None, None, dtype, c.fmt, None, dtype)


def quantize_mx_packed(x: torch.Tensor, qmap: torch.Tensor, axes, block_size: int, quant_max: float,
                       force_scale_power_of_two: bool = False,
                       scale_qmap: Optional[torch.Tensor] = None) -> PackedMX:
    """``quantize_mx`` with packed codes and scales."""
    xc, ax, outer, L, inner = _block_view(x, axes)
    ec = formats.classify(qmap)
    sc = None if force_scale_power_of_two or scale_qmap is None else formats.classify(scale_qmap)
    bias = pot_bias(quant_max) if force_scale_power_of_two else 0
    scale = torch.empty(_scale_shape(xc, ax, block_size), dtype=torch.uint8, device=x.device)
    codes = torch.empty(xc.shape, dtype=torch.uint8, device=x.device)
    st = load().vh_quantize_mx(
        ptr(xc), dtype_code(xc.dtype), outer, L, inner, block_size, float(quant_max),
        1 if force_scale_power_of_two else 0, ctypes.byref(sc.fmt) if sc else None, None, 0,
        ctypes.byref(ec.fmt), ptr(scale), VH_U8, bias, ptr(codes), VH_U8, None, ctypes.c_void_p(stream_of(x)))
    _lib.check(st, "vh_quantize_mx")
    return PackedMX(codes, scale, ec, sc, bool(force_scale_power_of_two), bias, block_size, ax)


def unpack_mx_scale(p: PackedMX, dtype=torch.bfloat16) -> torch.Tensor:
    """Reference-form block scales of a ``PackedMX``."""
    if p.pot:
        b = p.scale.to(torch.int32)
        v = torch.ldexp(torch.ones_like(b, dtype=torch.float32), b - p.bias)
        v = torch.where(b == 255, torch.full_like(v, float("inf")), v)
        return v.to(dtype)
    return _elementwise("dequantize", p.scale, None, None, None, dtype, p.scale_fmt.fmt, None, dtype)
