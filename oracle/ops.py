"""The ``quantized_ops`` operators restated on the CPU (test only).

Each function follows the reference function it names, op for op, so every
intermediate is rounded to the same dtype as there (bfloat16 where the
reference computes in bfloat16).  Citations are into
``src/voyager_compiler/`` of the reference.
"""

import math
from typing import List, Optional, Sequence

import torch

QMAP_SIZE = 2**16
FP32_MIN_NORMAL = 2.0**-126

LINEAR_LAYOUT = "xc,kc->xk"
MATMUL_LAYOUT = "xc,ck->xk"


def repeat_per_block(scale, input, block_size):
    """Per-block parameters expanded to ``input``'s shape;
    ``ops/quantized.py:124-144``."""
    while scale.ndim < input.ndim:
        scale = scale.unsqueeze(0)
    for d, n in enumerate(input.shape):
        if scale.shape[d] != n:
            scale = torch.repeat_interleave(scale, block_size, d)
    if list(scale.shape) != list(input.shape):
        scale = scale[tuple(slice(n) for n in input.shape)]
    if input.is_contiguous():
        return scale
    return torch.empty_like(input, dtype=scale.dtype).copy_(scale)


def vmap(input, table):
    """``table[bits(bf16(input))]`` in ``input``'s dtype and layout;
    ``ops/quantized.py:147-184`` (one gather instead of the chunk loop)."""
    in_dtype = input.dtype
    x = input.to(torch.bfloat16) if input.dtype != torch.bfloat16 else input
    idx = x.view(torch.int16).to(torch.int32) & 0xFFFF
    out = torch.empty_like(x)
    out.copy_(table[idx].to(x.dtype))
    return out.to(in_dtype)


def encode(input, codebook, bounds=None):
    """1-D codebook search; ``ops/quantized.py:232-287`` (one table only)."""
    assert codebook.dim() == 1
    edges = bounds if bounds is not None else (codebook[:-1] + codebook[1:]) / 2
    index = torch.searchsorted(edges, input.bfloat16().float())
    picked = index if bounds is not None else codebook[index]
    return picked.to(input.dtype)


def decode(input, codebook):
    """``codebook[long(input)]``; ``ops/quantized.py:290-315`` (1-D)."""
    assert codebook.dim() == 1
    return codebook[input.to(torch.long)].to(input.dtype)


def quantize(input, scale, zero_point=None, axes=None, block_size=None,
             qmap=None, output_code=None, seed=None):
    """``ops/quantized.py:449-515`` (nearest rounding only)."""
    assert seed is None
    if block_size is not None:
        scale = repeat_per_block(scale, input, block_size)
        if zero_point is not None:
            zero_point = repeat_per_block(zero_point, input, block_size)
    if zero_point is None:
        x = input / scale
    else:
        x = input / scale + zero_point
    if qmap is None:
        return x
    if qmap.numel() == QMAP_SIZE and qmap.dim() == 1:
        return vmap(x, qmap)
    return encode(x, qmap, output_code)


def dequantize(input, scale, zero_point=None, axes=None, block_size=None,
               input_qmap=None, output_qmap=None):
    """``ops/quantized.py:518-571``."""
    if input_qmap is not None:
        input = vmap(input, input_qmap)
    if block_size is not None:
        scale = repeat_per_block(scale, input, block_size)
        if zero_point is not None:
            zero_point = repeat_per_block(zero_point, input, block_size)
    if zero_point is None:
        out = input * scale
    else:
        out = (input - zero_point) * scale
    if output_qmap is not None:
        out = vmap(out, output_qmap)
    return out


def reshape_to_blocks(a, axes, block_size):
    """Zero-pad the blocked axes to whole blocks and split each into
    ``[count, block]``; ``quantization/mx_utils.py:66-125``."""
    axes = sorted(x + a.ndim if x < 0 else x for x in axes)
    for i in range(len(axes)):
        axes[i] += i
        a = torch.unsqueeze(a, dim=axes[i] + 1)
    orig = a.size()
    pad = [0, 0] * len(orig)
    padded = False
    for ax in axes:
        n = orig[ax]
        if n % block_size:
            pad[2 * ax] = block_size - n % block_size
            padded = True
    if padded:
        a = torch.nn.functional.pad(a, list(reversed(pad)), mode="constant")
    shape = list(a.size())
    for ax in axes:
        if shape[ax] >= block_size:
            shape[ax + 1] = block_size
            shape[ax] = shape[ax] // block_size
        else:
            shape[ax + 1] = shape[ax]
            shape[ax] = 1
    return a.view(shape), axes


def shared_exponents(a, axes):
    """``floor(log2(amax))`` over ``axes`` in float32, ``amax == 0`` taken
    as float32's smallest normal; ``quantization/mx_utils.py:16-63``
    (``method="max"``, ``ebits=0``)."""
    s = a
    for ax in axes:
        s, _ = torch.max(torch.abs(s), dim=ax, keepdim=True)
    amax = s.float()
    lg = torch.log2(amax + FP32_MIN_NORMAL * (amax == 0).float())
    return torch.floor(lg).to(s.dtype)


def calculate_mx_qparam(input, axes, block_size, quant_max, force_scale_power_of_two=False,
                        scale_qmap=None, global_scale=None):
    """``ops/quantized.py:958-1031``."""
    assert block_size > 0
    axes = [axes] if isinstance(axes, int) else list(axes)
    axes = [x + input.ndim if x < 0 else x for x in axes]
    blocked, axes = reshape_to_blocks(input, axes, block_size)
    red = [x + 1 for x in axes]
    if force_scale_power_of_two:
        e = shared_exponents(blocked, red)
        e = e - math.floor(math.log2(quant_max))
        for ax in reversed(axes):
            e = torch.squeeze(e, dim=ax + 1)
        scale = 2**e
    else:
        amax = torch.amax(torch.abs(blocked), dim=red)
        scale = amax / quant_max
        if global_scale is not None:
            scale = scale / global_scale
        if scale_qmap is not None:
            scale = vmap(scale, scale_qmap)
    return torch.where(scale > 0.0, scale, 1.0)


def quantize_mx(input, qmap, axes, block_size, quant_max, force_scale_power_of_two=False,
                scale_qmap=None, output_code=None, seed=None, global_scale=None):
    """``(scale, codes)``; ``ops/quantized.py:1070-1115``."""
    scale = calculate_mx_qparam(input, axes, block_size, quant_max,
                                force_scale_power_of_two, scale_qmap, global_scale)
    el = scale if global_scale is None else scale * global_scale
    return scale, quantize(input, el, None, axes, block_size, qmap, output_code, seed)


def dequantize_mx_parts(input, scale, code, block_size):
    """``_dequantize_mx`` / ``_decode_and_scale``; ``ops/quantized.py:574-591``."""
    if code is None and scale is None:
        return input
    if code is not None:
        input = decode(input, code)
    if scale is not None:
        input = input * repeat_per_block(scale, input, block_size)
    return input


def dequantize_mx(input, scale, block_size, code=None, global_scale=None):
    """``ops/quantized.py:1118-1150``."""
    out = dequantize_mx_parts(input, scale, code, block_size)
    if global_scale is not None:
        out = out * global_scale
    return out


def quantize_affine(input, qmap, axes, block_size, quant_min, quant_max, scale_qmap=None):
    """``(scale, zero_point, value)``; ``ops/quantized.py:1218-1283``."""
    assert block_size > 0
    (axis,) = axes
    axes = [axis % input.ndim]
    blocked, baxes = reshape_to_blocks(input, axes, block_size)
    red = [x + 1 for x in baxes]
    low = torch.amin(blocked, dim=red)
    high = torch.amax(blocked, dim=red)
    scale = (high - low) / (quant_max - quant_min)
    scale = torch.where(scale > 0.0, scale, 1.0)
    if scale_qmap is not None:
        scale = vmap(scale, scale_qmap)
        scale = torch.where(scale > 0.0, scale, 1.0)
    zp = -low / scale + quant_min
    if scale_qmap is not None:
        zp = vmap(zp, scale_qmap)
    value = quantize(input, scale, zp, axes, block_size, qmap)
    return scale, zp, value


def _parse_layout(layout):
    ops, out = layout.split("->")
    act, w = ops.split(",")
    assert act in ("xc", "cx") and w in ("kc", "ck") and out in ("xk", "kx"), layout
    return act, w, out


def _gemm_in_layout(op, native, a, w, layout, out_dtype, *rest):
    """``ops/layout.py:231-260``."""
    sa, sw, so = _parse_layout(layout)
    na, nw, no = _parse_layout(native)
    if sa != na:
        a = a.mT
    if sw != nw:
        w = w.mT
    if out_dtype is not None:
        a, w = a.float(), w.float()
        rest = [None if r is None else r.float() for r in rest]
    out = op(a, w, *rest)
    if out_dtype is not None:
        out = out.to(out_dtype)
    return out.mT.contiguous() if so != no else out


def linear(input, weight, bias=None, layout=LINEAR_LAYOUT, out_dtype=None):
    """``quantized_ops.linear``; ``ops/layout.py:263-275``."""
    return _gemm_in_layout(torch.ops.aten.linear, LINEAR_LAYOUT, input, weight, layout,
                           out_dtype, bias)


def matmul(input, other, layout=MATMUL_LAYOUT, out_dtype=None):
    """``quantized_ops.matmul``; ``ops/layout.py:278-284``."""
    return _gemm_in_layout(torch.ops.aten.matmul, MATMUL_LAYOUT, input, other, layout,
                           out_dtype)


def _with_xk(layout):
    a, w, _ = _parse_layout(layout)
    return f"{a},{w}->xk"


def linear_mx(input, weight, bias=None, input_scale=None, weight_scale=None, block_size=None,
              input_code=None, weight_code=None, alpha=None, layout=LINEAR_LAYOUT,
              out_dtype=None):
    """``ops/quantized.py:651-723`` without the outlier (CSR) term."""
    _, _, so = _parse_layout(layout)
    x = dequantize_mx_parts(input, input_scale, input_code, block_size)
    w = dequantize_mx_parts(weight, weight_scale, weight_code, block_size)
    dtype = x.dtype if out_dtype is None else out_dtype
    acc = torch.promote_types(dtype, torch.float32)
    out = linear(x, w, bias if alpha is None else None, layout=_with_xk(layout), out_dtype=acc)
    if alpha is not None:
        out = out * alpha
        if bias is not None:
            out = out + bias
    out = out.to(dtype)
    return out.mT.contiguous() if so != "xk" else out


def matmul_mx(input, other, input_scale=None, weight_scale=None, block_size=None,
              input_code=None, weight_code=None, alpha=None, layout=MATMUL_LAYOUT,
              out_dtype=None):
    """``ops/quantized.py:742-805`` without the outlier (CSR) term."""
    _, _, so = _parse_layout(layout)
    x = dequantize_mx_parts(input, input_scale, input_code, block_size)
    w = dequantize_mx_parts(other, weight_scale, weight_code, block_size)
    dtype = x.dtype if out_dtype is None else out_dtype
    acc = torch.promote_types(dtype, torch.float32)
    out = matmul(x, w, layout=_with_xk(layout), out_dtype=acc)
    if alpha is not None:
        out = out * alpha
    out = out.to(dtype)
    return out.mT.contiguous() if so != "xk" else out


def per_tensor_scale(x, quant_max):
    """Calibrated per-tensor symmetric scale ``amax / quant_max`` in ``x``'s
    dtype, as the amax observer computes it for a single observation
    (``quantization/fake_quantize.py:414-437``: amax, ``sf = amax / qmax``,
    kept where ``amax > 0`` and finite)."""
    amax = torch.amax(torch.abs(x))
    sf = amax / quant_max
    one = torch.ones((), dtype=x.dtype)
    sf = torch.where(amax > 0.0, sf, one)
    sf = torch.where(torch.isfinite(amax), sf, one)
    return sf
