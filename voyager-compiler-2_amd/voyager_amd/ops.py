"""The ``quantized_ops`` operator library on MI355X.

Defines the namespace with the reference's schema strings, byte for byte
(``src/voyager_compiler/ops/quantized.py:147, 449-453, 518-522, 651-658,
596-603, 742-748, 958-962, 1070-1075, 1118-1121, 1218-1222, 1286-1289,
1396-1402, 1493-1497, 1567-1571``; ``ops/layout.py:176-181, 221-228``),
a fake (meta) kernel for each op so FX shape propagation works, and a CUDA-key
kernel (PyTorch-ROCm routes HIP tensors there) that validates arguments,
allocates outputs with torch's caching allocator and launches the HIP library
on the current stream.  There is no CPU kernel: the reference's CPU path is the
oracle of the tests, not part of this package.

Because the reference defines the same namespace, the two cannot be loaded
in one process.
"""

import ctypes
from typing import List, Optional, Sequence

import torch

from . import _lib, formats
from ._lib import Format, Param, VH_U8, dtype_code, load, ptr, stream_of

QMAP_SIZE = formats.QMAP_SIZE

from .registry import cuda_kernel, fake_kernel
from .schemas import LINEAR_LAYOUT, MATMUL_LAYOUT, SCHEMAS  # noqa: F401


# ----------------------------------------------------------------- helpers
def _require_gpu(*tensors):
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError("voyager_amd quantized_ops run on the GPU only; got a CPU tensor")


def _is_table(q: Optional[torch.Tensor]) -> bool:
    return q is not None and q.numel() == QMAP_SIZE and q.dim() == 1


def _fmt_of(table: torch.Tensor) -> formats.Classified:
    return formats.classify(table)


def _layout_order(x: torch.Tensor):
    """Dims of ``x`` in memory order when ``x`` is densely packed in a
    permuted layout (which an elementwise result keeps), else None."""
    if x.is_contiguous() or x.dim() == 0:
        return None
    order = sorted(range(x.dim()), key=lambda d: (x.stride(d), -d), reverse=True)
    if x.permute(order).is_contiguous():
        return order
    return None


def _param(p: Optional[torch.Tensor], shape: Sequence[int], block_size: Optional[int],
           dtype: torch.dtype, name: str, order=None, own_precision: bool = False):
    """``vh_param`` of a scale / zero point read against a tensor of
    ``shape`` (already in memory order when ``order`` is given).  Follows
    ``repeat_per_block`` (``ops/quantized.py:124-144``) with a block size and
    torch broadcasting without one."""
    if p is None:
        return None, None
    # How eager torch (CPU) combines a tensor with a 0-d tensor of a wider
    # float dtype: mul and div use the 0-d value at its own precision (then
    # round once), add and sub round it to the tensor's dtype first.  So a
    # float scale keeps its dtype (the kernels read any float dtype into
    # float32) and a zero point takes the compute dtype; a wider n-d
    # parameter has already widened `dtype`, where either is exact.
    if not (own_precision and p.dtype in (torch.bfloat16, torch.float16, torch.float32)):
        p = p.to(dtype)
    nd = len(shape)
    if p.dim() > nd:
        raise ValueError(f"{name} has more dims ({p.dim()}) than the input ({nd})")
    while p.dim() < nd:
        p = p.unsqueeze(0)
    if order is not None:
        p = p.permute(order)
    prm = Param()
    prm.dtype = dtype_code(p.dtype)
    if p.numel() == 1:
        p = p.reshape(()).contiguous()
        prm.ptr = p.data_ptr()
        prm.scalar = 1
        return prm, p
    p = p.contiguous()
    prm.ptr = p.data_ptr()
    for d in range(nd):
        n, m = shape[d], p.shape[d]
        prm.div[d] = 1
        if m == n:
            prm.stride[d] = p.stride(d)
        elif block_size is not None:
            if m * block_size < n:
                raise ValueError(f"{name}: {m} blocks of {block_size} cannot cover {n} elements on dim {d}")
            prm.div[d] = block_size
            prm.stride[d] = p.stride(d)
        elif m == 1:
            prm.stride[d] = 0
        else:
            raise ValueError(f"{name} of shape {list(p.shape)} does not broadcast to {list(shape)}")
    return prm, p


def _shape_arr(shape):
    return (ctypes.c_int64 * max(len(shape), 1))(*shape) if len(shape) else (ctypes.c_int64 * 1)(1)


def _elementwise(kind: str, x: torch.Tensor, scale, zp, block_size, cdt, fmt_a: Optional[Format],
                 fmt_b: Optional[Format], out_dtype: torch.dtype):
    """Run vh_quantize / vh_dequantize over ``x`` keeping its layout."""
    lib_ = load()
    order = _layout_order(x)
    xv = x.permute(order) if order is not None else x.contiguous()
    shape = list(xv.shape)
    sp, keep_s = _param(scale, shape, block_size, cdt, "scale", order, own_precision=True)
    zpp, keep_z = _param(zp, shape, block_size, cdt, "zero_point", order)
    out = torch.empty(shape, dtype=out_dtype, device=x.device)
    args_common = (ptr(xv), dtype_code(xv.dtype), _shape_arr(shape), len(shape),
                   ctypes.byref(sp) if sp else None, ctypes.byref(zpp) if zpp else None, dtype_code(cdt))
    if kind == "quantize":
        st = lib_.vh_quantize(*args_common, ctypes.byref(fmt_a) if fmt_a is not None else None, ptr(out),
                              dtype_code(out_dtype), ctypes.c_void_p(stream_of(x)))
    else:
        st = lib_.vh_dequantize(*args_common, ctypes.byref(fmt_a) if fmt_a is not None else None,
                                ctypes.byref(fmt_b) if fmt_b is not None else None, ptr(out),
                                dtype_code(out_dtype), ctypes.c_void_p(stream_of(x)))
    _lib.check(st, f"vh_{kind}")
    del keep_s, keep_z  # launched on the stream; the allocator tracks stream use
    if order is not None:
        inv = [0] * len(order)
        for i, d in enumerate(order):
            inv[d] = i
        out = out.permute(inv)
    return out


def _record(t: Optional[torch.Tensor], x: torch.Tensor):
    if t is not None and t.is_cuda:
        t.record_stream(torch.cuda.current_stream(x.device))


# ----------------------------------------------------------------- vmap
def _vmap_cuda(input, qmap):
    _require_gpu(input, qmap)
    c = _fmt_of(qmap)
    return _elementwise("quantize", input, None, None, None, input.dtype, c.fmt, None, input.dtype)


cuda_kernel("vmap")(_vmap_cuda)


@fake_kernel("vmap")
def _vmap_fake(input, qmap):
    return torch.empty_like(input)


# ----------------------------------------------------------------- quantize
def _quantize_dtype(input, scale, zero_point):
    d = torch.result_type(input, scale)
    if zero_point is not None:
        probe = torch.empty([1] * max(input.dim(), 1), dtype=d, device="meta")
        d = torch.result_type(probe, zero_point)
    return d


def _quantize_sr(input, scale, zero_point, block_size, qmap, seed, cdt):
    """``quantize`` with a seed (``ops/quantized.py:318-446``): the division,
    then stochastic rounding between the levels of ``qmap``, through
    ``vh_quantize_sr``; elements in logical row-major order (the order of the
    random bytes), result contiguous in ``cdt``."""
    levels = formats.sr_levels(qmap)
    if levels.dim() != 1:
        raise NotImplementedError("quantized_ops.quantize: stochastic rounding against per-head codebooks is not "
                                  "supported on the GPU")
    if levels.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        levels = levels.to(torch.float32)
    if seed.dtype != torch.int64 or seed.numel() != 1:
        raise ValueError("quantized_ops.quantize: seed must be an int64 scalar")
    x = input.contiguous()
    shape = list(x.shape)
    sp, keep_s = _param(scale, shape, block_size, cdt, "scale", own_precision=True)
    zpp, keep_z = _param(zero_point, shape, block_size, cdt, "zero_point")
    out = torch.empty(shape, dtype=cdt, device=x.device)
    sd = seed.reshape(()).contiguous()
    st = load().vh_quantize_sr(ptr(x), dtype_code(x.dtype), _shape_arr(shape), len(shape),
                               ctypes.byref(sp) if sp else None, ctypes.byref(zpp) if zpp else None, dtype_code(cdt),
                               ptr(levels), dtype_code(levels.dtype), levels.numel(), ptr(sd), ptr(out),
                               dtype_code(cdt), ctypes.c_void_p(stream_of(x)))
    _lib.check(st, "vh_quantize_sr")
    del keep_s, keep_z
    return out


def _quantize_cuda(input, scale, zero_point=None, axes=None, block_size=None, qmap=None,
                   output_code=None, seed=None):
    _require_gpu(input, scale, zero_point, qmap, seed)
    cdt = _quantize_dtype(input, scale, zero_point)
    if seed is not None and qmap is not None:
        return _quantize_sr(input, scale, zero_point, block_size, qmap, seed, cdt)
    if qmap is not None and not _is_table(qmap):
        raise NotImplementedError("quantized_ops.quantize: codebook (searchsorted) maps are not supported yet")
    fmt = _fmt_of(qmap).fmt if qmap is not None else None
    return _elementwise("quantize", input, scale, zero_point, block_size, cdt, fmt, None, cdt)


cuda_kernel("quantize")(_quantize_cuda)


@fake_kernel("quantize")
def _quantize_fake(input, scale, zero_point=None, axes=None, block_size=None, qmap=None,
                   output_code=None, seed=None):
    return torch.empty_like(input, dtype=_quantize_dtype(input, scale, zero_point))


# ----------------------------------------------------------------- dequantize
def _dequantize_dtype(input, scale, zero_point):
    d = input.dtype
    if zero_point is not None:
        d = torch.result_type(input, zero_point)
    probe = torch.empty([1] * max(input.dim(), 1), dtype=d, device="meta")
    return torch.result_type(probe, scale)


def _dequantize_cuda(input, scale, zero_point=None, axes=None, block_size=None, input_qmap=None,
                     output_qmap=None):
    _require_gpu(input, scale, zero_point, input_qmap, output_qmap)
    cdt = _dequantize_dtype(input, scale, zero_point)
    fi = _fmt_of(input_qmap).fmt if input_qmap is not None else None
    fo = _fmt_of(output_qmap).fmt if output_qmap is not None else None
    return _elementwise("dequantize", input, scale, zero_point, block_size, cdt, fi, fo, cdt)


cuda_kernel("dequantize")(_dequantize_cuda)


@fake_kernel("dequantize")
def _dequantize_fake(input, scale, zero_point=None, axes=None, block_size=None, input_qmap=None,
                     output_qmap=None):
    return torch.empty_like(input, dtype=_dequantize_dtype(input, scale, zero_point))


# ----------------------------------------------------------------- block views
def _block_view(x: torch.Tensor, axes):
    """``x`` as contiguous ``[outer, L, inner]`` around its one blocked axis."""
    axes = [axes] if isinstance(axes, int) else list(axes)
    if len(axes) != 1:
        raise NotImplementedError("block scaling along more than one axis is not supported on the GPU")
    ax = axes[0] + x.dim() if axes[0] < 0 else axes[0]
    if not 0 <= ax < x.dim():
        raise IndexError(f"axis {axes[0]} out of range for a {x.dim()}-d tensor")
    xc = x.contiguous()
    outer = 1
    for n in xc.shape[:ax]:
        outer *= n
    inner = 1
    for n in xc.shape[ax + 1:]:
        inner *= n
    return xc, ax, outer, xc.shape[ax], inner


def _scale_shape(x: torch.Tensor, ax: int, block_size: int):
    shape = list(x.shape)
    shape[ax] = -(-shape[ax] // block_size)
    return shape


def _fmt_ref(c: Optional[formats.Classified]):
    return None if c is None else ctypes.byref(c.fmt)


def _mx_launch(x, axes, block_size, quant_max, pot, scale_qmap, global_scale, qmap, want_codes):
    if block_size <= 0:
        raise AssertionError("block_size must be > 0")
    xc, ax, outer, L, inner = _block_view(x, axes)
    cdt = xc.dtype
    scale = torch.empty(_scale_shape(xc, ax, block_size), dtype=cdt, device=x.device)
    codes = torch.empty_like(xc) if want_codes else None
    sc = _fmt_of(scale_qmap) if (scale_qmap is not None and not pot) else None
    ec = _fmt_of(qmap) if want_codes else None
    gs = None
    if global_scale is not None and not pot:
        gs = global_scale.reshape(()).contiguous()
    st = load().vh_quantize_mx(
        ptr(xc), dtype_code(cdt), outer, L, inner, block_size, float(quant_max), 1 if pot else 0, _fmt_ref(sc),
        ptr(gs), dtype_code(gs.dtype) if gs is not None else 0, _fmt_ref(ec), ptr(scale), dtype_code(cdt), 0,
        ptr(codes), dtype_code(cdt), None, ctypes.c_void_p(stream_of(x)))
    _lib.check(st, "vh_quantize_mx")
    return scale, codes


def _calculate_mx_qparam_cuda(input, axes, block_size, quant_max, force_scale_power_of_two=False,
                              scale_qmap=None, global_scale=None):
    _require_gpu(input, scale_qmap, global_scale)
    scale, _ = _mx_launch(input, axes, block_size, quant_max, force_scale_power_of_two, scale_qmap, global_scale,
                          None, False)
    return scale


cuda_kernel("calculate_mx_qparam")(_calculate_mx_qparam_cuda)


@fake_kernel("calculate_mx_qparam")
def _calculate_mx_qparam_fake(input, axes, block_size, quant_max, force_scale_power_of_two=False,
                              scale_qmap=None, global_scale=None):
    axes = [axes] if isinstance(axes, int) else list(axes)
    ax = axes[0] % input.dim()
    return input.new_empty(_scale_shape(input, ax, block_size))


def _quantize_mx_cuda(input, qmap, axes, block_size, quant_max, force_scale_power_of_two=False,
                      scale_qmap=None, output_code=None, seed=None, global_scale=None):
    _require_gpu(input, qmap, scale_qmap, global_scale, seed)
    if seed is not None:
        # ops/quantized.py:1097-1115: the block scales, then quantize with the seed
        if global_scale is not None:
            raise NotImplementedError("quantized_ops.quantize_mx: stochastic rounding with a global scale is not "
                                      "supported on the GPU")
        scale, _ = _mx_launch(input, axes, block_size, quant_max, force_scale_power_of_two, scale_qmap, None, None,
                              False)
        cdt = _quantize_dtype(input, scale, None)
        return scale, _quantize_sr(input, scale, None, block_size, qmap, seed, cdt)
    if not _is_table(qmap):
        raise NotImplementedError("quantized_ops.quantize_mx: codebook (searchsorted) maps are not supported yet")
    return _mx_launch(input, axes, block_size, quant_max, force_scale_power_of_two, scale_qmap, global_scale, qmap,
                      True)


cuda_kernel("quantize_mx")(_quantize_mx_cuda)


@fake_kernel("quantize_mx")
def _quantize_mx_fake(input, qmap, axes, block_size, quant_max, force_scale_power_of_two=False,
                      scale_qmap=None, output_code=None, seed=None, global_scale=None):
    axes = [axes] if isinstance(axes, int) else list(axes)
    ax = axes[0] % input.dim()
    return input.new_empty(_scale_shape(input, ax, block_size)), torch.empty_like(input)


def _quantize_affine_cuda(input, qmap, axes, block_size, quant_min, quant_max, scale_qmap=None):
    _require_gpu(input, qmap, scale_qmap)
    if block_size <= 0:
        raise AssertionError("block_size must be > 0")
    if len(axes) != 1:
        raise ValueError("quantize_affine takes exactly one axis")
    if not _is_table(qmap):
        raise NotImplementedError("quantized_ops.quantize_affine: codebook maps are not supported yet")
    xc, ax, outer, L, inner = _block_view(input, axes)
    cdt = xc.dtype
    sshape = _scale_shape(xc, ax, block_size)
    scale = torch.empty(sshape, dtype=cdt, device=input.device)
    zp = torch.empty(sshape, dtype=cdt, device=input.device)
    codes = torch.empty_like(xc)
    sc = _fmt_of(scale_qmap) if scale_qmap is not None else None
    ec = _fmt_of(qmap)
    st = load().vh_quantize_affine(ptr(xc), dtype_code(cdt), outer, L, inner, block_size, float(quant_min),
                                   float(quant_max), _fmt_ref(sc), _fmt_ref(ec), ptr(scale), ptr(zp), ptr(codes),
                                   dtype_code(cdt), ctypes.c_void_p(stream_of(input)))
    _lib.check(st, "vh_quantize_affine")
    return scale, zp, codes


cuda_kernel("quantize_affine")(_quantize_affine_cuda)


@fake_kernel("quantize_affine")
def _quantize_affine_fake(input, qmap, axes, block_size, quant_min, quant_max, scale_qmap=None):
    ax = axes[0] % input.dim()
    s = input.new_empty(_scale_shape(input, ax, block_size))
    return s, torch.empty_like(s), torch.empty_like(input)


# ----------------------------------------------------------------- dequantize_mx
def decode_table(code: torch.Tensor) -> torch.Tensor:
    """The 65,536-entry bfloat16 table of ``decode`` (``ops/quantized.py:290-315``):
    entry ``v`` is ``code[long(v)]`` (negative indices counting from the end,
    as torch indexing does), NaN where torch would raise.  Built on the
    codebook's device with no host round trip, and cached on the codebook
    tensor itself (a codebook is a graph buffer; an in-place change or a new
    tensor at a reused address rebuilds it)."""
    cached = getattr(code, "_vh_decode_table", None)
    if cached is not None and cached[0] == code._version and cached[1] == code.data_ptr():
        return cached[2]
    dev = code.device
    v = torch.arange(QMAP_SIZE, dtype=torch.int32, device=dev).to(torch.int16).view(torch.bfloat16).float()
    n = code.numel()
    vals = code.detach().reshape(-1).to(torch.float32)
    fin = torch.isfinite(v)
    idx = torch.where(fin, v, torch.zeros_like(v)).trunc().to(torch.int64)
    ok = fin & (idx >= -n) & (idx < n)
    idx = torch.where(idx < 0, idx + n, idx).clamp(0, n - 1)
    table = torch.where(ok, vals[idx], torch.full_like(v, float("nan"))).to(torch.bfloat16)
    try:
        code._vh_decode_table = (code._version, code.data_ptr(), table)
    except (AttributeError, RuntimeError):
        pass
    return table


def _dequantize_mx_cuda(input, scale, block_size, code=None, global_scale=None):
    _require_gpu(input, scale, code, global_scale)
    if code is not None and code.dim() != 1:
        raise NotImplementedError("dequantize_mx: region (per-head) codebooks are not supported yet")
    fi = _fmt_of(decode_table(code)).fmt if code is not None else None
    dec_dtype = input.dtype if code is None else input.dtype
    probe = torch.empty([1] * max(input.dim(), 1), dtype=dec_dtype, device="meta")
    cdt = torch.result_type(probe, scale)
    out = _elementwise("dequantize", input, scale, None, block_size, cdt, fi, None, cdt)
    if global_scale is not None:
        out = out * global_scale
    return out


cuda_kernel("dequantize_mx")(_dequantize_mx_cuda)


@fake_kernel("dequantize_mx")
def _dequantize_mx_fake(input, scale, block_size, code=None, global_scale=None):
    dtype = torch.promote_types(input.dtype, scale.dtype)
    if global_scale is not None:
        dtype = torch.promote_types(dtype, global_scale.dtype)
    return input.new_empty(input.shape, dtype=dtype)
