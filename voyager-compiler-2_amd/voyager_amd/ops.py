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
import math
from typing import List, Optional, Sequence

import torch

from . import _lib, formats
from ._lib import Codebook, Format, Param, VH_U8, dtype_code, load, ptr, stream_of

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


# ----------------------------------------------------------------- codebooks
_CB_DTYPES = (torch.bfloat16, torch.float16, torch.float32)


def _floor_f32(e: torch.Tensor) -> torch.Tensor:
    """``e`` as float32, each value the largest float32 not above it: a
    search of bfloat16 (hence float32) values answers against it as against
    ``e`` itself."""
    e32 = e.to(torch.float32)
    if e.dtype in _CB_DTYPES:
        return e32.contiguous()
    down = torch.nextafter(e32, torch.full_like(e32, float("-inf")))
    return torch.where(e32.to(e.dtype) > e, down, e32).contiguous()


def _region_grid(codebook: torch.Tensor, shape) -> tuple:
    """The region grid of ``codebook`` over a contiguous tensor of ``shape``
    (``_region_view``, ``ops/quantized.py:193-229``): ``(regions, Param)``,
    the table of element ``(i_0..i_n)`` being ``sum_d (i_d / div[d]) *
    stride[d]`` in row-major order over the grid."""
    prm = Param()
    if codebook.dim() == 1:
        prm.scalar = 1
        return 1, prm
    counts = list(codebook.shape[:-1])
    if len(counts) != len(shape):
        raise ValueError(f"a {counts} region codebook tiles {len(counts)} axes, "
                         f"but the tensor reaching it has {len(shape)}")
    if any(n % c for n, c in zip(shape, counts)):
        raise ValueError(f"a {counts} region codebook does not divide the {list(shape)} tensor reaching it")
    stride = 1
    for d in reversed(range(len(counts))):
        prm.div[d] = max(shape[d] // counts[d], 1)
        prm.stride[d] = stride if counts[d] > 1 else 0
        stride *= counts[d]
    return stride, prm


def _cached_on(t: torch.Tensor, attr: str, key, build):
    """``build()`` cached on tensor ``t`` under ``key`` (its version and
    address included, so an in-place change or a new tensor rebuilds)."""
    key = (t._version, t.data_ptr()) + key
    hit = getattr(t, attr, None)
    if hit is not None and hit[0] == key:
        return hit[1]
    value = build()
    try:
        setattr(t, attr, (key, value))
    except (AttributeError, RuntimeError):
        pass
    return value


def _codebook_desc(codebook: torch.Tensor, shape, bounds: Optional[torch.Tensor], encode: bool):
    """``vh_codebook`` for ``codebook`` (``[k]`` or ``[*counts, k]``) over a
    contiguous tensor of ``shape``, and the device tensors it points to.
    encode: the edges are ``bounds`` (the result is the index) or the
    entries' midpoints in their dtype (the result is the entry), as
    ``encode`` (``ops/quantized.py:232-287``) takes them."""
    if codebook.dtype not in _CB_DTYPES:
        raise NotImplementedError(f"codebook entries of dtype {codebook.dtype} are not supported on the GPU")
    regions, grid = _region_grid(codebook, shape)
    k = codebook.shape[-1]
    cb = Codebook()
    cb.k = k
    cb.regions = regions
    cb.region = grid
    keep = []
    if not encode or bounds is None:
        entries = codebook.reshape(regions, k).contiguous()
        cb.entries = entries.data_ptr()
        cb.entries_dtype = dtype_code(entries.dtype)
        keep.append(entries)
    if encode:
        if bounds is None:
            edges = _cached_on(codebook, "_vh_cb_edges", (), lambda: _floor_f32(
                (codebook[..., :-1] + codebook[..., 1:]) / 2).reshape(regions, k - 1))
        else:
            if codebook.dim() == 1 and bounds.dim() != 1:
                raise NotImplementedError("a 1-D codebook with multi-dimensional bounds is not supported on the GPU")
            if bounds.numel() % regions:
                raise ValueError(f"{bounds.numel()} bounds do not split into {regions} region tables")
            edges = _cached_on(bounds, "_vh_cb_edges", (regions,),
                               lambda: _floor_f32(bounds).reshape(regions, -1))
        cb.edges = edges.data_ptr()
        cb.nedges = edges.shape[-1]
        keep.append(edges)
    return cb, keep


def _encode_cuda(x, scale, zero_point, block_size, cdt, codebook, bounds):
    """``quantize`` against a codebook: the division as ``quantize`` does it,
    then ``encode`` (``ops/quantized.py:232-287``) in one pass."""
    xc = x.contiguous()
    shape = list(xc.shape)
    sp, keep_s = _param(scale, shape, block_size, cdt, "scale", own_precision=True)
    zpp, keep_z = _param(zero_point, shape, block_size, cdt, "zero_point")
    cb, keep = _codebook_desc(codebook, shape, bounds, True)
    out = torch.empty(shape, dtype=cdt, device=x.device)
    st = load().vh_quantize_codebook(ptr(xc), dtype_code(xc.dtype), _shape_arr(shape), len(shape),
                                     ctypes.byref(sp) if sp else None, ctypes.byref(zpp) if zpp else None,
                                     dtype_code(cdt), ctypes.byref(cb), ptr(out), ctypes.c_void_p(stream_of(x)))
    _lib.check(st, "vh_quantize_codebook")
    del keep_s, keep_z, keep
    return out


def decode_codes(x, code, scale=None, block_size=None):
    """``decode`` then, with a scale, ``* repeat_per_block(scale)``
    (``ops/quantized.py:290-315, 574-591``): a 1-D codebook read by
    bfloat16 codes goes through its 65,536-entry table; any other codebook
    (a region grid, float16 or float32 codes) through ``vh_decode_codebook``."""
    if code.dim() == 1 and x.dtype == torch.bfloat16:
        fi = _fmt_of(decode_table(code)).fmt
        if scale is None:
            return _elementwise("quantize", x, None, None, None, x.dtype, fi, None, x.dtype)
        probe = torch.empty([1] * max(x.dim(), 1), dtype=x.dtype, device="meta")
        cdt = torch.result_type(probe, scale)
        return _elementwise("dequantize", x, scale, None, block_size, cdt, fi, None, cdt)
    if x.dtype not in _CB_DTYPES:
        raise NotImplementedError(f"codebook indices of dtype {x.dtype} are not supported on the GPU")
    xc = x.contiguous()
    shape = list(xc.shape)
    out_dtype = x.dtype
    sp, keep_s = None, None
    if scale is not None:
        probe = torch.empty([1] * max(x.dim(), 1), dtype=x.dtype, device="meta")
        out_dtype = torch.result_type(probe, scale)
        sp, keep_s = _param(scale, shape, block_size, out_dtype, "scale", own_precision=True)
    cb, keep = _codebook_desc(code, shape, None, False)
    out = torch.empty(shape, dtype=out_dtype, device=x.device)
    st = load().vh_decode_codebook(ptr(xc), dtype_code(xc.dtype), _shape_arr(shape), len(shape), ctypes.byref(cb),
                                   1 if code.dim() == 1 else 0, ctypes.byref(sp) if sp else None, ptr(out),
                                   dtype_code(out_dtype), ctypes.c_void_p(stream_of(x)))
    _lib.check(st, "vh_decode_codebook")
    del keep_s, keep
    return out


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
        return _encode_cuda(input, scale, zero_point, block_size, cdt, qmap, output_code)
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
def _axes_list(x: torch.Tensor, axes) -> List[int]:
    """The blocked axes, non-negative and ascending (``_reshape_to_blocks``,
    ``quantization/mx_utils.py:66-80``)."""
    axes = [axes] if isinstance(axes, int) else list(axes)
    out = []
    for a in axes:
        ax = a + x.dim() if a < 0 else a
        if not 0 <= ax < max(x.dim(), 1):
            raise IndexError(f"axis {a} out of range for a {x.dim()}-d tensor")
        out.append(ax)
    if len(set(out)) != len(out):
        raise ValueError(f"repeated block axes {axes}")
    return sorted(out)


def _block_view(x: torch.Tensor, axes):
    """``x`` as contiguous ``[outer, L, inner]`` around its one blocked axis."""
    axes = _axes_list(x, axes)
    if len(axes) != 1:
        raise ValueError("one block axis expected")
    ax = axes[0]
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


def _mx_scale(x, axes, block_size, quant_max, pot, scale_qmap, global_scale):
    """``calculate_mx_qparam`` (``ops/quantized.py:958-1031``).  One axis:
    the block-scale kernel.  Several: a block's scale depends on nothing but
    its max |x|, so ``vh_block_amax`` reduces the blocked axes one at a time
    and the block-scale kernel turns each max into its scale (blocks of
    one)."""
    if block_size <= 0:
        raise AssertionError("block_size must be > 0")
    axes = _axes_list(x, axes)
    if len(axes) == 1:
        scale, _ = _mx_launch(x, axes, block_size, quant_max, pot, scale_qmap, global_scale, None, False)
        return scale
    a = x.contiguous()
    lib_ = load()
    for ax in axes:
        outer = math.prod(a.shape[:ax])
        inner = math.prod(a.shape[ax + 1:])
        shape = list(a.shape)
        shape[ax] = -(-shape[ax] // block_size)
        out = torch.empty(shape, dtype=a.dtype, device=a.device)
        _lib.check(lib_.vh_block_amax(ptr(a), dtype_code(a.dtype), outer, a.shape[ax], inner, block_size, ptr(out),
                                      ctypes.c_void_p(stream_of(x))), "vh_block_amax")
        a = out
    scale, _ = _mx_launch(a, [a.dim() - 1], 1, quant_max, pot, scale_qmap, global_scale, None, False)
    return scale


def _calculate_mx_qparam_cuda(input, axes, block_size, quant_max, force_scale_power_of_two=False,
                              scale_qmap=None, global_scale=None):
    _require_gpu(input, scale_qmap, global_scale)
    return _mx_scale(input, axes, block_size, quant_max, force_scale_power_of_two, scale_qmap, global_scale)


cuda_kernel("calculate_mx_qparam")(_calculate_mx_qparam_cuda)


@fake_kernel("calculate_mx_qparam")
def _calculate_mx_qparam_fake(input, axes, block_size, quant_max, force_scale_power_of_two=False,
                              scale_qmap=None, global_scale=None):
    return input.new_empty(_scale_shape_axes(input, axes, block_size))


def _scale_shape_axes(x, axes, block_size):
    shape = list(x.shape)
    for ax in _axes_list(x, axes):
        shape[ax] = -(-shape[ax] // block_size)
    return shape


def _quantize_mx_cuda(input, qmap, axes, block_size, quant_max, force_scale_power_of_two=False,
                      scale_qmap=None, output_code=None, seed=None, global_scale=None):
    _require_gpu(input, qmap, scale_qmap, global_scale, seed, output_code)
    if seed is None and _is_table(qmap) and len(_axes_list(input, axes)) == 1:
        # one pass: block scales and codes
        return _mx_launch(input, axes, block_size, quant_max, force_scale_power_of_two, scale_qmap, global_scale,
                          qmap, True)
    # ops/quantized.py:1097-1115: the block scales, then quantize (with the
    # seed, against the codebook, or per block over several axes) by
    # scale * global_scale, which the dequantize kernel forms as eager torch
    # does (the 0-d global scale at its own precision, one rounding)
    scale = _mx_scale(input, axes, block_size, quant_max, force_scale_power_of_two, scale_qmap, global_scale)
    el = scale
    if global_scale is not None:
        el = _elementwise("dequantize", scale, global_scale.reshape(()), None, None, scale.dtype, None, None,
                          scale.dtype)
    cdt = _quantize_dtype(input, el, None)
    if seed is not None:
        return scale, _quantize_sr(input, el, None, block_size, qmap, seed, cdt)
    if _is_table(qmap):
        return scale, _elementwise("quantize", input, el, None, block_size, cdt, _fmt_of(qmap).fmt, None, cdt)
    return scale, _encode_cuda(input, el, None, block_size, cdt, qmap, output_code)


cuda_kernel("quantize_mx")(_quantize_mx_cuda)


@fake_kernel("quantize_mx")
def _quantize_mx_fake(input, qmap, axes, block_size, quant_max, force_scale_power_of_two=False,
                      scale_qmap=None, output_code=None, seed=None, global_scale=None):
    return input.new_empty(_scale_shape_axes(input, axes, block_size)), torch.empty_like(input)


def _quantize_affine_cuda(input, qmap, axes, block_size, quant_min, quant_max, scale_qmap=None):
    _require_gpu(input, qmap, scale_qmap)
    if block_size <= 0:
        raise AssertionError("block_size must be > 0")
    if len(axes) != 1:
        raise ValueError("quantize_affine takes exactly one axis")
    xc, ax, outer, L, inner = _block_view(input, axes)
    cdt = xc.dtype
    sshape = _scale_shape(xc, ax, block_size)
    scale = torch.empty(sshape, dtype=cdt, device=input.device)
    zp = torch.empty(sshape, dtype=cdt, device=input.device)
    table = _is_table(qmap)
    codes = torch.empty_like(xc) if table else None
    sc = _fmt_of(scale_qmap) if scale_qmap is not None else None
    ec = _fmt_of(qmap) if table else None
    st = load().vh_quantize_affine(ptr(xc), dtype_code(cdt), outer, L, inner, block_size, float(quant_min),
                                   float(quant_max), _fmt_ref(sc), _fmt_ref(ec), ptr(scale), ptr(zp), ptr(codes),
                                   dtype_code(cdt), ctypes.c_void_p(stream_of(input)))
    _lib.check(st, "vh_quantize_affine")
    if not table:
        # a codebook: quantize (ops/quantized.py:1282) searches it with the
        # block's scale and zero point
        codes = _encode_cuda(xc, scale, zp, block_size, _quantize_dtype(xc, scale, zp), qmap, None)
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
    if code is not None:
        out = decode_codes(input, code, scale, block_size)
    else:
        probe = torch.empty([1] * max(input.dim(), 1), dtype=input.dtype, device="meta")
        cdt = torch.result_type(probe, scale)
        out = _elementwise("dequantize", input, scale, None, block_size, cdt, None, None, cdt)
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
