"""The outlier (CSR) ops of ``quantized_ops`` on the GPU.

A converted graph whose activation spec filters outliers
(``quantization/quantize_pt2e.py:738-752, 906-944, 1088-1116``) splits the
activation with ``quantize_mx_outlier`` into MX-quantized inliers and a CSR
stream of the exact outliers, and its ``linear_mx`` / ``matmul_mx`` adds the
stream's product with the decoded weight (``A_data``, ``A_indices``,
``A_indptr``; ``ops/quantized.py:709-720``).  Here:

* ``filter_outlier`` / ``quantize_mx_outlier`` (``ops/quantized.py:1286-1458``)
  run ``vh_filter_outlier`` (segment counts with the inliers, a scan per
  matrix, the fill; a small workspace from torch's allocator), then the
  package's ``quantize_mx`` on the inliers;
* ``slice_csr_tensor`` (``:1493-1545``) runs ``vh_slice_csr``;
* ``spmm_csr`` (``:1567-1645``) decodes ``B`` with the package's
  ``dequantize_mx`` and runs ``vh_spmm_csr``; ``linear_mx`` / ``matmul_mx``
  call ``spmm_into`` with their float32 GEMM product as the base, so the
  sum is rounded to the output dtype once, as in the reference.

Every output has the shape the reference gives it, so nothing here waits on
the device: the CSR capacity is fixed by the shapes (``max_pct``,
``size_factor``).  The reference logs the outlier sparsity of each
``filter_outlier`` call; that needs a device-to-host read and is left out.
"""

import ctypes
import math
from typing import Optional

import torch

from . import _lib
from ._lib import dtype_code, load, ptr, stream_of
from .ops import _quantize_mx_cuda, _require_gpu
from .registry import cuda_kernel, fake_kernel

FLOAT_DTYPES = (torch.bfloat16, torch.float16, torch.float32)
_LAYOUTS = {"kc": 0, "ck": 1}


def threshold_in(dtype: torch.dtype, threshold: float) -> float:
    """The threshold as ``torch.abs(input) >= threshold`` compares it: a
    Python float converted to the tensor's dtype through float32."""
    return float(torch.tensor(float(threshold), dtype=torch.float32).to(dtype).float())


def _float_dtype(t: torch.Tensor, what: str) -> None:
    if t.dtype not in FLOAT_DTYPES:
        raise NotImplementedError(f"quantized_ops.{what}: {t.dtype} is not supported on the GPU "
                                  "(bfloat16, float16 or float32)")


def _int32(t: torch.Tensor) -> torch.Tensor:
    return t if t.dtype == torch.int32 else t.to(torch.int32)


def _max_nnz(mat_shape, max_pct: float) -> int:
    return int(math.prod(mat_shape) * max_pct)


# ----------------------------------------------------------------- filter
def filter_outlier(input: torch.Tensor, threshold: float, max_pct: float = 0.01, indptr_offset: int = 0):
    """``(data, indices, indptr, inliers)``: per matrix of the last two dims,
    the non-zero elements with ``|x| >= threshold`` as a CSR of
    ``int(rows * cols * max_pct)`` slots (``ops/quantized.py:1322-1374``),
    row pointers plus ``indptr_offset``; ``inliers`` is ``input`` with
    every element whose magnitude reaches the threshold zeroed."""
    _require_gpu(input)
    if threshold is None:
        raise TypeError("filter_outlier: threshold must be a float, got None")
    if input.dim() < 2:
        raise ValueError(f"filter_outlier: expected a tensor of at least 2 dims, got {input.dim()}")
    _float_dtype(input, "filter_outlier")
    batch_shape = tuple(input.shape[:-2])
    rows, cols = input.shape[-2:]
    cap = _max_nnz((rows, cols), max_pct)
    nb = int(math.prod(batch_shape))
    x = input.contiguous()
    data = torch.empty(*batch_shape, cap, dtype=input.dtype, device=input.device)
    indices = torch.empty(*batch_shape, cap, dtype=torch.int32, device=input.device)
    indptr = torch.empty(*batch_shape, rows + 1, dtype=torch.int32, device=input.device)
    inliers = torch.empty_like(x)
    if nb == 0:
        return data, indices, indptr, inliers
    thr = threshold_in(input.dtype, threshold)
    lib_ = load()
    nbytes = lib_.vh_filter_outlier_workspace_bytes(nb, rows, cols)
    work = torch.empty((nbytes + 15) // 16, 16, dtype=torch.uint8, device=input.device)
    st = lib_.vh_filter_outlier(ptr(x), dtype_code(x.dtype), nb, rows, cols, ctypes.c_float(thr), cap,
                                int(indptr_offset), ptr(data), ptr(indices), ptr(indptr), ptr(inliers), ptr(work),
                                work.numel(), ctypes.c_void_p(stream_of(x)))
    _lib.check(st, "vh_filter_outlier")
    return data, indices, indptr, inliers


def _filter_outlier_cuda(input, threshold, max_pct=0.01):
    return filter_outlier(input, threshold, max_pct)


def _quantize_mx_outlier_cuda(self, qmap, axes, block_size, quant_max, force_scale_power_of_two=False,
                              scale_qmap=None, output_code=None, threshold=None, max_pct=0.01, indptr_offset=0):
    """``ops/quantized.py:1405-1458``: the filter, then ``quantize_mx`` of
    the inliers; ``(data, indices, indptr, scale, inliers)``."""
    data, indices, indptr, inliers = filter_outlier(self, threshold, max_pct, indptr_offset)
    scale, codes = _quantize_mx_cuda(inliers, qmap, axes, block_size, quant_max, force_scale_power_of_two,
                                     scale_qmap, output_code)
    return data, indices, indptr, scale, codes


cuda_kernel("filter_outlier")(_filter_outlier_cuda)
cuda_kernel("quantize_mx_outlier")(_quantize_mx_outlier_cuda)


@fake_kernel("filter_outlier")
def _filter_outlier_fake(input, threshold, max_pct=0.01):
    batch_shape = input.shape[:-2]
    cap = _max_nnz(input.shape[-2:], max_pct)
    indptr = input.new_empty((*batch_shape, input.shape[-2] + 1), dtype=torch.int32)
    indices = input.new_empty((*batch_shape, cap), dtype=torch.int32)
    data = input.new_empty((*batch_shape, cap))
    return data, indices, indptr, torch.empty_like(input)


@fake_kernel("quantize_mx_outlier")
def _quantize_mx_outlier_fake(input, qmap, axes, block_size, quant_max, force_scale_power_of_two=False,
                              scale_qmap=None, output_code=None, threshold=None, max_pct=0.01, indptr_offset=0):
    batch_shape = input.shape[:-2]
    cap = _max_nnz(input.shape[-2:], max_pct)
    indptr = input.new_empty((*batch_shape, input.shape[-2] + 1), dtype=torch.int32)
    indices = input.new_empty((*batch_shape, cap), dtype=torch.int32)
    data = input.new_empty((*batch_shape, cap))
    scale_shape = list(input.shape)
    for axis in axes:
        scale_shape[axis] = math.ceil(scale_shape[axis] / block_size)
    scale = input.new_empty(scale_shape)
    inliers = torch.empty_like(input, memory_format=torch.contiguous_format)
    return data, indices, indptr, scale, inliers


# ----------------------------------------------------------------- slice
def _slice_csr_tensor_cuda(data, indices, indptr, dim=0, start=None, end=None, size_factor=1.0):
    """``ops/quantized.py:1500-1545`` on one CSR matrix (1-D data, indices
    and indptr); the output holds ``int(len(data) * size_factor)`` slots."""
    _require_gpu(data, indices, indptr)
    dim = dim + 2 if dim < 0 else dim
    if dim not in (0, 1):
        raise ValueError(f"Cannot slice sparse CSR matrix along dim {dim}")
    if data.dim() != 1 or indices.dim() != 1 or indptr.dim() != 1:
        raise NotImplementedError("quantized_ops.slice_csr_tensor: one CSR matrix (1-D data, indices, indptr) "
                                  "on the GPU")
    if start is None or end is None:
        raise TypeError("slice_csr_tensor: start and end are required")
    _float_dtype(data, "slice_csr_tensor")
    rows = indptr.numel() - 1
    cap = data.shape[0]
    out_cap = int(data.shape[0] * size_factor)
    start, end = int(start), int(end)
    if dim == 0:
        if not (0 <= start <= end <= rows):
            raise IndexError(f"slice_csr_tensor: rows [{start}, {end}) out of range for {rows} rows")
        n_ptr = end - start + 1
    else:
        if start < 0:
            raise ValueError("slice_csr_tensor: a column slice starts at a non-negative column")
        n_ptr = rows + 1
    ix, ip = _int32(indices).contiguous(), _int32(indptr).contiguous()
    dv = data.contiguous()
    out_data = torch.empty(out_cap, dtype=data.dtype, device=data.device)
    out_indices = torch.empty(out_cap, dtype=torch.int32, device=data.device)
    out_indptr = torch.empty(n_ptr, dtype=torch.int32, device=data.device)
    st = load().vh_slice_csr(ptr(dv), dtype_code(dv.dtype), ptr(ix), ptr(ip), rows, cap, dim, start, end, out_cap,
                             ptr(out_data), ptr(out_indices), ptr(out_indptr), ctypes.c_void_p(stream_of(dv)))
    _lib.check(st, "vh_slice_csr")
    return out_data, out_indices, out_indptr.to(indptr.dtype)


cuda_kernel("slice_csr_tensor")(_slice_csr_tensor_cuda)


@fake_kernel("slice_csr_tensor")
def _slice_csr_tensor_fake(data, indices, indptr, dim=0, start=None, end=None, size_factor=1.0):
    fake_indptr = torch.empty_like(indptr)
    if dim == 0 or dim == -2:
        return torch.empty_like(data), torch.empty_like(indices), fake_indptr[start: end + 1]
    return torch.empty_like(data), torch.empty_like(indices), fake_indptr


# ----------------------------------------------------------------- product
def spmm_into(data: torch.Tensor, indices: torch.Tensor, indptr: torch.Tensor, B: torch.Tensor, weight_layout: str,
              out_dtype: torch.dtype, base: Optional[torch.Tensor] = None) -> torch.Tensor:
    """CSR (``data``/``indices``/``indptr``, batch dims leading) times the
    decoded dense ``B`` (stored as ``weight_layout`` says), summed in
    float32 per output in stored entry order, plus ``base`` (float32, the
    shape of the result) when given, rounded once to ``out_dtype``."""
    if weight_layout not in _LAYOUTS:
        raise AssertionError(weight_layout)
    _float_dtype(data, "spmm_csr")
    _float_dtype(B, "spmm_csr")
    if out_dtype not in FLOAT_DTYPES:
        raise NotImplementedError(f"quantized_ops.spmm_csr: out_dtype {out_dtype} is not supported on the GPU")
    batch_shape = tuple(indptr.shape[:-1])
    nb = int(math.prod(batch_shape))
    rows = indptr.shape[-1] - 1
    cap = data.shape[-1]
    if B.dim() > 2:
        Bb = B.reshape(nb, B.shape[-2], B.shape[-1]).contiguous()
        b_stride = Bb.shape[-2] * Bb.shape[-1]
    else:
        Bb, b_stride = B.contiguous(), 0
    K, N = (Bb.shape[-1], Bb.shape[-2]) if weight_layout == "kc" else (Bb.shape[-2], Bb.shape[-1])
    out = torch.empty(*batch_shape, rows, N, dtype=out_dtype, device=data.device)
    if base is not None:
        if base.dtype != torch.float32 or tuple(base.shape) != tuple(out.shape):
            raise RuntimeError(f"spmm_csr: base must be float32 {list(out.shape)}, got {base.dtype} "
                               f"{list(base.shape)}")
        base = base.contiguous()
    if out.numel() == 0:
        return out
    dv = data.reshape(nb, cap).contiguous()
    ix = _int32(indices).reshape(nb, -1).contiguous()
    ip = _int32(indptr).reshape(nb, rows + 1).contiguous()
    if ix.shape[-1] != cap:
        raise RuntimeError("spmm_csr: data and indices differ in length")
    work = torch.empty(nb, rows + 1, dtype=torch.int32, device=data.device)
    st = load().vh_spmm_csr(ptr(dv), dtype_code(dv.dtype), ptr(ix), ptr(ip), nb, rows, cap, ptr(Bb),
                            dtype_code(Bb.dtype), _LAYOUTS[weight_layout], K, N, b_stride, ptr(base), ptr(out),
                            dtype_code(out_dtype), ptr(work), ctypes.c_void_p(stream_of(dv)))
    _lib.check(st, "vh_spmm_csr")
    return out


def _spmm_csr_cuda(data, indices, indptr, B, B_scale=None, B_code=None, block_size=None, weight_layout="kc", *,
                   out_dtype=None):
    """``ops/quantized.py:1574-1645``: ``B`` decoded (code, then block
    scale) as the GEMM decodes it, then the product."""
    from .gemm import _decode

    _require_gpu(data, indices, indptr, B, B_scale, B_code)
    assert weight_layout in ("kc", "ck"), weight_layout
    Bd = _decode(B, B_scale, B_code, block_size)
    return spmm_into(data, indices, indptr, Bd, weight_layout, Bd.dtype if out_dtype is None else out_dtype)


cuda_kernel("spmm_csr")(_spmm_csr_cuda)


@fake_kernel("spmm_csr")
def _spmm_csr_fake(data, indices, indptr, B, B_scale=None, B_code=None, block_size=None, weight_layout="kc", *,
                   out_dtype=None):
    batch_shape = indptr.shape[:-1]
    X = indptr.shape[-1] - 1
    K = B.shape[-1] if weight_layout == "ck" else B.shape[-2]
    return data.new_empty((*batch_shape, X, K), dtype=out_dtype)
