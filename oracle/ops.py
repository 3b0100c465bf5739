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


def vmap(input, table, chunk_size=1024 * 1024):
    """``table[bits(bf16(input))]`` in ``input``'s dtype and layout;
    ``ops/quantized.py:147-184``.  Gathers in chunks of ``chunk_size``
    elements in memory order, as the reference's eager path does, so the
    CPU baseline times the same loop."""
    in_dtype = input.dtype
    x = input.to(torch.bfloat16) if input.dtype != torch.bfloat16 else input
    idx = x.view(torch.int16)
    order = sorted(range(x.ndim), key=x.stride, reverse=True)
    if x.permute(order).is_contiguous():
        out = torch.empty_like(x)
    else:
        order = list(range(x.ndim))
        out = torch.empty_like(x, memory_format=torch.contiguous_format)
    idx_flat = idx.permute(order).reshape(-1)
    out_flat = out.permute(order).view(-1)
    for start in range(0, idx_flat.numel(), chunk_size):
        end = min(start + chunk_size, idx_flat.numel())
        out_flat[start:end] = table[idx_flat[start:end].to(torch.int32) & 0xFFFF].to(x.dtype)
    return out.to(in_dtype)


def region_view(input, codebook):
    """``_region_view``, ``ops/quantized.py:193-229``: ``input`` split by the
    ``[*counts, k]`` grid of ``codebook`` with the region axes first, and the
    permutation back."""
    counts = tuple(codebook.shape[:-1])
    if len(counts) != input.dim():
        raise ValueError(f"a {list(counts)} region codebook tiles {len(counts)} axes, "
                         f"but the tensor reaching it has {input.dim()}")
    if any(n % c for n, c in zip(input.shape, counts)):
        raise ValueError(f"a {list(counts)} region codebook does not divide the "
                         f"{list(input.shape)} tensor reaching it")
    split = []
    for n, c in zip(input.shape, counts):
        split += [c, n // c]
    order = list(range(0, 2 * len(counts), 2)) + list(range(1, 2 * len(counts), 2))
    inverse = [0] * len(order)
    for pos, ax in enumerate(order):
        inverse[ax] = pos
    return input.reshape(split).permute(order), inverse


def encode(input, codebook, bounds=None):
    """Codebook search, one table or a region grid; ``ops/quantized.py:232-287``."""
    edges = bounds if bounds is not None else (codebook[..., :-1] + codebook[..., 1:]) / 2
    if codebook.dim() == 1:
        index = torch.searchsorted(edges, input.bfloat16().float())
        picked = index if bounds is not None else codebook[index]
        return picked.to(input.dtype)
    moved, inverse = region_view(input, codebook)
    regions = codebook.numel() // codebook.shape[-1]
    flat = moved.reshape(regions, -1).bfloat16().float()
    table = codebook.reshape(regions, -1)
    index = torch.searchsorted(edges.reshape(regions, -1).contiguous(), flat.contiguous())
    picked = index if bounds is not None else table.gather(1, index)
    picked = picked.view(moved.shape).permute(inverse)
    return picked.reshape(input.shape).to(input.dtype)


def decode(input, codebook):
    """The entry each index names, one table or a region grid;
    ``ops/quantized.py:290-315``."""
    index = input.to(torch.long)
    if codebook.dim() == 1:
        return codebook[index].to(input.dtype)
    moved, inverse = region_view(index, codebook)
    regions = codebook.numel() // codebook.shape[-1]
    picked = codebook.reshape(regions, -1).gather(1, moved.reshape(regions, -1))
    picked = picked.view(moved.shape).permute(inverse)
    return picked.reshape(index.shape).to(input.dtype)


# ------------------------------------------------------ stochastic rounding
# Philox4x32-10 (Salmon et al., SC'11): round multipliers, key increments.
PHILOX_M = (0xD2511F53, 0xCD9E8D57)
PHILOX_W = (0x9E3779B9, 0xBB67AE85)
MASK32 = 0xFFFFFFFF


def _mulhilo32(a, b):
    """High and low words of ``a * b``: uint32 values held in int64, the
    product taken over the 16-bit halves of ``b`` so nothing overflows
    (``ops/quantized.py:327-336``)."""
    lo_part = a * (b & 0xFFFF)
    hi_part = a * (b >> 16)
    low = lo_part + ((hi_part & 0xFFFF) << 16)
    return (hi_part >> 16) + (low >> 32), low & MASK32


def philox(counter, seed):
    """``_philox``, ``ops/quantized.py:339-360``: the four words of the
    Philox4x32-10 draw of each int64 ``counter`` (high 64 counter bits zero)
    under the 64-bit key ``seed``; int64 ``[*counter.shape, 4]``."""
    c0, c1 = counter & MASK32, (counter >> 32) & MASK32
    c2 = torch.zeros_like(counter)
    c3 = torch.zeros_like(counter)
    k0, k1 = seed & MASK32, (seed >> 32) & MASK32
    for _ in range(10):
        hi0, lo0 = _mulhilo32(c0, PHILOX_M[0])
        hi1, lo1 = _mulhilo32(c2, PHILOX_M[1])
        c0, c1, c2, c3 = hi1 ^ c1 ^ k0, lo1, hi0 ^ c3 ^ k1, lo0
        k0 = (k0 + PHILOX_W[0]) & MASK32
        k1 = (k1 + PHILOX_W[1]) & MASK32
    return torch.stack([c0, c1, c2, c3], -1)


def random_bytes(seed, shape):
    """``_random_bytes``, ``ops/quantized.py:363-381``: element ``i`` takes
    byte ``i % 4`` of word ``i % 16 // 4`` of draw ``i // 16``."""
    numel = math.prod(shape)
    words = philox(torch.arange(-(-numel // 16)), seed)
    shifts = torch.arange(0, 32, 8)
    return ((words[..., None] >> shifts) & 0xFF).flatten()[:numel].view(shape)


def qmap_levels(qmap):
    """``qmap_levels``, ``ops/quantized.py:384-396``: a table's distinct finite values,
    ascending, float32, one +0."""
    table = qmap.float()
    return torch.unique(table[torch.isfinite(table)]) + 0.0


def stochastic_round(input, qmap, seed):
    """``_stochastic_round`` / ``_neighbors``, ``ops/quantized.py:399-446``."""
    levels = qmap_levels(qmap) if qmap.numel() == QMAP_SIZE else qmap
    levels = levels.float()
    value = input.float().clamp(levels[0], levels[-1])
    upper = torch.searchsorted(levels, value).clamp(max=levels.numel() - 1)
    high = levels[upper]
    low = torch.where(high == value, high, levels[(upper - 1).clamp(min=0)])
    noise = random_bytes(seed, input.shape) / 256
    near = torch.where(value < 0, high, low)
    far = torch.where(value < 0, low, high)
    away = value.abs() + noise * (high - low) >= far.abs()
    return torch.where(away, far, near).to(input.dtype)


def quantize(input, scale, zero_point=None, axes=None, block_size=None,
             qmap=None, output_code=None, seed=None):
    """``ops/quantized.py:449-515``; with a ``seed``, stochastic rounding."""
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
    if seed is not None:
        return stochastic_round(x, qmap, seed)
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
              out_dtype=None, A_data=None, A_indices=None, A_indptr=None):
    """``ops/quantized.py:651-723``, the outlier (CSR) term included."""
    _, sw, so = _parse_layout(layout)
    x = dequantize_mx_parts(input, input_scale, input_code, block_size)
    w = dequantize_mx_parts(weight, weight_scale, weight_code, block_size)
    dtype = x.dtype if out_dtype is None else out_dtype
    acc = torch.promote_types(dtype, torch.float32)
    out = linear(x, w, bias if alpha is None else None, layout=_with_xk(layout), out_dtype=acc)
    if alpha is not None:
        out = out * alpha
        if bias is not None:
            out = out + bias
    if A_data is not None:
        out = out + spmm_csr(A_data, A_indices, A_indptr, weight, weight_scale, weight_code, block_size,
                             sw, out_dtype=acc)
    out = out.to(dtype)
    return out.mT.contiguous() if so != "xk" else out


def matmul_mx(input, other, input_scale=None, weight_scale=None, block_size=None,
              input_code=None, weight_code=None, alpha=None, layout=MATMUL_LAYOUT,
              out_dtype=None, A_data=None, A_indices=None, A_indptr=None):
    """``ops/quantized.py:742-805``, the outlier (CSR) term included."""
    _, sw, so = _parse_layout(layout)
    x = dequantize_mx_parts(input, input_scale, input_code, block_size)
    w = dequantize_mx_parts(other, weight_scale, weight_code, block_size)
    dtype = x.dtype if out_dtype is None else out_dtype
    acc = torch.promote_types(dtype, torch.float32)
    out = matmul(x, w, layout=_with_xk(layout), out_dtype=acc)
    if alpha is not None:
        out = out * alpha
    if A_data is not None:
        out = out + spmm_csr(A_data, A_indices, A_indptr, other, weight_scale, weight_code, block_size,
                             sw, out_dtype=acc)
    out = out.to(dtype)
    return out.mT.contiguous() if so != "xk" else out


# ------------------------------------------------------------ conv2d

def _pair(v):
    return tuple(v) if isinstance(v, (list, tuple)) else (v, v)


def conv2d(input, weight, bias=None, stride=(1, 1), padding=(0, 0), dilation=(1, 1), groups=1,
           layout="nchw", out_dtype=None):
    """``quantized_ops.conv2d``, ``ops/layout.py:187-214``: aten's conv2d on
    NCHW maps, or NHWC ones with an HWIO weight when dense."""
    assert layout in ("nchw", "nhwc"), layout
    nhwc = layout == "nhwc"
    if nhwc:
        input = input.permute(0, 3, 1, 2)
        if groups == 1:
            weight = weight.permute(3, 2, 0, 1)
    if out_dtype is not None:
        input, weight = input.float(), weight.float()
        bias = None if bias is None else bias.float()
    out = torch.ops.aten.conv2d(input, weight, bias, _pair(stride), _pair(padding), _pair(dilation), groups)
    if out_dtype is not None:
        out = out.to(out_dtype)
    return out.permute(0, 2, 3, 1) if nhwc else out


def conv2d_mx(input, weight, bias=None, stride=1, padding=0, dilation=1, groups=1, input_scale=None,
              weight_scale=None, block_size=None, input_code=None, weight_code=None, layout="nchw",
              out_dtype=None):
    """``ops/quantized.py:606-643``: both operands decoded, then ``conv2d``."""
    x = dequantize_mx_parts(input, input_scale, input_code, block_size)
    w = dequantize_mx_parts(weight, weight_scale, weight_code, block_size)
    return conv2d(x, w, bias, stride, padding, dilation, groups, layout, out_dtype)


# ------------------------------------------------------------ outliers (CSR)

def pad_csr(values, col_indices, crow_indices, max_nnz):
    """``_pad_csr``, ``ops/quantized.py:1292-1319``: a CSR stream padded to
    ``max_nnz`` slots (data 0, index -1), or cut to its first ``max_nnz``
    entries with the row pointers clamped there.  Returns
    ``(data, indices, crow_indices)``."""
    nse = int(crow_indices[-1])
    if max_nnz >= nse:
        data = torch.nn.functional.pad(values, (0, max_nnz - nse), mode="constant", value=0)
        indices = torch.nn.functional.pad(col_indices, (0, max_nnz - nse), mode="constant", value=-1)
        return data, indices, crow_indices
    return values[:max_nnz], col_indices[:max_nnz], crow_indices.clamp(max=max_nnz)


def filter_outlier(input, threshold, max_pct=0.01):
    """``ops/quantized.py:1322-1374``: ``(data, indices, indptr, inliers)``,
    the elements with ``|x| >= threshold`` of each matrix (last two dims) as
    a padded CSR of ``int(rows * cols * max_pct)`` slots."""
    is_outlier = torch.abs(input) >= threshold
    inliers = torch.where(is_outlier, 0, input)
    outliers = torch.where(is_outlier, input, 0)
    batch_shape, mat_shape = input.shape[:-2], input.shape[-2:]
    max_nnz = int(math.prod(mat_shape) * max_pct)
    per_matrix = outliers.reshape(int(math.prod(batch_shape)), *mat_shape)
    parts = []
    for mat in per_matrix:
        csr = mat.to_sparse_csr()
        parts.append(pad_csr(csr.values(), csr.col_indices().to(torch.int32),
                             csr.crow_indices().to(torch.int32), max_nnz))
    data = torch.stack([p[0] for p in parts]).reshape(*batch_shape, -1)
    indices = torch.stack([p[1] for p in parts]).reshape(*batch_shape, -1)
    indptr = torch.stack([p[2] for p in parts]).reshape(*batch_shape, -1)
    return data, indices, indptr, inliers


def quantize_mx_outlier(input, qmap, axes, block_size, quant_max, force_scale_power_of_two=False,
                        scale_qmap=None, output_code=None, threshold=None, max_pct=0.01, indptr_offset=0):
    """``ops/quantized.py:1405-1458``: ``(data, indices, indptr, scale,
    inliers)``."""
    data, indices, indptr, inliers = filter_outlier(input, threshold, max_pct)
    if indptr_offset:
        indptr = indptr + indptr_offset
    scale, codes = quantize_mx(inliers, qmap, axes, block_size, quant_max, force_scale_power_of_two,
                               scale_qmap, output_code)
    return data, indices, indptr, scale, codes


def slice_csr_tensor(data, indices, indptr, dim=0, start=None, end=None, size_factor=1.0):
    """``ops/quantized.py:1500-1545``: rows (dim 0) or columns (dim 1)
    ``[start, end)`` of one CSR matrix, padded to ``int(len(data) *
    size_factor)`` slots."""
    dim = dim + 2 if dim < 0 else dim
    if dim not in (0, 1):
        raise ValueError(f"Cannot slice sparse CSR matrix along dim {dim}")
    if dim == 0:
        first, last = int(indptr[start]), int(indptr[end])
        new_indptr = indptr[start:end + 1] - first
        values, cols = data[first:last], indices[first:last]
    else:
        keep = (indices >= start) & (indices < end)
        lengths = (indptr[1:] - indptr[:-1]).to(torch.int64)
        nse = int(indptr[-1])
        counts = torch.segment_reduce(keep[:nse].to(torch.float32), "sum", lengths=lengths).to(indptr.dtype)
        new_indptr = torch.empty_like(indptr)
        new_indptr[0] = 0
        new_indptr[1:] = counts.cumsum(0).to(indptr.dtype)
        values, cols = data[keep], indices[keep] - start
    return pad_csr(values, cols, new_indptr, int(data.shape[0] * size_factor))


def spmm_csr(data, indices, indptr, B, B_scale=None, B_code=None, block_size=None, weight_layout="kc",
             out_dtype=None):
    """``ops/quantized.py:1574-1645``: the CSR matrices (batch dims leading)
    times ``B`` decoded (code, then block scale), in float32 through
    ``torch.sparse.mm``; rows rebased on their first pointer, clamped and made
    non-decreasing, columns clamped into ``B``."""
    assert weight_layout in ("kc", "ck"), weight_layout
    B = dequantize_mx_parts(B, B_scale, B_code, block_size)
    if weight_layout == "kc":
        B = B.mT
    batch_shape = indptr.shape[:-1]
    nb = int(math.prod(batch_shape))
    indptr = indptr.reshape(-1, indptr.shape[-1])
    indices = indices.reshape(-1, indices.shape[-1])
    data = data.reshape(-1, data.shape[-1])
    if B.ndim > 2:
        B = B.reshape(nb, B.shape[-2], B.shape[-1])
    outs = []
    for i in range(nb):
        Bi = B[i] if B.ndim == 3 else B
        crow = (indptr[i] - indptr[i][0]).clamp(0, data.shape[-1])
        crow = torch.cummax(crow, 0).values
        end = int(crow[-1])
        csr = torch.sparse_csr_tensor(crow, indices[i, :end].clamp(0, Bi.shape[0] - 1), data[i, :end],
                                      dtype=torch.float32, size=(indptr[i].numel() - 1, Bi.shape[0]))
        outs.append(torch.sparse.mm(csr, Bi.to(torch.float32)).to(B.dtype if out_dtype is None else out_dtype))
    return torch.stack(outs).reshape(*batch_shape, -1, B.shape[-1])


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


# ------------------------------------------------------------ attention twins
HADAMARD_SIZE = 16


def hadamard_rotate(x, axis, matrix):
    """``ops/quantized.py:1038-1067``: runs of 16 along ``axis`` (last or
    second-to-last, zero-padded to whole runs) times ``matrix`` in float32."""
    axis %= x.ndim
    assert axis >= x.ndim - 2
    pad = -x.shape[axis] % HADAMARD_SIZE
    if pad:
        x = torch.nn.functional.pad(x, (0, 0) * (x.ndim - 1 - axis) + (0, pad))
    runs = x.float().unflatten(axis, (-1, HADAMARD_SIZE))
    m = matrix.float()
    out = runs @ m if axis == x.ndim - 1 else m.T @ runs
    return out.flatten(axis, axis + 1).to(x.dtype)


def quantize_mx_transpose(input, qmap, block_size, quant_max, force_scale_power_of_two=False, scale_qmap=None,
                          output_code=None, seed=None, global_scale=None, transpose_seed=None,
                          transpose_global_scale=None, hadamard=None):
    """``ops/quantized.py:1168-1215``."""
    t = input.mT
    if hadamard is not None:
        t = hadamard_rotate(t, -1, hadamard)
    args = (qmap, (-1,), block_size, quant_max, force_scale_power_of_two, scale_qmap, output_code)
    return (*quantize_mx(input, *args, seed, global_scale), *quantize_mx(t, *args, transpose_seed,
                                                                         transpose_global_scale))


def _masked(scores, mask):
    """``ops/quantized.py:924-932``."""
    if mask is None:
        return scores
    if mask.dtype == torch.bool:
        return scores.masked_fill(~mask, float("-inf"))
    return scores + mask


def sdpa_mx(query, key, value, attn_mask=None, dropout_p=0.0, is_causal=False, query_residual=None,
            key_residual=None, value_residual=None, residual_mask=None, scale=None, enable_gqa=False,
            query_scale=None, key_scale=None, value_scale=None, block_size=None, input_code=None,
            weight_code=None, probs_qmap=None, probs_quant_max=None, probs_scale_qmap=None, probs_code=None,
            force_scale_power_of_two=False):
    """``ops/quantized.py:834-921``."""
    if is_causal and attn_mask is not None:
        raise ValueError("is_causal excludes an explicit attn_mask")
    query = dequantize_mx_parts(query, query_scale, input_code, block_size)
    key = dequantize_mx_parts(key, key_scale, weight_code, block_size)
    value = dequantize_mx_parts(value, value_scale, weight_code, block_size)
    residual = key_residual is not None
    if enable_gqa:
        g = query.shape[-3] // key.shape[-3]
        key, value = key.repeat_interleave(g, dim=-3), value.repeat_interleave(g, dim=-3)
        if residual:
            key_residual = key_residual.repeat_interleave(g, dim=-3)
            value_residual = value_residual.repeat_interleave(g, dim=-3)
    if scale is None:
        scale = 1.0 / math.sqrt(query.shape[-1])
    scores = torch.matmul(query, key.transpose(-1, -2)) * scale
    if is_causal:
        attn_mask = torch.ones(scores.shape[-2:], dtype=torch.bool).tril()
    scores = _masked(scores, attn_mask)
    keys = scores.shape[-1]
    if residual:
        rs = _masked((query_residual @ key_residual.transpose(-1, -2)) * scale, residual_mask)
        scores = torch.cat([scores, rs], dim=-1)
    probs = torch.softmax(scores, dim=-1)
    probs, residual_probs = probs[..., :keys], probs[..., keys:]
    if probs_qmap is not None:
        ps, probs = quantize_mx(probs, probs_qmap, [-1], block_size, probs_quant_max, force_scale_power_of_two,
                                probs_scale_qmap, probs_code)
        probs = dequantize_mx_parts(probs, ps, input_code, block_size)
    out = torch.matmul(probs, value)
    if residual:
        out = out + torch.matmul(residual_probs, value_residual)
    return out
