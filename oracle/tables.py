"""64K-entry quantization tables, restated for the oracle (test only).

Entry ``i`` of a table is the value the bfloat16 whose bit pattern reads
``i`` rounds to.  Follows ``quantization/fake_quantize.py:68-139`` and the
format builders in ``quantization/dtypes/{fp8,posit,normal_float}.py``.
"""

import functools
import math

import torch

from .qspec import float_format, int_range, parse_codebook_dtype, posit_format

QMAP_SIZE = 2**16


def all_bf16() -> torch.Tensor:
    """Every bfloat16 bit pattern, pattern ``i`` at index ``i``."""
    return torch.arange(QMAP_SIZE, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)


def _round_even(a: torch.Tensor) -> torch.Tensor:
    """Round-half-even of ``a`` as ``dtypes/fp8.py:47-51`` computes it."""
    mag = torch.abs(a)
    on_half_even = ((mag - 0.5) % 2 == 0).to(a.dtype)
    return torch.sign(a) * (torch.floor(mag + 0.5) - on_half_even)


def minifloat(a: torch.Tensor, bits: int, ebits: int, max_norm: float) -> torch.Tensor:
    """Round float32 ``a`` to a minifloat grid; ``dtypes/fp8.py:69-135``
    with ``round="even"``, ``saturate_normals=True`` and subnormals kept.

    ``bits`` counts the mantissa plus sign and implicit bit (``mbits + 2``).
    """
    exp = torch.floor(torch.log2(torch.abs(a) + (a == 0).to(a.dtype)))
    exp = exp.clip(min=2 - 2 ** (ebits - 1))
    out = a / (2**exp) * (2 ** (bits - 2))
    out = _round_even(out)
    out = out / (2 ** (bits - 2)) * (2**exp)
    out = torch.clamp(out, min=-max_norm, max=max_norm)
    out[a == float("inf")] = float("inf")
    out[a == -float("inf")] = -float("inf")
    return out


def posit(values: torch.Tensor, nbits: int, es: int) -> torch.Tensor:
    """Posit rounding of ``values`` by bit manipulation of their float32
    encoding; ``dtypes/posit.py:8-73`` with ``round_to_even=True``."""
    raw = values.clone().to(torch.float).view(torch.int32)
    scale = ((raw & 0x7F800000) >> 23) - 127
    frac = raw & 0x7FFFFF
    pos = scale >= 0
    max_scale = (nbits - 2) * (1 << es)
    dominated = torch.where(pos, scale > max_scale, scale < -max_scale)
    run = torch.where(pos, 1 + (scale >> es), -(scale >> es))
    regime = torch.where(pos, (1 << (run + 1)) - 1, 0) ^ 1
    expo = scale % (1 << es)
    pbits = (regime << (23 + es)) | (expo << 23) | frac
    length = 2 + run + es + 23
    last = 1 << (length - nbits)
    guard = last >> 1
    sticky = guard - 1
    lb = (pbits & last) != 0
    gb = (pbits & guard) != 0
    sb = (pbits & sticky) != 0
    round_up = ((lb & gb) | (gb & sb)) & ~dominated
    exp_cut = torch.clamp(2 + run + es - nbits, min=0, max=es)
    scale = scale & (-1 << exp_cut)
    scale = torch.clamp(scale, min=-max_scale, max=max_scale)
    frac_cut = torch.clamp(length - nbits, min=0, max=23)
    frac = frac & (-1 << frac_cut)
    out = ((scale + 127) << 23) | frac
    out = torch.where(round_up, out + (1 << (frac_cut + exp_cut)), out)
    out = out.view(torch.float) * torch.sign(values)
    threshold = math.pow(2, math.floor(-(nbits - 1) * (1 << es) + 2 ** (es - 1)))
    out = torch.where(values.abs() < threshold, 0, out)
    out = torch.where(values == 0, 0, out)
    out = torch.where(torch.isfinite(values), out, torch.nan)
    return out.to(values.dtype)


def normal_map(k: int = 4, offset: float = 0.9677083, extra: bool = True) -> torch.Tensor:
    """NormalFloat levels in [-1, 1]; ``dtypes/normal_float.py:4-33``."""
    from scipy.stats import norm

    n = 2 ** (k - 1)
    if extra:
        pos = norm.ppf(torch.linspace(offset, 0.5, n + 1)[:-1]).tolist()
        zeros = [0]
        neg = (-norm.ppf(torch.linspace(offset, 0.5, n)[:-1])).tolist()
    else:
        pos = norm.ppf(torch.linspace(offset, 0.5, n)[:-1]).tolist()
        zeros = [0] * 2
        neg = (-norm.ppf(torch.linspace(offset, 0.5, n)[:-1])).tolist()
    vals = torch.Tensor(pos + zeros + neg).sort().values
    vals /= vals.max()
    assert vals.numel() == 2**k
    return vals


def nf_round(values: torch.Tensor, k: int, grid=None):
    """``dtypes/normal_float.py:36-62``: index of the nearest level (first
    on ties, computed in ``values``' dtype) and the levels."""
    levels = normal_map(k=k)
    if grid is not None:
        levels = levels.to(grid) * grid.max()
        levels = grid[torch.abs(levels[:, None] - grid).argmin(-1)]
    levels = levels.to(dtype=values.dtype)
    clamped = torch.clamp(values, min=levels.amin(), max=levels.amax())
    idx = torch.argmin(torch.abs(levels - clamped.unsqueeze(-1)), dim=-1)
    return idx, levels


def table_levels(table: torch.Tensor) -> torch.Tensor:
    """Distinct finite entries, ascending, one +0; ``ops/quantized.py:384-396``."""
    t = table.float()
    return torch.unique(t[torch.isfinite(t)]) + 0.0


def entry_levels(dtype: str) -> torch.Tensor:
    """Symmetric grid of a codebook entry dtype; ``fake_quantize.py:125-139``."""
    lv = table_levels(quantization_map(dtype))
    return lv[lv >= -lv.max()]


@functools.lru_cache(maxsize=None)
def quantization_map(dtype):
    """The bfloat16 table of ``dtype``; ``fake_quantize.py:68-122``."""
    v = all_bf16()
    if dtype is None:
        return v
    if (b := int_range(dtype)) is not None:
        return torch.clamp(torch.round(v), *b)
    if (f := float_format(dtype)) is not None:
        if not f.signed:
            v = torch.abs(v)
        v = torch.clamp(v, -f.max_norm, f.max_norm)
        return minifloat(v.float(), f.mbits + 2, f.ebits, f.max_norm).to(torch.bfloat16)
    if (p := posit_format(dtype)) is not None:
        return posit(v, *p)
    if (c := parse_codebook_dtype(dtype)) is not None:
        bits, entry = c
        grid = None if entry is None else entry_levels(entry)
        idx, levels = nf_round(v, bits, grid=grid)
        return levels[idx]
    raise ValueError(f"Unsupported dtype: {dtype}")


def codebook_index_table(value_table: torch.Tensor):
    """What convert swaps in for a codebook dtype: ``values = unique(table)``
    and the int64 index table ``searchsorted(values, table)``;
    ``quantization/quantize_pt2e.py:753-791``.  Returns ``(index_table,
    entries, midpoints)``."""
    values = torch.unique(value_table)
    index = torch.searchsorted(values, value_table).to(torch.int64)
    mid = (values[:-1] + values[1:]) / 2
    return index, values, mid
