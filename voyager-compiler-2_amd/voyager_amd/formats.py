"""Numeric formats: the spec-string vocabulary, closed-form descriptors of the
65,536-entry quantization maps, and classification of a caller's map.

The reference expresses every elementwise format as a bfloat16-indexed table
(``ops/quantized.py:147-190``; built by ``quantization/fake_quantize.py:68-122``).
The GPU kernels evaluate closed forms instead.  ``classify`` picks the closed
form for a caller's table on the host and then *verifies it on the device*:
``vh_build_table`` rebuilds all 65,536 entries from the closed form and the
table is accepted only if every entry matches (NaN matching NaN).  A table no
closed form reproduces is gathered from device memory (``FMT_LUT``), so any
table the reference accepts gives the reference's answer.
"""

import ctypes
import functools
import math
import re
from typing import NamedTuple, Optional, Tuple

import numpy as np
import torch

from . import _lib
from ._lib import (FMT_HW_E4M3, FMT_IDENTITY, FMT_INT, FMT_LUT, FMT_MINIFLOAT, FMT_POSIT, FMT_SIGNED,
                   FMT_STEPS, MAX_STEPS, Format)

QMAP_SIZE = 2**16

# ----------------------------------------------------------------- spec grammar
# Follows quantization/qspec.py:87-273 of the reference.


def int_range(dtype: str) -> Optional[Tuple[int, int]]:
    """``(min, max)`` of ``int<N>`` (signed) or ``uint<N>``; None otherwise."""
    m = re.fullmatch(r"(u?)int(\d+)", dtype, re.IGNORECASE)
    if not m:
        return None
    n = int(m.group(2))
    return (0, 2**n - 1) if m.group(1) else (-(2 ** (n - 1)), 2 ** (n - 1) - 1)


class FloatFormat(NamedTuple):
    bits: int
    ebits: int
    mbits: int
    ieee: bool
    max_norm: float

    @property
    def signed(self) -> bool:
        return self.bits == self.ebits + self.mbits + 1


def float_format(dtype: str) -> Optional[FloatFormat]:
    """``fp<B>_e<X>m<Y>[_ieee]``: ``B = X+Y+1`` signed, ``X+Y`` unsigned; an
    IEEE-style format (``X > 4`` or ``_ieee``) reserves its top exponent;
    ``fp8_e4m3`` reaches 448."""
    m = re.fullmatch(r"fp(\d+)_e(\d+)m(\d+)(_ieee)?", dtype, re.IGNORECASE)
    if not m:
        return None
    bits, eb, mb = (int(v) for v in m.group(1, 2, 3))
    if bits not in (eb + mb, eb + mb + 1):
        raise ValueError(f"{dtype}: {bits} bits is neither {eb}+{mb} nor {eb}+{mb}+1")
    ieee = eb > 4 or m.group(4) is not None
    emax = 2 ** (eb - 1) - 1 if ieee else 2 ** (eb - 1)
    top = 1.75 if dtype.lower() == "fp8_e4m3" else 2 - 2.0**-mb
    return FloatFormat(bits, eb, mb, ieee, 2.0**emax * top)


def posit_format(dtype: str) -> Optional[Tuple[int, int]]:
    m = re.fullmatch(r"posit(\d+)_(\d+)", dtype, re.IGNORECASE)
    return (int(m.group(1)), int(m.group(2))) if m else None


def parse_codebook_dtype(dtype: str):
    """``lut<I>[_to_<E>]`` -> ``(I, E or None)``; entries must be signed."""
    m = re.fullmatch(r"lut(\d+)(?:_to_(\w+))?", dtype)
    if not m:
        return None
    bits, entry = m.groups()
    if entry is not None:
        b, f = int_range(entry), float_format(entry)
        if (b is None or b[0] == 0) and (f is None or not f.signed):
            raise ValueError(f"{dtype}: a lookup table's entries must be a signed int or float")
    return int(bits), entry


def quant_min_max(dtype: str):
    """The representable range a qscheme implies for ``dtype``."""
    if (b := int_range(dtype)) is not None:
        return b
    if (f := float_format(dtype)) is not None:
        return -f.max_norm, f.max_norm
    if (p := posit_format(dtype)) is not None:
        mx = (2 ** (2 ** p[1])) ** (p[0] - 2)
        return -mx, mx
    if (c := parse_codebook_dtype(dtype)) is not None:
        mx = 1 if c[1] is None else quant_min_max(c[1])[1]
        return -mx, mx
    raise ValueError(f"Unsupported dtype: {dtype}")


_ABBREV = {"qmin": "quant_min", "qmax": "quant_max", "qs": "qscheme", "ahl": "amax_history_len",
           "ax": "ch_axis", "bs": "block_size", "pot": "power_2_scale", "scale": "scale_dtype",
           "othr": "outlier_threshold", "opct": "outlier_pct", "sr": "stochastic_rounding",
           "gs": "global_scale"}
_SCHEMES = ("per_tensor_symmetric", "per_channel_symmetric", "microscaling", "group_wise_affine")


def _int_or_tuple(v: str):
    v = v.strip()
    if v.startswith("(") and v.endswith(")"):
        return tuple(int(x) for x in v[1:-1].split(","))
    return int(v)


def _bool(v: str) -> bool:
    if v not in ("0", "1", "false", "true"):
        raise ValueError(f"Expected 0, 1, false or true but got '{v}'")
    return v in ("1", "true")


def _scheme(v: str) -> str:
    if v not in _SCHEMES:
        raise ValueError(f"'{v}' is not a valid QScheme")
    return v


_TYPES = {"quant_min": float, "quant_max": float, "qscheme": _scheme, "amax_history_len": int,
          "ch_axis": _int_or_tuple, "block_size": _int_or_tuple, "power_2_scale": _bool,
          "scale_dtype": str, "outlier_threshold": float, "outlier_pct": float,
          "stochastic_rounding": _bool, "global_scale": _bool}


def parse_spec(s: str) -> dict:
    """``"int8,qs=microscaling,bs=16,ax=-1"`` -> keyword dict, with the range a
    qscheme implies filled in (``qspec.py:230-273``)."""
    if not s:
        raise ValueError("String quantization_spec is None or empty")
    fields = re.split(r",(?![^()]*\))", s)
    out = {"dtype": fields[0]}
    for item in fields[1:]:
        if "=" not in item:
            raise ValueError(f"Expected key=value format but got '{item}'")
        k, v = item.split("=")
        k = _ABBREV.get(k, k)
        if k not in _TYPES:
            raise ValueError(f"Unknown argument '{k}'. Valid keys: {', '.join(_TYPES)}")
        out[k] = _TYPES[k](v)
    if out.get("qscheme") is not None:
        lo, hi = quant_min_max(out["dtype"])
        out.setdefault("quant_min", float(lo))
        out.setdefault("quant_max", float(hi))
        if out["qscheme"] in _SCHEMES[:2]:
            out.setdefault("amax_history_len", 64)
    return out


# ----------------------------------------------------------------- descriptors
def _bf16(x: float) -> float:
    return torch.tensor(x, dtype=torch.float32).bfloat16().item()


def _bf16_bits(x: float) -> int:
    return torch.tensor([x], dtype=torch.float32).bfloat16().view(torch.int16).item() & 0xFFFF


def int_format(lo: int, hi: int) -> Format:
    f = Format()
    f.kind, f.p0, f.p1 = FMT_INT, int(lo), int(hi)
    return f


def minifloat_format(ebits: int, mbits: int, signed: bool, max_norm: float) -> Format:
    f = Format()
    f.kind, f.p0, f.p1 = FMT_MINIFLOAT, ebits, mbits
    f.flags = FMT_SIGNED if signed else 0
    f.emin = 2 - 2 ** (ebits - 1)
    f.max_norm = max_norm
    f.clamp_bf16 = _bf16(max_norm)
    if (ebits, mbits, signed, max_norm) == (4, 3, True, 448.0):
        f.flags |= FMT_HW_E4M3  # OCP E4M3: the hardware converter (verified like any closed form)
    return f


def posit_fmt(nbits: int, es: int) -> Format:
    f = Format()
    f.kind, f.p0, f.p1 = FMT_POSIT, nbits, es
    f.thresh = math.pow(2, math.floor(-(nbits - 1) * (1 << es) + 2 ** (es - 1)))
    return f


def identity_format() -> Format:
    f = Format()
    f.kind = FMT_IDENTITY
    return f


def format_for_dtype(dtype: str) -> Format:
    """Closed form of ``get_quantization_map(dtype)`` for int, minifloat and
    posit dtypes (codebooks go through ``codebook_format``)."""
    if (b := int_range(dtype)) is not None:
        return int_format(*b)
    if (fl := float_format(dtype)) is not None:
        return minifloat_format(fl.ebits, fl.mbits, fl.signed, fl.max_norm)
    if (p := posit_format(dtype)) is not None:
        return posit_fmt(*p)
    raise ValueError(f"no closed form for dtype {dtype!r}")


def build_table(fmt: Format, device) -> torch.Tensor:
    """The 65,536-entry bfloat16 table of ``fmt``, built on the GPU."""
    lib = _lib.load()
    out = torch.empty(QMAP_SIZE, dtype=torch.int16, device=device)
    _lib.check(lib.vh_build_table(ctypes.byref(fmt), ctypes.c_void_p(out.data_ptr()),
                                  ctypes.c_void_p(torch.cuda.current_stream(out.device).cuda_stream)),
               "vh_build_table")
    return out.view(torch.bfloat16)


def _nf_levels(k: int, grid: Optional[torch.Tensor]) -> torch.Tensor:
    """NormalFloat levels (``dtypes/normal_float.py:4-33``), scaled to the
    grid's largest value and snapped to the nearest grid point (first on
    ties), as ``quantize_to_nf`` does (``normal_float.py:52-56``)."""
    from scipy.stats import norm

    n = 2 ** (k - 1)
    upper = norm.ppf(torch.linspace(0.9677083, 0.5, n + 1)[:-1]).tolist()
    lower = (-norm.ppf(torch.linspace(0.9677083, 0.5, n)[:-1])).tolist()
    v = torch.Tensor(upper + [0] + lower).sort().values
    v /= v.max()
    if grid is not None:
        v = v.to(grid) * grid.max()
        v = grid[torch.abs(v[:, None] - grid).argmin(-1)]
    return v


def _all_bf16() -> torch.Tensor:
    return torch.arange(QMAP_SIZE, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)


@functools.lru_cache(maxsize=None)
def _codebook_value_table(dtype: str) -> torch.Tensor:
    """Host table of a ``lut<I>[_to_<E>]`` dtype: each bfloat16 value clamped
    to the levels' range and moved to the nearest level, the first on ties,
    with the distance taken in bfloat16 (``normal_float.py:57-62``).  Built
    once per dtype on the host, like the reference's cached tables."""
    bits, entry = parse_codebook_dtype(dtype)
    grid = None
    if entry is not None:
        if (b := int_range(entry)) is not None:
            hi = b[1]
            grid = torch.arange(-hi, hi + 1, dtype=torch.float32)
        else:
            tab = quantization_map(entry, "cuda").float().cpu()
            lv = torch.unique(tab[torch.isfinite(tab)]) + 0.0
            grid = lv[lv >= -lv.max()]
    levels = _nf_levels(bits, grid).to(torch.bfloat16)
    v = _all_bf16()
    c = torch.clamp(v, min=levels.amin(), max=levels.amax())
    idx = torch.argmin(torch.abs(levels - c.unsqueeze(-1)), dim=-1)
    return levels[idx]


def quantization_map(dtype: Optional[str], device="cuda") -> torch.Tensor:
    """``get_quantization_map`` (``fake_quantize.py:68-122``): the bfloat16
    table of ``dtype`` on ``device``; None gives the identity."""
    if dtype is None:
        return build_table(identity_format(), device)
    if parse_codebook_dtype(dtype) is not None:
        return _codebook_value_table(dtype).to(device)
    return build_table(format_for_dtype(dtype), device)


def codebook_tables(dtype: str, device="cuda"):
    """What convert passes a codebook dtype's ops
    (``quantization/quantize_pt2e.py:753-791``): the int64 index table
    ``searchsorted(unique(table), table)``, the entries and their midpoints."""
    table = _codebook_value_table(dtype)
    values = torch.unique(table)
    index = torch.searchsorted(values, table).to(torch.int64)
    mid = (values[:-1] + values[1:]) / 2
    return index.to(device), values.to(device), mid.to(device)


# ----------------------------------------------------------------- classification
def _keys(bits: np.ndarray) -> np.ndarray:
    b = bits.astype(np.int64) & 0xFFFF
    return np.where(b & 0x8000, (~b) & 0xFFFF, b | 0x8000)


_ALL_BITS = np.arange(QMAP_SIZE, dtype=np.int64)
_NAN_IN = (_ALL_BITS & 0x7FFF) > 0x7F80
_KEY_ORDER = np.argsort(_keys(_ALL_BITS), kind="stable")


def _steps_from_bits(out_bits: np.ndarray) -> Optional[Format]:
    """Run-length form of a table along the value order of its inputs, or
    None when it has more than ``MAX_STEPS`` runs or its NaN inputs disagree."""
    nan_vals = np.unique(out_bits[_NAN_IN])
    if nan_vals.size != 1:
        return None
    order = _KEY_ORDER[~_NAN_IN[_KEY_ORDER]]
    seq = out_bits[order]
    starts = np.flatnonzero(np.diff(seq)) + 1
    if starts.size + 1 > MAX_STEPS:
        return None
    f = Format()
    f.kind = FMT_STEPS
    f.nsteps = int(starts.size)
    keys = _keys(order[starts])
    vals = np.concatenate([seq[:1], seq[starts]])
    for i, k in enumerate(keys):
        f.thr_key[i] = int(k)
    for i, v in enumerate(vals):
        f.val[i] = int(v)
    f.nan_out = int(nan_vals[0])
    hit = np.flatnonzero(vals == nan_vals[0])
    f.nan_level = int(hit[0]) if hit.size else 0
    return f


def _float_of_bits(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << 16).view(np.float32)


def _candidates(out_bits: np.ndarray):
    """Closed forms that might reproduce a bfloat16 value table."""
    vals = _float_of_bits(out_bits)
    fin = np.isfinite(vals)
    if np.array_equal(out_bits, _ALL_BITS & 0xFFFF):
        yield identity_format()
        return
    fv = vals[fin]
    if fv.size == 0:
        return
    if np.all(fv == np.round(fv)) and np.all(np.isnan(vals[~fin])):
        yield int_format(int(fv.min()), int(fv.max()))
    pos = fv[fv > 0]
    if pos.size:
        mx, mn = float(pos.max()), float(pos.min())
        signed = bool((fv < 0).any())
        for eb in range(1, 9):
            for mb in range(0, 11):
                for ieee in (False, True):
                    emax = 2 ** (eb - 1) - 1 if (ieee or eb > 4) else 2 ** (eb - 1)
                    top = 1.75 if (eb, mb, signed, ieee) == (4, 3, True, False) else 2 - 2.0**-mb
                    max_norm = 2.0**emax * top
                    emin = 2 - 2 ** (eb - 1)
                    if _bf16(max_norm) != mx or _bf16(2.0 ** (emin - mb)) != mn:
                        continue
                    yield minifloat_format(eb, mb, signed, max_norm)
        for n in range(3, 17):
            for es in range(0, 4):
                if float(2 ** ((n - 2) * (1 << es))) == mx:
                    yield posit_fmt(n, es)


def _same_table(a: torch.Tensor, b: torch.Tensor) -> bool:
    """Bit-equal bfloat16 tables, any NaN matching any NaN."""
    ai, bi = a.view(torch.int16), b.view(torch.int16)
    af, bf = a.view(torch.bfloat16), b.view(torch.bfloat16)
    return bool(((ai == bi) | (torch.isnan(af) & torch.isnan(bf))).all().item())


class Classified(NamedTuple):
    fmt: Format
    lut: Optional[torch.Tensor]  # keeps a FMT_LUT table alive
    index_table: bool           # entries are codebook indices (packed code == entry)


def _bf16_view_of_table(table: torch.Tensor) -> torch.Tensor:
    """The caller's table as the bfloat16 bit patterns a vmap writes into a
    bfloat16 output (index tables are converted, ``ops/quantized.py:179-182``)."""
    if table.dtype == torch.bfloat16:
        return table.contiguous()
    return table.to(torch.bfloat16).contiguous()


def classify(table: torch.Tensor) -> Classified:
    """Closed form of a 65,536-entry table, verified on the device; cached on
    the tensor (tables are shared graph buffers that are never mutated,
    ``fake_quantize.py:74-77``; an in-place change invalidates the cache)."""
    if table.dim() != 1 or table.numel() != QMAP_SIZE:
        raise ValueError(f"expected a {QMAP_SIZE}-entry 1-D quantization map, got shape {list(table.shape)}")
    cached = getattr(table, "_vh_classified", None)
    if cached is not None and cached[0] == table._version and cached[1] == table.data_ptr():
        return cached[2]
    dev_table = _bf16_view_of_table(table)
    bits = dev_table.view(torch.int16).cpu().numpy().astype(np.int64) & 0xFFFF
    index_table = not table.dtype.is_floating_point
    result = None
    for cand in ([] if index_table else list(_candidates(bits))):
        if _same_table(build_table(cand, table.device), dev_table):
            result = Classified(cand, None, False)
            break
    if result is None:
        steps = _steps_from_bits(bits)
        if steps is not None and _same_table(build_table(steps, table.device), dev_table):
            result = Classified(steps, None, index_table)
    if result is None:
        lut = dev_table.view(torch.int16).clone()
        f = Format()
        f.kind = FMT_LUT
        f.lut = lut.data_ptr()
        result = Classified(f, lut, False)
    try:
        table._vh_classified = (table._version, table.data_ptr(), result)
    except (AttributeError, RuntimeError):
        pass
    return result


def sr_levels(qmap: torch.Tensor) -> torch.Tensor:
    """The levels stochastic rounding rounds between
    (``qmap_levels``, ``ops/quantized.py:384-396``): a 65,536-entry table's
    distinct finite entries, ascending, with one +0 (float32, computed on the
    host once per table and cached on it); a smaller map is a codebook whose
    entries are the levels as given."""
    if qmap.dim() != 1 or qmap.numel() != QMAP_SIZE:
        return qmap
    cached = getattr(qmap, "_vh_sr_levels", None)
    if cached is not None and cached[0] == qmap._version and cached[1] == qmap.data_ptr():
        return cached[2]
    vals = qmap.detach().cpu().to(torch.float32).numpy()
    lv = (np.unique(vals[np.isfinite(vals)]) + np.float32(0.0)).astype(np.float32)
    levels = torch.from_numpy(lv).to(qmap.device)
    try:
        qmap._vh_sr_levels = (qmap._version, qmap.data_ptr(), levels)
    except (AttributeError, RuntimeError):
        pass
    return levels


def describe(fmt: Format) -> str:
    names = {FMT_IDENTITY: "identity", FMT_INT: "int", FMT_MINIFLOAT: "minifloat", FMT_POSIT: "posit",
             FMT_STEPS: "steps", FMT_LUT: "lut"}
    return f"{names[fmt.kind]}(p0={fmt.p0}, p1={fmt.p1}, flags={fmt.flags}, nsteps={fmt.nsteps})"
