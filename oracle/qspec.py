"""Spec-string vocabulary, restated for the oracle (test infrastructure only).

Follows ``quantization/qspec.py:87-273`` of the reference.
"""

import re
from typing import NamedTuple, Optional, Tuple


def int_range(dtype: str) -> Optional[Tuple[int, int]]:
    """``(min, max)`` of ``int<N>`` / ``uint<N>``; ``qspec.py:87-102``."""
    m = re.fullmatch(r"(u?)int(\d+)", dtype, re.IGNORECASE)
    if m is None:
        return None
    n = int(m.group(2))
    if m.group(1):
        return 0, 2**n - 1
    return -(2 ** (n - 1)), 2 ** (n - 1) - 1


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
    """Minifloat ``fp<B>_e<X>m<Y>[_ieee]``; ``qspec.py:122-156``.

    More than four exponent bits (or ``_ieee``) reserve the top exponent;
    ``fp8_e4m3`` gives up only the all-ones mantissa (max 448).
    """
    m = re.fullmatch(r"fp(\d+)_e(\d+)m(\d+)(_ieee)?", dtype, re.IGNORECASE)
    if m is None:
        return None
    bits, ebits, mbits = (int(g) for g in m.group(1, 2, 3))
    if bits not in (ebits + mbits, ebits + mbits + 1):
        raise ValueError(f"{dtype}: bad width")
    ieee = ebits > 4 or m.group(4) is not None
    emax = 2 ** (ebits - 1) - 1 if ieee else 2 ** (ebits - 1)
    if dtype.lower() == "fp8_e4m3":
        max_norm = 2.0**emax * 1.75
    else:
        max_norm = 2.0**emax * (2 - 2.0**-mbits)
    return FloatFormat(bits, ebits, mbits, ieee, max_norm)


def posit_format(dtype: str) -> Optional[Tuple[int, int]]:
    """``posit<N>_<es>``; ``qspec.py:159-171``."""
    m = re.fullmatch(r"posit(\d+)_(\d+)", dtype, re.IGNORECASE)
    if m is None:
        return None
    return int(m.group(1)), int(m.group(2))


def parse_codebook_dtype(dtype: str):
    """``lut<I>[_to_<E>]`` -> ``(I, E or None)``; ``qspec.py:196-227``."""
    m = re.fullmatch(r"lut(\d+)(?:_to_(\w+))?", dtype)
    if m is None:
        return None
    bits, entry = m.groups()
    if entry is not None:
        bounds = int_range(entry)
        fmt = float_format(entry)
        if (bounds is None or bounds[0] == 0) and (fmt is None or not fmt.signed):
            raise ValueError(f"{dtype}: entries must be signed")
    return int(bits), entry


def quant_min_max(dtype: str):
    """Representable range of a dtype; ``qspec.py:174-193``."""
    if (b := int_range(dtype)) is not None:
        return b
    if (f := float_format(dtype)) is not None:
        return -f.max_norm, f.max_norm
    if (p := posit_format(dtype)) is not None:
        bits, es = p
        mx = (2 ** (2**es)) ** (bits - 2)
        return -mx, mx
    if (c := parse_codebook_dtype(dtype)) is not None:
        mx = 1 if c[1] is None else quant_min_max(c[1])[1]
        return -mx, mx
    raise ValueError(f"Unsupported dtype: {dtype}")
