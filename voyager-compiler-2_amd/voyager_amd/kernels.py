"""Bind the package's kernels onto a ``quantized_ops`` library.

Importing this module defines nothing.  :func:`register` binds the CUDA-key
kernels (which launch the HIP library through its C ABI) -- and, on request,
the fake kernels -- onto any ``torch.library.Library`` whose namespace has the
reference's schemas defined: the reference's own ``quantized_ops_lib``
(``src/voyager_compiler/ops/quantized.py:97``), or the standalone namespace
``voyager_amd.library`` defines.
"""

from typing import Iterable, List, Optional

import torch

from . import conv, gemm, ops, sparse, twins  # noqa: F401  (fill the registry; no side effects)
from .registry import CUDA_KERNELS, FAKE_KERNELS


def names() -> List[str]:
    """Every op the package has a CUDA kernel for."""
    return sorted(CUDA_KERNELS)


def register(lib: torch.library.Library, *, fakes: bool = False, allow_override: bool = False,
             only: Optional[Iterable[str]] = None) -> List[str]:
    """Register the CUDA kernels of the ops in ``only`` (default: all of
    them) on ``lib``, plus their fake kernels when ``fakes``.

    ``allow_override`` replaces kernels already registered from Python for
    the same op and dispatch key, e.g. the reference's torch.compile CUDA
    kernels of ``quantize`` / ``dequantize`` / ``quantize_mx`` /
    ``quantize_affine`` (``ops/quantized.py:100-109``).  Returns the ops
    registered."""
    todo = names() if only is None else list(only)
    for name in todo:
        if name not in CUDA_KERNELS:
            raise KeyError(f"voyager_amd has no kernel for quantized_ops.{name}")
    for name in todo:
        lib.impl(name, CUDA_KERNELS[name], "CUDA", allow_override=allow_override)
        if fakes and name in FAKE_KERNELS:
            torch.library.register_fake(f"{lib.ns}::{name}", FAKE_KERNELS[name], lib=lib,
                                        allow_override=allow_override)
    return todo
