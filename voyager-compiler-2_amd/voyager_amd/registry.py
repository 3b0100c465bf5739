"""Collects the package's operator kernels without registering anything.

Modules that implement ``quantized_ops`` operators mark their CUDA-key and
fake kernels with :func:`cuda_kernel` / :func:`fake_kernel`; nothing touches
the torch dispatcher until :func:`voyager_amd.kernels.register` binds them
onto a ``torch.library.Library`` the caller owns.
"""

from typing import Callable, Dict

#: op name -> the CUDA-key kernel (launches the HIP library)
CUDA_KERNELS: Dict[str, Callable] = {}
#: op name -> the fake (meta) kernel used by FX shape propagation
FAKE_KERNELS: Dict[str, Callable] = {}


def cuda_kernel(name: str):
    def mark(fn):
        if name in CUDA_KERNELS:
            raise RuntimeError(f"two CUDA kernels for quantized_ops.{name}")
        CUDA_KERNELS[name] = fn
        return fn

    return mark


def fake_kernel(name: str):
    def mark(fn):
        if name in FAKE_KERNELS:
            raise RuntimeError(f"two fake kernels for quantized_ops.{name}")
        FAKE_KERNELS[name] = fn
        return fn

    return mark
