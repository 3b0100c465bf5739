"""ctypes binding of ``libvoyager_hip.so`` (the C ABI in ``include/voyager_hip.h``).

The library is built in-tree by ``__graft_entry__.build()`` into
``voyager_amd/_lib/libvoyager_hip.so``.  Loading fails loudly when it is
missing: the package has no CPU or PyTorch fallback for its ops.
"""

import ctypes
import os
from typing import Optional

import torch

LIB_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib")
LIB_PATH = os.path.join(LIB_DIR, "libvoyager_hip.so")

VH_OK = 0

VH_BF16, VH_F32, VH_F16, VH_U8, VH_I64 = 0, 1, 2, 3, 4

FMT_IDENTITY, FMT_INT, FMT_MINIFLOAT, FMT_POSIT, FMT_STEPS, FMT_LUT = range(6)
FMT_SIGNED = 1
FMT_HW_E4M3 = 2
MAX_STEPS = 64
MAX_DIMS = 6

_DTYPE_CODE = {
    torch.bfloat16: VH_BF16,
    torch.float32: VH_F32,
    torch.float16: VH_F16,
    torch.uint8: VH_U8,
    torch.int64: VH_I64,
}


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODE[dtype]
    except KeyError:
        raise TypeError(f"voyager_amd: unsupported dtype {dtype}") from None


class Format(ctypes.Structure):
    """``vh_format``: a quantization map in closed form."""

    _fields_ = [
        ("kind", ctypes.c_int32),
        ("p0", ctypes.c_int32),
        ("p1", ctypes.c_int32),
        ("flags", ctypes.c_int32),
        ("emin", ctypes.c_int32),
        ("max_norm", ctypes.c_float),
        ("clamp_bf16", ctypes.c_float),
        ("thresh", ctypes.c_float),
        ("nsteps", ctypes.c_int32),
        ("nan_out", ctypes.c_uint16),
        ("nan_level", ctypes.c_uint16),
        ("thr_key", ctypes.c_uint16 * MAX_STEPS),
        ("val", ctypes.c_uint16 * MAX_STEPS),
        ("lut", ctypes.c_void_p),
    ]


class Param(ctypes.Structure):
    """``vh_param``: broadcast/block indexing of a scale or zero point."""

    _fields_ = [
        ("ptr", ctypes.c_void_p),
        ("dtype", ctypes.c_int32),
        ("scalar", ctypes.c_int32),
        ("div", ctypes.c_int64 * MAX_DIMS),
        ("stride", ctypes.c_int64 * MAX_DIMS),
    ]


class Codebook(ctypes.Structure):
    """``vh_codebook``: codebook tables under a region grid."""

    _fields_ = [
        ("edges", ctypes.c_void_p),
        ("nedges", ctypes.c_int32),
        ("k", ctypes.c_int32),
        ("entries", ctypes.c_void_p),
        ("entries_dtype", ctypes.c_int32),
        ("regions", ctypes.c_int64),
        ("region", Param),
    ]


_lib: Optional[ctypes.CDLL] = None

_P = ctypes.c_void_p
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64
_F32 = ctypes.c_float

_SIGNATURES = {
    "vh_last_error": ([], ctypes.c_char_p),
    "vh_abi_version": ([], _I32),
    "vh_build_table": ([ctypes.POINTER(Format), _P, _P], _I32),
    "vh_quantize": (
        [_P, _I32, ctypes.POINTER(_I64), _I32, ctypes.POINTER(Param), ctypes.POINTER(Param), _I32,
         ctypes.POINTER(Format), _P, _I32, _P],
        _I32,
    ),
    "vh_quantize_sr": ([_P, _I32, _P, _I32, _P, _P, _I32, _P, _I32, _I32, _P, _P, _I32, _P], _I32),
    "vh_stream_2to1": ([_P, _I64, _P, _P], _I32),
    "vh_quantize_codebook": (
        [_P, _I32, ctypes.POINTER(_I64), _I32, ctypes.POINTER(Param), ctypes.POINTER(Param), _I32,
         ctypes.POINTER(Codebook), _P, _P],
        _I32,
    ),
    "vh_decode_codebook": (
        [_P, _I32, ctypes.POINTER(_I64), _I32, ctypes.POINTER(Codebook), _I32, ctypes.POINTER(Param), _P, _I32, _P],
        _I32,
    ),
    "vh_block_amax": ([_P, _I32, _I64, _I64, _I64, _I64, _P, _P], _I32),
    "vh_quantize_mx8_f16": ([_P, _I64, _I64, _P, _P, _P], _I32),
    "vh_mx8_bake_f16": ([_P, _P, _I32, _I64, _I64, _P, _P, _P], _I32),
    "vh_gemm_mx8_f16": ([_P, _P, _P, _P, _I64, _I64, _I64, _P, _P, _I64, _P, _I64, _I32, _I32, _P], _I32),
    "vh_dequantize": (
        [_P, _I32, ctypes.POINTER(_I64), _I32, ctypes.POINTER(Param), ctypes.POINTER(Param), _I32,
         ctypes.POINTER(Format), ctypes.POINTER(Format), _P, _I32, _P],
        _I32,
    ),
    "vh_quantize_mx": (
        [_P, _I32, _I64, _I64, _I64, _I64, _F32, _I32, ctypes.POINTER(Format), _P, _I32,
         ctypes.POINTER(Format), _P, _I32, _I32, _P, _I32, _P, _P],
        _I32,
    ),
    "vh_quantize_affine": (
        [_P, _I32, _I64, _I64, _I64, _I64, _F32, _F32, ctypes.POINTER(Format), ctypes.POINTER(Format),
         _P, _P, _P, _I32, _P],
        _I32,
    ),
    "vh_decode_bytes": ([_P, _I64, _P, _P, _P], _I32),
    # vh_gemm takes a vh_gemm_desc*; voyager_amd.gemm.GemmDesc mirrors it.
    "vh_gemm": ([_P, _P], _I32),
    "vh_gemm_workspace_bytes": ([_P], _I64),
    "vh_gemm_plan": ([_P, ctypes.POINTER(_I32), ctypes.POINTER(_I32), ctypes.POINTER(_I32)], _I32),
    "vh_quantize_mx_rows16": ([_P, _I32, _I64, _I64, _I64, ctypes.c_float, ctypes.POINTER(Format),
                               ctypes.POINTER(Format), _P, _P, _P, _P], _I32),
    "vh_pack_nf4": ([_P, _I64, _I64, _P, _P], _I32),
    # x_levels, x_scale, M, w_packed, w_scale, w_scale_fmt, levels16 (host), N, K, epilogue*, y, stream
    "vh_gemv_nf4": ([_P, _P, _I64, _P, _P, ctypes.POINTER(Format), _P, _I64, _I64, _P, _P, _P], _I32),
    "vh_gemm_nf4": ([_P, _P, ctypes.POINTER(Format), _I64, _P, _P, ctypes.POINTER(Format), _P, _I64, _I64, _P,
                     _P, _I64, _I32, _I32, _P, _I64, _P], _I32),
    "vh_gemm_nf4_plan": ([_I64, _I64, _I64, _P, _P, _P], _I32),
    "vh_nf4_decode_bf16": ([_P, _P, ctypes.POINTER(Format), _I64, _P, _P, ctypes.POINTER(Format), _P, _I64, _I64,
                            _P, _P, _P], _I32),
    "vh_gemv_nf4_m1": ([_P, _I32, ctypes.c_float, ctypes.POINTER(Format), ctypes.POINTER(Format), _P, _P,
                        ctypes.POINTER(Format), _P, _I64, _I64, _P, _P, _P], _I32),
    # decoder-layer decode step
    "vh_rmsnorm_mx8": ([_P, _P, _I64, _I64, _F32, _P, _P, _P, _P], _I32),
    "vh_mx8_bake": ([_P, _P, _I32, _I64, _I64, _I32, _P, _P, _P, _P, _P], _I32),
    "vh_gemv_mx8": ([_P, _I64, _I64, _P, _P, _I64, _I32, _I32, _P, _P, _P, _P, _P, _P, _P], _I32),
    "vh_kivi_bake": ([_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _P, _P], _I32),
    "vh_kivi_bake_residual": ([_P, _P, _I64, _I64, _P, _P, _P], _I32),
    # vh_kivi_attention takes a vh_kivi_desc*; voyager_amd.decode.KiviDesc mirrors it.
    "vh_kivi_attention": ([_P, _P], _I32),
    "vh_conv_im2col": ([_P, _I32, _P, _I32, _I32, _I64, _P, _P], _I32),
    "vh_conv_pack_weight": ([_P, _I32, _P, _I32, _I32, _I64, _P, _P], _I32),
    "vh_nhwc_to_nchw": ([_P, _I32, _I64, _I64, _I64, _P, _P], _I32),
    "vh_filter_outlier": ([_P, _I32, _I64, _I64, _I64, _F32, _I64, _I32, _P, _P, _P, _P, _P, _I64, _P], _I32),
    "vh_filter_outlier_workspace_bytes": ([_I64, _I64, _I64], _I64),
    "vh_filter_outlier_noalloc": ([_P, _I32, _I64, _I64, _I64, _F32, _I64, _I32, _P, _P, _P, _P, _P], _I32),
    "vh_slice_csr": ([_P, _I32, _P, _P, _I64, _I64, _I32, _I64, _I64, _I64, _P, _P, _P, _P], _I32),
    "vh_spmm_csr": ([_P, _I32, _P, _P, _I64, _I64, _I64, _P, _I32, _I32, _I64, _I64, _I64, _P, _P, _I32, _P, _P],
                    _I32),
}

DECODE_ERR_FP16_RANGE = 1
DECODE_ERR_WEIGHT_RANGE = 2
DECODE_ERR_KV_CODE = 4
DECODE_ERR_KV_FULL = 8
DECODE_ERR_KV_STATE = 16
KIVI_RES_CAP = 128
FILTER_NOALLOC_SCRATCH_BYTES = 8 << 20
GEMV_STORE, GEMV_RESIDUAL, GEMV_SWIGLU = 0, 1, 2

#: ``VH_ABI_VERSION`` of the header these bindings follow.
ABI_VERSION = 2

#: Every symbol ``include/voyager_hip.h`` declares.
EXPORTED = tuple(_SIGNATURES)


def load() -> ctypes.CDLL:
    """Load the HIP library once; raise if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"voyager_amd: HIP library not built ({LIB_PATH} missing); "
            "run __graft_entry__.build() first"
        )
    lib = ctypes.CDLL(LIB_PATH)
    lib.vh_abi_version.restype = _I32
    if lib.vh_abi_version() != ABI_VERSION:
        raise RuntimeError(f"voyager_amd: {LIB_PATH} has ABI version {lib.vh_abi_version()}, this package binds "
                           f"version {ABI_VERSION}; rebuild it with __graft_entry__.build()")
    for name, (args, res) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    _lib = lib
    return lib


def check(status: int, what: str) -> None:
    if status != VH_OK:
        msg = load().vh_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed (status {status}): {msg}")


def stream_of(t: torch.Tensor) -> int:
    """The current HIP stream of ``t``'s device, as a raw handle."""
    return torch.cuda.current_stream(t.device).cuda_stream


def ptr(t: Optional[torch.Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())
