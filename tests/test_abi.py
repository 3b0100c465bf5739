"""The C ABI without a GPU: the built library loads, exports every function
``include/voyager_hip.h`` declares, the package's ctypes table names exactly
those, and the host-side entry points that compute nothing on the device
answer (the ABI version, the error getter, workspace sizes)."""

import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "voyager_hip.h")


def _declared():
    text = open(HEADER).read()
    return set(re.findall(r"^(?:const char\*|int|int64_t)\s+(vh_\w+)\(", text, re.M))


def _library():
    from voyager_amd import _lib

    assert os.path.exists(_lib.LIB_PATH), f"{_lib.LIB_PATH} is not built (run __graft_entry__.build())"
    return ctypes.CDLL(_lib.LIB_PATH)


def test_header_declares_the_entry_points():
    names = _declared()
    assert len(names) >= 26
    for must in ("vh_quantize", "vh_quantize_mx", "vh_dequantize", "vh_quantize_affine", "vh_gemm",
                 "vh_quantize_sr", "vh_filter_outlier", "vh_spmm_csr", "vh_conv_im2col"):
        assert must in names


def test_library_exports_every_declared_symbol():
    lib = _library()
    missing = [n for n in sorted(_declared()) if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"


def test_ctypes_table_matches_the_header():
    from voyager_amd import _lib

    assert set(_lib.EXPORTED) == _declared()


def test_host_side_entry_points():
    lib = _library()
    lib.vh_abi_version.restype = ctypes.c_int32
    from voyager_amd import _lib

    macro = re.search(r"#define VH_ABI_VERSION (\d+)", open(HEADER).read())
    assert macro and int(macro.group(1)) == _lib.ABI_VERSION == lib.vh_abi_version()
    lib.vh_last_error.restype = ctypes.c_char_p
    assert isinstance(lib.vh_last_error(), bytes)
    lib.vh_filter_outlier_workspace_bytes.restype = ctypes.c_int64
    lib.vh_filter_outlier_workspace_bytes.argtypes = [ctypes.c_int64] * 3
    small = lib.vh_filter_outlier_workspace_bytes(1, 4, 100)
    big = lib.vh_filter_outlier_workspace_bytes(3, 2048, 14336)
    assert 0 < small < big and big % 16 == 0
    assert lib.vh_filter_outlier_workspace_bytes(-1, 4, 4) == 0


@pytest.mark.parametrize("fn", ["vh_quantize", "vh_gemm", "vh_spmm_csr", "vh_filter_outlier", "vh_quantize_sr"])
def test_ctypes_signatures_are_bound(fn):
    from voyager_amd import _lib

    lib = _lib.load()
    f = getattr(lib, fn)
    assert f.restype is not None and f.argtypes is not None and len(f.argtypes) >= 2
