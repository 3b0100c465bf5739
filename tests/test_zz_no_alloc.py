"""vh_filter_outlier_noalloc through the C ABI against vh_filter_outlier
(the same filter with a caller's workspace): bit-identical CSR arrays and
inliers on two calls in a row, the second smaller (the scratch keeps the
first call's contents), plus the size limit and its error."""

import ctypes

import pytest
import torch

from voyager_amd import _lib
from voyager_amd._lib import dtype_code, load

pytestmark = pytest.mark.gpu


def _outputs(shape, cap, dtype, dev):
    *batch, rows, cols = shape
    return (torch.full((*batch, cap), 7, dtype=dtype, device=dev),
            torch.full((*batch, cap), -7, dtype=torch.int32, device=dev),
            torch.full((*batch, rows + 1), -7, dtype=torch.int32, device=dev),
            torch.full(shape, 3, dtype=dtype, device=dev))


def _run(x, thr, cap, offset, noalloc):
    lib = load()
    *batch, rows, cols = x.shape
    nb = 1
    for n in batch:
        nb *= n
    data, indices, indptr, inl = _outputs(list(x.shape), cap, x.dtype, x.device)
    stream = ctypes.c_void_p(torch.cuda.current_stream(x.device).cuda_stream)
    common = (ctypes.c_void_p(x.data_ptr()), dtype_code(x.dtype), nb, rows, cols, ctypes.c_float(thr), cap, offset,
              ctypes.c_void_p(data.data_ptr()), ctypes.c_void_p(indices.data_ptr()),
              ctypes.c_void_p(indptr.data_ptr()), ctypes.c_void_p(inl.data_ptr()))
    if noalloc:
        st = lib.vh_filter_outlier_noalloc(*common, stream)
    else:
        nbytes = lib.vh_filter_outlier_workspace_bytes(nb, rows, cols)
        work = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=x.device)
        st = lib.vh_filter_outlier(*common, ctypes.c_void_p(work.data_ptr()), work.numel(), stream)
    _lib.check(st, "filter")
    return data, indices, indptr, inl


def _same(a, b, what):
    for u, v, name in zip(a, b, ("data", "indices", "indptr", "inliers")):
        assert torch.equal(u.view(torch.int16) if u.dtype == torch.bfloat16 else u,
                           v.view(torch.int16) if v.dtype == torch.bfloat16 else v), f"{what}: {name} differs"


def test_noalloc_matches_workspace_entry_point_twice():
    g = torch.Generator().manual_seed(5)
    # first call: many outliers in every segment (more than the 16 each
    # segment stages), batch 2, 3.5 segments per row
    big = (torch.randn(2, 700, 7000, generator=g) * 3).bfloat16().cuda()
    exp = _run(big, 2.0, 400_000, 5, noalloc=False)
    got = _run(big, 2.0, 400_000, 5, noalloc=True)
    torch.cuda.synchronize()
    _same(got, exp, "first call")
    # second call: smaller, few outliers, ragged columns, fp32; the scratch
    # still holds the first call's counts and staged values
    small = torch.randn(130, 2050, generator=g).cuda()
    small[::7, ::13] *= 40
    exp = _run(small, 30.0, 900, 0, noalloc=False)
    got = _run(small, 30.0, 900, 0, noalloc=True)
    torch.cuda.synchronize()
    _same(got, exp, "second call")
    assert int(got[2][-1]) > 16  # outliers were found


def test_noalloc_rejects_sizes_beyond_its_scratch():
    lib = load()
    rows, cols = 40_000, 14_336
    need = lib.vh_filter_outlier_workspace_bytes(1, rows, cols)
    assert need > _lib.FILTER_NOALLOC_SCRATCH_BYTES
    x = torch.zeros(8, dtype=torch.bfloat16, device="cuda")  # never read: the size check comes first
    st = lib.vh_filter_outlier_noalloc(ctypes.c_void_p(x.data_ptr()), dtype_code(x.dtype), 1, rows, cols,
                                       ctypes.c_float(1.0), 10, 0, ctypes.c_void_p(x.data_ptr()),
                                       ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(x.data_ptr()),
                                       ctypes.c_void_p(x.data_ptr()), None)
    assert st == 1
    assert b"fixed scratch" in lib.vh_last_error()


_CAPTURE_CHILD = r"""
import ctypes, sys
import torch
from voyager_amd import _lib
from voyager_amd._lib import dtype_code, load

lib = load()
dev = torch.device("cuda:0")
g = torch.Generator().manual_seed(9)
x = (torch.randn(300, 4100, generator=g) * 3).bfloat16().to(dev)
rows, cols, cap, thr = 300, 4100, 20_000, 2.5

def outputs():
    return (torch.full((cap,), 7, dtype=torch.bfloat16, device=dev), torch.full((cap,), -7, dtype=torch.int32, device=dev),
            torch.full((rows + 1,), -7, dtype=torch.int32, device=dev), torch.full((rows, cols), 3, dtype=torch.bfloat16, device=dev))

def args(o, stream):
    return (ctypes.c_void_p(x.data_ptr()), dtype_code(x.dtype), 1, rows, cols, ctypes.c_float(thr), cap, 0,
            *[ctypes.c_void_p(t.data_ptr()) for t in o], ctypes.c_void_p(stream))

got = outputs()
graph = torch.cuda.CUDAGraph()
side = torch.cuda.Stream()
side.wait_stream(torch.cuda.current_stream())
with torch.cuda.stream(side):
    with torch.cuda.graph(graph):
        # the library's first call in this process, made under capture
        st = lib.vh_filter_outlier_noalloc(*args(got, torch.cuda.current_stream().cuda_stream))
_lib.check(st, "noalloc under capture")
torch.cuda.current_stream().wait_stream(side)
work = torch.empty(lib.vh_filter_outlier_workspace_bytes(1, rows, cols), dtype=torch.uint8, device=dev)
for rep in range(3):
    for t, v in zip(got, (7, -7, -7, 3)):
        t.fill_(v)
    exp = outputs()
    st = lib.vh_filter_outlier(*args(exp, torch.cuda.current_stream().cuda_stream)[:-1],
                               ctypes.c_void_p(work.data_ptr()), work.numel(),
                               ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    _lib.check(st, "workspace entry point")
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    for u, v, name in zip(got, exp, ("data", "indices", "indptr", "inliers")):
        a = u.view(torch.int16) if u.dtype == torch.bfloat16 else u
        b = v.view(torch.int16) if v.dtype == torch.bfloat16 else v
        assert torch.equal(a, b), f"replay {rep}: {name} differs"
    assert int(got[2][-1]) > 16
print("ok", flush=True)
"""


def test_noalloc_first_call_under_graph_capture():
    """In a fresh interpreter, the entry point's first call (which looks up
    the device's scratch address) is made under HIP graph capture; three
    replays, each after an eager call of the workspace entry point, equal
    that call's outputs bit for bit."""
    import os
    import subprocess
    import sys

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, PYTHONPATH=os.pathsep.join([root, os.path.join(root, "voyager-compiler-2_amd")]))
    print("noalloc capture child: start", flush=True)
    r = subprocess.run([sys.executable, "-c", _CAPTURE_CHILD], capture_output=True, text=True, env=env, timeout=240)
    assert r.returncode == 0 and r.stdout.strip().endswith("ok"), (r.stdout[-1000:], r.stderr[-3000:])
