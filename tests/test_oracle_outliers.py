"""Pins of the oracle's outlier (CSR) ops against what fixes them without the
reference: a brute-force row-major scan in plain Python (which elements are
outliers, their slot order, the capacity cut, the clamped row pointers, the
padding), dense reconstruction, slices of the dense matrix, and float64
products of the densified CSR (``ops/quantized.py:1286-1645``)."""

import math
import struct

import numpy as np
import pytest
import torch

from oracle import ops as O
from oracle import tables as T


def _bf16_round(f: float) -> float:
    """float32(f) rounded to bfloat16, half to even, in integer arithmetic."""
    u = struct.unpack("<I", struct.pack("<f", f))[0]
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return struct.unpack("<f", struct.pack("<I", u << 16))[0]


def _brute_csr(mat, thr, cap):
    """Row-major scan of a 2-D list of floats: (data, indices, indptr) with
    the reference's capacity rules, built entry by entry."""
    entries, counts = [], []
    for row in mat:
        n = 0
        for j, v in enumerate(row):
            if abs(v) >= thr and v != 0.0:
                entries.append((v, j))
                n += 1
        counts.append(n)
    indptr, run = [0], 0
    for n in counts:
        run += n
        indptr.append(min(run, cap))
    kept = entries[:cap]
    data = [v for v, _ in kept] + [0.0] * (cap - len(kept))
    idx = [j for _, j in kept] + [-1] * (cap - len(kept))
    return data, idx, indptr


def _rand(shape, seed, scale=1.0, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(dtype)


@pytest.mark.parametrize("shape,thr,pct", [((6, 10), 1.5, 0.2), ((6, 10), 0.5, 0.2), ((2, 3, 7), 1.0, 0.3),
                                           ((4, 8), 10.0, 0.1), ((5, 5), 1.2, 0.0)])
def test_filter_outlier_matches_row_major_scan(shape, thr, pct):
    x = _rand(shape, 1)
    x.view(-1)[3] = 0.0
    data, idx, indptr, inl = O.filter_outlier(x, thr, pct)
    rows, cols = shape[-2:]
    cap = int(rows * cols * pct)
    thr_b = _bf16_round(thr)
    mats = x.float().reshape(-1, rows, cols).tolist()
    for b, mat in enumerate(mats):
        d, i, p = _brute_csr(mat, thr_b, cap)
        assert data.reshape(len(mats), cap)[b].float().tolist() == d
        assert idx.reshape(len(mats), cap)[b].tolist() == i
        assert indptr.reshape(len(mats), rows + 1)[b].tolist() == p
    assert data.dtype == x.dtype and idx.dtype == torch.int32 and indptr.dtype == torch.int32
    flat = x.float().reshape(-1).tolist()
    want_inl = [0.0 if abs(v) >= thr_b else v for v in flat]
    assert inl.float().reshape(-1).tolist() == want_inl


def test_filter_outlier_dense_reconstruction():
    """With room for every outlier, inliers + the densified CSR == input,
    bit for bit, and the first row pointer is 0."""
    x = _rand((3, 16, 40), 2, 2.0)
    data, idx, indptr, inl = O.filter_outlier(x, 3.0, 0.5)
    dense = inl.clone()
    for b in range(3):
        assert int(indptr[b, 0]) == 0
        for r in range(16):
            for j in range(int(indptr[b, r]), int(indptr[b, r + 1])):
                assert dense[b, r, int(idx[b, j])] == 0
                dense[b, r, int(idx[b, j])] = data[b, j]
    assert torch.equal(dense.view(torch.int16), x.view(torch.int16))


def test_filter_outlier_threshold_rounds_to_input_dtype():
    """3.140625 is bf16(3.141): an outlier of a bf16 tensor, not of a float32
    one; NaN is never an outlier; -0 and 0 are outliers of a threshold <= 0
    but stay out of the CSR."""
    xb = torch.tensor([[3.140625, 1.0]], dtype=torch.bfloat16)
    assert O.filter_outlier(xb, 3.141, 1.0)[2].tolist() == [0, 1]
    assert O.filter_outlier(xb.float(), 3.141, 1.0)[2].tolist() == [0, 0]
    xs = torch.tensor([[float("nan"), -0.0, 0.0, 2.0]], dtype=torch.bfloat16)
    data, idx, indptr, inl = O.filter_outlier(xs, -1.0, 1.0)
    assert indptr.tolist() == [0, 1] and idx.tolist() == [3, -1, -1, -1]
    assert torch.isnan(inl[0, 0]) and inl[0, 1:].tolist() == [0.0, 0.0, 0.0]


def test_quantize_mx_outlier_quantizes_the_inliers():
    x = _rand((8, 64), 3, 2.0)
    tab = T.quantization_map("int8")
    data, idx, indptr, scale, codes = O.quantize_mx_outlier(x, tab, [-1], 16, 127.0, True, threshold=4.0,
                                                            max_pct=0.05, indptr_offset=7)
    d2, i2, p2, inl = O.filter_outlier(x, 4.0, 0.05)
    s_ref, c_ref = O.quantize_mx(inl, tab, [-1], 16, 127.0, True)
    assert torch.equal(data, d2) and torch.equal(idx, i2) and torch.equal(indptr, p2 + 7)
    assert torch.equal(scale, s_ref) and torch.equal(codes, c_ref)


def _dense_of(data, idx, indptr, rows, cols):
    m = np.zeros((rows, cols))
    for r in range(rows):
        for j in range(int(indptr[r]), int(indptr[r + 1])):
            m[r, int(idx[j])] = float(data[j])
    return m


@pytest.mark.parametrize("dim,start,end,factor", [(0, 2, 7, 1.0), (0, 0, 12, 0.25), (1, 5, 30, 1.0),
                                                  (1, 0, 40, 0.1), (-1, 10, 11, 1.0), (0, 4, 4, 1.0)])
def test_slice_csr_matches_dense_slice(dim, start, end, factor):
    x = _rand((12, 40), 4, 2.0)
    data, idx, indptr, _ = O.filter_outlier(x, 2.0, 0.2)
    nd, ni, np_ = O.slice_csr_tensor(data, idx, indptr, dim, start, end, factor)
    cap = int(data.shape[0] * factor)
    assert nd.shape[0] == ni.shape[0] == cap
    dense = _dense_of(data, idx, indptr, 12, 40)
    part = dense[start:end] if dim == 0 else dense[:, start:end]
    d, i, p = _brute_csr(part.tolist(), 0.0, cap)
    assert ni.tolist() == i and np_.tolist() == p
    assert nd.float().tolist() == d


def test_spmm_csr_matches_float64_product():
    """Both layouts, a batch of CSR matrices, B decoded from int8 codes with
    power-of-two block scales; float64 product of the densified CSR."""
    x = _rand((2, 9, 64), 5, 2.0)
    data, idx, indptr, _ = O.filter_outlier(x, 1.5, 0.3)
    w = _rand((24, 64), 6, 0.02)
    tab = T.quantization_map("int8")
    ws, wc = O.quantize_mx(w, tab, [-1], 16, 127.0, True)
    wd = O.dequantize_mx_parts(wc, ws, None, 16).double().numpy()
    for layout, B, S in (("kc", wc, ws), ("ck", wc.mT.contiguous(), ws.mT.contiguous())):
        got = O.spmm_csr(data, idx, indptr, B, S, None, 16, layout, out_dtype=torch.float32)
        assert got.shape == (2, 9, 24) and got.dtype == torch.float32
        for b in range(2):
            ref = _dense_of(data[b], idx[b], indptr[b], 9, 64) @ wd.T
            np.testing.assert_allclose(got[b].double().numpy(), ref, rtol=1e-6, atol=1e-6 * np.abs(ref).max())


def test_spmm_csr_rebases_and_clamps_row_pointers():
    """Row pointers that start past 0 name a span of data; columns past B
    are clamped to its last row (``ops/quantized.py:1620-1631``)."""
    data = torch.tensor([1.0, 2.0, 3.0, 0.0])
    idx = torch.tensor([0, 5, 1, -1], dtype=torch.int32)  # 5 is past K = 3
    indptr = torch.tensor([10, 11, 13], dtype=torch.int32)
    B = torch.arange(6, dtype=torch.float32).reshape(2, 3)  # "kc": [N = 2, K = 3]
    got = O.spmm_csr(data, idx, indptr, B, weight_layout="kc")
    Bt = B.T.double().numpy()
    ref = np.stack([1.0 * Bt[0], 2.0 * Bt[2] + 3.0 * Bt[1]])
    np.testing.assert_array_equal(got.double().numpy(), ref)


def test_linear_mx_outlier_term_matches_float64():
    """quantize_mx_outlier -> linear_mx with the CSR: float64 of
    (deq(codes) + dense(CSR)) deq(W)^T, rounded to bf16 (1e-2 bar)."""
    x = _rand((16, 128), 7, 1.0)
    x[3, 5] = 40.0
    x[9, 100] = -33.0
    tab = T.quantization_map("int8")
    w = _rand((48, 128), 8, 0.02)
    ws, wc = O.quantize_mx(w, tab, [-1], 16, 127.0, True)
    data, idx, indptr, xs, xc = O.quantize_mx_outlier(x, tab, [-1], 16, 127.0, True, threshold=3.0, max_pct=0.05)
    y = O.linear_mx(xc, wc, input_scale=xs, weight_scale=ws, block_size=16, A_data=data, A_indices=idx,
                    A_indptr=indptr)
    a = O.dequantize_mx_parts(xc, xs, None, 16).double().numpy() + _dense_of(data, idx, indptr, 16, 128)
    ref = a @ O.dequantize_mx_parts(wc, ws, None, 16).double().numpy().T
    err = np.abs(y.double().numpy() - ref).max() / np.abs(ref).max()
    assert err < 1e-2
    y0 = O.linear_mx(xc, wc, input_scale=xs, weight_scale=ws, block_size=16)
    assert not torch.equal(y, y0)  # the outliers count
