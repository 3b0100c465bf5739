"""The outlier (CSR) path on the GPU against the oracle on the same inputs:
filter_outlier / quantize_mx_outlier and slice_csr_tensor bit-exact (data,
indices, row pointers, inliers, scales and codes); spmm_csr within float32
summation-order error (it sums each output in stored order, torch's sparse
mm in its own); linear_mx / matmul_mx with the CSR term within the 1e-2 GEMM
bar (``ops/quantized.py:651-819, 1286-1645``)."""

import pytest
import torch

import voyager_amd.library  # noqa: F401  (defines quantized_ops)
from helpers import assert_same_bits, max_rel_err
from oracle import ops as O
from oracle import tables as T

pytestmark = pytest.mark.gpu

Q = torch.ops.quantized_ops
DEV = "cuda"


def _rand(shape, seed, scale=1.0, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(dtype)


def _with_outliers(shape, seed, rate=0.001, factor=20.0):
    """N(0,1) with a `rate` fraction of entries multiplied by `factor`, the
    outlier pattern of the MXINT8 benchmark input."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=g)
    x = torch.where(torch.rand(*shape, generator=g) < rate, x * factor, x)
    return x.bfloat16()


def _check_filter(got, exp, what):
    for name, g, e in zip(("data", "indices", "indptr", "inliers"), got, exp):
        assert_same_bits(g, e, f"{what} {name}")


FILTER_CASES = [
    ("bf16 vector rows", (64, 256), torch.bfloat16, 2.5, 0.01),
    ("bf16 batched, ragged rows", (3, 33, 70), torch.bfloat16, 1.0, 0.05),
    ("fp16", (17, 64), torch.float16, 1.5, 0.1),
    ("fp32 vector rows", (9, 130), torch.float32, 1.2, 0.1),
    ("fp32 ragged rows", (5, 7), torch.float32, 0.8, 0.3),
    ("capacity overflow", (32, 96), torch.bfloat16, 0.5, 0.01),
    ("no capacity", (8, 16), torch.bfloat16, 1.0, 0.0),
    ("one row", (1, 4096), torch.bfloat16, 2.0, 0.02),
    ("no outliers", (16, 64), torch.bfloat16, 100.0, 0.01),
    ("config-1 activations", (256, 4096), torch.bfloat16, 6.0, 0.002),
]


@pytest.mark.parametrize("what,shape,dtype,thr,pct", FILTER_CASES, ids=[c[0] for c in FILTER_CASES])
def test_filter_outlier_bit_exact(what, shape, dtype, thr, pct):
    x = _with_outliers(shape, 11, rate=0.01, factor=8.0).to(dtype)
    exp = O.filter_outlier(x, thr, pct)
    got = Q.filter_outlier(x.to(DEV), thr, pct)
    _check_filter(got, exp, what)


def test_filter_outlier_specials():
    """NaN stays an inlier; +-inf are outliers; 0 and -0 reach a threshold
    <= 0 but stay out of the stream; the threshold rounds to bf16 first."""
    x = _rand((4, 24), 12)
    x[0, :6] = torch.tensor([float("nan"), float("inf"), -float("inf"), 0.0, -0.0, 3.140625])
    for thr in (-1.0, 3.141, 1.0):
        exp = O.filter_outlier(x, thr, 0.5)
        got = Q.filter_outlier(x.to(DEV), thr, 0.5)
        _check_filter(got, exp, f"specials thr={thr}")


def test_filter_outlier_large_matrix_reconstructs():
    """A [2048, 14336] prefill activation at 0.1% outliers: the stream and
    the inliers rebuild the input exactly, and equal the oracle's."""
    x = _with_outliers((2048, 14336), 13)
    data, idx, indptr, inl = Q.filter_outlier(x.to(DEV), 5.0, 0.002)
    n = int(indptr[-1])
    assert 0 < n < data.numel() and int(indptr[0]) == 0
    rows = torch.repeat_interleave(torch.arange(2048, device=DEV), (indptr[1:] - indptr[:-1]).long())
    rebuilt = inl.clone()
    rebuilt[rows, idx[:n].long()] = data[:n]
    assert torch.equal(rebuilt.view(torch.int16), x.to(DEV).view(torch.int16))
    assert bool((idx[n:] == -1).all()) and bool((data[n:] == 0).all())
    _check_filter((data, idx, indptr, inl), O.filter_outlier(x, 5.0, 0.002), "large")


@pytest.mark.parametrize("fmt", ["int8", "nf4"])
@pytest.mark.parametrize("offset", [0, 123])
def test_quantize_mx_outlier_bit_exact(fmt, offset):
    x = _with_outliers((2, 48, 512), 14)
    if fmt == "int8":
        args = (T.quantization_map("int8"), [-1], 16, 127.0, True)
        kw = {}
    else:
        index, _, mid = T.codebook_index_table(T.quantization_map("lut4_to_int6"))
        args = (index, [-1], 64, 31.0, False)
        kw = dict(scale_qmap=T.quantization_map("fp8_e5m3"), output_code=mid)
    exp = O.quantize_mx_outlier(x, *args, **kw, threshold=4.0, max_pct=0.01, indptr_offset=offset)
    dev_args = tuple(a.to(DEV) if torch.is_tensor(a) else a for a in args)
    dev_kw = {k: v.to(DEV) for k, v in kw.items()}
    got = Q.quantize_mx_outlier(x.to(DEV), *dev_args, **dev_kw, threshold=4.0, max_pct=0.01,
                                indptr_offset=offset)
    for name, g, e in zip(("data", "indices", "indptr", "scale", "codes"), got, exp):
        assert_same_bits(g, e, f"{fmt} offset={offset} {name}")


SLICES = [(0, 0, 40, 1.0), (0, 7, 19, 1.0), (0, 5, 5, 1.0), (0, 0, 40, 0.2), (1, 0, 256, 1.0),
          (1, 64, 192, 1.0), (1, 250, 256, 1.0), (1, 0, 128, 0.1), (-1, 17, 18, 0.5), (-2, 3, 30, 0.5)]


@pytest.mark.parametrize("dim,start,end,factor", SLICES)
def test_slice_csr_bit_exact(dim, start, end, factor):
    x = _with_outliers((40, 256), 15, rate=0.02, factor=10.0)
    data, idx, indptr, _ = O.filter_outlier(x, 3.0, 0.05)
    exp = O.slice_csr_tensor(data, idx, indptr, dim, start, end, factor)
    got = Q.slice_csr_tensor(data.to(DEV), idx.to(DEV), indptr.to(DEV), dim, start, end, factor)
    for name, g, e in zip(("data", "indices", "indptr"), got, exp):
        assert_same_bits(g, e, f"slice dim={dim} [{start},{end}) x{factor} {name}")


def _weights(kind, N, K, seed):
    w = _rand((N, K), seed, 0.02)
    if kind == "bf16":
        return w, None, None, None
    if kind == "int8":
        s, c = O.quantize_mx(w, T.quantization_map("int8"), [-1], 16, 127.0, True)
        return c, s, None, 16
    index, entries, _ = T.codebook_index_table(T.quantization_map("lut4_to_int6"))
    s, c = O.quantize_mx(w, index, [-1], 64, 31.0, False, T.quantization_map("fp8_e5m3"))
    return c, s, entries, 64


SPMM_CASES = [("bf16", "kc", 37, 256, 100, None), ("int8", "kc", 64, 4096, 512, torch.float32),
              ("int8", "ck", 64, 4096, 384, None), ("nf4", "kc", 16, 1024, 256, torch.float32),
              ("bf16", "ck", 8, 14336, 64, torch.float32), ("int8", "kc", 256, 14336, 48, None)]


@pytest.mark.parametrize("kind,layout,M,K,N,out_dtype", SPMM_CASES)
def test_spmm_csr_matches_oracle(kind, layout, M, K, N, out_dtype):
    x = _with_outliers((M, K), 16, rate=0.01)
    data, idx, indptr, _ = O.filter_outlier(x, 3.0, 0.02)
    B, S, code, bs = _weights(kind, N, K, 17)
    if layout == "ck":
        B = B.mT.contiguous()
        S = None if S is None else S.mT.contiguous()
    exp = O.spmm_csr(data, idx, indptr, B, S, code, bs, layout, out_dtype=out_dtype)
    dv = lambda t: None if t is None else t.to(DEV)  # noqa: E731
    got = Q.spmm_csr(dv(data), dv(idx), dv(indptr), dv(B), dv(S), dv(code), bs, layout, out_dtype=out_dtype)
    assert got.dtype == exp.dtype and got.shape == exp.shape
    tol = 1e-5 if exp.dtype == torch.float32 else 2.0**-8
    assert max_rel_err(got, exp) < tol


def test_spmm_csr_batched_and_rebased():
    """Batched CSR (3-D input) against one B and against a batch of B; row
    pointers that start at an offset (quantize_mx_outlier's indptr_offset)."""
    x = _with_outliers((3, 20, 512), 18, rate=0.02)
    data, idx, indptr, _ = O.filter_outlier(x, 2.5, 0.05)
    indptr = indptr + 1000
    B1 = _rand((96, 512), 19, 0.02)
    B3 = _rand((3, 96, 512), 20, 0.02)
    for B in (B1, B3):
        exp = O.spmm_csr(data, idx, indptr, B, out_dtype=torch.float32)
        got = Q.spmm_csr(data.to(DEV), idx.to(DEV), indptr.to(DEV), B.to(DEV), out_dtype=torch.float32)
        assert got.shape == exp.shape == (3, 20, 96)
        assert max_rel_err(got, exp) < 1e-5


@pytest.mark.parametrize("variant", ["plain", "bias", "alpha_bias", "fp32_out", "kx", "batched"])
def test_linear_mx_with_outlier_term(variant):
    """quantize_mx_outlier -> linear_mx(A_data, A_indices, A_indptr) as a
    converted graph runs it, against the oracle (1e-2)."""
    shape = (2, 64, 512) if variant == "batched" else (128, 512)
    x = _with_outliers(shape, 21, rate=0.005)
    tab = T.quantization_map("int8")
    wc, ws, _, _ = _weights("int8", 192, 512, 22)
    bias = _rand((192,), 23) if variant in ("bias", "alpha_bias") else None
    alpha = torch.tensor(0.5, dtype=torch.bfloat16) if variant == "alpha_bias" else None
    out_dtype = torch.float32 if variant == "fp32_out" else None
    layout = "xc,kc->kx" if variant == "kx" else "xc,kc->xk"
    data, idx, indptr, xs, xc = O.quantize_mx_outlier(x, tab, [-1], 16, 127.0, True, threshold=5.0, max_pct=0.01)
    exp = O.linear_mx(xc, wc, bias, input_scale=xs, weight_scale=ws, block_size=16, alpha=alpha, layout=layout,
                      out_dtype=out_dtype, A_data=data, A_indices=idx, A_indptr=indptr)
    d = lambda t: None if t is None else t.to(DEV)  # noqa: E731
    g = Q.quantize_mx_outlier(x.to(DEV), tab.to(DEV), [-1], 16, 127.0, True, threshold=5.0, max_pct=0.01)
    got = Q.linear_mx(g[4], d(wc), d(bias), input_scale=g[3], weight_scale=d(ws), block_size=16, alpha=d(alpha),
                      A_data=g[0], A_indices=g[1], A_indptr=g[2], layout=layout, out_dtype=out_dtype)
    assert got.dtype == exp.dtype and got.shape == exp.shape
    assert max_rel_err(got, exp) < 1e-2
    plain = Q.linear_mx(g[4], d(wc), d(bias), input_scale=g[3], weight_scale=d(ws), block_size=16, alpha=d(alpha),
                        layout=layout, out_dtype=out_dtype)
    assert max_rel_err(got, exp) < max_rel_err(plain, exp)  # the outlier term is applied


def test_matmul_mx_with_outlier_term():
    x = _with_outliers((64, 256), 24, rate=0.01)
    tab = T.quantization_map("int8")
    wc, ws, _, _ = _weights("int8", 128, 256, 25)
    other, other_s = wc.mT.contiguous(), ws.mT.contiguous()  # [K, N], blocks along K
    data, idx, indptr, xs, xc = O.quantize_mx_outlier(x, tab, [-1], 16, 127.0, True, threshold=4.0, max_pct=0.02)
    exp = O.matmul_mx(xc, other, input_scale=xs, weight_scale=other_s, block_size=16, A_data=data, A_indices=idx,
                      A_indptr=indptr)
    got = Q.matmul_mx(xc.to(DEV), other.to(DEV), input_scale=xs.to(DEV), weight_scale=other_s.to(DEV),
                      block_size=16, A_data=data.to(DEV), A_indices=idx.to(DEV), A_indptr=indptr.to(DEV))
    assert max_rel_err(got, exp) < 1e-2


def test_outlier_linear_replays_under_hip_graph_capture():
    """quantize_mx_outlier + linear_mx captured after an eager run: every
    replay, with eager work between them, equals the eager result."""
    x = _with_outliers((96, 512), 26, rate=0.01).to(DEV)
    tab = T.quantization_map("int8").to(DEV)
    wc, ws, _, _ = _weights("int8", 256, 512, 27)
    wc, ws = wc.to(DEV), ws.to(DEV)

    def step():
        g = Q.quantize_mx_outlier(x, tab, [-1], 16, 127.0, True, threshold=4.0, max_pct=0.01)
        return Q.linear_mx(g[4], wc, input_scale=g[3], weight_scale=ws, block_size=16, A_data=g[0],
                           A_indices=g[1], A_indptr=g[2])

    eager = step()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = step()
    for _ in range(3):
        torch.randn(1 << 16, device=DEV).sum()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
