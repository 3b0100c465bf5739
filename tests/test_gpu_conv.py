"""quantized_ops.conv2d / conv2d_mx on the GPU (im2col + the bf16 MFMA GEMM)
against the oracle (``ops/layout.py:187-214``, ``ops/quantized.py:596-643``)
within the 1e-2 GEMM bar, and within one bf16 ulp of a float64 convolution
of the same operands."""

import pytest
import torch

import voyager_amd.library  # noqa: F401  (defines quantized_ops)
from helpers import assert_within_bf16_ulps, max_rel_err
from oracle import ops as O
from oracle import tables as T

pytestmark = pytest.mark.gpu

Q = torch.ops.quantized_ops
TOL = 1e-2

CASES = [
    # N, C, H, W, K, KH, KW, stride, padding, dilation, groups, layout, bias, out_dtype
    (2, 16, 14, 14, 32, 3, 3, (1, 1), (1, 1), (1, 1), 1, "nchw", True, None),
    (2, 16, 15, 13, 24, 3, 3, (2, 2), (1, 0), (1, 1), 1, "nhwc", True, None),
    (1, 32, 12, 12, 64, 3, 3, (1, 1), (2, 2), (2, 2), 2, "nchw", False, None),
    (2, 8, 10, 10, 8, 3, 3, (1, 1), (1, 1), (1, 1), 8, "nhwc", True, None),
    (1, 3, 32, 32, 16, 7, 7, (2, 2), (3, 3), (1, 1), 1, "nchw", True, torch.float32),
    (3, 40, 9, 11, 48, 1, 1, (1, 1), (0, 0), (1, 1), 1, "nhwc", False, torch.float32),
]


def _operands(N, C, H, W, K, KH, KW, groups, layout, bias, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(N, C, H, W, generator=g).bfloat16()
    w = (torch.randn(K, C // groups, KH, KW, generator=g) * 0.1).bfloat16()
    b = torch.randn(K, generator=g).bfloat16() if bias else None
    if layout == "nhwc":
        x = x.permute(0, 2, 3, 1).contiguous()
        if groups == 1:
            w = w.permute(2, 3, 1, 0).contiguous()
    return x, w, b


@pytest.mark.parametrize("case", CASES, ids=[f"{c[11]}-g{c[10]}-k{c[5]}-s{c[7][0]}" for c in CASES])
def test_conv2d(case):
    N, C, H, W, K, KH, KW, stride, padding, dilation, groups, layout, bias, out_dtype = case
    x, w, b = _operands(N, C, H, W, K, KH, KW, groups, layout, bias, sum(case[:7]))
    exp = O.conv2d(x, w, b, stride, padding, dilation, groups, layout, out_dtype)
    d = lambda t: None if t is None else t.cuda()  # noqa: E731
    got = Q.conv2d(d(x), d(w), d(b), stride, padding, dilation, groups, layout=layout, out_dtype=out_dtype)
    assert got.shape == exp.shape and got.dtype == exp.dtype
    assert max_rel_err(got, exp) < TOL
    ref64 = O.conv2d(x.double(), w.double(), None if b is None else b.double(), stride, padding, dilation, groups,
                     layout)
    if got.dtype == torch.bfloat16:
        assert_within_bf16_ulps(got, ref64, ulps=1.0, atol=1e-5 * float(ref64.abs().max()), what="conv2d")
    else:
        assert max_rel_err(got, ref64) < 1e-5


@pytest.mark.parametrize("layout", ["nchw", "nhwc"])
def test_conv2d_mx_int8(layout):
    """MX-int8 feature maps and filters, blocks of 16 along the channels."""
    N, C, H, W, K = 2, 32, 10, 10, 48
    g = torch.Generator().manual_seed(5)
    x = torch.randn(N, C, H, W, generator=g).bfloat16()
    w = (torch.randn(K, C, 3, 3, generator=g) * 0.05).bfloat16()
    tab = T.quantization_map("int8")
    cax = 3 if layout == "nhwc" else 1
    if layout == "nhwc":
        x = x.permute(0, 2, 3, 1).contiguous()
        w = w.permute(2, 3, 1, 0).contiguous()
    xs, xc = O.quantize_mx(x, tab, [cax], 16, 127.0, True)
    ws, wc = O.quantize_mx(w, tab, [2 if layout == "nhwc" else 1], 16, 127.0, True)
    exp = O.conv2d_mx(xc, wc, None, 1, 1, 1, 1, xs, ws, 16, layout=layout)
    got = Q.conv2d_mx(xc.cuda(), wc.cuda(), None, [1, 1], [1, 1], [1, 1], 1, input_scale=xs.cuda(),
                      weight_scale=ws.cuda(), block_size=16, layout=layout)
    assert got.shape == exp.shape and max_rel_err(got, exp) < TOL
