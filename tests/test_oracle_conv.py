"""The oracle's conv2d twin (``ops/layout.py:187-214``) against a direct
float64 convolution written from the definition: NCHW and NHWC (HWIO
weights when dense), stride, padding, dilation, groups, bias."""

import numpy as np
import pytest
import torch

from oracle import ops as O


def direct_conv(x, w, b, stride, padding, dilation, groups):
    """NCHW x, OIHW w (float64 numpy); out[n, k, oh, ow]."""
    N, C, H, W = x.shape
    K, Cg, KH, KW = w.shape
    (sh, sw), (ph, pw), (dh, dw) = stride, padding, dilation
    OH = (H + 2 * ph - dh * (KH - 1) - 1) // sh + 1
    OW = (W + 2 * pw - dw * (KW - 1) - 1) // sw + 1
    xp = np.zeros((N, C, H + 2 * ph, W + 2 * pw))
    xp[:, :, ph:ph + H, pw:pw + W] = x
    out = np.zeros((N, K, OH, OW))
    Kg = K // groups
    for k in range(K):
        g = k // Kg
        for kh in range(KH):
            for kw in range(KW):
                patch = xp[:, g * Cg:(g + 1) * Cg, kh * dh: kh * dh + sh * (OH - 1) + 1: sh,
                           kw * dw: kw * dw + sw * (OW - 1) + 1: sw]
                out[:, k] += np.einsum("nchw,c->nhw", patch, w[k, :, kh, kw])
        if b is not None:
            out[:, k] += b[k]
    return out


@pytest.mark.parametrize("layout,stride,padding,dilation,groups,bias", [
    ("nchw", (1, 1), (1, 1), (1, 1), 1, True), ("nhwc", (2, 1), (1, 0), (1, 1), 1, False),
    ("nchw", (1, 2), (2, 1), (2, 1), 2, True), ("nhwc", (1, 1), (1, 1), (1, 1), 4, True)])
def test_conv2d_twin_matches_direct_convolution(layout, stride, padding, dilation, groups, bias):
    g = torch.Generator().manual_seed(groups)
    x = torch.randn(2, 4, 7, 6, generator=g, dtype=torch.float64)
    w = torch.randn(8, 4 // groups, 3, 2, generator=g, dtype=torch.float64)
    b = torch.randn(8, generator=g, dtype=torch.float64) if bias else None
    ref = direct_conv(x.numpy(), w.numpy(), None if b is None else b.numpy(), stride, padding, dilation, groups)
    if layout == "nhwc":
        xin = x.permute(0, 2, 3, 1).contiguous()
        win = w.permute(2, 3, 1, 0).contiguous() if groups == 1 else w
        got = O.conv2d(xin, win, b, stride, padding, dilation, groups, layout).permute(0, 3, 1, 2)
    else:
        got = O.conv2d(x, w, b, stride, padding, dilation, groups, layout)
    np.testing.assert_allclose(got.numpy(), ref, rtol=1e-12, atol=1e-12)
