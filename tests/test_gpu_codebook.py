"""Codebook search / lookup (one table and region grids) and block scales over
several axes on the GPU, bit for bit against the oracle."""

import pytest
import torch

import voyager_amd.library  # noqa: F401  (defines quantized_ops)
from helpers import assert_same_bits
from oracle import ops as O
from oracle import tables as T

pytestmark = pytest.mark.gpu

Q = torch.ops.quantized_ops

NF4 = torch.tensor([-1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
                    -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
                    0.07958029955625534, 0.16093020141124725, 0.24611230194568634, 0.33791524171829224,
                    0.44070982933044434, 0.5626170039176941, 0.7229568362236023, 1.0])


def _x(g, shape, dtype=torch.bfloat16, scale=1.0):
    x = torch.randn(shape, generator=g) * scale
    flat = x.view(-1)
    sp = torch.tensor([0.0, -0.0, float("inf"), -float("inf"), float("nan"), 1e-40, 0.5, -1.0, 1.0])
    flat[: sp.numel()] = sp
    return x.to(dtype)


def _cuda(*ts):
    return [t.cuda() if t is not None else None for t in ts]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16])
@pytest.mark.parametrize("code_dtype", [torch.float32, torch.bfloat16])
def test_quantize_1d_codebook(dtype, code_dtype):
    g = torch.Generator().manual_seed(21)
    x = _x(g, (33, 70), dtype, 0.7)
    s = (torch.rand(33, 3, generator=g) + 0.2).to(dtype)  # blocks of 32 along the last axis (partial)
    code = NF4.to(code_dtype)
    bounds = (NF4[:-1] + NF4[1:]) / 2
    exp = O.quantize(x, s, None, [-1], 32, code)
    got = Q.quantize(*_cuda(x, s), None, [-1], 32, code.cuda())
    assert_same_bits(got, exp, "entries")
    exp = O.quantize(x, s, None, [-1], 32, code, bounds)
    got = Q.quantize(*_cuda(x, s), None, [-1], 32, code.cuda(), bounds.cuda())
    assert_same_bits(got, exp, "indices")


def test_quantize_codebook_zero_point_and_scalar_scale():
    g = torch.Generator().manual_seed(22)
    x = _x(g, (4, 257), torch.bfloat16, 3.0)
    s = torch.tensor(0.37)
    z = (torch.randn(4, 1, generator=g)).bfloat16()
    code = torch.tensor([-4.0, -1.5, 0.0, 0.25, 2.0, 8.0])
    exp = O.quantize(x, s, z, qmap=code)
    got = Q.quantize(*_cuda(x, s, z), qmap=code.cuda())
    assert_same_bits(got, exp, "zero point")


@pytest.mark.parametrize("bounds", [False, True])
def test_quantize_per_head_codebooks(bounds):
    g = torch.Generator().manual_seed(23)
    B, H, S, D = 2, 8, 19, 64
    x = _x(g, (B, H, S, D), torch.bfloat16, 2.0)
    code = torch.sort(torch.randn(1, H, 1, 1, 16, generator=g) * 2, dim=-1).values
    bnd = (code[..., :-1] + code[..., 1:]) / 2 if bounds else None
    s = torch.tensor(1.0, dtype=torch.bfloat16)
    exp = O.quantize(x, s, qmap=code, output_code=bnd)
    got = Q.quantize(*_cuda(x, s), qmap=code.cuda(), output_code=bnd.cuda() if bounds else None)
    assert_same_bits(got, exp, "per head")
    # decode back through the same tables, with and without a block scale
    if bounds:
        sc = (torch.rand(B, H, S, 2, generator=g) + 0.5).bfloat16()
        exp_d = O.dequantize_mx(exp, sc, 32, code)
        got_d = Q.dequantize_mx(got, sc.cuda(), 32, code.cuda())
        assert_same_bits(got_d, exp_d, "per-head decode")


def test_region_grid_over_two_axes_and_errors():
    g = torch.Generator().manual_seed(24)
    x = _x(g, (6, 40), torch.float32, 1.5)
    code = torch.sort(torch.randn(3, 4, 7, generator=g), dim=-1).values
    s = torch.tensor(0.5)
    exp = O.quantize(x, s, qmap=code)
    got = Q.quantize(*_cuda(x, s), qmap=code.cuda())
    assert_same_bits(got, exp, "grid")
    with pytest.raises(ValueError, match="does not divide"):
        Q.quantize(torch.zeros(5, 40, device="cuda"), s.cuda(), qmap=code.cuda())


@pytest.mark.parametrize("code_dtype", [torch.bfloat16, torch.float32])
def test_dequantize_mx_codebook_code_dtypes(code_dtype):
    g = torch.Generator().manual_seed(25)
    idx = torch.randint(-16, 16, (48, 128), generator=g).float()
    idx.view(-1)[:4] = torch.tensor([float("nan"), 16.0, -17.0, 2.7])
    sc = (torch.rand(48, 4, generator=g) + 0.1).bfloat16()
    code = NF4.to(code_dtype)
    for dt in (torch.bfloat16, torch.float32):
        x = idx.to(dt)
        # out-of-range indices raise on the CPU; the GPU writes NaN there
        ok = ~(torch.isnan(x) | (x.long() >= 16) | (x.long() < -16))
        safe = torch.where(ok, x, torch.zeros_like(x))
        exp = O.dequantize_mx(safe, sc, 32, code)
        exp = torch.where(ok, exp, torch.full_like(exp, float("nan")))
        got = Q.dequantize_mx(x.cuda(), sc.cuda(), 32, code.cuda())
        assert_same_bits(got, exp, f"codes {dt}")


def test_quantize_mx_and_affine_with_codebook():
    g = torch.Generator().manual_seed(26)
    x = _x(g, (16, 320), torch.bfloat16, 1.0)
    bounds = (NF4[:-1] + NF4[1:]) / 2
    exp = O.quantize_mx(x, NF4, [-1], 64, 1.0, output_code=bounds)
    got = Q.quantize_mx(x.cuda(), NF4.cuda(), [-1], 64, 1.0, output_code=bounds.cuda())
    assert_same_bits(got[0], exp[0], "scales")
    assert_same_bits(got[1], exp[1], "indices")
    lv = torch.arange(16).float()
    exp = O.quantize_affine(x, lv, [-1], 32, 0, 15)
    got = Q.quantize_affine(x.cuda(), lv.cuda(), [-1], 32, 0, 15)
    for a, b, what in zip(got, exp, ("scale", "zero point", "codes")):
        assert_same_bits(a, b, what)


@pytest.mark.parametrize("pot", [True, False])
@pytest.mark.parametrize("shape,axes,bs", [((6, 40, 72), [1, 2], 32), ((3, 5, 7), [0, -1], 4),
                                           ((70, 33), [-2, -1], 16)])
def test_block_scales_over_two_axes(pot, shape, axes, bs):
    g = torch.Generator().manual_seed(27)
    x = (torch.randn(shape, generator=g) * torch.exp(torch.randn(shape, generator=g) * 2)).bfloat16()
    x.view(-1)[::53] = 0.0
    if not pot:
        x.view(-1)[5] = float("nan")
    tab = T.quantization_map("int8")
    stab = T.quantization_map("fp8_e5m3") if not pot else None
    exp = O.calculate_mx_qparam(x, axes, bs, 127.0, pot, stab)
    got = Q.calculate_mx_qparam(x.cuda(), axes, bs, 127.0, pot, stab.cuda() if stab is not None else None)
    assert_same_bits(got, exp, "scales")
    es, ec = O.quantize_mx(x, tab, axes, bs, 127.0, pot, stab)
    gs, gc = Q.quantize_mx(x.cuda(), tab.cuda(), axes, bs, 127.0, pot, stab.cuda() if stab is not None else None)
    assert_same_bits(gs, es, "quantize_mx scales")
    assert_same_bits(gc, ec, "quantize_mx codes")


def test_matmul_mx_with_region_codebook_operand():
    g = torch.Generator().manual_seed(28)
    M, K, N = 64, 128, 96
    code = torch.sort(torch.randn(2, 1, 16, generator=g), dim=-1).values.bfloat16()
    xi = torch.randint(0, 16, (M, K), generator=g).bfloat16()
    w = torch.randn(K, N, generator=g).bfloat16()
    exp = O.matmul_mx(xi, w, input_code=code).float()
    got = Q.matmul_mx(xi.cuda(), w.cuda(), input_code=code.cuda()).float().cpu()
    assert torch.allclose(got, exp, rtol=1e-2, atol=1e-2 * exp.abs().max().item())


@pytest.mark.parametrize("case", ["seed", "codebook", "two_axes"])
def test_quantize_mx_global_scale_unfused(case):
    """quantize_mx with a 0-d global scale on the paths that quantize after
    the block scales (stochastic rounding, a codebook, blocks over two axes):
    scales and codes bit-exact, the elements divided by scale * global_scale
    as eager torch forms it."""
    g = torch.Generator().manual_seed(29)
    x = (torch.randn(24, 256, generator=g) * 300).bfloat16()
    e4m3 = T.quantization_map("fp8_e4m3")
    gs = (x.float().abs().amax() / (6.0 * 448.0)).to(torch.float32)
    axes, qmap, seed, oc = [-1], T.quantization_map("fp4_e2m1"), None, None
    if case == "seed":
        seed = torch.tensor(1234, dtype=torch.int64)
    elif case == "codebook":
        qmap = torch.tensor([-6.0, -3.0, -1.0, 0.0, 1.0, 3.0, 6.0])
    else:
        axes = [0, 1]
    es, ec = O.quantize_mx(x, qmap, axes, 16, 6.0, False, e4m3, oc, seed, gs)
    gs_, gc = Q.quantize_mx(x.cuda(), qmap.cuda(), axes, 16, 6.0, False, e4m3.cuda(), oc,
                            seed.cuda() if seed is not None else None, gs.cuda())
    assert_same_bits(gs_, es, f"{case} scales")
    assert_same_bits(gc, ec, f"{case} codes")
