"""Every GEMM tile the dispatcher picks at the configurations' shapes, run
and checked: config 2's four FP8 shapes at M = 2048 (packed E4M3 and the
reference-form quantize -> linear -> dequantize chain), config 4's posit8
GEMM at 2048 x 4096 x 4096, bf16 shapes that select each direct-to-LDS tile,
and a tile_hint sweep over every tile at one ragged mid size.

Each case asserts the kernel ``vh_gemm`` ran (``vh_gemm_plan``, logged per
launch through ``gemm.plan_log``) and compares the result with the oracle's
op sequence (``quantize_pt2e.py:538-600``: ``dequantize(linear(xq, wq), s)``;
``ops/layout.py:231-260``) within 1e-2 max-abs-normalized error, and with a
float32 product of the same operand values."""

import pytest
import torch

import voyager_amd.library  # noqa: F401  (defines quantized_ops)
from helpers import max_rel_err
from oracle import ops as O
from oracle import tables as T
from voyager_amd import gemm, packed

pytestmark = pytest.mark.gpu

TOL = 1e-2
FP8_DIRECT_TILES = [20, 21, 23, 24, 30, 31, 32, 33, 34, 35, 36, 37, 40, 41, 42, 43, 44, 45, 46, 47, 48]
BF16_DIRECT_TILES = [31, 33, 35, 37, 41]
STAGED_TILES = [2, 3, 4, 5, 6, 7, 8, 9, 10]


def _rand(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).bfloat16()


class _Plans:
    """Collects (family, tile, splits, M, N, K) of every vh_gemm launch."""

    def __enter__(self):
        self.log = []
        gemm.plan_log = self.log
        return self.log

    def __exit__(self, *exc):
        gemm.plan_log = None


# config 2: (K, N) -> the direct-to-LDS tile of the packed E4M3 GEMM and of
# the bf16 GEMM the reference-form chain runs
CFG2 = [
    ((4096, 4096), 31, 31),
    ((4096, 1024), 37, 35),
    ((4096, 14336), 44, 41),
    ((14336, 4096), 31, 31),
]


@pytest.mark.parametrize("kn,fp8_tile,bf16_tile", CFG2, ids=[f"K{k}_N{n}" for (k, n), _, _ in CFG2])
def test_cfg2_fp8_shapes(kn, fp8_tile, bf16_tile):
    K, N = kn
    M = 2048
    print(f"cfg2 K={K} N={N}", flush=True)
    x, w = _rand((M, K), 0), _rand((N, K), 1, 0.02)
    tab = T.quantization_map("fp8_e4m3")
    ident = T.quantization_map(None)
    sx, sw = O.per_tensor_scale(x, 448.0), O.per_tensor_scale(w, 448.0)
    s = sx * sw  # bf16 product, as convert forms it (quantize_pt2e.py:609-613)
    xq, wq = O.quantize(x, sx, qmap=tab), O.quantize(w, sw, qmap=tab)
    exp = O.dequantize(O.linear(xq, wq), s, input_qmap=ident)
    ref32 = (xq.float() @ wq.float().T) * s.float()
    d = "cuda"
    cx = packed.quantize_packed(x.to(d), sx.to(d), tab.to(d))
    cw = packed.quantize_packed(w.to(d), sw.to(d), tab.to(d))
    with _Plans() as log:
        got = gemm.linear_fp8(cx, cw, s.to(d))
    assert log == [(gemm.FAMILY_DIRECT_FP8, fp8_tile, 1, M, N, K)]
    assert max_rel_err(got, exp) < TOL
    assert max_rel_err(got, ref32) < TOL
    Q = torch.ops.quantized_ops
    gq = Q.quantize(x.to(d), sx.to(d), qmap=tab.to(d))
    gw = Q.quantize(w.to(d), sw.to(d), qmap=tab.to(d))
    with _Plans() as log:
        lin = Q.linear(gq, gw)
    assert log == [(gemm.FAMILY_DIRECT_BF16, bf16_tile, 1, M, N, K)]
    got2 = Q.dequantize(lin, s.to(d), input_qmap=ident.to(d))
    assert max_rel_err(got2, exp) < TOL
    # the two GPU paths multiply the same exact products
    assert max_rel_err(got2, got) < TOL


def test_cfg4_posit8_gemm_full_size():
    """Config 4's posit8 GEMM at its full shape, 2048 x 4096 x 4096: both
    operands posit8-cast (a direct cast, quantize_pt2e.py:557-561), then
    the bf16 GEMM."""
    M, N, K = 2048, 4096, 4096
    x, w = _rand((M, K), 1), _rand((N, K), 2, 0.02)
    tab = T.quantization_map("posit8_1")
    one = torch.tensor(1.0, dtype=torch.bfloat16)
    xq, wq = O.quantize(x, one, qmap=tab), O.quantize(w, one, qmap=tab)
    exp = O.linear(xq, wq)
    ref32 = xq.float() @ wq.float().T
    d = "cuda"
    cx = packed.quantize_packed(x.to(d), one.to(d), tab.to(d))
    cw = packed.quantize_packed(w.to(d), one.to(d), tab.to(d))
    lut = gemm.posit8_lut(tab.to(d))
    with _Plans() as log:
        got = gemm.linear_posit8(cx, cw, lut)
    assert log == [(gemm.FAMILY_DIRECT_BF16, 31, 1, M, N, K)]
    assert max_rel_err(got, exp) < TOL
    assert max_rel_err(got, ref32) < TOL
    # the reference-form chain: quantize (posit table) then quantized_ops.linear
    Q = torch.ops.quantized_ops
    with _Plans() as log:
        got2 = Q.linear(Q.quantize(x.to(d), one.to(d), qmap=tab.to(d)), Q.quantize(w.to(d), one.to(d), qmap=tab.to(d)))
    assert log == [(gemm.FAMILY_DIRECT_BF16, 31, 1, M, N, K)]
    assert max_rel_err(got2, exp) < TOL


@pytest.mark.parametrize("M,N,K,tile", [
    (2048, 14336, 4096, 41),   # >= 384 tiles of 256 x 256
    (2048, 4096, 4096, 31),    # >= 224 tiles of 256 x 128
    (1024, 3584, 2048, 33),    # >= 224 tiles of 128 x 128
    (256, 4096, 4096, 35),     # fewer: 128 x 64
])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_bf16_direct_tiles(M, N, K, tile, out_dtype):
    """quantized_ops.linear on bf16 operands at shapes that select each
    automatic direct-to-LDS tile, bf16 and float32 results."""
    print(f"bf16 M={M} N={N} K={K} tile={tile} {out_dtype}", flush=True)
    x, w = _rand((M, K), M + 3), _rand((N, K), N + 4, 0.05)
    of = None if out_dtype == torch.bfloat16 else out_dtype
    exp = O.linear(x, w, out_dtype=of)
    ref32 = x.float() @ w.float().T
    with _Plans() as log:
        got = torch.ops.quantized_ops.linear(x.cuda(), w.cuda(), out_dtype=of)
    assert log == [(gemm.FAMILY_DIRECT_BF16, tile, 1, M, N, K)]
    assert got.dtype == out_dtype
    assert max_rel_err(got, exp) < TOL
    assert max_rel_err(got, ref32) < (TOL if out_dtype == torch.bfloat16 else 1e-5)


def _fp8_operands(M, N, K, seed):
    tab = T.quantization_map("fp8_e4m3")
    x, w = _rand((M, K), seed), _rand((N, K), seed + 1, 0.02)
    sx, sw = O.per_tensor_scale(x, 448.0), O.per_tensor_scale(w, 448.0)
    s = sx * sw
    xq, wq = O.quantize(x, sx, qmap=tab), O.quantize(w, sw, qmap=tab)
    exp = O.dequantize(O.linear(xq, wq), s, input_qmap=T.quantization_map(None))
    d = "cuda"
    cx = packed.quantize_packed(x.to(d), sx.to(d), tab.to(d))
    cw = packed.quantize_packed(w.to(d), sw.to(d), tab.to(d))
    return cx, cw, s.to(d), exp, xq, wq


SWEEP = (520, 776, 1040)  # ragged against every tile; K a multiple of 16, not of 128


@pytest.mark.parametrize("tile", FP8_DIRECT_TILES + STAGED_TILES)
def test_fp8_tile_sweep(tile):
    """Every E4M3 tile (direct-to-LDS 20..48, register-staged 2..10) at one
    ragged mid size against the oracle."""
    M, N, K = SWEEP
    cx, cw, s, exp, _, _ = _fp8_operands(M, N, K, 50)
    with _Plans() as log:
        got = gemm.linear_fp8(cx, cw, s, tile_hint=tile)
    fam = gemm.FAMILY_DIRECT_FP8 if tile in FP8_DIRECT_TILES else gemm.FAMILY_STAGED
    assert log == [(fam, tile, 1, M, N, K)]
    assert max_rel_err(got, exp) < TOL


@pytest.mark.parametrize("tile", BF16_DIRECT_TILES + STAGED_TILES)
def test_bf16_tile_sweep(tile):
    """Every bf16 tile at one ragged mid size (float32 result with alpha and
    bias: the float32 epilogue of each tile) against float64."""
    M, N, K = SWEEP
    a, b = _rand((M, K), 60), _rand((N, K), 61, 0.05)
    bias = _rand((N,), 62)
    alpha = torch.tensor(0.75)
    d = gemm.GemmDesc()
    ac, bc = a.cuda(), b.cuda()
    out = torch.empty(M, N, dtype=torch.float32, device="cuda")
    bias32 = bias.float().cuda()
    al = alpha.float().cuda()
    d.A, d.B, d.C = ac.data_ptr(), bc.data_ptr(), out.data_ptr()
    d.M, d.N, d.K = M, N, K
    d.lda, d.ldb, d.ldc = K * 2, K * 2, N
    d.a_fmt = d.b_fmt = gemm.OP_BF16
    d.tile_hint = tile
    d.epi = gemm._epilogue(gemm.EPI_PLAIN, torch.float32, al, bias32)
    with _Plans() as log:
        gemm.run(d, ac.device)
    fam = gemm.FAMILY_DIRECT_BF16 if tile in BF16_DIRECT_TILES else gemm.FAMILY_STAGED
    assert log == [(fam, tile, 1, M, N, K)]
    ref = (a.double() @ b.double().T) * 0.75 + bias.double()
    assert max_rel_err(out, ref) < 1e-5


@pytest.mark.parametrize("fam,tile", [("bf16", t) for t in BF16_DIRECT_TILES] +
                         [("fp8", t) for t in (20, 24, 31, 35, 41, 44, 48)])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_direct_tile_bias_epilogue(fam, tile, out_dtype):
    """The direct-to-LDS tiles' bias instantiation (plain epilogue with alpha
    and a bias, bf16 or float32 bias alternating with the tile, bf16 or
    float32 output) at one ragged size against float64.  Alpha brings the
    products to the bias's magnitude (E4M3 grid values are up to 448), so a
    wrong or missing bias moves the result far past the tolerance."""
    M, N, K = SWEEP
    if fam == "bf16":
        a, b = _rand((M, K), 70), _rand((N, K), 71, 0.05)
        ac, bc = a.cuda(), b.cuda()
        av, bv = a.double(), b.double()
        fmt, lda, family, al, tol32 = gemm.OP_BF16, K * 2, gemm.FAMILY_DIRECT_BF16, 0.75, 1e-5
    else:
        ac, bc, _, _, xq, wq = _fp8_operands(M, N, K, 72)
        av, bv = xq.double(), wq.double()
        # fp32 sums of ~1e5-sized products: 1e-4 of the largest output
        fmt, lda, family, al, tol32 = gemm.OP_FP8, K, gemm.FAMILY_DIRECT_FP8, 2.0 ** -16, 1e-4
    bias = _rand((N,), 73)
    bias_dev = bias.cuda() if tile % 2 else bias.float().cuda()
    alpha = torch.tensor(al, device="cuda")
    out = torch.empty(M, N, dtype=out_dtype, device="cuda")
    d = gemm.GemmDesc()
    d.A, d.B, d.C = ac.data_ptr(), bc.data_ptr(), out.data_ptr()
    d.M, d.N, d.K = M, N, K
    d.lda, d.ldb, d.ldc = lda, lda, N
    d.a_fmt = d.b_fmt = fmt
    d.tile_hint = tile
    d.epi = gemm._epilogue(gemm.EPI_PLAIN, out_dtype, alpha, bias_dev)
    with _Plans() as log:
        gemm.run(d, ac.device)
    assert log == [(family, tile, 1, M, N, K)]
    ref = (av @ bv.T) * al + bias.double()
    assert max_rel_err(out, ref) < (TOL if out_dtype == torch.bfloat16 else tol32)
    # the bias is a visible part of the result
    assert max_rel_err(ref - bias.double(), ref) > 10 * (TOL if out_dtype == torch.bfloat16 else tol32)


def test_posit8_in_staging_tiles():
    """The posit8 operands decoded in the register-staged kernel's staging
    (a tile hint), every staged tile, against the oracle."""
    M, N, K = SWEEP
    tab = T.quantization_map("posit8_1")
    one = torch.tensor(1.0, dtype=torch.bfloat16)
    x, w = _rand((M, K), 70), _rand((N, K), 71, 0.02)
    exp = O.linear(O.quantize(x, one, qmap=tab), O.quantize(w, one, qmap=tab))
    d = "cuda"
    cx = packed.quantize_packed(x.to(d), one.to(d), tab.to(d))
    cw = packed.quantize_packed(w.to(d), one.to(d), tab.to(d))
    lut = gemm.posit8_lut(tab.to(d))
    for tile in STAGED_TILES:
        with _Plans() as log:
            got = gemm.linear_posit8(cx, cw, lut, tile_hint=tile)
        assert log == [(gemm.FAMILY_STAGED, tile, 1, M, N, K)], tile
        assert max_rel_err(got, exp) < TOL, tile


def test_plan_follows_output_alignment():
    """A bf16 result whose rows are not 16-byte aligned cannot take the LDS
    epilogue: the plan falls back to the register-staged kernel, as the
    launch does."""
    M, N, K = 256, 1030, 256
    a, b = _rand((M, K), 80).cuda(), _rand((N, K), 81).cuda()
    with _Plans() as log:
        got = torch.ops.quantized_ops.linear(a, b)
    assert log[0][0] == gemm.FAMILY_STAGED
    assert max_rel_err(got, O.linear(a.cpu(), b.cpu())) < TOL


@pytest.mark.parametrize("ld", [1032, 1040])
def test_fp8_rows_in_wider_buffers(ld):
    """E4M3 operands of K = 1024 inside rows of ``ld`` bytes whose padding
    holds NaN codes: rows 16-byte aligned (1040) take the direct-to-LDS
    kernel, rows at 8 bytes past alignment (1032) the register-staged one
    (the direct kernel moves whole aligned 16-byte chunks); both match the
    oracle, so no padding byte enters a product."""
    M, N, K = 256, 384, 1024
    cx, cw, s, exp, _, _ = _fp8_operands(M, N, K, 90)
    bx = torch.full((M, ld), 0x7F, dtype=torch.uint8, device="cuda")
    bw = torch.full((N, ld), 0x7F, dtype=torch.uint8, device="cuda")
    bx[:, :K], bw[:, :K] = cx, cw
    with _Plans() as log:
        got = gemm.linear_fp8(bx[:, :K], bw[:, :K], s)
    assert log[0][0] == (gemm.FAMILY_DIRECT_FP8 if ld % 16 == 0 else gemm.FAMILY_STAGED)
    assert max_rel_err(got, exp) < TOL


def test_bf16_linear_odd_contraction():
    """quantized_ops.linear with K = 27 (a first convolution's C * kh * kw):
    K is zero-padded to whole 16-byte chunks, which adds nothing."""
    a, b = _rand((64, 27), 91).cuda(), _rand((40, 27), 92).cuda()
    got = torch.ops.quantized_ops.linear(a, b)
    assert max_rel_err(got, O.linear(a.cpu(), b.cpu())) < TOL
    a3 = _rand((3, 16, 27), 93).cuda()
    got3 = torch.ops.quantized_ops.linear(a3, b)
    assert max_rel_err(got3, O.linear(a3.cpu(), b.cpu())) < TOL
