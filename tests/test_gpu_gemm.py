"""GEMM ops on the GPU against the oracle (1e-2 max-abs-normalized, bf16
out, fp32 accumulation) and, where cheap, a float64 matmul."""

import pytest
import torch

import voyager_amd.library  # noqa: F401  (defines quantized_ops)
from helpers import assert_same_bits, assert_within_bf16_ulps, max_rel_err
from oracle import ops as O
from oracle import tables as T

pytestmark = pytest.mark.gpu

TOL = 1e-2


def _rand(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).bfloat16()


@pytest.mark.parametrize("M,N,K", [(64, 64, 64), (100, 70, 136), (256, 512, 1024), (1, 4096, 4096), (333, 129, 72)])
def test_linear_bf16(M, N, K):
    x, w = _rand((M, K), 1), _rand((N, K), 2, 0.05)
    exp = O.linear(x, w)
    got = torch.ops.quantized_ops.linear(x.cuda(), w.cuda())
    assert got.dtype == torch.bfloat16
    assert max_rel_err(got, exp) < TOL
    ref64 = x.double() @ w.double().T
    assert max_rel_err(got, ref64) < TOL


def test_linear_layouts_bias_and_out_dtype():
    x, w, b = _rand((48, 96), 3), _rand((80, 96), 4), _rand((80,), 5)
    for layout, xs, ws in [("xc,kc->xk", x, w), ("xc,ck->xk", x, w.T.contiguous()),
                           ("cx,ck->xk", x.T.contiguous(), w.T.contiguous()), ("xc,kc->kx", x, w)]:
        exp = O.linear(xs, ws, b, layout=layout, out_dtype=torch.float32)
        got = torch.ops.quantized_ops.linear(xs.cuda(), ws.cuda(), b.cuda(), layout=layout, out_dtype=torch.float32)
        assert got.dtype == torch.float32 and list(got.shape) == list(exp.shape)
        assert max_rel_err(got, exp) < 1e-5, layout


def test_matmul_batched():
    a, b = _rand((2, 3, 40, 64), 6), _rand((2, 3, 64, 24), 7)
    exp = O.matmul(a, b)
    got = torch.ops.quantized_ops.matmul(a.cuda(), b.cuda())
    assert list(got.shape) == [2, 3, 40, 24]
    assert max_rel_err(got, exp) < TOL
    exp = O.matmul(a, b, out_dtype=torch.float32)
    got = torch.ops.quantized_ops.matmul(a.cuda(), b.cuda(), out_dtype=torch.float32)
    assert max_rel_err(got, exp) < 1e-5


def _cfg1():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(256, 4096, generator=g)
    x = torch.where(torch.rand(256, 4096, generator=g) < 0.001, x * 20, x).bfloat16()
    w = (torch.randn(4096, 4096, generator=g) * 0.02).bfloat16()
    return x, w


def test_linear_mx_mxint8_cfg1():
    """Config 1 end to end through the reference op sequence:
    quantize_mx(X), quantize_mx(W), linear_mx."""
    x, w = _cfg1()
    tab = T.quantization_map("int8")
    sx, cx = O.quantize_mx(x, tab, [-1], 16, 127.0, True)
    sw, cw = O.quantize_mx(w, tab, [-1], 16, 127.0, True)
    exp = O.linear_mx(cx, cw, input_scale=sx, weight_scale=sw, block_size=16)
    gsx, gcx = torch.ops.quantized_ops.quantize_mx(x.cuda(), tab.cuda(), [-1], 16, 127.0, True)
    gsw, gcw = torch.ops.quantized_ops.quantize_mx(w.cuda(), tab.cuda(), [-1], 16, 127.0, True)
    assert_same_bits(gsx, sx, "x scale")
    assert_same_bits(gcw, cw, "w codes")
    got = torch.ops.quantized_ops.linear_mx(gcx, gcw, input_scale=gsx, weight_scale=gsw, block_size=16)
    assert got.dtype == torch.bfloat16
    assert max_rel_err(got, exp) < TOL
    # the packed MX-int8 GEMM (codes + scale bytes decoded in the GEMM)
    from voyager_amd import gemm, packed

    px = packed.quantize_mx_packed(x.cuda(), tab.cuda(), [-1], 16, 127.0, True)
    pw = packed.quantize_mx_packed(w.cuda(), tab.cuda(), [-1], 16, 127.0, True)
    got2 = gemm.linear_mxint8(px.codes, px.scale, pw.codes, pw.scale, 16, px.bias, pw.bias)
    assert max_rel_err(got2, exp) < TOL
    # both GPU paths compute the same exact products; only summation order differs
    assert max_rel_err(got2, got) < 1e-2


def _deq_mxint8(p):
    """Exact float64 values of packed MX-int8 operands: code * 2**(byte - bias)."""
    c = p.codes.cpu().view(torch.int8).double()
    e = p.scale.cpu().long() - p.bias
    e = e.repeat_interleave(p.block_size, dim=1)[:, : c.shape[1]]
    return c * torch.pow(2.0, e.double())


@pytest.mark.parametrize("M,N,K,block,hint,split,tile", [
    (256, 4096, 4096, 16, 0, 0, 51),     # config 1: automatic tile and split
    (256, 4096, 4096, 16, 50, 1, 50),    # bf16 operands, unsplit
    (130, 200, 1024, 16, 50, 3, 50),     # ragged M / N; 16 stages in splits of 6, 6, 4
    (130, 200, 1024, 32, 51, 2, 51),
    (64, 128, 64, 16, 52, 0, 52),        # a single K stage
    (300, 520, 640, 16, 53, 5, 53),
    (70, 260, 1152, 32, 54, 4, 54),
    (256, 4096, 4096, 16, 55, 4, 55),    # producer / consumer waves
    (130, 200, 1024, 16, 55, 3, 55),
    (300, 520, 640, 32, 56, 1, 56),
    (64, 128, 64, 16, 55, 0, 55),
    (2048, 4096, 256, 16, 0, 0, 56),     # a grid that fills the GPU: automatic 56, unsplit
        (256, 4096, 4096, 16, 60, 0, 60),    # fp16 operands, 256 x 64: automatic split (4)
    (2048, 1024, 4096, 16, 60, 0, 60),   # 128 tiles: split 2
    (256, 4096, 4096, 16, 60, 1, 60),
    (300, 200, 1024, 16, 60, 3, 60),     # ragged M / N; 4 K granules in splits of 2, 2
    (130, 520, 768, 16, 60, 2, 60),      # 3 K granules (256 each) in splits of 2, 1
    (512, 256, 256, 16, 60, 0, 60),
    (300, 520, 640, 32, 60, 1, 51),      # 32-element blocks: the fp16 kernel does not apply
])
def test_linear_mxint8_split_k(M, N, K, block, hint, split, tile):
    """The MX-int8 kernels (tiles 50..56, K split across workgroups with fp32
    partials added in split order) against the exact float64 product of the
    decoded operands, and against the register-staged kernel (tile 4).  The
    split adds the same exact products in another order, so the two GPU
    results agree to fp32 rounding."""
    from voyager_amd import gemm, packed

    tab = T.quantization_map("int8").cuda()
    x = _rand((M, K), 30).cuda()
    w = _rand((N, K), 31, 0.02).cuda()
    px = packed.quantize_mx_packed(x, tab, [-1], block, 127.0, True)
    pw = packed.quantize_mx_packed(w, tab, [-1], block, 127.0, True)
    ref = _deq_mxint8(px) @ _deq_mxint8(pw).T
    gemm.plan_log = log = []
    try:
        got = gemm.linear_mxint8(px.codes, px.scale, pw.codes, pw.scale, block, px.bias, pw.bias, tile_hint=hint,
                                 split_k=split)
    finally:
        gemm.plan_log = None
    assert [(f, t) for f, t, *_ in log] == [(gemm.FAMILY_MXI8, tile)]
    assert max_rel_err(got, ref) < TOL
    old = gemm.linear_mxint8(px.codes, px.scale, pw.codes, pw.scale, block, px.bias, pw.bias, tile_hint=4)
    assert max_rel_err(got, old) < 1e-2
    # fp32 output with alpha and bias: the reduce kernel's epilogue
    alpha = torch.tensor(0.75, device="cuda")
    bias = _rand((N,), 32).cuda()
    got32 = gemm.linear_mxint8(px.codes, px.scale, pw.codes, pw.scale, block, px.bias, pw.bias,
                               out_dtype=torch.float32, bias=bias, alpha=alpha, tile_hint=hint, split_k=split)
    ref32 = ref * 0.75 + bias.cpu().double()
    assert got32.dtype == torch.float32
    assert max_rel_err(got32, ref32) < 1e-5


@pytest.mark.parametrize("M,N,K", [(1030, 520, 1024), (2048, 4096, 4096)])
def test_linear_mxint8_two_pass(M, N, K, monkeypatch):
    """Grids past ``mxint8_two_pass_pays`` rebase both packed operands to
    exact fp16 rows (``bake_mx8_f16``) and run the fp16 GEMM
    (``linear_mx8_f16``), with no ``vh_gemm`` launch: against the exact
    float64 product of the decoded operands and the in-staging decode
    kernel, bf16 and float32 results with alpha and bias."""
    from voyager_amd import gemm, packed

    monkeypatch.setattr(gemm, "MXI8_TWO_PASS_MIN_WORK", 0)
    assert gemm.mxint8_two_pass_pays(M, N, K)
    tab = T.quantization_map("int8").cuda()
    x = _rand((M, K), 34).cuda()
    w = _rand((N, K), 35, 0.02).cuda()
    px = packed.quantize_mx_packed(x, tab, [-1], 16, 127.0, True)
    pw = packed.quantize_mx_packed(w, tab, [-1], 16, 127.0, True)
    ref = _deq_mxint8(px) @ _deq_mxint8(pw).T
    gemm.plan_log = log = []
    try:
        got = gemm.linear_mxint8(px.codes, px.scale, pw.codes, pw.scale, 16, px.bias, pw.bias)
    finally:
        gemm.plan_log = None
    assert log == [] and got.dtype == torch.bfloat16 and list(got.shape) == [M, N]
    assert max_rel_err(got, ref) < TOL
    staged = gemm.linear_mxint8(px.codes, px.scale, pw.codes, pw.scale, 16, px.bias, pw.bias, tile_hint=4)
    assert max_rel_err(got, staged) < 1e-2
    alpha = torch.tensor(0.75, device="cuda")
    bias = _rand((N,), 36).cuda()
    got32 = gemm.linear_mxint8(px.codes, px.scale, pw.codes, pw.scale, 16, px.bias, pw.bias, out_dtype=torch.float32,
                               bias=bias, alpha=alpha)
    assert max_rel_err(got32, ref * 0.75 + bias.cpu().double()) < 1e-5


def test_linear_mxint8_fp16_operands_exponent_range():
    """k_gemm_mx8h rebases each row to its largest block exponent: rows whose
    blocks span 2**-40 .. 2**20 (blocks more than 24 binades below the row's
    largest are flushed) and rows of equal exponents, against the exact
    float64 product, with a float32 result."""
    from voyager_amd import gemm, packed

    M, N, K = 256, 128, 1024
    tab = T.quantization_map("int8").cuda()
    g = torch.Generator().manual_seed(33)
    ex = torch.randint(-40, 21, (M, K // 16), generator=g).repeat_interleave(16, dim=1)
    x = (torch.randn(M, K, generator=g) * torch.pow(2.0, ex.float())).bfloat16().cuda()
    ew = torch.randint(-12, 4, (N, K // 16), generator=g).repeat_interleave(16, dim=1)
    w = (torch.randn(N, K, generator=g) * torch.pow(2.0, ew.float())).bfloat16().cuda()
    px = packed.quantize_mx_packed(x, tab, [-1], 16, 127.0, True)
    pw = packed.quantize_mx_packed(w, tab, [-1], 16, 127.0, True)
    ref = _deq_mxint8(px) @ _deq_mxint8(pw).T
    for split in (1, 4):
        got = gemm.linear_mxint8(px.codes, px.scale, pw.codes, pw.scale, 16, px.bias, pw.bias,
                                 out_dtype=torch.float32, tile_hint=60, split_k=split)
        assert max_rel_err(got, ref) < 1e-5
        # row by row: each row's own largest term sets its scale
        rel = ((got.cpu().double() - ref).abs().amax(dim=1) / ref.abs().amax(dim=1)).max().item()
        assert rel < 1e-5


def test_gemm_workspace_query():
    """vh_gemm_workspace_bytes: split partials for small MX-int8 grids, none
    for grids that fill the GPU or for other formats."""
    import ctypes

    from voyager_amd import gemm
    from voyager_amd._lib import load

    def q(M, N, K, a_fmt=2, split=0):
        d = gemm.GemmDesc()
        d.M, d.N, d.K = M, N, K
        d.lda, d.ldb = K, K
        d.a_fmt = d.b_fmt = a_fmt
        d.a_block = d.b_block = 16
        d.split_k = split
        return load().vh_gemm_workspace_bytes(ctypes.c_void_p(ctypes.addressof(d)))

    assert q(256, 4096, 4096) == 4 * 256 * 4096 * 4
    assert q(4096, 4096, 4096) == 0
    assert q(256, 4096, 4096, a_fmt=0) == 0
    assert q(256, 4096, 4096, split=1) == 0
    assert q(130, 200, 1024, split=3) == 3 * 130 * 200 * 4


@pytest.mark.parametrize("M", [1, 16])
@pytest.mark.parametrize("K,N", [(4096, 1024), (14336, 4096)])
def test_linear_mx_mxnf4_cfg3(M, K, N):
    vt = T.quantization_map("lut4_to_int6")
    index, entries, mid = T.codebook_index_table(vt)
    stab = T.quantization_map("fp8_e5m3")
    x, w = _rand((M, K), 10), _rand((N, K), 11, 0.02)
    sx, cx = O.quantize_mx(x, index, [-1], 64, 31.0, False, stab, mid)
    sw, cw = O.quantize_mx(w, index, [-1], 64, 31.0, False, stab)
    exp = O.linear_mx(cx, cw, input_scale=sx, weight_scale=sw, block_size=64, input_code=entries,
                      weight_code=entries)
    d = "cuda"
    gsx, gcx = torch.ops.quantized_ops.quantize_mx(x.to(d), index.to(d), [-1], 64, 31.0, False, stab.to(d), mid.to(d))
    gsw, gcw = torch.ops.quantized_ops.quantize_mx(w.to(d), index.to(d), [-1], 64, 31.0, False, stab.to(d))
    assert_same_bits(gcw, cw, "w codes")
    got = torch.ops.quantized_ops.linear_mx(gcx, gcw, input_scale=gsx, weight_scale=gsw, block_size=64,
                                            input_code=entries.to(d), weight_code=entries.to(d))
    assert max_rel_err(got, exp) < TOL


@pytest.mark.parametrize("M,K,N", [(256, 4096, 1024), (2048, 4096, 1024), (130, 384, 200)])
def test_linear_fp8_per_tensor(M, K, N):
    """Config 2's path: quantize X and W to E4M3 with amax scales,
    linear(xq, wq) in bf16, then dequantize by the bf16 scale product."""
    x, w = _rand((M, K), 20), _rand((N, K), 21, 0.02)
    tab = T.quantization_map("fp8_e4m3")
    sx = O.per_tensor_scale(x, 448.0)
    sw = O.per_tensor_scale(w, 448.0)
    s = sx * sw  # the scale product is formed in bf16 at convert
    xq = O.quantize(x, sx, qmap=tab)
    wq = O.quantize(w, sw, qmap=tab)
    ident = T.quantization_map(None)
    exp = O.dequantize(O.linear(xq, wq), s, input_qmap=ident)
    from voyager_amd import gemm, packed

    d = "cuda"
    cx = packed.quantize_packed(x.to(d), sx.to(d), tab.to(d))
    cw = packed.quantize_packed(w.to(d), sw.to(d), tab.to(d))
    assert torch.equal(cx.cpu(), xq.float().to(torch.float8_e4m3fn).view(torch.uint8))
    got = gemm.linear_fp8(cx, cw, s.to(d))
    assert max_rel_err(got, exp) < TOL
    ref64 = (xq.double() @ wq.double().T) * s.double()
    assert max_rel_err(got, ref64) < TOL
    # the reference-form ops give the same answer
    gq = torch.ops.quantized_ops.quantize(x.to(d), sx.to(d), qmap=tab.to(d))
    gw = torch.ops.quantized_ops.quantize(w.to(d), sw.to(d), qmap=tab.to(d))
    got2 = torch.ops.quantized_ops.dequantize(torch.ops.quantized_ops.linear(gq, gw), s.to(d),
                                              input_qmap=ident.to(d))
    assert max_rel_err(got2, exp) < TOL


def test_packed_gemms_take_strided_views():
    """The packed-operand linears address rows as base + row * ld: column-
    strided views are copied first (same result as the contiguous operands),
    row-strided ones are read in place, and a misshapen ``out`` is refused."""
    from voyager_amd import gemm, packed

    d = "cuda"
    x, w = _rand((192, 512), 22).to(d), _rand((256, 512), 23, 0.02).to(d)
    tab = T.quantization_map("fp8_e4m3").to(d)
    sx, sw = O.per_tensor_scale(x.cpu(), 448.0).to(d), O.per_tensor_scale(w.cpu(), 448.0).to(d)
    s = sx * sw
    cx, cw = packed.quantize_packed(x, sx, tab), packed.quantize_packed(w, sw, tab)
    ref = gemm.linear_fp8(cx, cw, s)
    cxt = cx.t().contiguous().t()          # column-strided view of the same codes
    wide = torch.zeros(256, 640, dtype=torch.uint8, device=d)
    wide[:, :512] = cw
    assert torch.equal(gemm.linear_fp8(cxt, wide[:, :512], s), ref)  # rows 640 bytes apart
    with pytest.raises(RuntimeError, match="out must be"):
        gemm.linear_fp8(cx, cw, s, out=torch.empty(192, 256, dtype=torch.float32, device=d))
    with pytest.raises(RuntimeError, match="one-byte"):
        gemm.linear_fp8(x, cw, s)
    # MX-int8 codes and scale bytes likewise
    t8 = T.quantization_map("int8").to(d)
    px = packed.quantize_mx_packed(x, t8, [-1], 16, 127.0, True)
    pw = packed.quantize_mx_packed(w, t8, [-1], 16, 127.0, True)
    r8 = gemm.linear_mxint8(px.codes, px.scale, pw.codes, pw.scale, 16, px.bias, pw.bias)
    got8 = gemm.linear_mxint8(px.codes.t().contiguous().t(), px.scale.t().contiguous().t(), pw.codes, pw.scale, 16,
                              px.bias, pw.bias)
    assert torch.equal(got8, r8)


def test_linear_posit8():
    """Config 4's GEMM at a reduced M: posit8-cast operands, bf16 GEMM."""
    x, w = _rand((256, 4096), 30), _rand((512, 4096), 31, 0.02)
    tab = T.quantization_map("posit8_1")
    one = torch.tensor(1.0, dtype=torch.bfloat16)
    xq, wq = O.quantize(x, one, qmap=tab), O.quantize(w, one, qmap=tab)
    exp = O.linear(xq, wq)
    from voyager_amd import gemm, packed

    d = "cuda"
    cx = packed.quantize_packed(x.to(d), one.to(d), tab.to(d))
    cw = packed.quantize_packed(w.to(d), one.to(d), tab.to(d))
    lut = gemm.posit8_lut(tab.to(d))
    got = gemm.linear_posit8(cx, cw, lut)
    assert max_rel_err(got, exp) < TOL
    # the in-staging decode (taken with a tile hint) agrees as well
    assert max_rel_err(gemm.linear_posit8(cx, cw, lut, tile_hint=10), exp) < TOL


@pytest.mark.parametrize("n", [16 * 1024, 1000, 15, 16 * 4096 + 7])
def test_decode_bytes(n):
    """vh_decode_bytes: every byte through the posit8 table, whole 16-byte
    rows and a ragged tail, against the oracle's values of the codes."""
    from voyager_amd import gemm, packed

    tab = T.quantization_map("posit8_1")
    g = torch.Generator().manual_seed(33)
    x = (torch.randn(n, generator=g) * 3).bfloat16()
    one = torch.tensor(1.0, dtype=torch.bfloat16)
    codes = packed.quantize_packed(x.cuda(), one.cuda(), tab.cuda())
    got = gemm.decode_bytes(codes, gemm.posit8_lut(tab.cuda())).cpu()
    assert_same_bits(got, O.quantize(x, one, qmap=tab), f"n={n}")


@pytest.mark.parametrize("M,K,N", [
    (1, 4096, 4096), (16, 4096, 4096), (1, 4096, 1024), (16, 4096, 1024), (1, 4096, 14336),
    (16, 4096, 14336), (1, 14336, 4096), (16, 14336, 4096),
    # ragged: K ranges of 0-2 blocks (empty waves), chunks padded past the
    # range end, one row per lane (M == 1) and four (M > 1), four tiles per
    # workgroup (N / 16 >= 512 with K <= 2048)
    (5, 320, 48), (1, 1088, 2048), (3, 2048, 8192), (1, 2048, 8192), (2, 960, 8192)])
def test_linear_nf4_gemv_cfg3(M, K, N):
    """Config 3's decode GEMV on baked 4-bit weights against the oracle's
    linear_mx of the same quantized operands."""
    from voyager_amd import gemm

    vt = T.quantization_map("lut4_to_int6")
    index, entries, mid = T.codebook_index_table(vt)
    stab = T.quantization_map("fp8_e5m3")
    g = torch.Generator().manual_seed(40)
    x = torch.randn(M, K, generator=g).bfloat16()
    w = (torch.randn(N, K, generator=g) * 0.02).bfloat16()
    sx, cx = O.quantize_mx(x, index, [-1], 64, 31.0, False, stab, mid)
    sw, cw = O.quantize_mx(w, index, [-1], 64, 31.0, False, stab)
    exp = O.linear_mx(cx, cw, input_scale=sx, weight_scale=sw, block_size=64, input_code=entries,
                      weight_code=entries)
    d = "cuda"
    wb = gemm.bake_nf4_weight(w.to(d), index.to(d), stab.to(d), entries.to(d))
    got = gemm.linear_nf4(x.to(d), wb, index.to(d), stab.to(d))
    assert got.dtype == torch.bfloat16 and list(got.shape) == [M, N]
    assert max_rel_err(got, exp) < TOL
    if M == 1:
        # the one-launch path (the row quantized inside the GEMV) is the
        # two-launch path bit for bit: same levels, scales and sums
        two = gemm.linear_nf4(x.to(d), wb, index.to(d), stab.to(d), fused=False)
        one = gemm.linear_nf4(x.to(d), wb, index.to(d), stab.to(d), fused=True)
        assert_same_bits(one, two, "one launch vs two")
        assert torch.equal(got, one)


@pytest.mark.parametrize("two_pass", [False, True])
@pytest.mark.parametrize("M,K,N,tile,splits", [(17, 1024, 256, 0, 0), (64, 4096, 1024, 0, 0), (300, 576, 1040, 1, 1),
                                               (300, 576, 1040, 2, 3), (2048, 4096, 4096, 0, 0), (33, 64, 16, 0, 0),
                                               (40, 4160, 48, 1, 7)])
def test_linear_nf4_prefill(M, K, N, tile, splits, two_pass):
    """MXNF4 linear_mx above the GEMV's 16 rows, on the GEMV's baked weight,
    fused (both operands decoded while the GEMM stages them) and in two
    passes (both decoded once, then the bf16 GEMM): against the oracle's
    linear_mx (1e-2), and -- both operands decoded exactly as the reference
    decodes them, which the two-pass decode shows bit for bit -- within one
    bf16 ulp of the float64 product of the oracle's decoded operands (plus
    the float32 accumulation allowance); ragged rows, columns and block
    counts, bf16 and float32 results with alpha and bias."""
    from voyager_amd import gemm, packed

    vt = T.quantization_map("lut4_to_int6")
    index, entries, mid = T.codebook_index_table(vt)
    stab = T.quantization_map("fp8_e5m3")
    g = torch.Generator().manual_seed(M + K + N)
    x = torch.randn(M, K, generator=g).bfloat16()
    x[0, :64] = 0  # an all-zero block
    w = (torch.randn(N, K, generator=g) * 0.02).bfloat16()
    sx, cx = O.quantize_mx(x, index, [-1], 64, 31.0, False, stab, mid)
    sw, cw = O.quantize_mx(w, index, [-1], 64, 31.0, False, stab)
    exp = O.linear_mx(cx, cw, input_scale=sx, weight_scale=sw, block_size=64, input_code=entries,
                      weight_code=entries)
    xd = O.dequantize_mx_parts(cx, sx, entries, 64).double()
    wd = O.dequantize_mx_parts(cw, sw, entries, 64).double()
    d = "cuda"
    wb = gemm.bake_nf4_weight(w.to(d), index.to(d), stab.to(d), entries.to(d))
    t, sp = gemm.nf4_prefill_plan(M, N, K, tile, splits)
    print(f"nf4 prefill M={M} K={K} N={N}: tile {t}, {sp} K splits", flush=True)
    if two_pass:
        px = packed.quantize_mx_packed(x.to(d), index.to(d), [-1], 64, 31.0, False, stab.to(d))
        xo, wo = gemm.nf4_decode_bf16(px, wb)
        assert torch.equal(xo.cpu().double(), xd) and torch.equal(wo.cpu().double(), wd)
    got = gemm.linear_nf4_prefill(x.to(d), wb, index.to(d), stab.to(d), tile=tile, splits=splits, two_pass=two_pass)
    assert got.dtype == torch.bfloat16 and list(got.shape) == [M, N]
    assert max_rel_err(got, exp) < TOL
    assert_within_bf16_ulps(got, xd @ wd.T, 1.0, 2.0**-14 * (xd.abs() @ wd.abs().T), "prefill")
    if M > 16 and two_pass == gemm.nf4_two_pass_pays(M, N, K):
        assert torch.equal(got, gemm.linear_nf4(x.to(d), wb, index.to(d), stab.to(d)))
    alpha = torch.tensor(0.75, device=d)
    bias = (torch.randn(N, generator=g)).bfloat16()
    got32 = gemm.linear_nf4_prefill(x.to(d), wb, index.to(d), stab.to(d), out_dtype=torch.float32, bias=bias.to(d),
                                    alpha=alpha, tile=tile, splits=splits, two_pass=two_pass)
    ref = (xd @ wd.T) * 0.75 + bias.double()
    assert max_rel_err(got32, ref) < 1e-5


@pytest.mark.parametrize("K,N", [(1024, 64), (4096, 8192)])
def test_linear_nf4_one_launch_special_blocks(K, N):
    """The one-launch M = 1 path on blocks of zeros, NaN, +-inf, tiny and
    large values, with alpha and bias and a float32 output: bit for bit the
    two-launch path, and the finite outputs within tolerance of the
    oracle."""
    from voyager_amd import gemm

    vt = T.quantization_map("lut4_to_int6")
    index, entries, mid = T.codebook_index_table(vt)
    stab = T.quantization_map("fp8_e5m3")
    g = torch.Generator().manual_seed(42)
    x = torch.randn(1, K, generator=g)
    x[0, 0:64] = 0.0
    x[0, 70] = float("nan")
    x[0, 130] = float("inf")
    x[0, 200] = -float("inf")
    x[0, 256:320] *= 1e-30
    x[0, 320:384] *= 3e4
    x = x.bfloat16()
    w = (torch.randn(N, K, generator=g) * 0.02).bfloat16()
    d = "cuda"
    wb = gemm.bake_nf4_weight(w.to(d), index.to(d), stab.to(d), entries.to(d))
    alpha = torch.tensor(0.75)
    bias = torch.randn(N, generator=g)
    args = (x.to(d), wb, index.to(d), stab.to(d), torch.float32, bias.to(d), alpha.to(d))
    two = gemm.linear_nf4(*args, fused=False)
    one = gemm.linear_nf4(*args, fused=True)
    assert_same_bits(one, two, "one launch vs two")
    sx, cx = O.quantize_mx(x, index, [-1], 64, 31.0, False, stab, mid)
    sw, cw = O.quantize_mx(w, index, [-1], 64, 31.0, False, stab)
    exp = O.linear_mx(cx, cw, input_scale=sx, weight_scale=sw, block_size=64, input_code=entries,
                      weight_code=entries).float() * 0.75 + bias
    fin = torch.isfinite(exp)
    assert torch.equal(torch.isfinite(one.cpu()), fin)
    assert max_rel_err(one.cpu()[fin], exp[fin]) < TOL


@pytest.mark.parametrize("M,K", [(1, 4096), (16, 14336), (5, 320)])
def test_quantize_mx_rows16(M, K):
    """vh_quantize_mx_rows16 (the decode GEMV's activation quantize) writes
    the same scales and level bytes as vh_quantize_mx, its scales
    block-major [K/64][16]; the scales match the oracle's bit for bit."""
    import ctypes

    from voyager_amd import _lib, formats, gemm

    vt = T.quantization_map("lut4_to_int6")
    index, entries, mid = T.codebook_index_table(vt)
    stab = T.quantization_map("fp8_e5m3")
    x = _rand((M, K), 41, 2.0)
    sx, _ = O.quantize_mx(x, index, [-1], 64, 31.0, False, stab, mid)
    d = "cuda"
    xd = x.to(d)
    ec, sc = formats.classify(index.to(d)), formats.classify(stab.to(d))
    lut = torch.arange(256, dtype=torch.uint8, device=d)
    nb = K // 64
    xs_t = torch.full((nb, 16), float("nan"), device=d)
    xl_t = torch.empty(M, K, dtype=torch.uint8, device=d)
    xs = torch.empty(M, nb, device=d)
    xl = torch.empty(M, K, dtype=torch.uint8, device=d)
    lib = _lib.load()
    _lib.check(lib.vh_quantize_mx_rows16(ctypes.c_void_p(xd.data_ptr()), _lib.VH_BF16, M, K, 64, 31.0,
                                         ctypes.byref(sc.fmt), ctypes.byref(ec.fmt), ctypes.c_void_p(xs_t.data_ptr()),
                                         ctypes.c_void_p(xl_t.data_ptr()), ctypes.c_void_p(lut.data_ptr()), None),
               "vh_quantize_mx_rows16")
    _lib.check(lib.vh_quantize_mx(ctypes.c_void_p(xd.data_ptr()), _lib.VH_BF16, M, K, 1, 64, 31.0, 0,
                                  ctypes.byref(sc.fmt), None, 0, ctypes.byref(ec.fmt), ctypes.c_void_p(xs.data_ptr()),
                                  _lib.VH_F32, 0, ctypes.c_void_p(xl.data_ptr()), _lib.VH_U8,
                                  ctypes.c_void_p(lut.data_ptr()), None), "vh_quantize_mx")
    assert torch.equal(xl_t, xl)
    assert_same_bits(xs_t[:, :M].T.contiguous().cpu(), xs.cpu(), "block-major scales")
    assert_same_bits(xs.cpu(), sx.float(), "scales vs oracle")
    assert torch.isnan(xs_t[:, M:]).all()  # rows past M untouched


@pytest.mark.parametrize("M,N,K", [(64, 256, 512), (7, 96, 160)])
def test_linear_mx_nvfp4(M, N, K):
    """NVFP4 as the reference's converted graph runs it: quantize_mx of both
    operands to fp4_e2m1 with fp8_e4m3 block scales over 16 and a float32
    global scale each (ops/quantized.py:1076-1115), then linear_mx with the
    global scales' product as alpha (:651-723); codes and scales bit-exact,
    the product within 1e-2 of the oracle and of float64."""
    fp4, e4m3 = T.quantization_map("fp4_e2m1"), T.quantization_map("fp8_e4m3")
    x, w = _rand((M, K), 31, 3.0), _rand((N, K), 32, 0.02)

    def gscale(t):
        return (t.float().abs().amax() / (6.0 * 448.0)).clamp_min(torch.finfo(torch.float32).tiny)

    gx, gw = gscale(x), gscale(w)
    exs, exc = O.quantize_mx(x, fp4, [-1], 16, 6.0, False, e4m3, None, None, gx)
    ews, ewc = O.quantize_mx(w, fp4, [-1], 16, 6.0, False, e4m3, None, None, gw)
    alpha = gx * gw
    exp = O.linear_mx(exc, ewc, input_scale=exs, weight_scale=ews, block_size=16, alpha=alpha)
    Q = torch.ops.quantized_ops
    d = lambda t: t.cuda()  # noqa: E731
    gxs, gxc = Q.quantize_mx(d(x), d(fp4), [-1], 16, 6.0, False, d(e4m3), None, None, d(gx))
    gws, gwc = Q.quantize_mx(d(w), d(fp4), [-1], 16, 6.0, False, d(e4m3), None, None, d(gw))
    for g, e, what in ((gxs, exs, "x scale"), (gxc, exc, "x codes"), (gws, ews, "w scale"), (gwc, ewc, "w codes")):
        assert_same_bits(g, e, what)
    got = Q.linear_mx(gxc, gwc, input_scale=gxs, weight_scale=gws, block_size=16, alpha=d(alpha))
    assert got.dtype == exp.dtype and max_rel_err(got, exp) < TOL
    ref64 = (O.dequantize_mx_parts(exc, exs, None, 16).double() @ O.dequantize_mx_parts(ewc, ews, None, 16).double().T
             ) * alpha.double()
    assert max_rel_err(got, ref64) < TOL


@pytest.mark.parametrize("M,N,K,batch", [(2048, 1024, 4096, 0), (512, 1030, 256, 0), (300, 520, 136, 3)])
def test_gemm_float32_results(M, N, K, batch):
    """Float32 results of the bf16 GEMM (the direct-to-LDS kernel's float32
    epilogue where the rows allow it): alpha and bias, a ragged N, and a
    batch (each batch's result at its own offset), against float64."""
    from voyager_amd import gemm

    g = torch.Generator().manual_seed(M + N)
    shape_a = (batch, M, K) if batch else (M, K)
    shape_b = (batch, N, K) if batch else (N, K)
    a = torch.randn(*shape_a, generator=g).bfloat16()
    b = (torch.randn(*shape_b, generator=g) * 0.05).bfloat16()
    bias = torch.randn(N, generator=g).bfloat16()
    alpha = torch.tensor(0.75)
    got = gemm.gemm_bf16(a.cuda(), b.cuda(), torch.float32, bias.cuda(), alpha.cuda())
    ref = (a.double() @ b.double().mT) * 0.75 + bias.double()
    assert got.dtype == torch.float32 and got.shape == ref.shape
    assert max_rel_err(got, ref) < 1e-5


def _mx8_f16_decoded(x16, ex):
    return x16.cpu().double() * torch.pow(2.0, ex.cpu().double()).unsqueeze(1)


@pytest.mark.parametrize("M,K", [(256, 4096), (7, 1024), (300, 640), (5, 6144), (3, 14336)])
def test_quantize_mx8_f16_exact(M, K):
    """The activation quantize of the small-M MX-int8 path: each row's fp16
    values times 2**E_row are exactly the reference's decoded quantize_mx
    (codes times block scales), NaN and infinities included.  Rows of up to
    256 blocks, up to 512 (two per thread kept in registers) and longer (the
    two-pass kernel)."""
    from voyager_amd import gemm

    g = torch.Generator().manual_seed(M + K)
    x = (torch.randn(M, K, generator=g) * torch.exp(torch.randn(M, 1, generator=g) * 3)).bfloat16()
    # a NaN block takes scale 1 (exponent 0) and sets its row's E; keep the
    # row's other blocks within 24 binades of it, where nothing is flushed
    x[0] = torch.randn(K, generator=g).bfloat16()
    x[0, :3] = torch.tensor([float("nan"), float("inf"), -1.0])
    x[1, 16:32] = 0.0
    tab = T.quantization_map("int8")
    s, c = O.quantize_mx(x, tab, [-1], 16, 127.0, True)
    exp = O.dequantize_mx(c, s, 16).double()
    x16, ex = gemm.quantize_mx8_f16(x.cuda())
    got = _mx8_f16_decoded(x16, ex)
    same = (got == exp) | (torch.isnan(got) & torch.isnan(exp))
    assert bool(same.all()), (~same).nonzero()[:5]


@pytest.mark.parametrize("N,K", [(64, 512), (48, 6144), (16, 20480)])
def test_mx8_f16_bake_flushes_only_far_blocks(N, K):
    """Weight baking: exact where a block is within 24 binades of its row's
    largest, zero below; rows of up to 256 blocks, up to 1024 (kept in
    registers) and longer (the two-pass kernel)."""
    from voyager_amd import gemm, packed

    g = torch.Generator().manual_seed(5)
    ew = torch.randint(-40, 1, (N, K // 16), generator=g)
    ew[:, 0] = 0
    w = (torch.randn(N, K, generator=g) * torch.pow(2.0, ew.float()).repeat_interleave(16, dim=1)).bfloat16()
    tab = T.quantization_map("int8")
    pw = packed.quantize_mx_packed(w.cuda(), tab.cuda(), [-1], 16, 127.0, True)
    s, c = O.quantize_mx(w, tab, [-1], 16, 127.0, True)
    exp = O.dequantize_mx(c, s, 16).double()
    bw = gemm.bake_mx8_f16(pw.codes.view(torch.int8), pw.scale, pw.bias)
    got = _mx8_f16_decoded(bw.w, bw.e)
    e_blk = torch.floor(torch.log2(exp.abs().view(N, K // 16, 16).amax(-1).clamp_min(1e-300))).repeat_interleave(16, 1)
    far = e_blk < (e_blk.amax(1, keepdim=True) - 24 + 1)  # within the flush margin of a block's code range
    assert torch.equal(got[~far], exp[~far])
    assert bool((got[far].abs() <= exp[far].abs()).all())


@pytest.mark.parametrize("M,N,K,tile,splits", [(256, 4096, 4096, -1, 0), (256, 4096, 4096, 1, 2),
                                               (256, 4096, 4096, 2, 2), (256, 4096, 4096, 3, 8),
                                               (33, 520, 1024, -1, 0), (130, 264, 768, 0, 3),
                                               # one split: the GEMM's own epilogue (ragged rows and
                                               # tiles), and N % 8 != 0 through the reduction
                                               (2048, 4096, 1024, -1, 0), (256, 4096, 4096, 1, 1),
                                               (130, 264, 768, 0, 1), (33, 520, 1024, 2, 1),
                                               (1100, 136, 512, 3, 1), (50, 260, 512, 0, 1),
                                               # the 64x64 small-M tile: automatic at M <= 256, ragged
                                               # rows and tiles, its own epilogue and split
                                               (16, 4096, 4096, -1, 0), (256, 4096, 4096, 4, 1),
                                               (33, 520, 1024, 4, 1), (130, 264, 768, 4, 2)])
def test_linear_mx8_f16(M, N, K, tile, splits):
    """The small-M MX-int8 linear on exact fp16 operands against the exact
    float64 product of the reference's decoded operands, bf16 and fp32
    results (alpha and bias in the reduction's epilogue, or the GEMM's own
    with one split)."""
    from voyager_amd import gemm, packed

    tab = T.quantization_map("int8").cuda()
    x = _rand((M, K), 40).cuda()
    w = _rand((N, K), 41, 0.02).cuda()
    px = packed.quantize_mx_packed(x, tab, [-1], 16, 127.0, True)
    pw = packed.quantize_mx_packed(w, tab, [-1], 16, 127.0, True)
    ref = _deq_mxint8(px) @ _deq_mxint8(pw).T
    bw = gemm.bake_mx8_f16(pw.codes.view(torch.int8), pw.scale, pw.bias)
    x16, ex = gemm.quantize_mx8_f16(x)
    got = gemm.linear_mx8_f16(x16, ex, bw, tile=tile, splits=splits)
    assert got.dtype == torch.bfloat16
    assert max_rel_err(got, ref) < TOL
    alpha = torch.tensor(0.75, device="cuda")
    bias = _rand((N,), 42).cuda()
    got32 = gemm.linear_mx8_f16(x16, ex, bw, out_dtype=torch.float32, bias=bias, alpha=alpha, tile=tile,
                                splits=splits)
    assert max_rel_err(got32, ref * 0.75 + bias.cpu().double()) < 1e-5
    # the packed path's result agrees
    old = gemm.linear_mxint8(px.codes, px.scale, pw.codes, pw.scale, 16, px.bias, pw.bias)
    assert max_rel_err(got, old) < TOL


@pytest.mark.parametrize("M", [256, 100])
def test_mx8_f16_small_tile_matches(M):
    """One split: every tile accumulates each output over K in the same
    order, so the 64x64 tile's result is the 64x128 tile's bit for bit."""
    from voyager_amd import gemm, packed

    tab = T.quantization_map("int8").cuda()
    x = _rand((M, 4096), 43).cuda()
    w = _rand((1024, 4096), 44, 0.02).cuda()
    pw = packed.quantize_mx_packed(w, tab, [-1], 16, 127.0, True)
    bw = gemm.bake_mx8_f16(pw.codes.view(torch.int8), pw.scale, pw.bias)
    x16, ex = gemm.quantize_mx8_f16(x)
    a = gemm.linear_mx8_f16(x16, ex, bw, tile=1, splits=1)
    b = gemm.linear_mx8_f16(x16, ex, bw, tile=4, splits=1)
    assert torch.equal(a, b)
    assert gemm.mx8_f16_plan(M, 4096, 4096)[0] == 4
