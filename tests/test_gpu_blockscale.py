"""quantize_mx / calculate_mx_qparam / dequantize_mx / quantize_affine on the
GPU against the oracle, at the configs' shapes and on edge blocks."""

import pytest
import torch

import voyager_amd.library  # noqa: F401  (defines quantized_ops)
from helpers import assert_same_bits
from oracle import ops as O
from oracle import tables as T

pytestmark = pytest.mark.gpu


def cfg1_x():
    """Config 1's activations: seed 0, N(0,1) [256,4096], 0.1% outliers x20."""
    g = torch.Generator().manual_seed(0)
    x = torch.randn(256, 4096, generator=g)
    out = torch.rand(256, 4096, generator=g) < 0.001
    return torch.where(out, x * 20, x).bfloat16(), g


def test_mxint8_cfg1_activation():
    x, _ = cfg1_x()
    tab = T.quantization_map("int8")
    es, ec = O.quantize_mx(x, tab, [-1], 16, 127.0, True)
    gs, gc = torch.ops.quantized_ops.quantize_mx(x.cuda(), tab.cuda(), [-1], 16, 127.0, True)
    assert_same_bits(gs, es, "scale")
    assert_same_bits(gc, ec, "codes")
    assert_same_bits(torch.ops.quantized_ops.calculate_mx_qparam(x.cuda(), [-1], 16, 127.0, True), es, "qparam")


def test_mxint8_packed_matches_ref_form():
    from voyager_amd import packed

    x, _ = cfg1_x()
    tab = T.quantization_map("int8")
    es, ec = O.quantize_mx(x, tab, [-1], 16, 127.0, True)
    p = packed.quantize_mx_packed(x.cuda(), tab.cuda(), [-1], 16, 127.0, True)
    assert_same_bits(packed.unpack_mx_scale(p), es, "packed scale")
    # packed int8 has no -0: compare codes with -0 read as +0
    ec = torch.where(ec == 0, torch.zeros_like(ec), ec)
    assert_same_bits(packed.unpack_codes(p.codes, tab.cuda()), ec, "packed codes")


def _edge_blocks(block):
    rows = [
        [0.0] * block,
        [float("nan")] + [1.0] * (block - 1),
        [float("inf")] + [1.0] * (block - 1),
        [-float("inf")] + [2.0] * (block - 1),
        [2.0**-127] + [0.0] * (block - 1),
        [2.0**-128] + [2.0**-130] * (block - 1),
        [3e38] + [1.0] * (block - 1),
        [127.5, -127.5] + [0.25] * (block - 2),
        [-0.0] * block,
        [1e-40, -2e-40] + [0.0] * (block - 2),
    ]
    return torch.tensor(rows, dtype=torch.float32).bfloat16()


@pytest.mark.parametrize("block", [16, 32, 64])
def test_mx_edge_blocks(block):
    x = _edge_blocks(block)
    for dtype, qmax in [("int8", 127.0), ("fp8_e4m3", 448.0)]:
        tab = T.quantization_map(dtype)
        es, ec = O.quantize_mx(x, tab, [-1], block, qmax, True)
        gs, gc = torch.ops.quantized_ops.quantize_mx(x.cuda(), tab.cuda(), [-1], block, qmax, True)
        assert_same_bits(gs, es, f"{dtype} scale")
        assert_same_bits(gc, ec, f"{dtype} codes")


@pytest.mark.parametrize("dtype", ["lut4_to_int6", "lut3_to_int4", "lut2_to_int3"])
@pytest.mark.parametrize("rows,L", [(1, 4096), (16, 1024), (10, 640), (512, 1024)])
def test_mx_index_packed_edge_blocks(dtype, rows, L):
    """Packed codebook indices and E5M3 scale bytes -- the decode-size lane
    kernel up to 2**18 elements, the eight-per-thread row kernel beyond --
    for codebooks of 16, 8 and 4 levels (15, 7 and 3 thresholds: the key
    table is padded past them), on blocks of zeros, NaN, +-inf, subnormals
    and huge values among random ones of a wide range: the oracle's indices
    and scales bit for bit."""
    from voyager_amd import packed

    vt = T.quantization_map(dtype)
    index, entries, mid = T.codebook_index_table(vt)
    qmax = float(entries.abs().max())
    stab = T.quantization_map("fp8_e5m3")
    g = torch.Generator().manual_seed(rows * L)
    x = torch.randn(rows, L, generator=g) * torch.exp(torch.randn(rows, L, generator=g) * 2)
    e = _edge_blocks(64).float()
    nb = min(e.shape[0], L // 64)
    x[0, :nb * 64] = e[:nb].reshape(-1)
    x[-1, L - nb * 64:] = e[:nb].flip(0).reshape(-1)
    x = x.bfloat16()
    es, ec = O.quantize_mx(x, index, [-1], 64, qmax, False, stab)
    p = packed.quantize_mx_packed(x.cuda(), index.cuda(), [-1], 64, qmax, False, stab.cuda())
    assert torch.equal(p.codes.cpu().to(torch.int64), ec.to(torch.int64)), f"{dtype} indices"
    assert_same_bits(packed.unpack_mx_scale(p), es, f"{dtype} scales")


def test_mxnf4_cfg3_shapes():
    vt = T.quantization_map("lut4_to_int6")
    index, entries, mid = T.codebook_index_table(vt)
    stab = T.quantization_map("fp8_e5m3")
    g = torch.Generator().manual_seed(1)
    for shape, sc in [((1, 4096), 1.0), ((16, 14336), 1.0), ((1024, 4096), 0.02)]:
        x = (torch.randn(*shape, generator=g) * sc).bfloat16()
        es, ec = O.quantize_mx(x, index, [-1], 64, 31.0, False, stab, mid)
        gs, gc = torch.ops.quantized_ops.quantize_mx(x.cuda(), index.cuda(), [-1], 64, 31.0, False, stab.cuda(),
                                                     mid.cuda())
        assert_same_bits(gs, es, f"scale {shape}")
        assert_same_bits(gc, ec, f"codes {shape}")
        # decode and scale, as linear_mx does
        exp = O.dequantize_mx(ec, es, 64, entries)
        got = torch.ops.quantized_ops.dequantize_mx(gc, gs, 64, entries.cuda())
        assert_same_bits(got, exp, f"dequantize_mx {shape}")


def test_decode_table_follows_the_codebook_tensor():
    """dequantize_mx with per-call codebooks (ops/quantized.py:290-315): a
    second, different 16-entry codebook allocated where a freed one lived
    (same size, same address, version 0) must decode with its own entries,
    and an in-place change to a codebook must be seen."""
    g = torch.Generator().manual_seed(11)
    codes = torch.randint(0, 16, (64, 128), generator=g).to(torch.bfloat16)
    scale = torch.pow(2.0, torch.randint(-3, 3, (64, 2), generator=g).float()).bfloat16()
    books = [torch.randn(16, generator=g).bfloat16() for _ in range(3)]
    ptrs = []
    for book in books:
        dev = book.cuda()
        ptrs.append(dev.data_ptr())
        got = torch.ops.quantized_ops.dequantize_mx(codes.cuda(), scale.cuda(), 64, dev)
        assert_same_bits(got, O.dequantize_mx(codes, scale, 64, book), f"codebook at {dev.data_ptr():#x}")
        del dev, got
        torch.cuda.synchronize()
    # the caching allocator hands the freed block back: the case a pointer-keyed cache got wrong
    assert len(set(ptrs)) < len(ptrs)
    dev = books[0].cuda()
    torch.ops.quantized_ops.dequantize_mx(codes.cuda(), scale.cuda(), 64, dev)
    dev.mul_(-2)
    got = torch.ops.quantized_ops.dequantize_mx(codes.cuda(), scale.cuda(), 64, dev)
    assert_same_bits(got, O.dequantize_mx(codes, scale, 64, (books[0] * -2).bfloat16()), "after an in-place change")


def test_mx_generic_paths():
    """Column blocks (axis 0), partial blocks, odd lengths, fp32 input."""
    g = torch.Generator().manual_seed(6)
    tab = T.quantization_map("int8")
    x = (torch.randn(50, 37, generator=g) * 3).bfloat16()
    for axes in ([0], [-1], [1]):
        es, ec = O.quantize_mx(x, tab, axes, 16, 127.0, True)
        gs, gc = torch.ops.quantized_ops.quantize_mx(x.cuda(), tab.cuda(), axes, 16, 127.0, True)
        assert_same_bits(gs, es, f"scale axes={axes}")
        assert_same_bits(gc, ec, f"codes axes={axes}")
    xf = (torch.randn(8, 96, generator=g) * 5).float()
    es, ec = O.quantize_mx(xf, tab, [-1], 32, 127.0, True)
    gs, gc = torch.ops.quantized_ops.quantize_mx(xf.cuda(), tab.cuda(), [-1], 32, 127.0, True)
    assert_same_bits(gs, es, "fp32 scale")
    assert_same_bits(gc, ec, "fp32 codes")
    # partial last block on the row path (L % 8 == 0, L % block != 0)
    x2 = (torch.randn(7, 40, generator=g)).bfloat16()
    es, ec = O.quantize_mx(x2, tab, [-1], 16, 127.0, True)
    gs, gc = torch.ops.quantized_ops.quantize_mx(x2.cuda(), tab.cuda(), [-1], 16, 127.0, True)
    assert_same_bits(gs, es, "partial scale")
    assert_same_bits(gc, ec, "partial codes")


def test_mx_nonpot_without_scale_map():
    g = torch.Generator().manual_seed(7)
    x = (torch.randn(32, 256, generator=g)).bfloat16()
    tab = T.quantization_map("fp8_e4m3")
    es, ec = O.quantize_mx(x, tab, [-1], 32, 448.0, False)
    gs, gc = torch.ops.quantized_ops.quantize_mx(x.cuda(), tab.cuda(), [-1], 32, 448.0, False)
    assert_same_bits(gs, es, "scale")
    assert_same_bits(gc, ec, "codes")


@pytest.mark.parametrize("axis", [-2, -1])
def test_quantize_affine_kivi(axis):
    """KIVI 2-bit: keys grouped along tokens (axis -2), values along channels
    (axis -1), group 32, fp16_e5m10 scale/zero-point map."""
    g = torch.Generator().manual_seed(8)
    x = torch.randn(2, 8, 256, 128, generator=g).bfloat16()
    x[0, 0, :3, :5] = torch.tensor(float("nan"))
    x[1, 2, 5, :] = 7.0  # constant rows / columns
    qtab = T.quantization_map("uint2")
    stab = T.quantization_map("fp16_e5m10")
    es, ez, ev = O.quantize_affine(x, qtab, [axis], 32, 0.0, 3.0, stab)
    gs, gz, gv = torch.ops.quantized_ops.quantize_affine(x.cuda(), qtab.cuda(), [axis], 32, 0.0, 3.0, stab.cuda())
    assert_same_bits(gs, es, "scale")
    assert_same_bits(gz, ez, "zero point")
    assert_same_bits(gv, ev, "codes")
    # read back (dequantize with the group zero point)
    exp = O.dequantize(ev, es, ez, [axis], 32)
    got = torch.ops.quantized_ops.dequantize(gv, gs, gz, [axis], 32)
    assert_same_bits(got, exp, "dequantize")


def test_quantize_affine_partial_blocks():
    g = torch.Generator().manual_seed(9)
    x = torch.randn(3, 50, 24, generator=g).bfloat16()
    qtab = T.quantization_map("uint2")
    for axis in (-2, -1):
        es, ez, ev = O.quantize_affine(x, qtab, [axis], 32, 0.0, 3.0)
        gs, gz, gv = torch.ops.quantized_ops.quantize_affine(x.cuda(), qtab.cuda(), [axis], 32, 0.0, 3.0)
        assert_same_bits(gs, es, f"scale {axis}")
        assert_same_bits(gz, ez, f"zp {axis}")
        assert_same_bits(gv, ev, f"codes {axis}")


@pytest.mark.parametrize("gdtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", [(64, 256), (3, 16, 96)])
def test_nvfp4_global_scale_bit_exact(gdtype, shape):
    """NVFP4's two-level scaling (ops/quantized.py:1016-1021, 1094-1115):
    fp4_e2m1 codes, fp8_e4m3 block scales over 16 elements, and a 0-d
    global scale that divides out the tensor's magnitude before the block
    scales are quantized and multiplies them back into the elements'
    divisor; calculate_mx_qparam and quantize_mx bit-exact."""
    g = torch.Generator().manual_seed(sum(shape))
    x = (torch.randn(*shape, generator=g) * 7).bfloat16()
    fp4, e4m3 = T.quantization_map("fp4_e2m1"), T.quantization_map("fp8_e4m3")
    gs = (x.float().abs().amax() / (6.0 * 448.0)).clamp_min(torch.finfo(torch.float32).tiny).to(gdtype)
    es = O.calculate_mx_qparam(x, [-1], 16, 6.0, False, e4m3, gs)
    got = torch.ops.quantized_ops.calculate_mx_qparam(x.cuda(), [-1], 16, 6.0, False, e4m3.cuda(), gs.cuda())
    assert_same_bits(got, es, "scale")
    es2, ec2 = O.quantize_mx(x, fp4, [-1], 16, 6.0, False, e4m3, None, None, gs)
    gs2, gc2 = torch.ops.quantized_ops.quantize_mx(x.cuda(), fp4.cuda(), [-1], 16, 6.0, False, e4m3.cuda(), None,
                                                   None, gs.cuda())
    assert_same_bits(gs2, es2, "quantize_mx scale")
    assert_same_bits(gc2, ec2, "quantize_mx codes")
