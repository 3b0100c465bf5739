"""quantize / dequantize / packed codes on the GPU against the oracle."""

import pytest
import torch

import voyager_amd.library  # noqa: F401  (defines quantized_ops)
from helpers import assert_same_bits
from oracle import ops as O
from oracle import tables as T

pytestmark = pytest.mark.gpu


def _specials(n, g, scale=4.0, dtype=torch.bfloat16):
    x = torch.randn(n, generator=g) * scale
    sp = torch.tensor([0.0, -0.0, float("inf"), -float("inf"), float("nan"), 1e-40, -1e-39, 3e38, -3e38,
                       0.5, 1.5, 2.5, -2.5, 447.0, 449.0, 464.0, 480.0, 2.0**-133, 2.0**-126])
    x[: sp.numel()] = sp
    return x.to(dtype)


@pytest.mark.parametrize("dtype", ["int8", "fp8_e4m3", "posit8_1", "uint2", "fp8_e5m3", "lut4_to_int6"])
@pytest.mark.parametrize("scale", [1.0, 0.0173, 3.5])
def test_quantize_per_tensor(dtype, scale):
    g = torch.Generator().manual_seed(11)
    x = _specials(10007, g)
    s = torch.tensor(scale, dtype=torch.bfloat16)
    tab = T.quantization_map(dtype)
    exp = O.quantize(x, s, qmap=tab)
    got = torch.ops.quantized_ops.quantize(x.cuda(), s.cuda(), qmap=tab.cuda())
    assert_same_bits(got, exp, dtype)


def test_quantize_no_map_and_zero_point():
    g = torch.Generator().manual_seed(12)
    x = _specials(4096, g).view(64, 64)
    s = (torch.rand(64, 1, generator=g) + 0.1).bfloat16()
    z = (torch.randn(64, 1, generator=g)).bfloat16()
    assert_same_bits(torch.ops.quantized_ops.quantize(x.cuda(), s.cuda()), O.quantize(x, s), "no map")
    tab = T.quantization_map("uint2")
    exp = O.quantize(x, s, z, qmap=tab)
    got = torch.ops.quantized_ops.quantize(x.cuda(), s.cuda(), z.cuda(), qmap=tab.cuda())
    assert_same_bits(got, exp, "zero point")


def test_quantize_block_scales_and_layouts():
    g = torch.Generator().manual_seed(13)
    x = _specials(8 * 8 * 40 * 24, g).view(8, 8, 40, 24)
    s = (torch.rand(8, 8, 2, 24, generator=g) + 0.05).bfloat16()  # blocks of 32 along dim 2 (partial)
    z = torch.randn(8, 8, 2, 24, generator=g).bfloat16()
    tab = T.quantization_map("uint2")
    exp = O.quantize(x, s, z, [-2], 32, tab)
    got = torch.ops.quantized_ops.quantize(x.cuda(), s.cuda(), z.cuda(), [-2], 32, tab.cuda())
    assert_same_bits(got, exp, "blocked")
    # a permuted (dense) input keeps its layout
    xp = x.permute(0, 2, 1, 3)
    sp = s.permute(0, 2, 1, 3)
    exp = O.quantize(xp, sp, None, [1], 32, tab)
    got = torch.ops.quantized_ops.quantize(xp.cuda(), sp.cuda(), None, [1], 32, tab.cuda())
    assert got.stride() == xp.stride()
    assert_same_bits(got, exp, "permuted")


def test_quantize_float32_input():
    g = torch.Generator().manual_seed(14)
    x = _specials(5000, g, dtype=torch.float32)
    s = torch.tensor(0.37)
    tab = T.quantization_map("fp8_e4m3")
    exp = O.quantize(x, s, qmap=tab)
    got = torch.ops.quantized_ops.quantize(x.cuda(), s.cuda(), qmap=tab.cuda())
    assert_same_bits(got, exp, "fp32")


@pytest.mark.parametrize("dtype", ["int8", "fp8_e4m3", "posit8_1", "fp8_e5m3"])
def test_dequantize(dtype):
    g = torch.Generator().manual_seed(15)
    tab = T.quantization_map(dtype)
    x = O.quantize(_specials(3000, g), torch.tensor(0.25, dtype=torch.bfloat16), qmap=tab)
    s = torch.tensor(0.031, dtype=torch.bfloat16)
    ident = T.quantization_map(None)
    exp = O.dequantize(x, s, input_qmap=ident)
    got = torch.ops.quantized_ops.dequantize(x.cuda(), s.cuda(), input_qmap=ident.cuda())
    assert_same_bits(got, exp, "dequantize")
    i6 = T.quantization_map("int6")
    exp = O.dequantize(x, s, None, None, None, tab, i6)
    got = torch.ops.quantized_ops.dequantize(x.cuda(), s.cuda(), None, None, None, tab.cuda(), i6.cuda())
    assert_same_bits(got, exp, "dequantize with maps")


def test_dequantize_group_zero_point():
    g = torch.Generator().manual_seed(16)
    codes = torch.randint(0, 4, (2, 8, 64, 128), generator=g).bfloat16()
    s = (torch.rand(2, 8, 2, 128, generator=g) + 0.01).bfloat16()
    z = torch.randn(2, 8, 2, 128, generator=g).bfloat16()
    exp = O.dequantize(codes, s, z, [-2], 32)
    got = torch.ops.quantized_ops.dequantize(codes.cuda(), s.cuda(), z.cuda(), [-2], 32)
    assert_same_bits(got, exp, "kivi keys")


@pytest.mark.parametrize("dtype", ["int8", "fp8_e4m3", "posit8_1", "lut4_to_int6"])
def test_packed_codes_roundtrip(dtype):
    from voyager_amd import packed

    g = torch.Generator().manual_seed(17)
    x = _specials(9000, g)
    s = torch.tensor(0.5, dtype=torch.bfloat16)
    tab = T.quantization_map(dtype)
    exp = O.quantize(x, s, qmap=tab)
    codes = packed.quantize_packed(x.cuda(), s.cuda(), tab.cuda())
    assert codes.dtype == torch.uint8
    back = packed.unpack_codes(codes, tab.cuda())
    if dtype == "int8":  # packed int8 holds neither NaN nor -0: both pack as code 0
        exp = torch.where(torch.isnan(exp) | (exp == 0), torch.zeros_like(exp), exp)
    assert_same_bits(back, exp, dtype)
    if dtype == "fp8_e4m3":  # the bytes are OCP E4M3
        ref = exp.float().to(torch.float8_e4m3fn).view(torch.uint8)
        fin = ~torch.isnan(exp)
        assert torch.equal(codes.cpu()[fin], ref[fin])


def test_cpu_tensor_fails_loudly():
    x = torch.randn(16).bfloat16()
    with pytest.raises((RuntimeError, NotImplementedError)):
        torch.ops.quantized_ops.quantize(x, torch.tensor(1.0, dtype=torch.bfloat16))


@pytest.mark.parametrize("scale", [1.0, 0.0173, 3.5, 0.0078125, 2.0**-130, 1.5e38])
def test_quantize_packed_e4m3_every_bf16_pattern(scale):
    """The per-tensor E4M3 fast path (packed bytes for the FP8 GEMM): all
    65,536 bf16 patterns against the oracle's quantize, read back through the
    table entry's E4M3 byte.  A subnormal and a huge scale force the exact
    fallback; 0.0173 puts many quotients next to bf16 rounding midpoints."""
    from voyager_amd import packed

    x = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    s = torch.tensor(scale, dtype=torch.bfloat16)
    tab = T.quantization_map("fp8_e4m3")
    exp = O.quantize(x, s, qmap=tab)  # table values (bf16)
    got = packed.quantize_packed(x.cuda(), s.cuda(), tab.cuda()).cpu()
    back = packed.unpack_codes(got.cuda(), tab.cuda()).cpu()
    assert_same_bits(back, exp, f"scale {scale}")
    # the packed byte is the OCP E4M3 encoding of the table value, sign of zero included
    ref = exp.float().to(torch.float8_e4m3fn).view(torch.uint8)
    fin = ~torch.isnan(exp)
    assert torch.equal(got[fin], ref[fin])


def test_quantize_packed_e4m3_large_ragged():
    """The per-tensor E4M3 fast path on a tensor large enough for its
    8-groups-per-thread variant (over 2^24 elements), with a last workgroup
    that is partly past the end: every bf16 pattern 257 times, then 40 more."""
    from voyager_amd import packed

    pat = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    s = torch.tensor(0.0173, dtype=torch.bfloat16)
    tab = T.quantization_map("fp8_e4m3")
    exp = packed.quantize_packed(pat.cuda(), s.cuda(), tab.cuda()).cpu()
    back = packed.unpack_codes(exp.cuda(), tab.cuda()).cpu()
    assert_same_bits(back, O.quantize(pat, s, qmap=tab), "patterns")
    x = torch.cat([pat.cuda().repeat(257), pat[:40].cuda()])
    got = packed.quantize_packed(x, s.cuda(), tab.cuda())
    assert torch.equal(got[: 257 * 65536].view(257, 65536), exp.cuda().expand(257, 65536))
    assert torch.equal(got[257 * 65536:].cpu(), exp[:40])


@pytest.mark.parametrize("scale", [1.0, 0.0173, 0.25])
def test_posit8_elementwise_at_config4_size(scale):
    """Config 4's elementwise leg at its size: every bf16 pattern 1030 times
    plus a 48-element tail (67,502,128 elements, more than the config's
    64M) through the posit table quantize, packed and reference form, and the
    packed dequantize, with a unit, a general and a power-of-two scale.  At this size the quantize's
    grid-stride loop (256 workgroups x 1024 threads x 4 vectors a pass) runs
    nine passes, alternating its two load buffers, and the dequantize's
    gather loop (4096 workgroups, 65,536 units of 1024 codes a pass) a second,
    partial pass; the tail's last workgroup ends past the end.  Every
    65,536-pattern block is bit-exact against the oracle."""
    from voyager_amd import formats, packed
    from voyager_amd.ops import _elementwise

    R, tail = 1030, 48
    n = R * 65536 + tail
    # vectors of 8 past eight quantize passes; units of 1024 codes past one gather pass
    assert n % 16 == 0 and n // 8 > 8 * 256 * 1024 * 4 and n // 1024 > 4096 * 4 * 4
    pat = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    s = torch.tensor(scale, dtype=torch.bfloat16)
    s2 = torch.tensor(0.375, dtype=torch.bfloat16)
    tab = T.quantization_map("posit8_1")
    exp_ref = O.quantize(pat, s, qmap=tab)
    exp_deq = O.dequantize(exp_ref, s2)
    tab_d, s_d, s2_d = tab.cuda(), s.cuda(), s2.cuda()
    x = torch.cat([pat.cuda().repeat(R), pat[:tail].cuda()])

    def blocks(t):
        return t[: R * 65536].view(R, 65536)

    def check(got, exp, what):
        # the pattern block once against the oracle, then every repeat and the tail against it on the GPU
        assert_same_bits(got[:65536].cpu(), exp, what)
        g16 = got.view(torch.int16)
        assert torch.equal(blocks(g16), g16[:65536].expand(R, 65536)), what
        assert torch.equal(g16[R * 65536:], g16[:tail]), what

    ref = torch.ops.quantized_ops.quantize(x, s_d, qmap=tab_d)
    check(ref, exp_ref, "reference form")
    del ref
    codes = packed.quantize_packed(x, s_d, tab_d)
    assert torch.equal(blocks(codes), codes[:65536].expand(R, 65536)) and torch.equal(codes[R * 65536:],
                                                                                     codes[:tail])
    del x
    check(packed.unpack_codes(codes, tab_d), exp_ref, "packed, read back")
    deq = _elementwise("dequantize", codes, s2_d, None, None, torch.bfloat16, formats.classify(tab_d).fmt, None,
                       torch.bfloat16)
    check(deq, exp_deq, "packed dequantize with a scale")


@pytest.mark.parametrize("dtype", ["posit8_1", "posit8_0", "posit8_2", "posit16_1"])
@pytest.mark.parametrize("scale", [1.0, 0.0173, 3.5, 2.0**-130, 1.5e38, 0.25, 2.0**-20, 2.0**100, 2.0**-120])
def test_quantize_posit_every_bf16_pattern(dtype, scale):
    """The posit table path (per-tensor scale, whole 16-byte rows): all
    65,536 bf16 patterns, reference form and (8-bit posits) packed codes read
    back through the code table, against the oracle's closed-form posit
    rounding.  The patterns cover zero, the flush region below the threshold,
    the saturating region above maxpos and the non-finite inputs; the
    subnormal and huge scales force the exact-division fallback; a unit scale
    takes q = x, and the other powers of two skip the rounding-midpoint test
    (their quotients, subnormal and overflowing ones included, are the
    products by the exact reciprocal)."""
    from voyager_amd import packed

    x = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    s = torch.tensor(scale, dtype=torch.bfloat16)
    tab = T.quantization_map(dtype)
    exp = O.quantize(x, s, qmap=tab)
    got = torch.ops.quantized_ops.quantize(x.cuda(), s.cuda(), qmap=tab.cuda()).cpu()
    assert_same_bits(got, exp, f"{dtype} reference form, scale {scale}")
    if dtype.startswith("posit8"):
        codes = packed.quantize_packed(x.cuda(), s.cuda(), tab.cuda())
        back = packed.unpack_codes(codes, tab.cuda()).cpu()
        assert_same_bits(back, exp, f"{dtype} packed, scale {scale}")


@pytest.mark.parametrize("dtype", ["posit8_1", "int8", "fp8_e4m3", "fp8_e5m3", "uint2"])
@pytest.mark.parametrize("scale", [None, 0.0173, 3.5])
def test_dequantize_packed_table(dtype, scale):
    """dequantize of packed codes to bf16 (the per-workgroup 256-entry table
    path, taken for whole 16-code rows): every code, with and without a
    scalar scale, against the oracle's dequantize of the reference-form
    values.  A 40-code tail that takes the generic kernel must agree too."""
    from voyager_amd import formats, packed
    from voyager_amd.ops import _elementwise

    tab = T.quantization_map(dtype)
    g = torch.Generator().manual_seed(21)
    x = _specials(4096 * 16, g)
    codes = packed.quantize_packed(x.cuda(), torch.tensor(1.0, dtype=torch.bfloat16).cuda(), tab.cuda())
    vals = O.quantize(x, torch.tensor(1.0, dtype=torch.bfloat16), qmap=tab)
    if "int" in dtype:  # an integer code has no negative zero or NaN: both pack as code 0
        vals = torch.where((vals == 0) | torch.isnan(vals), torch.zeros_like(vals), vals)
    fmt = formats.classify(tab.cuda()).fmt
    for n in (codes.numel(), 40):
        c, v = codes[:n], vals[:n]
        if scale is None:
            got = _elementwise("dequantize", c, None, None, None, torch.bfloat16, fmt, None, torch.bfloat16).cpu()
            assert_same_bits(got, v, f"{dtype} n={n}")
        else:
            sv = torch.tensor(scale, dtype=torch.bfloat16)
            got = _elementwise("dequantize", c, sv.cuda(), None, None, torch.bfloat16, fmt, None,
                               torch.bfloat16).cpu()
            assert_same_bits(got, O.dequantize(v, sv), f"{dtype} n={n} scale {scale}")


@pytest.mark.parametrize("op", ["quantize", "dequantize"])
@pytest.mark.parametrize("sdtype", [torch.float32, torch.float16])
def test_zero_dim_scale_of_another_dtype(op, sdtype):
    """A bf16 tensor with a 0-d float32 / float16 scale and zero point, as
    eager torch (CPU) combines them: the division (multiplication) by the
    scale at its own precision, rounded once to bf16; the zero point
    rounded to bf16 before it is added (subtracted)."""
    g = torch.Generator().manual_seed(77)
    x = (torch.randn(64, 128, generator=g) * 5).bfloat16()
    s = torch.tensor(0.0123456789, dtype=sdtype)
    zp = torch.tensor(3.3, dtype=sdtype)
    tab = T.quantization_map("int8")
    if op == "quantize":
        exp = O.quantize(x, s, zp, qmap=tab)
        got = torch.ops.quantized_ops.quantize(x.cuda(), s.cuda(), zp.cuda(), qmap=tab.cuda())
    else:
        exp = O.dequantize(x, s, zp)
        got = torch.ops.quantized_ops.dequantize(x.cuda(), s.cuda(), zp.cuda())
    assert got.dtype == exp.dtype == torch.bfloat16
    assert_same_bits(got, exp, f"{op} {sdtype}")


@pytest.mark.parametrize("n", [8 * 1000 + 8 * 7, 8 * ((1 << 21) + 333)])
def test_stream_2to1_writes_each_high_byte(n):
    """The bench's streaming ceiling kernel (vh_stream_2to1) reads every
    16-byte group and writes its elements' high bytes: a ragged size on the
    4-group path and one past 2^21 groups on the 8-group path."""
    import ctypes

    from voyager_amd import _lib

    x = torch.randint(-32768, 32768, (n,), dtype=torch.int32).to(torch.int16).cuda()
    out = torch.full((n,), 7, dtype=torch.uint8, device="cuda")
    st = _lib.load().vh_stream_2to1(ctypes.c_void_p(x.data_ptr()), n // 8, ctypes.c_void_p(out.data_ptr()),
                                    ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    _lib.check(st, "vh_stream_2to1")
    exp = ((x.int() >> 8) & 0xFF).to(torch.uint8)
    assert torch.equal(out, exp)
