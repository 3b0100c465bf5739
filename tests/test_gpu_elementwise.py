"""quantize / dequantize / packed codes on the GPU against the oracle."""

import pytest
import torch

import voyager_amd  # noqa: F401  (registers quantized_ops)
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
