"""Stochastic rounding on the GPU (``vh_quantize_sr``) against the oracle's
restatement of ``ops/quantized.py:318-515``: codes bit-exact (NaN as NaN)
for tables and codebooks, per-tensor and block scales, zero points, fp32
and bf16 inputs, permuted layouts, specials, and ``quantize_mx`` with a
seed."""

import pytest
import torch

import voyager_amd.library  # noqa: F401  (defines quantized_ops)
from helpers import assert_same_bits
from oracle import ops as O
from oracle import tables as T

pytestmark = pytest.mark.gpu

Q = torch.ops.quantized_ops
DEV = "cuda"


def _x(shape, seed, scale=3.0, dtype=torch.bfloat16, specials=True):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(*shape, generator=g) * scale).to(dtype)
    if specials and x.numel() >= 8:
        x.view(-1)[:8] = torch.tensor([float("nan"), float("inf"), -float("inf"), 0.0, -0.0, 1e6, -1e-30, 2.5])
    return x


SEEDS = [0, 1, 2**40 + 3, -5]


@pytest.mark.parametrize("name", ["int8", "int4", "fp4_e2m1", "fp8_e4m3", "posit8_1", "uint2"])
@pytest.mark.parametrize("seed", SEEDS)
def test_quantize_sr_tables(name, seed):
    tab = T.quantization_map(name)
    x = _x((33, 65), 1)
    s = torch.tensor(0.75, dtype=torch.bfloat16)
    sd = torch.tensor(seed, dtype=torch.int64)
    exp = O.quantize(x, s, qmap=tab, seed=sd)
    got = Q.quantize(x.to(DEV), s.to(DEV), qmap=tab.to(DEV), seed=sd.to(DEV))
    assert_same_bits(got, exp, f"{name} seed={seed}")


@pytest.mark.parametrize("case", ["fp32 input", "zero point", "block scale", "permuted", "ragged", "codebook"])
def test_quantize_sr_variants(case):
    tab = T.quantization_map("int8")
    sd = torch.tensor(123456789, dtype=torch.int64)
    s, zp, bs = torch.tensor(0.5, dtype=torch.bfloat16), None, None
    if case == "fp32 input":
        x = _x((17, 40), 2, dtype=torch.float32)
        s = torch.tensor(0.3, dtype=torch.float32)
    elif case == "zero point":
        x = _x((16, 64), 3)
        tab = T.quantization_map("uint4")
        s, zp = torch.tensor(0.4, dtype=torch.bfloat16), torch.tensor(7.0, dtype=torch.bfloat16)
    elif case == "block scale":
        x = _x((8, 96), 4)
        g = torch.Generator().manual_seed(5)
        s, bs = (torch.rand(8, 6, generator=g) + 0.25).bfloat16(), 16
    elif case == "permuted":
        x = _x((48, 20), 6).t()  # logical order differs from memory order
    elif case == "ragged":
        x = _x((1, 37), 7)
    else:
        index, entries, _ = T.codebook_index_table(T.quantization_map("lut4_to_int6"))
        tab = entries  # a 1-D codebook: its entries are the levels
        x = _x((12, 50), 8, scale=20.0)
        s = torch.tensor(1.0, dtype=torch.bfloat16)
    exp = O.quantize(x, s, zp, None, bs, tab, None, sd)
    d = lambda t: None if t is None else t.to(DEV)  # noqa: E731
    got = Q.quantize(x.to(DEV), s.to(DEV), d(zp), None, bs, tab.to(DEV), None, sd.to(DEV))
    assert_same_bits(got.contiguous(), exp.contiguous(), case)


@pytest.mark.parametrize("fmt", ["int8 pot", "fp4 e4m3 scales"])
def test_quantize_mx_sr(fmt):
    x = _x((24, 256), 9, specials=False)
    sd = torch.tensor(31337, dtype=torch.int64)
    if fmt == "int8 pot":
        args = (T.quantization_map("int8"), [-1], 16, 127.0, True, None)
    else:
        args = (T.quantization_map("fp4_e2m1"), [-1], 32, 6.0, False, T.quantization_map("fp8_e4m3"))
    es, ec = O.quantize_mx(x, *args, seed=sd)
    dev_args = tuple(a.to(DEV) if torch.is_tensor(a) else a for a in args)
    gs, gc = Q.quantize_mx(x.to(DEV), *dev_args, seed=sd.to(DEV))
    assert_same_bits(gs, es, f"{fmt} scale")
    assert_same_bits(gc, ec, f"{fmt} codes")


def test_quantize_sr_large_is_unbiased_and_matches():
    """A 1M-element tensor: bit-exact, and the codes average to the input
    within the rule's 1/256 bias bound plus sampling error."""
    tab = T.quantization_map("int4")
    g = torch.Generator().manual_seed(10)
    x = (torch.rand(1024, 1024, generator=g) * 12 - 6).bfloat16()
    s = torch.tensor(1.0, dtype=torch.bfloat16)
    sd = torch.tensor(2024, dtype=torch.int64)
    got = Q.quantize(x.to(DEV), s.to(DEV), qmap=tab.to(DEV), seed=sd.to(DEV))
    assert_same_bits(got, O.quantize(x, s, qmap=tab, seed=sd), "1M")
    bias = (got.double().cpu() - x.double()).mean().item()
    assert abs(bias) < 1 / 256 + 0.01
