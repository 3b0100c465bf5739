"""A seeded random sweep of the element and block ops on the GPU against the
oracle, bit-exact (NaN as NaN): shapes of 1-4 dims with odd sizes, bf16 and
fp32 inputs, random formats, axes, block sizes, scale maps and parameter
broadcasts.  Each case prints what it drew, so a failure names its inputs."""

import random

import pytest
import torch

import voyager_amd.library  # noqa: F401  (defines quantized_ops)
from helpers import assert_same_bits
from oracle import ops as O
from oracle import tables as T

pytestmark = pytest.mark.gpu

Q = torch.ops.quantized_ops
FORMATS = ["int8", "int4", "uint4", "fp8_e4m3", "fp8_e5m2", "fp4_e2m1", "fp6_e3m2", "posit8_1", "uint2"]
QMAX = {"int8": 127.0, "int4": 7.0, "uint4": 15.0, "fp8_e4m3": 448.0, "fp8_e5m2": 57344.0, "fp4_e2m1": 6.0,
        "fp6_e3m2": 28.0, "posit8_1": 4096.0, "uint2": 3.0}


def _input(rng, shape, dtype):
    g = torch.Generator().manual_seed(rng.randrange(1 << 30))
    x = torch.randn(*shape, generator=g) * rng.choice([0.01, 1.0, 30.0])
    x = x.to(dtype)
    flat = x.view(-1)
    for v in rng.sample([0.0, -0.0, float("nan"), float("inf"), 1e-30, 65000.0], k=min(3, flat.numel())):
        flat[rng.randrange(flat.numel())] = v
    return x


def _shape(rng):
    nd = rng.randint(1, 4)
    return [rng.choice([1, 3, 7, 16, 33, 64, 96]) for _ in range(nd)]


@pytest.mark.parametrize("seed", range(24))
def test_quantize_dequantize_sweep(seed):
    rng = random.Random(seed)
    shape = _shape(rng)
    dtype = rng.choice([torch.bfloat16, torch.float32])
    fmt = rng.choice(FORMATS)
    tab = T.quantization_map(fmt)
    x = _input(rng, shape, dtype)
    # per-tensor or broadcast per-channel scale along a random dim
    if rng.random() < 0.5 or len(shape) == 1:
        s = torch.tensor(rng.choice([0.5, 0.013, 3.0]), dtype=dtype)
    else:
        d = rng.randrange(len(shape))
        sshape = [1] * len(shape)
        sshape[d] = shape[d]
        g = torch.Generator().manual_seed(seed)
        s = (torch.rand(*sshape, generator=g) + 0.05).to(dtype)
    print(f"seed {seed}: shape {shape} {dtype} {fmt} scale {list(s.shape)}", flush=True)
    q_exp = O.quantize(x, s, qmap=tab)
    q_got = Q.quantize(x.cuda(), s.cuda(), qmap=tab.cuda())
    assert_same_bits(q_got, q_exp, "quantize")
    d_exp = O.dequantize(q_exp, s)
    d_got = Q.dequantize(q_exp.cuda(), s.cuda())
    assert_same_bits(d_got, d_exp, "dequantize")


@pytest.mark.parametrize("seed", range(24))
def test_quantize_mx_sweep(seed):
    rng = random.Random(1000 + seed)
    shape = _shape(rng)
    if len(shape) == 1:
        shape = [3] + shape
    dtype = rng.choice([torch.bfloat16, torch.float32])
    fmt = rng.choice(FORMATS)
    tab = T.quantization_map(fmt)
    ax = rng.randrange(len(shape))
    bs = rng.choice([8, 16, 32, 64])
    pot = rng.random() < 0.5
    smap = None if pot else T.quantization_map(rng.choice(["fp8_e4m3", "fp8_e5m3", None]))
    x = _input(rng, shape, dtype)
    print(f"seed {seed}: shape {shape} {dtype} {fmt} axis {ax} block {bs} pot {pot} smap "
          f"{None if smap is None else smap.shape}", flush=True)
    es, ec = O.quantize_mx(x, tab, [ax], bs, QMAX[fmt], pot, smap)
    gs, gc = Q.quantize_mx(x.cuda(), tab.cuda(), [ax], bs, QMAX[fmt], pot, None if smap is None else smap.cuda())
    assert_same_bits(gs, es, "scale")
    assert_same_bits(gc, ec, "codes")
    assert_same_bits(Q.dequantize_mx(gc, gs, bs), O.dequantize_mx(ec, es, bs), "dequantize_mx")


@pytest.mark.parametrize("seed", range(12))
def test_quantize_affine_sweep(seed):
    rng = random.Random(2000 + seed)
    shape = _shape(rng)
    if len(shape) == 1:
        shape = [5] + shape
    dtype = rng.choice([torch.bfloat16, torch.float32])
    fmt = rng.choice(["uint2", "uint4"])
    qmax = {"uint2": 3.0, "uint4": 15.0}[fmt]
    ax = rng.randrange(len(shape))
    bs = rng.choice([8, 16, 32])
    smap = T.quantization_map(rng.choice(["fp16_e5m10", "fp8_e4m3"])) if rng.random() < 0.5 else None
    x = _input(rng, shape, dtype)
    x = torch.nan_to_num(x, nan=0.0, posinf=10.0, neginf=-10.0)  # min/max blocks stay finite
    print(f"seed {seed}: shape {shape} {dtype} {fmt} axis {ax} block {bs}", flush=True)
    tab = T.quantization_map(fmt)
    exp = O.quantize_affine(x, tab, [ax], bs, 0.0, qmax, smap)
    got = Q.quantize_affine(x.cuda(), tab.cuda(), [ax], bs, 0.0, qmax, None if smap is None else smap.cuda())
    for name, g, e in zip(("scale", "zero_point", "codes"), got, exp):
        assert_same_bits(g, e, name)
