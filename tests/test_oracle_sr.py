"""Pins of the oracle's stochastic rounding (``ops/quantized.py:318-446``):
Philox4x32-10 against the published Random123 known-answer vectors, the
per-element byte layout and the rounding rule against plain-Python
restatements in float32 (numpy), the levels of tables against their
enumerated grids, and the rule's unbiasedness."""

import numpy as np
import pytest
import torch

from oracle import ops as O
from oracle import tables as T

M = (0xD2511F53, 0xCD9E8D57)
W = (0x9E3779B9, 0xBB67AE85)


def philox_ref(ctr, key):
    """Philox4x32-10 on Python ints, any 128-bit counter and 64-bit key."""
    c, k = list(ctr), list(key)
    for _ in range(10):
        p0, p1 = c[0] * M[0], c[2] * M[1]
        c = [(p1 >> 32) ^ c[1] ^ k[0], p1 & 0xFFFFFFFF, (p0 >> 32) ^ c[3] ^ k[1], p0 & 0xFFFFFFFF]
        k = [(k[0] + W[0]) & 0xFFFFFFFF, (k[1] + W[1]) & 0xFFFFFFFF]
    return c


@pytest.mark.parametrize("ctr,key,out", [
    ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF,) * 4, (0xFFFFFFFF,) * 2, (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
])
def test_philox_known_answers(ctr, key, out):
    """Random123's philox4x32_10 known-answer vectors."""
    assert tuple(philox_ref(ctr, key)) == out


@pytest.mark.parametrize("seed", [0, 12345, 2**33 + 7, -1, -(2**40) - 3])
def test_oracle_philox_matches_reference_rounds(seed):
    counters = torch.tensor([0, 1, 2, 2**32 + 5, 2**40 + 17], dtype=torch.int64)
    got = O.philox(counters, torch.tensor(seed, dtype=torch.int64))
    key = (seed & 0xFFFFFFFF, (seed >> 32) & 0xFFFFFFFF)
    for i, c in enumerate(counters.tolist()):
        assert got[i].tolist() == philox_ref((c & 0xFFFFFFFF, c >> 32, 0, 0), key)
    if seed == 0:
        assert tuple(got[0].tolist()) == (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)


def test_random_bytes_layout():
    seed = 987654321
    got = O.random_bytes(torch.tensor(seed), (3, 13)).reshape(-1).tolist()
    for i, b in enumerate(got):
        word = philox_ref((i // 16, 0, 0, 0), (seed & 0xFFFFFFFF, seed >> 32))[(i % 16) // 4]
        assert b == (word >> (8 * (i % 4))) & 0xFF


def _sr_ref(values, levels, noise):
    """The rounding rule per element, float32 arithmetic in numpy."""
    f = np.float32
    out = []
    for v, r in zip(values, noise):
        v = f(v)
        if not np.isnan(v):
            v = min(max(v, levels[0]), levels[-1])
        up = next((i for i, lv in enumerate(levels) if lv >= v), len(levels))  # NaN runs past the end
        up = min(up, len(levels) - 1)
        high = levels[up]
        low = high if high == v else levels[max(up - 1, 0)]
        near, far = (high, low) if v < 0 else (low, high)
        lhs = f(np.abs(v) + f(f(r) * f(high - low)))
        out.append(far if lhs >= abs(far) else near)
    return out


@pytest.mark.parametrize("name", ["int4", "fp4_e2m1", "fp8_e4m3", "posit8_1"])
def test_stochastic_round_rule(name):
    tab = T.quantization_map(name)
    g = torch.Generator().manual_seed(3)
    x = (torch.randn(200, generator=g) * 4).bfloat16()
    x[:6] = torch.tensor([float("nan"), float("inf"), -float("inf"), 0.0, -0.0, 1e6])
    seed = torch.tensor(42)
    got = O.stochastic_round(x, tab, seed).float().tolist()
    levels = [np.float32(v) for v in O.qmap_levels(tab).tolist()]
    noise = (O.random_bytes(seed, x.shape).double() / 256).tolist()
    want = [float(v) for v in _sr_ref(x.float().tolist(), levels, noise)]
    assert got == want
    assert got[0] == float(levels[-2])  # NaN: searchsorted past the end, then the level below


def test_levels_of_fp8_table_are_its_grid():
    lv = O.qmap_levels(T.quantization_map("fp8_e4m3"))
    grid = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float()
    grid = torch.unique(grid[torch.isfinite(grid)]) + 0.0
    assert torch.equal(lv, grid) and lv.numel() == 253
    uz = O.qmap_levels(T.quantization_map("uint4"))
    assert uz[0].item() == 0.0 and not torch.signbit(uz[0])


def test_stochastic_round_is_unbiased():
    """4096 copies of a value between two int8 levels round to a mean within
    the 1/256 bias bound plus sampling error of the value."""
    tab = T.quantization_map("int8")
    x = torch.full((4096,), 10.3, dtype=torch.float32)
    out = O.stochastic_round(x, tab, torch.tensor(7)).double()
    assert set(out.unique().tolist()) == {10.0, 11.0}
    assert abs(out.mean().item() - 10.3) < 1 / 256 + 3 * 0.5 / 64


def test_quantize_with_seed_divides_first():
    tab = T.quantization_map("int8")
    x = torch.tensor([[3.0, -5.5, 7.25, 100.0]], dtype=torch.bfloat16)
    s = torch.tensor(0.5, dtype=torch.bfloat16)
    got = O.quantize(x, s, qmap=tab, seed=torch.tensor(1))
    assert torch.equal(got, O.stochastic_round(x / s, tab, torch.tensor(1)))
    assert got.dtype == torch.bfloat16
