"""Pins of the oracle's codebook search and lookup (``oracle.ops.encode`` /
``decode``, restating ``ops/quantized.py:193-315``) and of its block scales
over several axes (``calculate_mx_qparam``, ``ops/quantized.py:958-1031``).

The checks are independent of the restated code:
  * encode against a brute-force nearest-entry search in exact arithmetic
    (ties to the lower entry; NaN and +inf to the last, -inf to the first:
    torch.searchsorted's left bisection);
  * region grids against an explicit loop over the regions, each slice of
    the tensor searched or looked up in its own table;
  * power-of-two block scales over two axes against a per-tile loop with
    ``math.frexp``.
A planted mistake (a transposed grid) must fail the region check.
"""

import math

import pytest
import torch

from oracle import ops as O


def _bf16_values(g, n, scale=3.0):
    return (torch.randn(n, generator=g) * scale).bfloat16()


def _nearest(v: float, entries) -> int:
    """Index of the entry nearest ``v``; ties to the lower index."""
    if math.isnan(v) or v == math.inf:
        return len(entries) - 1
    if v == -math.inf:
        return 0
    best, arg = None, 0
    for j, c in enumerate(entries):
        d = abs(v - c)
        if best is None or d < best:
            best, arg = d, j
    return arg


def _codebook(g, k):
    # distinct bfloat16 entries: every midpoint is exact in float32
    while True:
        c = torch.sort(_bf16_values(g, k)).values
        if torch.unique(c).numel() == k:
            return c.float()


@pytest.mark.parametrize("k", [2, 5, 16])
def test_encode_is_nearest_entry(k):
    g = torch.Generator().manual_seed(100 + k)
    code = _codebook(g, k)
    mids = ((code[:-1] + code[1:]) / 2).bfloat16().float()
    x = torch.cat([_bf16_values(g, 400).float(), code, mids,
                   torch.tensor([float("nan"), float("inf"), -float("inf"), 0.0, -0.0])])
    got = O.encode(x, code)
    idx = O.encode(x, code, (code[:-1] + code[1:]) / 2)
    for i, v in enumerate(x.tolist()):
        # a value at an exact midpoint (midpoints of bfloat16 entries that
        # are themselves bfloat16) takes the lower entry
        j = _nearest(v, code.tolist())
        assert int(idx[i]) == j, (v, int(idx[i]), j)
        assert got[i].item() == code[j].item()


def test_encode_rounds_to_bfloat16_first():
    code = torch.tensor([0.0, 1.0])
    # 0.5 + 2**-12 rounds to 0.5 in bfloat16: the midpoint, so the lower entry
    x = torch.tensor([0.5 + 2.0**-12, 0.5 + 2.0**-7])
    assert O.encode(x, code).tolist() == [0.0, 1.0]


def _region_loop(x, code, fn):
    """Apply ``fn(slice, table)`` to each region of the grid of ``code``."""
    counts = code.shape[:-1]
    out = torch.empty_like(x)
    tiles = [n // c for n, c in zip(x.shape, counts)]
    for r in range(math.prod(counts)):
        rest, ridx = r, []
        for c in reversed(counts):
            ridx.append(rest % c)
            rest //= c
        ridx = ridx[::-1]
        sl = tuple(slice(i * t, (i + 1) * t) for i, t in zip(ridx, tiles))
        out[sl] = fn(x[sl], code[tuple(ridx)])
    return out


def test_region_encode_and_decode_follow_the_grid():
    g = torch.Generator().manual_seed(7)
    x = _bf16_values(g, 2 * 6 * 4 * 8).float().view(2, 6, 4, 8)
    counts = (1, 3, 2, 1)
    code = torch.stack([_codebook(g, 9) for _ in range(math.prod(counts))]).view(*counts, 9)
    bounds = (code[..., :-1] + code[..., 1:]) / 2

    def brute(xs, table):
        return torch.tensor([table[_nearest(v, table.tolist())].item() for v in xs.reshape(-1).tolist()]
                            ).view(xs.shape)

    want = _region_loop(x, code, brute)
    assert torch.equal(O.encode(x, code), want)
    idx = O.encode(x, code, bounds)
    want_idx = _region_loop(x, code, lambda xs, t: torch.tensor(
        [float(_nearest(v, t.tolist())) for v in xs.reshape(-1).tolist()]).view(xs.shape))
    assert torch.equal(idx, want_idx)
    # decode reads each region's own table
    dec = O.decode(idx, code)
    want_dec = _region_loop(idx, code, lambda xs, t: t[xs.long()])
    assert torch.equal(dec, want_dec)
    assert torch.equal(dec, want)
    # a transposed grid (regions taken column-major) reads other tables
    wrong = code.permute(0, 2, 1, 3, 4).reshape(*counts, 9)
    assert not torch.equal(O.decode(idx, wrong), want_dec)


def test_region_grid_errors():
    code = torch.zeros(1, 3, 4)
    with pytest.raises(ValueError, match="tiles 2 axes"):
        O.encode(torch.zeros(2, 6, 1), code)
    with pytest.raises(ValueError, match="does not divide"):
        O.encode(torch.zeros(2, 5), code)


def test_decode_1d_negative_index_counts_from_the_end():
    code = torch.tensor([1.0, 2.0, 3.0])
    assert O.decode(torch.tensor([-1.0, 0.0, 2.0]), code).tolist() == [3.0, 1.0, 3.0]


@pytest.mark.parametrize("shape,axes,bs", [((6, 40, 72), [1, 2], 32), ((3, 5, 7), [0, 2], 4),
                                           ((70, 33), [0, 1], 16)])
def test_pot_scales_over_two_axes(shape, axes, bs):
    g = torch.Generator().manual_seed(9)
    x = (torch.randn(shape, generator=g) * torch.exp(torch.randn(shape, generator=g) * 3)).bfloat16()
    x.view(-1)[::97] = 0.0
    qmax = 127.0
    got = O.calculate_mx_qparam(x, axes, bs, qmax, force_scale_power_of_two=True)
    a0, a1 = axes
    nb0, nb1 = -(-shape[a0] // bs), -(-shape[a1] // bs)
    assert got.shape[a0] == nb0 and got.shape[a1] == nb1
    shift = math.floor(math.log2(qmax))
    xm = x.float().movedim((a0, a1), (0, 1))
    gm = got.float().movedim((a0, a1), (0, 1))
    for b0 in range(nb0):
        for b1 in range(nb1):
            tile = xm[b0 * bs:(b0 + 1) * bs, b1 * bs:(b1 + 1) * bs]
            amax = tile.abs().amax(dim=(0, 1))
            for i, a in enumerate(amax.reshape(-1).tolist()):
                e = (math.frexp(a)[1] - 1) if a > 0 else -126
                want = 2.0 ** (e - shift)
                if want < 2.0**-133:  # below bfloat16's subnormals: 0, taken as 1
                    want = 1.0
                assert gm[b0, b1].reshape(-1)[i].item() == want
