"""Pins of the oracle's split KIVI cache (``oracle.decode.KiviCacheRef``,
following ``codegen/transform/quant_folding.py:1025-1120, 1994-2065,
2634-2700``) on the CPU.

Keys are grouped along tokens in runs of 32 and values per token, so
quantizing the sequence chunk by chunk (as the folds do) must equal
quantizing every completed token at once; the residual holds exactly the
tokens past the last completed chunk, the fold happens on the step that
fills the residual's last slot, and the position counts every token."""

import torch

from oracle import decode as D


def _rand(g, *shape):
    return torch.randn(*shape, generator=g).bfloat16()


def test_folds_equal_quantizing_the_whole_sequence():
    g = torch.Generator().manual_seed(0)
    B, nkv, L = 2, 1, 128
    k0, v0 = _rand(g, B, nkv, 96, 128), _rand(g, B, nkv, 96, 128)
    kr, vr = _rand(g, B, nkv, 100, 128), _rand(g, B, nkv, 100, 128)
    ref = D.KiviCacheRef(k0, v0, kr, vr, residual_length=L)
    ks, vs = [k0, kr], [v0, vr]
    folded_at = []
    for step in range(200):
        k, v = _rand(g, B, nkv, 1, 128), _rand(g, B, nkv, 1, 128)
        assert ref.position == 96 + 100 + step
        if ref.append(k, v):
            folded_at.append(step)
        ks.append(k)
        vs.append(v)
    # the residual fills its 128th slot on step 27, then every 128 steps
    assert folded_at == [27, 155]
    allk, allv = torch.cat(ks, dim=2), torch.cat(vs, dim=2)
    n_main = 96 + 2 * L
    assert ref.n_main == n_main and ref.k_res.shape[2] == allk.shape[2] - n_main
    kp, vp = ref.past()
    # keys: the 96 starting tokens are 3 groups, each chunk 4 more: group-aligned throughout
    s, z, c = D.kivi_quantize(allk[:, :, :n_main], -2)
    assert torch.equal(kp[:, :, :n_main], D.kivi_dequantize(c, s, z, -2))
    s, z, c = D.kivi_quantize(allv[:, :, :n_main], -1)
    assert torch.equal(vp[:, :, :n_main], D.kivi_dequantize(c, s, z, -1))
    assert torch.equal(kp[:, :, n_main:], allk[:, :, n_main:])
    assert torch.equal(vp[:, :, n_main:], allv[:, :, n_main:])
