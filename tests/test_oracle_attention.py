"""Pins of the oracle's ``sdpa_mx``, ``hadamard_rotate`` and
``quantize_mx_transpose`` (``ops/quantized.py:834-921, 1038-1067,
1168-1215``) on the CPU, against independent computations:

* ``sdpa_mx`` against a float64 attention written head by head from the
  definition (query head h reads kv head h // group; one softmax over the
  main and residual keys; -inf where a bool mask is false), on MX-int8 codes
  with their block scales decoded exactly;
* causal masking against the explicit lower-triangular mask;
* ``hadamard_rotate`` against a per-run float64 product, and its
  second-to-last-axis form against the last-axis form of the transpose with
  a non-symmetric matrix (catches a transposed operand);
* ``quantize_mx_transpose``'s transposed half against ``quantize_mx`` with
  column blocks (a different code path of the oracle), transposed.
"""

import math

import torch

from oracle import ops as O
from oracle import tables as T


def _mx_int8(x, bs=16):
    tab = T.quantization_map("int8")
    return O.quantize_mx(x, tab, [-1], bs, 127.0, True)


def _exact(codes, scale, bs=16):
    return codes.double() * scale.double().repeat_interleave(bs, dim=-1)[..., : codes.shape[-1]]


def _attention64(q, k, v, kr=None, vr=None, qr=None, mask=None, rmask=None, scale=None):
    """float64 attention from the definition; q [B, H, L, D], k/v [B, G, T, D]."""
    B, H, L, D = q.shape
    G = k.shape[1]
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    out = torch.zeros(B, H, L, v.shape[-1], dtype=torch.float64)
    for b in range(B):
        for h in range(H):
            g = h // (H // G)
            s = (q[b, h] @ k[b, g].T) * scale
            if mask is not None:
                s = s.masked_fill(~mask, float("-inf"))
            vals = v[b, g]
            if kr is not None:
                rs = (qr[b, h] @ kr[b, g].T) * scale
                if rmask is not None:
                    rs = rs.masked_fill(~rmask, float("-inf"))
                s = torch.cat([s, rs], dim=-1)
                vals = torch.cat([vals, vr[b, g]], dim=0)
            p = torch.exp(s - s.max(dim=-1, keepdim=True).values)
            p = p / p.sum(dim=-1, keepdim=True)
            out[b, h] = p @ vals
    return out


def _max_rel(a, b):
    return float((a.double() - b.double()).abs().max() / b.double().abs().max())


def test_sdpa_mx_against_float64_definition():
    g = torch.Generator().manual_seed(0)
    B, H, G, L, T_, D, R = 2, 8, 2, 3, 64, 128, 5
    q = torch.randn(B, H, L, D, generator=g).bfloat16()
    k = torch.randn(B, G, T_, D, generator=g).bfloat16()
    v = torch.randn(B, G, T_, D, generator=g).bfloat16()
    qr = torch.randn(B, H, L, D, generator=g).bfloat16()
    kr = torch.randn(B, G, R, D, generator=g).bfloat16()
    vr = torch.randn(B, G, R, D, generator=g).bfloat16()
    mask = torch.rand(L, T_, generator=g) > 0.2
    rmask = torch.rand(L, R, generator=g) > 0.3
    (sq, cq), (sk, ck), (sv, cv) = _mx_int8(q), _mx_int8(k), _mx_int8(v)
    got = O.sdpa_mx(cq, ck, cv, mask, 0.0, False, qr, kr, vr, rmask, enable_gqa=True, query_scale=sq,
                    key_scale=sk, value_scale=sv, block_size=16)
    ref = _attention64(_exact(cq, sq), _exact(ck, sk), _exact(cv, sv), kr.double(), vr.double(), qr.double(),
                       mask, rmask)
    assert got.dtype == torch.bfloat16 and list(got.shape) == [B, H, L, D]
    assert _max_rel(got, ref) < 2e-2


def test_sdpa_mx_causal_is_the_lower_triangle():
    g = torch.Generator().manual_seed(1)
    q, k, v = (torch.randn(1, 2, 16, 32, generator=g).bfloat16() for _ in range(3))
    a = O.sdpa_mx(q, k, v, is_causal=True)
    b = O.sdpa_mx(q, k, v, attn_mask=torch.ones(16, 16, dtype=torch.bool).tril())
    assert torch.equal(a, b)
    ref = _attention64(q.double(), k.double(), v.double(), mask=torch.ones(16, 16, dtype=torch.bool).tril())
    assert _max_rel(a, ref) < 2e-2


def test_hadamard_rotate_runs_and_axes():
    g = torch.Generator().manual_seed(2)
    m = torch.randn(16, 16, generator=g)  # not symmetric: a transposed operand fails
    x = torch.randn(3, 20, 40, generator=g)
    got = O.hadamard_rotate(x, -1, m)
    assert list(got.shape) == [3, 20, 48]
    xp = torch.nn.functional.pad(x, (0, 8)).double()
    exp = torch.stack([xp[..., 16 * r:16 * r + 16] @ m.double() for r in range(3)], dim=-2).flatten(-2)
    assert torch.allclose(got.double(), exp, atol=1e-4)
    col = O.hadamard_rotate(x, -2, m)
    assert list(col.shape) == [3, 32, 40]
    assert torch.allclose(col, O.hadamard_rotate(x.mT, -1, m).mT, atol=1e-5)


def test_quantize_mx_transpose_matches_column_blocks():
    g = torch.Generator().manual_seed(3)
    x = (torch.randn(48, 80, generator=g) * 3).bfloat16()
    tab = T.quantization_map("int8")
    s, c, ts, tc = O.quantize_mx_transpose(x, tab, 16, 127.0, True)
    s0, c0 = O.quantize_mx(x, tab, [-1], 16, 127.0, True)
    assert torch.equal(s, s0) and torch.equal(c, c0)
    cs, cc = O.quantize_mx(x, tab, [0], 16, 127.0, True)  # blocks down the columns
    assert torch.equal(ts, cs.mT) and torch.equal(tc, cc.mT)
