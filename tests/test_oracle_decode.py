"""How the reference's quantized decode layer amplifies ulp-level input
differences (CPU, the oracle only).

The layer after attention re-quantizes its activations (MX-int8 of the
attention output, of RMSNorm(x1) and of the SwiGLU product), so moving an
element by one bf16 ulp can move a code, or a block's power-of-two scale,
and the layer output by a whole quantization step.  Here a small random
fraction of a config-5 attention output is moved by one ulp and the rest of
the oracle layer (o_proj, RMSNorm, gate / up, SwiGLU, down) is run again:
the layer output moves by more than half the 1e-2 parity bar.  This bounds
how closely any implementation whose attention is not bit-identical to the
reference's eager chain can follow it end to end."""

import torch

from oracle import decode as D


def test_ulp_differences_in_attention_move_the_layer_output():
    cfg = D.Config()
    w = D.random_layer(cfg, seed=0)
    mx = {}
    for k in ("wo", "wg", "wu", "wd"):
        s, c = D.mx8_quantize(w[k])
        mx[k] = (c, s)
    g = torch.Generator().manual_seed(1)
    B = 8
    x = torch.randn(B, cfg.hidden, generator=g).bfloat16()
    attn = (torch.randn(B, cfg.n_heads * cfg.head_dim, generator=g) * 0.3).bfloat16()

    def tail(a):
        x1 = x + D.mx8_linear(a, *mx["wo"])
        h2 = D.rms_norm(x1, w["ln2"], cfg.eps)
        act = torch.nn.functional.silu(D.mx8_linear(h2, *mx["wg"])) * D.mx8_linear(h2, *mx["wu"])
        return x1 + D.mx8_linear(act, *mx["wd"])

    base = tail(attn)
    moved = torch.rand(attn.shape, generator=g) < 0.0005
    step = torch.where(torch.rand(attn.shape, generator=g) < 0.5, 1, -1).to(torch.int16)
    pert = torch.where(moved, attn.view(torch.int16) + step, attn.view(torch.int16)).view(torch.bfloat16)
    assert 0 < int(moved.sum()) < 40
    out = tail(pert)
    err = float((out.double() - base.double()).abs().max() / base.double().abs().max())
    assert err > 5e-3, err
