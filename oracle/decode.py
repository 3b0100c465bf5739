"""One decode step of an MX-int8 / KIVI Llama decoder layer on the CPU
(TEST INFRASTRUCTURE ONLY: imported by tests, ``smoke()`` and the
``cpu_baseline`` leg of ``bench.py``).

The layer itself comes from the reference's pinned dependency
``transformers==5.13.0`` (``pyproject.toml:37``), which is not part of the
reference tree; its published eager algorithm is restated here:
``LlamaRMSNorm``, ``LlamaRotaryEmbedding`` (default RoPE), ``rotate_half`` /
``apply_rotary_pos_emb``, ``eager_attention_forward`` with ``repeat_kv`` and
``LlamaMLP`` (SwiGLU).  The reference quantizes that graph: every linear
becomes ``quantize_mx`` of its input followed by ``linear_mx`` on baked
weight codes (``quantization/quantize_pt2e.py:582-600``, ``:819-828``), and
the KV cache is split into a KIVI main part, quantized with
``quantize_affine`` and read back with ``dequantize``
(``examples/language_modeling/quantization_configs.py:171-207``,
``codegen/transform/quant_folding.py:1025-1120``), plus a full-precision
residual window.  The quantized ops come from ``oracle.ops``.

Pins (``tests/test_oracle_pins.py``): with plain bf16 linears and an
unquantized cache, ``decode_layer`` equals the installed transformers'
``LlamaDecoderLayer`` (eager attention) bit for bit; the KIVI round trip is
checked against a float64 restatement of the affine formula.
"""

import math
from dataclasses import dataclass
from typing import Dict, Optional, Tuple

import torch

from . import ops as O
from . import tables as T

MX_BLOCK = 16
KIVI_GROUP = 32


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """``LlamaRMSNorm.forward``."""
    h = x.to(torch.float32)
    var = h.pow(2).mean(-1, keepdim=True)
    h = h * torch.rsqrt(var + eps)
    return weight * h.to(x.dtype)


def rope_cos_sin(positions: torch.Tensor, head_dim: int, theta: float, dtype=torch.bfloat16):
    """``LlamaRotaryEmbedding`` (rope_type "default"): cos / sin tables
    ``[len(positions), head_dim]`` in ``dtype``."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.int64).float() / head_dim))
    freqs = positions.float()[:, None] * inv_freq[None, :]
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """``apply_rotary_pos_emb`` for one tensor; cos / sin broadcast over heads."""
    return (x * cos) + (rotate_half(x) * sin)


def eager_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scaling: float) -> torch.Tensor:
    """``eager_attention_forward`` without mask or dropout: q ``[B, nq, S, D]``,
    k / v ``[B, nkv, T, D]``; returns ``[B, S, nq, D]``."""
    groups = q.shape[1] // k.shape[1]
    ks = k[:, :, None].expand(-1, -1, groups, -1, -1).reshape(k.shape[0], -1, *k.shape[2:])
    vs = v[:, :, None].expand(-1, -1, groups, -1, -1).reshape(v.shape[0], -1, *v.shape[2:])
    w = torch.matmul(q, ks.transpose(2, 3).contiguous()) * scaling
    w = torch.nn.functional.softmax(w, dim=-1, dtype=torch.float32).to(q.dtype)
    out = torch.matmul(w, vs.contiguous())
    return out.transpose(1, 2).contiguous()


def int8_table() -> torch.Tensor:
    return T.quantization_map("int8")


def mx8_quantize(w: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """``quantize_mx(w, int8, [-1], 16, 127, force_scale_power_of_two=True)``:
    (scale, codes) in the reference form."""
    return O.quantize_mx(w, int8_table(), [-1], MX_BLOCK, 127.0, True)


def mx8_linear(x: torch.Tensor, w_codes: torch.Tensor, w_scale: torch.Tensor) -> torch.Tensor:
    """A converted MX-int8 linear: ``quantize_mx`` of the input, then
    ``linear_mx`` with the baked weight codes and scales."""
    sx, cx = mx8_quantize(x)
    return O.linear_mx(cx, w_codes, input_scale=sx, weight_scale=w_scale, block_size=MX_BLOCK)


def mx8_fake_quant(x: torch.Tensor) -> torch.Tensor:
    """The activation operand ``linear_mx`` forms: codes x scale (bf16)."""
    sx, cx = mx8_quantize(x)
    return O.dequantize_mx_parts(cx, sx, None, MX_BLOCK)


def kivi_quantize(x: torch.Tensor, axis: int) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """``quantize_affine`` with the KIVI spec ``uint2,bs=32,qs=group_wise_affine,
    ax=axis,scale=fp16_e5m10``: (scale, zero_point, codes)."""
    return O.quantize_affine(x, T.quantization_map("uint2"), [axis], KIVI_GROUP, 0.0, 3.0,
                             T.quantization_map("fp16_e5m10"))


def kivi_dequantize(codes, scale, zp, axis: int) -> torch.Tensor:
    """``dequantize(codes, scale, zp, axes=[axis], block_size=32)``."""
    return O.dequantize(codes, scale, zp, [axis], KIVI_GROUP)


@dataclass
class Config:
    hidden: int = 4096
    n_heads: int = 32
    n_kv_heads: int = 8
    head_dim: int = 128
    intermediate: int = 14336
    rope_theta: float = 500000.0
    eps: float = 1e-5


def random_layer(cfg: Config, seed: int = 0) -> Dict[str, torch.Tensor]:
    """A random-init layer in bf16: weights ~N(0, 0.02), norm weights 1 + N(0, 0.1)
    (so the RMSNorm gain is exercised)."""
    g = torch.Generator().manual_seed(seed)
    H, F = cfg.hidden, cfg.intermediate
    q, kv = cfg.n_heads * cfg.head_dim, cfg.n_kv_heads * cfg.head_dim

    def w(n, k):
        return (torch.randn(n, k, generator=g) * 0.02).bfloat16()

    return {
        "ln1": (1 + 0.1 * torch.randn(H, generator=g)).bfloat16(),
        "wq": w(q, H), "wk": w(kv, H), "wv": w(kv, H), "wo": w(H, q),
        "ln2": (1 + 0.1 * torch.randn(H, generator=g)).bfloat16(),
        "wg": w(F, H), "wu": w(F, H), "wd": w(H, F),
    }


def decode_layer(x: torch.Tensor, weights: Dict[str, torch.Tensor], k_past: torch.Tensor, v_past: torch.Tensor,
                 cos: torch.Tensor, sin: torch.Tensor, cfg: Config,
                 mx: Optional[Dict[str, Tuple[torch.Tensor, torch.Tensor]]] = None) -> Dict[str, torch.Tensor]:
    """One decode step of ``LlamaDecoderLayer`` for ``x [B, hidden]`` (one
    token per sequence) attending to ``k_past`` / ``v_past`` ``[B, nkv, T, D]``
    (already dequantized) plus the step's own key / value.  With ``mx`` (weight
    name -> (codes, scale)) every linear is the MX-int8 pair; otherwise plain
    bf16 ``F.linear``.  Returns the intermediates the GPU path also exposes."""
    B = x.shape[0]
    D, nq, nkv = cfg.head_dim, cfg.n_heads, cfg.n_kv_heads

    def lin(name, t):
        if mx is None:
            return torch.nn.functional.linear(t, weights[name])
        return mx8_linear(t, *mx[name])

    h1 = rms_norm(x, weights["ln1"], cfg.eps)
    q = lin("wq", h1).view(B, 1, nq, D).transpose(1, 2)
    k = lin("wk", h1).view(B, 1, nkv, D).transpose(1, 2)
    v = lin("wv", h1).view(B, 1, nkv, D).transpose(1, 2)
    c, s = cos[:, None, None, :], sin[:, None, None, :]
    q, k = apply_rope(q, c, s), apply_rope(k, c, s)
    keys = torch.cat((k_past, k), dim=2)
    values = torch.cat((v_past, v), dim=2)
    attn = eager_attention(q, keys, values, D ** -0.5).reshape(B, nq * D)
    x1 = x + lin("wo", attn)
    h2 = rms_norm(x1, weights["ln2"], cfg.eps)
    act = torch.nn.functional.silu(lin("wg", h2)) * lin("wu", h2)
    out = x1 + lin("wd", act)
    return {"h1": h1, "q": q, "k": k, "v": v, "attn": attn, "x1": x1, "h2": h2, "act": act, "out": out}


class KiviCacheRef:
    """The reference's split KIVI cache of one layer (test only).

    ``split_kv_cache`` (``codegen/transform/quant_folding.py:1025-1120``)
    keeps whole chunks of ``residual_length`` positions in the quantized main
    cache and the chunk being filled in a full-precision residual, position
    ``p`` in slot ``p mod residual_length``.  The attention reads the
    dequantized main cache followed by the residual.  After the step whose
    token lands in the residual's last slot, the fold quantizes the residual
    with the cache's own quantizer and stores it as the next chunk of the main
    cache (``_store_chunk``, ``:1994-2065``; run after the step by
    ``move_folds_out``, ``:2634-2700``).  Here the quantizer is the KIVI spec
    (``kivi_quantize``: keys grouped along tokens, values along channels),
    and the main cache is kept as its reference-form outputs, chunk by chunk.
    The starting main part may be any whole number of 32-token groups."""

    def __init__(self, k_main, v_main, k_res, v_res, residual_length: int = 128):
        self.length = residual_length
        self.k_chunks, self.v_chunks = [], []  # (scale, zp, codes) per stored run
        if k_main.shape[2]:
            self.k_chunks.append(kivi_quantize(k_main, -2))
            self.v_chunks.append(kivi_quantize(v_main, -1))
        self.n_main = k_main.shape[2]
        self.k_res, self.v_res = k_res.clone(), v_res.clone()
        self.folds = 0

    @property
    def position(self) -> int:
        return self.n_main + self.k_res.shape[2]

    def past(self):
        """Keys and values the step's attention reads before its own token:
        the dequantized main cache, then the residual (``[B, nkv, T, D]``)."""
        ks = [kivi_dequantize(c, s, z, -2) for s, z, c in self.k_chunks] + [self.k_res]
        vs = [kivi_dequantize(c, s, z, -1) for s, z, c in self.v_chunks] + [self.v_res]
        return torch.cat(ks, dim=2), torch.cat(vs, dim=2)

    def append(self, k, v) -> bool:
        """The step's key / value ``[B, nkv, 1, D]`` enter the residual; when
        they fill its last slot the chunk is folded.  Returns whether it was."""
        self.k_res = torch.cat((self.k_res, k), dim=2)
        self.v_res = torch.cat((self.v_res, v), dim=2)
        if self.k_res.shape[2] < self.length:
            return False
        self.k_chunks.append(kivi_quantize(self.k_res, -2))
        self.v_chunks.append(kivi_quantize(self.v_res, -1))
        self.n_main += self.length
        self.k_res, self.v_res = self.k_res[:, :, :0], self.v_res[:, :, :0]
        self.folds += 1
        return True
