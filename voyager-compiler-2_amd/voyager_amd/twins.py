"""The remaining ``quantized_ops`` operators a converted graph can hold.

* ``sdpa_mx`` (``ops/quantized.py:822-932``) -- attention over
  microscaling query / key / value codes, with an optional full-precision
  residual (a split KV cache) in the same softmax and an optional MX
  quantization of the probabilities.  CUDA kernel: the operands decode
  through the package's ``dequantize_mx`` (HIP), both products run on the
  package's bf16 MFMA GEMM, the probabilities quantize through its
  ``quantize_mx``; masking, concatenation and the softmax are torch
  elementwise ops.  Every intermediate is rounded to the dtype the
  reference's eager op sequence gives it.
* ``quantize_mx_transpose`` (``:1160-1215``) -- ``quantize_mx`` of a tensor
  and of its transpose (optionally Hadamard-rotated first), each on the HIP
  kernel.

These two are CUDA kernels like the package's others
(:func:`voyager_amd.kernels.register` binds them).  The accelerator-layout
twins below have no quantized arithmetic; they are registered only when this
package defines the namespace itself (``voyager_amd.library``), as torch
restatements on any device, so graphs whose data-layout passes retargeted
aten ops to them load and run:

* ``sdpa_kmajor`` / ``rms_norm_kmajor`` (``ops/layout.py:287-341``): aten's
  attention with query and key stored ``[..., head_dim, tokens]``, and RMS
  normalisation over the second-to-last dim of ``[..., hidden, tokens]``;
* the NHWC pool twins (``ops/layout.py:127-168``): aten's pool under its
  own name and schema on an NHWC activation, returning NHWC.
"""

import math
from typing import Optional

import torch
import torch.nn.functional as F

from .gemm import _decode, gemm_bf16
from .ops import _quantize_mx_cuda, _require_gpu
from .registry import cuda_kernel, fake_kernel
from .schemas import NHWC_POOLS

HADAMARD_RUN = 16  # elements per Hadamard block (ops/quantized.py:1035)


def _product(a: torch.Tensor, b_nk: torch.Tensor) -> torch.Tensor:
    """``a @ b_nk^T`` rounded to the operands' dtype, as an eager
    ``torch.matmul`` of two tensors of that dtype is: the package's MFMA GEMM
    for bf16 operands (fp32 accumulation, one rounding), torch otherwise."""
    if a.dtype == torch.bfloat16 and b_nk.dtype == torch.bfloat16 and a.shape[-1] % 8 == 0:
        return gemm_bf16(a, b_nk, torch.bfloat16)
    return torch.matmul(a, b_nk.mT)


def _apply_mask(scores: torch.Tensor, mask: Optional[torch.Tensor]) -> torch.Tensor:
    """A bool mask keeps where true (else -inf); a float mask is added."""
    if mask is None:
        return scores
    if mask.dtype == torch.bool:
        return scores.masked_fill(mask.logical_not(), float("-inf"))
    return scores + mask


@cuda_kernel("sdpa_mx")
def _sdpa_mx_cuda(query, key, value, attn_mask=None, dropout_p=0.0, is_causal=False, query_residual=None,
                  key_residual=None, value_residual=None, residual_mask=None, *, scale=None, enable_gqa=False,
                  query_scale=None, key_scale=None, value_scale=None, block_size=None, input_code=None,
                  weight_code=None, probs_qmap=None, probs_quant_max=None, probs_scale_qmap=None, probs_code=None,
                  force_scale_power_of_two=False):
    """``ops/quantized.py:834-921``.  ``dropout_p`` is ignored, as there."""
    _require_gpu(query, key, value, attn_mask, query_residual, key_residual, value_residual, residual_mask,
                 query_scale, key_scale, value_scale, input_code, weight_code, probs_qmap, probs_scale_qmap,
                 probs_code)
    if is_causal and attn_mask is not None:
        raise ValueError("is_causal excludes an explicit attn_mask")
    q = _decode(query, query_scale, input_code, block_size)
    k = _decode(key, key_scale, weight_code, block_size)
    v = _decode(value, value_scale, weight_code, block_size)
    with_residual = key_residual is not None
    kr, vr = key_residual, value_residual
    if enable_gqa:
        rep = q.shape[-3] // k.shape[-3]
        k, v = k.repeat_interleave(rep, dim=-3), v.repeat_interleave(rep, dim=-3)
        if with_residual:
            kr, vr = kr.repeat_interleave(rep, dim=-3), vr.repeat_interleave(rep, dim=-3)
    if scale is None:
        scale = 1.0 / math.sqrt(q.shape[-1])
    scores = _product(q, k) * scale
    if is_causal:
        attn_mask = torch.ones(scores.shape[-2:], dtype=torch.bool, device=scores.device).tril()
    scores = _apply_mask(scores, attn_mask)
    n_main = scores.shape[-1]
    if with_residual:
        rs = _apply_mask(_product(query_residual, kr) * scale, residual_mask)
        scores = torch.cat([scores, rs], dim=-1)
    probs = torch.softmax(scores, dim=-1)
    p_main, p_res = probs[..., :n_main], probs[..., n_main:]
    if probs_qmap is not None:
        p_scale, p_codes = _quantize_mx_cuda(p_main, probs_qmap, [-1], block_size, probs_quant_max,
                                             force_scale_power_of_two, probs_scale_qmap, probs_code)
        p_main = _decode(p_codes, p_scale, input_code, block_size)
    out = _product(p_main, v.mT.contiguous())
    if with_residual:
        out = out + _product(p_res, vr.mT.contiguous())
    return out


@fake_kernel("sdpa_mx")
def _sdpa_mx_fake(query, key, value, attn_mask=None, dropout_p=0.0, is_causal=False, query_residual=None,
                  key_residual=None, value_residual=None, residual_mask=None, **kwargs):
    return query.new_empty(*query.shape[:-1], value.shape[-1])


def hadamard_rotate(x: torch.Tensor, axis: int, matrix: torch.Tensor) -> torch.Tensor:
    """Runs of 16 elements along ``axis`` (the last or second-to-last) times
    ``matrix`` in float32, the axis zero-padded to whole runs first, the
    result in ``x``'s dtype (``ops/quantized.py:1038-1067``)."""
    axis %= x.ndim
    if axis < x.ndim - 2:
        raise ValueError(f"cannot rotate along axis {axis} of {x.ndim}")
    pad = (-x.shape[axis]) % HADAMARD_RUN
    if pad:
        spec = [0, 0] * (x.ndim - 1 - axis) + [0, pad]
        x = F.pad(x, spec)
    runs = x.float().unflatten(axis, (-1, HADAMARD_RUN))
    m = matrix.float()
    rot = runs @ m if axis == x.ndim - 1 else m.T @ runs
    return rot.flatten(axis, axis + 1).to(x.dtype)


@cuda_kernel("quantize_mx_transpose")
def _quantize_mx_transpose_cuda(input, qmap, block_size, quant_max, force_scale_power_of_two=False,
                                scale_qmap=None, output_code=None, seed=None, global_scale=None,
                                transpose_seed=None, transpose_global_scale=None, hadamard=None):
    """``ops/quantized.py:1168-1215``: ``(scale, codes, transpose_scale,
    transpose_codes)``."""
    _require_gpu(input, qmap, scale_qmap, output_code, seed, global_scale, transpose_seed,
                 transpose_global_scale, hadamard)
    t = input.mT
    if hadamard is not None:
        t = hadamard_rotate(t, -1, hadamard)
    common = (qmap, [-1], block_size, quant_max, force_scale_power_of_two, scale_qmap, output_code)
    s, c = _quantize_mx_cuda(input, *common, seed, global_scale)
    ts, tc = _quantize_mx_cuda(t, *common, transpose_seed, transpose_global_scale)
    return s, c, ts, tc


@fake_kernel("quantize_mx_transpose")
def _quantize_mx_transpose_fake(input, qmap, block_size, quant_max, force_scale_power_of_two=False,
                                scale_qmap=None, output_code=None, seed=None, global_scale=None,
                                transpose_seed=None, transpose_global_scale=None, hadamard=None):
    def pair(x):
        shape = list(x.shape)
        shape[-1] = -(-shape[-1] // block_size)
        return x.new_empty(shape), torch.empty_like(x)

    t = input.mT
    if hadamard is not None:
        shape = list(t.shape)
        shape[-1] += (-shape[-1]) % HADAMARD_RUN
        t = t.new_empty(shape)
    return (*pair(input), *pair(t))


# ------------------------------------------------ accelerator-layout twins
def _sdpa_kmajor(query, key, value, attn_mask=None, dropout_p=0.0, is_causal=False, *, scale=None,
                 enable_gqa=False, transpose_output=False):
    """``ops/layout.py:306-333``: query and key arrive ``[..., head_dim,
    tokens]``; the output is ``[..., tokens, head_dim]`` or, with
    ``transpose_output``, its transpose."""
    out = torch.ops.aten.scaled_dot_product_attention(query.mT.contiguous(), key.mT.contiguous(), value, attn_mask,
                                                      dropout_p, is_causal, scale=scale, enable_gqa=enable_gqa)
    return out.mT.contiguous() if transpose_output else out


def _rms_norm_kmajor(input, weight=None, eps=None):
    """``ops/layout.py:336-341``: RMS norm of ``[..., hidden, tokens]`` over
    ``hidden`` with a ``[hidden, 1]`` (or ``[hidden]``) weight."""
    hidden = input.shape[-2]
    w = None if weight is None else weight.reshape(hidden)
    return torch.ops.aten.rms_norm(input.mT, [hidden], w, eps).mT.contiguous()


def _nhwc_pool(aten_op):
    def run(input, *args):
        return aten_op(input.permute(0, 3, 1, 2), *args).permute(0, 2, 3, 1)

    return run


def register_layout_twins(lib) -> None:
    """Register the accelerator-layout twins as torch restatements
    (``CompositeExplicitAutograd``: any device, fake tensors trace through)
    on ``lib``, a library that has defined their schemas."""
    lib.impl("sdpa_kmajor", _sdpa_kmajor, "CompositeExplicitAutograd")
    lib.impl("rms_norm_kmajor", _rms_norm_kmajor, "CompositeExplicitAutograd")
    for op in NHWC_POOLS:
        lib.impl(op._schema.name.split("::")[1], _nhwc_pool(op), "CompositeExplicitAutograd")
