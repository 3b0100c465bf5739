"""GEMM ops: ``quantized_ops.linear`` / ``matmul`` (``ops/layout.py:216-284``)
and ``linear_mx`` / ``matmul_mx`` (``ops/quantized.py:651-819``) on the HIP
GEMM core (``vh_gemm``), plus the packed fp8 / MX-int8 / posit8 GEMMs a
lowered graph runs.

The reference computes every GEMM as an fp32 (or bf16) ``aten`` product of
decoded operands, rounded once to the output dtype.  Here the product is an
MFMA GEMM with fp32 accumulation; the epilogue applies ``alpha``, the bias and
the one rounding.  Results agree with the reference to the accumulation
order (the parity bar is 1e-2 max-abs-normalized error).
"""

import ctypes
from typing import NamedTuple, Optional, Tuple

import torch

from . import _lib, formats
from ._lib import FMT_HW_E4M3, FMT_MINIFLOAT, FMT_STEPS, VH_BF16, VH_F32, dtype_code, load, ptr, stream_of
from .ops import _dequantize_mx_cuda, _require_gpu, decode_codes
from .registry import cuda_kernel, fake_kernel
from .schemas import LINEAR_LAYOUT, MATMUL_LAYOUT

OP_BF16, OP_FP8, OP_MXI8, OP_P8 = 0, 1, 2, 3
EPI_PLAIN, EPI_ROUND_SCALE = 0, 1


class Epilogue(ctypes.Structure):
    _fields_ = [
        ("mode", ctypes.c_int32),
        ("out_dtype", ctypes.c_int32),
        ("scale", ctypes.c_void_p),
        ("scale_dtype", ctypes.c_int32),
        ("bias", ctypes.c_void_p),
        ("bias_dtype", ctypes.c_int32),
    ]


class GemmDesc(ctypes.Structure):
    _fields_ = [
        ("A", ctypes.c_void_p), ("B", ctypes.c_void_p), ("C", ctypes.c_void_p),
        ("M", ctypes.c_int64), ("N", ctypes.c_int64), ("K", ctypes.c_int64),
        ("lda", ctypes.c_int64), ("ldb", ctypes.c_int64), ("ldc", ctypes.c_int64),
        ("a_fmt", ctypes.c_int32), ("b_fmt", ctypes.c_int32),
        ("a_scale", ctypes.c_void_p), ("b_scale", ctypes.c_void_p),
        ("a_scale_ld", ctypes.c_int64), ("b_scale_ld", ctypes.c_int64),
        ("a_block", ctypes.c_int32), ("b_block", ctypes.c_int32),
        ("a_bias", ctypes.c_int32), ("b_bias", ctypes.c_int32),
        ("lut", ctypes.c_void_p),
        ("tile_hint", ctypes.c_int32),
        ("batch", ctypes.c_int64),
        ("batch_stride_a", ctypes.c_int64), ("batch_stride_b", ctypes.c_int64),
        ("batch_stride_c", ctypes.c_int64),
        ("batch_stride_a_scale", ctypes.c_int64), ("batch_stride_b_scale", ctypes.c_int64),
        ("epi", Epilogue),
        ("split_k", ctypes.c_int32),
        ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_int64),
    ]


FAMILY_STAGED, FAMILY_DIRECT_FP8, FAMILY_DIRECT_BF16, FAMILY_MXI8 = 1, 2, 3, 4

#: When set to a list, every ``vh_gemm`` launch appends ``(family, tile,
#: splits, M, N, K)`` of the kernel it runs (``vh_gemm_plan``), so tests can
#: assert which tile a shape takes.  None (the default) costs nothing.
plan_log = None


def plan(desc: GemmDesc):
    """``(family, tile, splits)`` of the kernel ``vh_gemm`` runs for ``desc``."""
    fam, tile, splits = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int32()
    st = load().vh_gemm_plan(ctypes.c_void_p(ctypes.addressof(desc)), ctypes.byref(fam), ctypes.byref(tile),
                             ctypes.byref(splits))
    _lib.check(st, "vh_gemm_plan")
    return fam.value, tile.value, splits.value


def run(desc: GemmDesc, device) -> None:
    if plan_log is not None:
        plan_log.append(plan(desc) + (desc.M, desc.N, desc.K))
    st = load().vh_gemm(ctypes.c_void_p(ctypes.addressof(desc)),
                        ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream))
    _lib.check(st, "vh_gemm")


def _epilogue(mode, out_dtype, scale=None, bias=None) -> Epilogue:
    e = Epilogue()
    e.mode = mode
    e.out_dtype = dtype_code(out_dtype)
    if scale is not None:
        e.scale = scale.data_ptr()
        e.scale_dtype = dtype_code(scale.dtype)
    if bias is not None:
        e.bias = bias.data_ptr()
        e.bias_dtype = dtype_code(bias.dtype)
    return e


def _rows(t: torch.Tensor) -> torch.Tensor:
    """``t`` [R, C] with unit column stride and rows at least C elements
    apart (the layout the kernels address as ``base + row * ld + col``);
    a copy when the view is laid out otherwise."""
    if t.dim() != 2:
        raise RuntimeError(f"expected a 2-D operand, got shape {list(t.shape)}")
    if t.stride(1) == 1 and t.stride(0) >= t.shape[1]:
        return t
    return t.contiguous()


def _bias_operand(bias: Optional[torch.Tensor]) -> Optional[torch.Tensor]:
    """A bias as the epilogues read it: bf16 and float32 as they are (every
    epilogue widens bf16 exactly), other dtypes converted to float32."""
    if bias is None:
        return None
    if bias.dtype not in (torch.bfloat16, torch.float32):
        bias = bias.to(torch.float32)
    return bias.contiguous()


def gemm_bf16(a: torch.Tensor, b: torch.Tensor, out_dtype, bias=None, alpha=None) -> torch.Tensor:
    """``a[..., M, K] . b[..., N, K]^T`` (bf16 operands, fp32 accumulation),
    ``* alpha + bias`` in fp32, one rounding to ``out_dtype``."""
    if a.dtype != torch.bfloat16 or b.dtype != torch.bfloat16:
        raise NotImplementedError(f"GEMM operands must be bfloat16 on the GPU (got {a.dtype}, {b.dtype})")
    K = a.shape[-1]
    if b.shape[-1] != K:
        raise RuntimeError(f"GEMM contraction mismatch: {list(a.shape)} vs {list(b.shape)}")
    if K % 8:  # the kernels move 16-byte chunks of each row: zero-pad K
        a = torch.nn.functional.pad(a, (0, -K % 8))
        b = torch.nn.functional.pad(b, (0, -K % 8))
        K = a.shape[-1]
    if b.dim() == 2 and a.dim() > 2:  # one GEMM over all leading dims
        lead = a.shape[:-1]
        return gemm_bf16(a.reshape(-1, K), b, out_dtype, bias, alpha).view(*lead, b.shape[0])
    batch_shape = torch.broadcast_shapes(a.shape[:-2], b.shape[:-2])
    M, N = a.shape[-2], b.shape[-2]
    a3 = a.expand(*batch_shape, M, K).reshape(-1, M, K).contiguous() if a.dim() > 2 else a.contiguous()
    bb = b.expand(*batch_shape, N, K) if b.dim() > 2 else b
    b3 = bb.reshape(-1, N, K).contiguous() if bb.dim() > 2 else bb.contiguous()
    nbat = 1
    for n in batch_shape:
        nbat *= n
    out = torch.empty(*batch_shape, M, N, dtype=out_dtype, device=a.device)
    if alpha is not None:
        alpha = alpha.reshape(()).to(torch.float32).contiguous()
    bias = _bias_operand(bias)
    d = GemmDesc()
    d.A, d.B, d.C = a3.data_ptr(), b3.data_ptr(), out.data_ptr()
    d.M, d.N, d.K = M, N, K
    d.lda, d.ldb, d.ldc = K * 2, K * 2, N
    d.a_fmt = d.b_fmt = OP_BF16
    d.batch = nbat
    d.batch_stride_a = M * K * 2 if a.dim() > 2 else 0
    d.batch_stride_b = N * K * 2 if bb.dim() > 2 else 0
    d.batch_stride_c = M * N
    d.epi = _epilogue(EPI_PLAIN, out_dtype, alpha, bias)
    run(d, a.device)
    return out


def _parse_layout(layout: str):
    ops_, out = layout.split("->")
    act, w = ops_.split(",")
    if act not in ("xc", "cx") or w not in ("kc", "ck") or out not in ("xk", "kx"):
        raise AssertionError(layout)
    return act, w, out


def _to_kc(act, w, a, b, native_w):
    """Operands as [.., M, K] and [.., N, K] from their stored layouts."""
    if act == "cx":
        a = a.mT
    # linear's native weight is kc ([N, K]); matmul's is ck ([K, N])
    if w == "ck":
        b = b.mT
    return a, b


def _gemm_in_layout(a, b, layout, out_dtype, bias, native, alpha=None):
    act, w, out_l = _parse_layout(layout)
    a, b = _to_kc(act, w, a, b, native)
    dtype = a.dtype if out_dtype is None else out_dtype
    if out_dtype is None and bias is not None and bias.dtype != a.dtype:
        dtype = torch.promote_types(a.dtype, bias.dtype)
    y = gemm_bf16(a, b, dtype, bias, alpha)
    return y.mT.contiguous() if out_l != "xk" else y


def _linear_cuda(input, weight, bias=None, *, layout=LINEAR_LAYOUT, out_dtype=None):
    _require_gpu(input, weight, bias)
    return _gemm_in_layout(input, weight, layout, out_dtype, bias, LINEAR_LAYOUT)


def _matmul_cuda(input, other, *, layout=MATMUL_LAYOUT, out_dtype=None):
    _require_gpu(input, other)
    return _gemm_in_layout(input, other, layout, out_dtype, None, MATMUL_LAYOUT)


cuda_kernel("linear")(_linear_cuda)
cuda_kernel("matmul")(_matmul_cuda)


def _gemm_shape(a, b, layout, bias, out_dtype):
    act, w, out_l = _parse_layout(layout)
    if act == "cx":
        a = a.mT
    if w == "ck":
        b = b.mT
    batch = torch.broadcast_shapes(a.shape[:-2], b.shape[:-2]) if (a.dim() > 2 or b.dim() > 2) else ()
    shape = [*batch, a.shape[-2], b.shape[-2]]
    if out_l == "kx":
        shape[-2], shape[-1] = shape[-1], shape[-2]
    dtype = a.dtype if out_dtype is None else out_dtype
    return shape, dtype


@fake_kernel("linear")
def _linear_fake(input, weight, bias=None, *, layout=LINEAR_LAYOUT, out_dtype=None):
    shape, dtype = _gemm_shape(input, weight, layout, bias, out_dtype)
    return input.new_empty(shape, dtype=dtype)


@fake_kernel("matmul")
def _matmul_fake(input, other, *, layout=MATMUL_LAYOUT, out_dtype=None):
    shape, dtype = _gemm_shape(input, other, layout, None, out_dtype)
    return input.new_empty(shape, dtype=dtype)


# ----------------------------------------------------------------- *_mx
def _decode(x, scale, code, block_size):
    """``_dequantize_mx`` (``ops/quantized.py:574-591``) on the GPU."""
    if code is None and scale is None:
        return x
    if scale is None:
        return decode_codes(x, code) if code is not None else x
    return _dequantize_mx_cuda(x, scale, block_size, code)


def _mx_common(kind, x, w, bias, input_scale, weight_scale, block_size, input_code, weight_code, alpha, A_data,
               A_indices, A_indptr, layout, out_dtype):
    _require_gpu(x, w, bias, input_scale, weight_scale, input_code, weight_code, alpha, A_data, A_indices,
                 A_indptr)
    xd = _decode(x, input_scale, input_code, block_size)
    wd = _decode(w, weight_scale, weight_code, block_size)
    dtype = xd.dtype if out_dtype is None else out_dtype
    act, wl, out_l = _parse_layout(layout)
    a, b = _to_kc(act, wl, xd, wd, None)
    acc_bias = bias if kind == "linear_mx" else None
    if a.dtype != torch.bfloat16 or b.dtype != torch.bfloat16:
        raise NotImplementedError(f"quantized_ops.{kind}: decoded operands must be bfloat16 on the GPU")
    if A_data is None:
        y = gemm_bf16(a, b, dtype, acc_bias, alpha)
    else:
        # The outlier product (ops/quantized.py:709-720, 789-802): the GEMM's
        # float32 result (alpha and bias applied) is the base the CSR product
        # of the decoded weight adds to before the one rounding to dtype.
        from .sparse import spmm_into

        if torch.promote_types(dtype, torch.float32) != torch.float32:
            raise NotImplementedError(f"quantized_ops.{kind}: {dtype} output with an outlier term")
        y32 = gemm_bf16(a, b, torch.float32, acc_bias, alpha)
        y = spmm_into(A_data, A_indices, A_indptr, wd, wl, dtype, base=y32)
    return y.mT.contiguous() if out_l != "xk" else y


def _linear_mx_cuda(input, weight, bias=None, *, input_scale=None, weight_scale=None, block_size=None,
                    input_code=None, weight_code=None, alpha=None, A_data=None, A_indices=None, A_indptr=None,
                    layout=LINEAR_LAYOUT, out_dtype=None):
    return _mx_common("linear_mx", input, weight, bias, input_scale, weight_scale, block_size, input_code,
                      weight_code, alpha, A_data, A_indices, A_indptr, layout, out_dtype)


def _matmul_mx_cuda(self, other, *, input_scale=None, weight_scale=None, block_size=None, input_code=None,
                    weight_code=None, alpha=None, A_data=None, A_indices=None, A_indptr=None,
                    layout=MATMUL_LAYOUT, out_dtype=None):
    return _mx_common("matmul_mx", self, other, None, input_scale, weight_scale, block_size, input_code,
                      weight_code, alpha, A_data, A_indices, A_indptr, layout, out_dtype)


cuda_kernel("linear_mx")(_linear_mx_cuda)
cuda_kernel("matmul_mx")(_matmul_mx_cuda)


@fake_kernel("linear_mx")
def _linear_mx_fake(input, weight, bias=None, **kwargs):
    shape, dtype = _gemm_shape(input, weight, kwargs.get("layout", LINEAR_LAYOUT), bias, kwargs.get("out_dtype"))
    return input.new_empty(shape, dtype=dtype)


@fake_kernel("matmul_mx")
def _matmul_mx_fake(self, other, **kwargs):
    shape, dtype = _gemm_shape(self, other, kwargs.get("layout", MATMUL_LAYOUT), None, kwargs.get("out_dtype"))
    return self.new_empty(shape, dtype=dtype)


# ----------------------------------------------------------------- packed GEMMs
def linear_fp8(xq: torch.Tensor, wq: torch.Tensor, scale: torch.Tensor, out: Optional[torch.Tensor] = None,
               tile_hint: int = 0) -> torch.Tensor:
    """Per-tensor FP8 linear as a lowered graph runs it: ``dequantize(linear(
    xq, wq), s)`` (``quantization/quantize_pt2e.py:538-600``) with E4M3 bytes
    ``xq`` [M, K] and ``wq`` [N, K] and the bf16 scale product ``s``: the fp32
    accumulator is rounded to bf16, multiplied by ``s`` and rounded again."""
    if xq.element_size() != 1 or wq.element_size() != 1:
        raise RuntimeError("linear_fp8: operands must hold one-byte E4M3 codes")
    xq, wq = _rows(xq), _rows(wq)
    M, K = xq.shape
    N = wq.shape[0]
    if wq.shape[1] != K:
        raise RuntimeError("linear_fp8: contraction mismatch")
    if out is None:
        out = torch.empty(M, N, dtype=torch.bfloat16, device=xq.device)
    elif (out.dtype != torch.bfloat16 or tuple(out.shape) != (M, N) or out.stride(1) != 1
          or out.stride(0) < N):
        raise RuntimeError("linear_fp8: out must be a bfloat16 [M, N] tensor with unit column stride")
    d = GemmDesc()
    d.A, d.B, d.C = xq.data_ptr(), wq.data_ptr(), out.data_ptr()
    d.M, d.N, d.K = M, N, K
    d.lda, d.ldb, d.ldc = xq.stride(0), wq.stride(0), out.stride(0)
    d.a_fmt = d.b_fmt = OP_FP8
    d.tile_hint = tile_hint
    d.epi = _epilogue(EPI_ROUND_SCALE, torch.bfloat16, scale)
    run(d, xq.device)
    return out


def linear_mxint8(x_codes, x_scale, w_codes, w_scale, block_size: int, bias_x: int, bias_w: int,
                  out_dtype=torch.bfloat16, bias=None, alpha=None, tile_hint: int = 0,
                  split_k: int = 0) -> torch.Tensor:
    """MX-int8 ``linear_mx`` on packed operands: int8 codes with biased
    power-of-two scale bytes, decoded exactly to bf16 in the GEMM's staging.
    Grids too small for the GPU split K (``split_k`` 0: automatic); the
    partials live in a workspace from torch's allocator.  With 16-element
    blocks, no tile or split asked for and ``mxint8_two_pass_pays``, both
    operands are rebased to exact fp16 rows (``bake_mx8_f16``) and
    multiplied by ``linear_mx8_f16`` instead."""
    x_codes, w_codes, x_scale, w_scale = _rows(x_codes), _rows(w_codes), _rows(x_scale), _rows(w_scale)
    M, K = x_codes.shape
    N = w_codes.shape[0]
    if w_codes.shape[1] != K:
        raise RuntimeError("linear_mxint8: contraction mismatch")
    if (block_size == 16 and tile_hint == 0 and split_k == 0 and K % 16 == 0
            and x_scale.shape == (M, K // 16) and w_scale.shape == (N, K // 16) and mxint8_two_pass_pays(M, N, K)):
        bx = bake_mx8_f16(x_codes.view(torch.int8), x_scale, bias_x)
        bw = bake_mx8_f16(w_codes.view(torch.int8), w_scale, bias_w)
        return linear_mx8_f16(bx.w, bx.e, bw, out_dtype, bias, alpha)
    out = torch.empty(M, N, dtype=out_dtype, device=x_codes.device)
    if alpha is not None:
        alpha = alpha.reshape(()).to(torch.float32).contiguous()
    bias = _bias_operand(bias)
    d = GemmDesc()
    d.A, d.B, d.C = x_codes.data_ptr(), w_codes.data_ptr(), out.data_ptr()
    d.M, d.N, d.K = M, N, K
    d.lda, d.ldb, d.ldc = x_codes.stride(0), w_codes.stride(0), N
    d.a_fmt = d.b_fmt = OP_MXI8
    d.a_scale, d.b_scale = x_scale.data_ptr(), w_scale.data_ptr()
    d.a_scale_ld, d.b_scale_ld = x_scale.stride(0), w_scale.stride(0)
    d.a_block = d.b_block = block_size
    d.a_bias, d.b_bias = bias_x, bias_w
    d.tile_hint = tile_hint
    d.split_k = split_k
    d.epi = _epilogue(EPI_PLAIN, out_dtype, alpha, bias)
    nbytes = load().vh_gemm_workspace_bytes(ctypes.c_void_p(ctypes.addressof(d)))
    ws = None
    if nbytes > 0:  # split-K partials (fp32), from torch's caching allocator
        ws = torch.empty(nbytes // 4, dtype=torch.float32, device=x_codes.device)
        d.workspace, d.workspace_bytes = ws.data_ptr(), nbytes
    run(d, x_codes.device)
    return out


def mxint8_two_pass_pays(M: int, N: int, K: int) -> bool:
    """Whether ``linear_mxint8`` rebases both operands to fp16 rows and runs
    the fp16 GEMM rather than decoding the codes in the GEMM's staging.
    Measured on MI355X (packed / two-pass, us): (K, N) = (4096, 4096) at
    M = 1024: 53.8 / 60.4, M = 2048: 87.0 / 76.7; (4096, 14336): 161.4 /
    134.9, 326.1 / 241.6; (14336, 4096): 181.4 / 164.8, 288.8 / 240.3."""
    return M >= MXI8_TWO_PASS_MIN_M and M * N * K >= MXI8_TWO_PASS_MIN_WORK


#: The two-pass MX-int8 linear needs at least these rows and this much work
#: (M * N * K).
MXI8_TWO_PASS_MIN_M = 1024
MXI8_TWO_PASS_MIN_WORK = 1 << 35


# ----------------------------------------------------------------- MX-int8, small M
class MX8F16Weight(NamedTuple):
    """An MX-int8 weight (block 16, power-of-two scales) baked for
    ``linear_mx8_f16``: each row as exact fp16 ``code * 2**(e - E)`` with the
    row's largest block exponent ``E``."""

    w: torch.Tensor  # float16 [N, K]
    e: torch.Tensor  # int32 [N]
    N: int
    K: int


def bake_mx8_f16(codes: torch.Tensor, scale_bytes: torch.Tensor, scale_bias: int) -> MX8F16Weight:
    """Bake packed MX-int8 weights (int8 codes [N, K], scale bytes [N, K / 16]
    as ``packed.quantize_mx_packed`` writes them)."""
    N, K = codes.shape
    if K % 16 or scale_bytes.shape != (N, K // 16):
        raise ValueError("bake_mx8_f16 needs [N, K] codes with one scale byte per 16 along K")
    c = codes.contiguous()
    sb = scale_bytes.contiguous()
    w = torch.empty(N, K, dtype=torch.float16, device=codes.device)
    e = torch.empty(N, dtype=torch.int32, device=codes.device)
    _lib.check(load().vh_mx8_bake_f16(ptr(c), ptr(sb), int(scale_bias), N, K, ptr(w), ptr(e),
                                      ctypes.c_void_p(stream_of(codes))), "vh_mx8_bake_f16")
    return MX8F16Weight(w, e, N, K)


def quantize_mx8_f16(x: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """``quantize_mx(x, int8, [-1], 16, 127, force_scale_power_of_two=True)``
    of the rows of a bf16 ``x`` [M, K], as the exact fp16 rows ``linear_mx8_f16``
    reads, and their exponents."""
    if x.dtype != torch.bfloat16 or x.dim() != 2:
        raise NotImplementedError("quantize_mx8_f16 takes a 2-D bfloat16 tensor")
    M, K = x.shape
    xc = x.contiguous()
    out = torch.empty(M, K, dtype=torch.float16, device=x.device)
    ex = torch.empty(M, dtype=torch.int32, device=x.device)
    _lib.check(load().vh_quantize_mx8_f16(ptr(xc), M, K, ptr(out), ptr(ex), ctypes.c_void_p(stream_of(x))),
               "vh_quantize_mx8_f16")
    return out, ex


def mx8_f16_plan(M: int, N: int, K: int) -> Tuple[int, int]:
    """(tile, splits) of ``linear_mx8_f16``.  Measured on MI355X at K = N =
    4096, one split storing through the GEMM's own epilogue unless stated:
    M = 2048 on 256x128 tiles 56.0 us (1226 TFLOP/s; 128x128 65.0; 256x128
    in two splits plus the reduction 92.5); M = 256 on 64x64 tiles (two
    waves, eight stages) 15.8 us (64x128 18.9; 64x64 in two splits plus the
    reduction 25.9); M = 128 / 64 / 16 on 64x64 tiles in two splits 15.1 /
    14.7 / 12.5 us (unsplit 15.7 / 15.7 / 15.5; 64x128 18.7 / 18.6 / 16.8);
    M = 512 on 64x128 tiles 21.5 us (64x64 30.1).  So: 64x64 while its grid
    is at most 256 workgroups, in two K splits while that grid is at most
    128; then 64x128 below 1024 rows (K split until the grid reaches 128
    workgroups, each split at least 512 elements); from 1024, 256x128."""
    if M >= 1024:
        return 3, 1
    t64 = -(-M // 64) * -(-N // 64)
    if t64 <= 256:
        return 4, (2 if t64 <= 128 and K % (2 * 512) == 0 else 1)
    tiles = -(-M // 64) * -(-N // 128)
    splits = 1
    while tiles * splits < 128 and K % (splits * 2 * 512) == 0 and splits < 8:
        splits *= 2
    return 1, splits


def linear_mx8_f16(x16: torch.Tensor, ex: torch.Tensor, weight: MX8F16Weight, out_dtype=torch.bfloat16, bias=None,
                   alpha=None, tile: int = -1, splits: int = 0) -> torch.Tensor:
    """MX-int8 ``linear_mx`` (``ops/quantized.py:651-723``) on the exact fp16
    operands of ``quantize_mx8_f16`` and ``bake_mx8_f16``: an fp16 GEMM over
    K splits and one reduction that applies ``2**(E_row + E_col)``, alpha,
    bias and the output rounding; unsplit, the GEMM's epilogue applies them
    itself."""
    x16 = x16.contiguous()
    M, K = x16.shape
    if K != weight.K:
        raise RuntimeError("linear_mx8_f16: contraction mismatch")
    N = weight.N
    t, sp = mx8_f16_plan(M, N, K)
    tile = t if tile < 0 else tile
    splits = sp if splits <= 0 else splits
    out = torch.empty(M, N, dtype=out_dtype, device=x16.device)
    if alpha is not None:
        alpha = alpha.reshape(()).to(torch.float32).contiguous()
    bias = _bias_operand(bias)
    epi = _epilogue(EPI_PLAIN, out_dtype, alpha, bias)
    # one split stores through the GEMM's own epilogue (rows of N outputs,
    # N a multiple of 8): no float32 partials
    direct = splits == 1 and N % 8 == 0
    part = None if direct else torch.empty(splits * M * N, dtype=torch.float32, device=x16.device)
    _lib.check(load().vh_gemm_mx8_f16(ptr(x16), ptr(ex), ptr(weight.w), ptr(weight.e), M, N, K,
                                      ctypes.c_void_p(ctypes.addressof(epi)), ptr(out), N, ptr(part),
                                      0 if part is None else part.numel() * 4, splits, tile,
                                      ctypes.c_void_p(stream_of(x16))),
               "vh_gemm_mx8_f16")
    return out


def posit8_lut(qmap: torch.Tensor) -> torch.Tensor:
    """256-entry bf16 decode table of posit8 packed codes (code -> entry)."""
    c = formats.classify(qmap)
    codes = torch.arange(256, dtype=torch.uint8, device=qmap.device)
    from .ops import _elementwise

    return _elementwise("dequantize", codes, None, None, None, torch.bfloat16, c.fmt, None, torch.bfloat16)


def decode_bytes(codes: torch.Tensor, lut: torch.Tensor) -> torch.Tensor:
    """bf16 ``lut[codes]`` for one-byte codes (``vh_decode_bytes``)."""
    c = codes.contiguous()
    if c.data_ptr() % 16:
        c = c.clone()
    out = torch.empty(c.shape, dtype=torch.bfloat16, device=c.device)
    st = load().vh_decode_bytes(ptr(c), c.numel(), ptr(lut.contiguous()), ptr(out), ctypes.c_void_p(stream_of(c)))
    _lib.check(st, "vh_decode_bytes")
    return out


def linear_posit8(x_codes, w_codes, lut: torch.Tensor, out_dtype=torch.bfloat16, tile_hint: int = 0):
    """Posit8 ``linear`` on packed codes (``quantize_pt2e.py:557-561``: a
    direct cast, the GEMM reads posit values as bf16), one rounding at the
    end.  Both operands are decoded through ``lut`` to bf16 (exact) and run
    through the bf16 GEMM; with a ``tile_hint`` the codes are decoded while
    the GEMM stages them instead."""
    x_codes, w_codes = _rows(x_codes), _rows(w_codes)
    M, K = x_codes.shape
    N = w_codes.shape[0]
    if w_codes.shape[1] != K:
        raise RuntimeError("linear_posit8: contraction mismatch")
    if tile_hint == 0 and K % 8 == 0:
        return gemm_bf16(decode_bytes(x_codes, lut), decode_bytes(w_codes, lut), out_dtype)
    out = torch.empty(M, N, dtype=out_dtype, device=x_codes.device)
    d = GemmDesc()
    d.A, d.B, d.C = x_codes.data_ptr(), w_codes.data_ptr(), out.data_ptr()
    d.M, d.N, d.K = M, N, K
    d.lda, d.ldb, d.ldc = x_codes.stride(0), w_codes.stride(0), N
    d.a_fmt = d.b_fmt = OP_P8
    d.lut = lut.data_ptr()
    d.tile_hint = tile_hint
    d.epi = _epilogue(EPI_PLAIN, out_dtype)
    run(d, x_codes.device)
    return out


# ----------------------------------------------------------------- MXNF4 GEMV
class NF4Weight(NamedTuple):
    """Weights baked for ``linear_nf4``: level indices packed two per byte in
    the GEMV's MFMA lane order, plus one scale-map code per 64-block."""

    packed: torch.Tensor      # uint8, N * K / 2
    scale: torch.Tensor       # uint8 [N / 16, K / 64, 16], tile-major (nf4_tile_scales)
    scale_fmt: "formats.Classified"
    levels: bytes             # the 16 int8 codebook levels
    N: int
    K: int


def _levels_of(entries: torch.Tensor) -> bytes:
    lv = entries.detach().float().cpu()
    if lv.numel() != 16 or not torch.equal(lv, lv.round()) or lv.abs().max() > 127:
        raise ValueError("linear_nf4 needs a 16-entry codebook of integer levels in [-127, 127]")
    return bytes(int(v) & 0xFF for v in lv.tolist())


def nf4_tile_scales(scale_bytes: torch.Tensor) -> torch.Tensor:
    """Weight scale bytes ``[N, K/64]`` -> the GEMV's tile-major layout
    ``[N/16, K/64, 16]`` (a tile's 16 bytes of a block contiguous)."""
    N, nb = scale_bytes.shape
    return scale_bytes.reshape(N // 16, 16, nb).transpose(1, 2).contiguous()


def bake_nf4_weight(w: torch.Tensor, index_table: torch.Tensor, scale_qmap: torch.Tensor,
                    entries: torch.Tensor) -> NF4Weight:
    """``quantize_mx(w, index_table, [-1], 64, 31, scale_qmap=...)`` once (as
    convert bakes weights, ``quantization/quantize_pt2e.py:819-828``), then
    packed for the GEMV: nibbles in MFMA lane order, scale bytes tile-major."""
    from . import packed as _packed

    N, K = w.shape
    p = _packed.quantize_mx_packed(w, index_table, [-1], 64, 31.0, False, scale_qmap)
    out = torch.empty(N * K // 2, dtype=torch.uint8, device=w.device)
    st = load().vh_pack_nf4(ctypes.c_void_p(p.codes.data_ptr()), N, K, ctypes.c_void_p(out.data_ptr()),
                            ctypes.c_void_p(stream_of(w)))
    _lib.check(st, "vh_pack_nf4")
    return NF4Weight(out, nf4_tile_scales(p.scale), p.scale_fmt, _levels_of(entries), N, K)


_level_lut_cache = {}


def _level_lut(levels: bytes, device) -> torch.Tensor:
    key = (levels, str(device))
    t = _level_lut_cache.get(key)
    if t is None:
        lut = list(levels) + [0] * (256 - len(levels))
        t = torch.tensor(lut, dtype=torch.uint8, device=device)
        _level_lut_cache[key] = t
    return t


def _nf4_fusable(x: torch.Tensor, ec, sc) -> bool:
    """Whether ``vh_gemv_nf4_m1`` can take this call: one bfloat16 row, a
    minifloat activation scale map and an index table of at most 16 levels."""
    f, s = ec.fmt, sc.fmt
    return (x.shape[0] == 1 and x.dtype == torch.bfloat16 and s.kind == FMT_MINIFLOAT
            and not (s.flags & FMT_HW_E4M3) and f.kind == FMT_STEPS and f.nsteps <= 15 and f.nan_level <= 15)


def _nf4_one_launch_pays(N: int, K: int) -> bool:
    """Every 16-column tile (pair of tiles from 512 tiles) quantizes the
    row again, which costs less than a second launch at K = 4096 (MI355X,
    weights from HBM: 5.7-6.3 us against 7.8-8.4 at N <= 4096; 12.0 against
    13.7 at N = 14336); at K = 14336 the two are even (16.0 / 15.7 us)."""
    return K <= 4096


def nf4_prefill_plan(M: int, N: int, K: int, tile: int = 0, splits: int = 0) -> Tuple[int, int]:
    """(tile, splits) ``vh_gemm_nf4`` takes for a shape."""
    t, sp, bm = ctypes.c_int32(tile), ctypes.c_int32(splits), ctypes.c_int64(0)
    _lib.check(load().vh_gemm_nf4_plan(M, N, K, ctypes.byref(t), ctypes.byref(sp), ctypes.byref(bm)),
               "vh_gemm_nf4_plan")
    return t.value, sp.value


def linear_nf4_prefill(x: torch.Tensor, weight: NF4Weight, index_table: torch.Tensor, scale_qmap: torch.Tensor,
                       out_dtype=torch.bfloat16, bias=None, alpha=None, tile: int = 0,
                       splits: int = 0, two_pass: Optional[bool] = None) -> torch.Tensor:
    """MXNF4 ``linear_mx`` at any M on the GEMV's baked weight: the
    activation's ``quantize_mx`` to index and scale bytes, then
    ``vh_gemm_nf4``, which decodes both operands while staging to the
    reference's ``bf16(level * scale)`` and multiplies them on the bf16 MFMA
    with float32 accumulation."""
    from . import packed as _packed

    M, K = x.shape
    if K != weight.K:
        raise RuntimeError("linear_nf4_prefill: contraction mismatch")
    px = _packed.quantize_mx_packed(x.contiguous(), index_table, [-1], 64, 31.0, False, scale_qmap)
    return gemm_nf4_packed(px, weight, out_dtype, bias, alpha, tile, splits, two_pass)


def nf4_decode_bf16(px, weight: NF4Weight, decode_x: bool = True, decode_w: bool = True):
    """``(x, w)``: the operands ``vh_gemm_nf4`` multiplies, decoded once to
    bf16 (``vh_nf4_decode_bf16``): the activation packed by
    ``quantize_mx_packed`` [M, K] and the baked weight's rows [N, K], each
    ``bf16(level * scale)`` as the reference decodes them; None where not
    asked for."""
    M, K = px.codes.shape
    if K != weight.K:
        raise RuntimeError("nf4_decode_bf16: contraction mismatch")
    dev = weight.packed.device
    xo = torch.empty(M, K, dtype=torch.bfloat16, device=dev) if decode_x else None
    wo = torch.empty(weight.N, K, dtype=torch.bfloat16, device=dev) if decode_w else None
    codes, scale = px.codes.contiguous(), px.scale.contiguous()
    lv = ctypes.create_string_buffer(weight.levels, 16)
    st = load().vh_nf4_decode_bf16(ptr(codes), ptr(scale), ctypes.byref(px.scale_fmt.fmt), M,
                                   ptr(weight.packed), ptr(weight.scale), ctypes.byref(weight.scale_fmt.fmt), lv,
                                   weight.N, K, ptr(xo), ptr(wo), ctypes.c_void_p(stream_of(weight.packed)))
    _lib.check(st, "vh_nf4_decode_bf16")
    return xo, wo


def nf4_two_pass_pays(M: int, N: int, K: int) -> bool:
    """Whether the prefill runs as two passes (both operands decoded once,
    then the bf16 GEMM) rather than ``vh_gemm_nf4``, which decodes each
    weight block once per row tile of the output.  Measured on MI355X
    (fused / two-pass, us): (K, N) = (4096, 4096) at M = 256: 35.1 / 37.5,
    M = 512: 49.8 / 37.4, M = 2048: 96.3 / 74.4; (4096, 14336): 78.0 / 57.8,
    95.4 / 79.5, 368.7 / 227.9; (14336, 4096): 77.1 / 90.1, 140.8 / 98.7,
    321.1 / 219.1.  The two-pass form holds the decoded weight (2 bytes per
    element) for the call."""
    return M >= NF4_TWO_PASS_MIN_M


#: Rows from which the two-pass MXNF4 prefill is taken.
NF4_TWO_PASS_MIN_M = 512


def gemm_nf4_packed(px, weight: NF4Weight, out_dtype=torch.bfloat16, bias=None, alpha=None, tile: int = 0,
                    splits: int = 0, two_pass: Optional[bool] = None) -> torch.Tensor:
    """``vh_gemm_nf4`` on an activation already packed by ``quantize_mx_packed``
    (index bytes [M, K] and scale codes [M, K / 64]); with ``two_pass`` (by
    default where ``nf4_two_pass_pays``) the operands decoded once by
    ``nf4_decode_bf16`` and multiplied by the bf16 GEMM instead, which gives
    the same products summed in another order."""
    M, K = px.codes.shape
    if K != weight.K:
        raise RuntimeError("gemm_nf4_packed: contraction mismatch")
    if two_pass is None:
        two_pass = nf4_two_pass_pays(M, weight.N, K)
    if two_pass:
        xo, wo = nf4_decode_bf16(px, weight)
        return gemm_bf16(xo, wo, out_dtype, bias, alpha)
    y = torch.empty(M, weight.N, dtype=out_dtype, device=px.codes.device)
    if alpha is not None:
        alpha = alpha.reshape(()).to(torch.float32).contiguous()
    bias = _bias_operand(bias)
    epi = _epilogue(EPI_PLAIN, out_dtype, alpha, bias)
    lv = ctypes.create_string_buffer(weight.levels, 16)
    tile, splits = nf4_prefill_plan(M, weight.N, K, tile, splits)
    part = torch.empty(splits * M * weight.N, dtype=torch.float32, device=y.device) if splits > 1 else None
    st = load().vh_gemm_nf4(ctypes.c_void_p(px.codes.data_ptr()), ctypes.c_void_p(px.scale.data_ptr()),
                            ctypes.byref(px.scale_fmt.fmt), M, ctypes.c_void_p(weight.packed.data_ptr()),
                            ctypes.c_void_p(weight.scale.data_ptr()), ctypes.byref(weight.scale_fmt.fmt), lv,
                            weight.N, weight.K, ctypes.c_void_p(ctypes.addressof(epi)),
                            ctypes.c_void_p(y.data_ptr()), weight.N, tile, splits, ptr(part),
                            0 if part is None else part.numel() * 4, ctypes.c_void_p(stream_of(y)))
    _lib.check(st, "vh_gemm_nf4")
    return y


def linear_nf4(x: torch.Tensor, weight: NF4Weight, index_table: torch.Tensor, scale_qmap: torch.Tensor,
               out_dtype=torch.bfloat16, bias=None, alpha=None, fused=None) -> torch.Tensor:
    """MXNF4 ``linear_mx`` on the baked weight.  At decode shapes (M <= 16)
    the activations are quantized like the reference's in-graph
    ``quantize_mx`` (one launch that emits their int8 levels and float32
    block scales), then the weight-streaming GEMV.  One bfloat16 row is
    quantized inside the GEMV instead (``vh_gemv_nf4_m1``: the same levels
    and scales, one launch) when the formats allow and the shape is small
    enough for that to pay (``_nf4_one_launch_pays``); ``fused`` = False
    keeps the two launches, True requires the one.  More rows take the
    prefill GEMM (``linear_nf4_prefill``)."""
    M, K = x.shape
    if K != weight.K:
        raise RuntimeError("linear_nf4: contraction mismatch")
    if M > 16:
        if fused:
            raise RuntimeError("linear_nf4: the one-launch path takes one row")
        return linear_nf4_prefill(x, weight, index_table, scale_qmap, out_dtype, bias, alpha)
    xc = x.contiguous()
    ec = formats.classify(index_table)
    sc = formats.classify(scale_qmap)
    one = _nf4_fusable(xc, ec, sc)
    if fused and not one:
        raise RuntimeError("linear_nf4: the one-launch path needs one bfloat16 row, a minifloat scale map and "
                           "an index table of at most 16 levels")
    if fused is None:
        fused = one and _nf4_one_launch_pays(weight.N, K)
    if fused:
        y = torch.empty(M, weight.N, dtype=out_dtype, device=x.device)
        if alpha is not None:
            alpha = alpha.reshape(()).to(torch.float32).contiguous()
        bias = _bias_operand(bias)
        epi = _epilogue(EPI_PLAIN, out_dtype, alpha, bias)
        lv = ctypes.create_string_buffer(weight.levels, 16)
        st = load().vh_gemv_nf4_m1(ctypes.c_void_p(xc.data_ptr()), dtype_code(xc.dtype), 31.0,
                                   ctypes.byref(sc.fmt), ctypes.byref(ec.fmt),
                                   ctypes.c_void_p(weight.packed.data_ptr()), ctypes.c_void_p(weight.scale.data_ptr()),
                                   ctypes.byref(weight.scale_fmt.fmt), lv, weight.N, weight.K,
                                   ctypes.c_void_p(ctypes.addressof(epi)), ctypes.c_void_p(y.data_ptr()),
                                   ctypes.c_void_p(stream_of(x)))
        _lib.check(st, "vh_gemv_nf4_m1")
        return y
    xl = torch.empty(M, K, dtype=torch.uint8, device=x.device)
    xs = torch.empty(K // 64, 16, dtype=torch.float32, device=x.device)  # block-major, rows past M unused
    lut = _level_lut(weight.levels, x.device)
    lib_ = load()
    st = lib_.vh_quantize_mx_rows16(ctypes.c_void_p(xc.data_ptr()), dtype_code(xc.dtype), M, K, 64, 31.0,
                                    ctypes.byref(sc.fmt), ctypes.byref(ec.fmt), ctypes.c_void_p(xs.data_ptr()),
                                    ctypes.c_void_p(xl.data_ptr()), ctypes.c_void_p(lut.data_ptr()),
                                    ctypes.c_void_p(stream_of(x)))
    _lib.check(st, "vh_quantize_mx_rows16")
    y = torch.empty(M, weight.N, dtype=out_dtype, device=x.device)
    if alpha is not None:
        alpha = alpha.reshape(()).to(torch.float32).contiguous()
    bias = _bias_operand(bias)
    epi = _epilogue(EPI_PLAIN, out_dtype, alpha, bias)
    lv = ctypes.create_string_buffer(weight.levels, 16)
    st = lib_.vh_gemv_nf4(ctypes.c_void_p(xl.data_ptr()), ctypes.c_void_p(xs.data_ptr()), M,
                          ctypes.c_void_p(weight.packed.data_ptr()), ctypes.c_void_p(weight.scale.data_ptr()),
                          ctypes.byref(weight.scale_fmt.fmt), lv, weight.N, weight.K,
                          ctypes.c_void_p(ctypes.addressof(epi)), ctypes.c_void_p(y.data_ptr()),
                          ctypes.c_void_p(stream_of(x)))
    _lib.check(st, "vh_gemv_nf4")
    return y
