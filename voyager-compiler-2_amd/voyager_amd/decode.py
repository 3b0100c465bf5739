"""Decode step of an MX-int8 / KIVI Llama decoder layer on the GPU.

The reference runs a converted decode graph whose linears are
``quantize_mx`` + ``linear_mx`` on baked weight codes
(``quantization/quantize_pt2e.py:582-600``, ``:819-828``) and whose KV cache
is a KIVI main part (``quantize_affine`` / ``dequantize`` with
``uint2,bs=32,qs=group_wise_affine,ax=-2|-1``,
``examples/language_modeling/quantization_configs.py:171-207``) plus a
full-precision residual window (``codegen/transform/quant_folding.py:1025-1120``).
This module is the lowered GPU form of that graph: weights are baked once into
the MX-int8 GEMV layout, the cache into the KIVI attention layout, and each
step is seven launches (``include/voyager_hip.h``, "decoder-layer decode
step").  Every buffer is allocated up front, so a step can be captured in a
HIP graph and replayed.
"""

import ctypes
import math
from typing import Dict, NamedTuple, Optional

import torch

from . import _lib, formats, packed
from ._lib import check, load, ptr
from .ops import _quantize_affine_cuda

MX_BLOCK = 16
KIVI_GROUP = 32
HEAD_DIM = 128
GQA = 4


def _stream(t: torch.Tensor) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


class ErrorFlag:
    """The device int32 the decode kernels OR ``DECODE_ERR_*`` bits into.
    Kernels never clear it: read it with :meth:`check`, which clears it."""

    def __init__(self, device):
        self.t = torch.zeros(1, dtype=torch.int32, device=device)

    _WHAT = (
        (_lib.DECODE_ERR_FP16_RANGE, "an activation block exceeds the fp16 range of the GEMV operand"),
        (_lib.DECODE_ERR_WEIGHT_RANGE, "a weight block exponent is outside [-24, 5]"),
        (_lib.DECODE_ERR_KV_CODE, "a KIVI chunk folded into the main cache held a value whose code is NaN"),
        (_lib.DECODE_ERR_KV_FULL, "the KIVI main cache had no room for a completed chunk"),
        (_lib.DECODE_ERR_KV_STATE, "the KIVI cache state was out of range (nothing was computed)"),
    )

    def check(self) -> None:
        """Synchronising check: clear the flag, and raise if a kernel flagged
        unrepresentable data since the last check."""
        v = int(self.t.item())
        if v:
            self.t.zero_()
            what = [msg for bit, msg in self._WHAT if v & bit]
            raise RuntimeError("voyager_amd decode: " + "; ".join(what))


class MX8Weight(NamedTuple):
    codes: torch.Tensor  # uint8, baked GEMV layout
    hb: torch.Tensor     # uint8, baked fp16 exponent bytes
    n_out: int           # output columns (gate/up pairs count once when paired)
    K: int
    paired: bool
    shift: Optional[torch.Tensor] = None  # int32 per weight row: the rebased rows' 2**shift, None when all 0


def bake_mx8(codes: torch.Tensor, scale: torch.Tensor, bias: int, paired: bool = False,
             rebase: bool = True) -> MX8Weight:
    """Bake packed MX-int8 weights ``[N, K]`` (codes one int8 per byte, scales
    as biased exponent bytes, as ``packed.quantize_mx_packed`` returns them).
    A row whose block exponents leave the GEMV operand's [-24, 5] is rebased
    to its largest (``rebase``; the row's blocks more than 29 binades under
    it are flushed), otherwise flagged; the bake reads back whether any row
    was (one synchronisation, at bake time)."""
    N, K = codes.shape
    if codes.dtype != torch.uint8 or scale.dtype != torch.uint8:
        raise TypeError("bake_mx8: codes and scales must be uint8")
    wc = torch.empty(N * K, dtype=torch.uint8, device=codes.device)
    wh = torch.empty(N * K // MX_BLOCK, dtype=torch.uint8, device=codes.device)
    shift = torch.empty(N, dtype=torch.int32, device=codes.device) if rebase else None
    flag = ErrorFlag(codes.device)
    st = load().vh_mx8_bake(ptr(codes.contiguous()), ptr(scale.contiguous()), int(bias), N, K, 1 if paired else 0,
                            ptr(wc), ptr(wh), ptr(shift), ptr(flag.t), _stream(codes))
    check(st, "vh_mx8_bake")
    flag.check()
    if shift is not None and not bool(shift.any()):
        shift = None
    return MX8Weight(wc, wh, N // 2 if paired else N, K, paired, shift)


def quantize_mx8_weight(w: torch.Tensor, paired: bool = False) -> MX8Weight:
    """``quantize_mx(w, int8, [-1], 16, 127, force_scale_power_of_two=True)``
    on the GPU, baked for the GEMV."""
    tab = formats.quantization_map("int8", w.device)
    p = packed.quantize_mx_packed(w, tab, [-1], MX_BLOCK, 127.0, True)
    return bake_mx8(p.codes, p.scale, p.bias, paired)


def rmsnorm_mx8(x: torch.Tensor, weight: torch.Tensor, eps: float, flag: ErrorFlag,
                fq: Optional[torch.Tensor] = None, h_out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``LlamaRMSNorm`` of each row of ``x [M, H]`` and the MX-int8 fake
    quantization (fp16) of the result; ``h_out`` receives the bf16 norm."""
    M, H = x.shape
    if fq is None:
        fq = torch.empty(M, H, dtype=torch.float16, device=x.device)
    st = load().vh_rmsnorm_mx8(ptr(x), ptr(weight), M, H, float(eps), ptr(h_out), ptr(fq), ptr(flag.t), _stream(x))
    check(st, "vh_rmsnorm_mx8")
    return fq


def gemv_mx8(x_fq: torch.Tensor, w: MX8Weight, flag: ErrorFlag, mode: int = _lib.GEMV_STORE,
             residual: Optional[torch.Tensor] = None, y: Optional[torch.Tensor] = None,
             fq_out: Optional[torch.Tensor] = None, tiles_per_block: int = 0,
             row_exp: Optional[torch.Tensor] = None):
    """``linear_mx`` of fake-quantized activations and baked weights.  STORE /
    RESIDUAL return ``y`` (bf16); SWIGLU returns the fp16 fake quantization
    of ``silu(gate) * up`` (and fills ``y`` with the bf16 product if given).
    ``row_exp`` (int32 [M]): ``x_fq`` holds rows rebased as
    ``gemm.quantize_mx8_f16`` writes them (row m times 2**-row_exp[m])."""
    M, K = x_fq.shape
    if K != w.K:
        raise ValueError(f"gemv_mx8: K mismatch ({K} vs {w.K})")
    if mode == _lib.GEMV_SWIGLU:
        if not w.paired:
            raise ValueError("gemv_mx8: SWIGLU needs a paired (gate/up) weight")
        if fq_out is None:
            fq_out = torch.empty(M, w.n_out, dtype=torch.float16, device=x_fq.device)
    elif y is None:
        y = torch.empty(M, w.n_out, dtype=torch.bfloat16, device=x_fq.device)
    if tiles_per_block == 0:
        tiles_per_block = 2 if (w.n_out // 16) >= 1024 and (w.n_out // 16) % 2 == 0 else 1
    st = load().vh_gemv_mx8(ptr(x_fq), M, K, ptr(w.codes), ptr(w.hb), w.n_out, mode, tiles_per_block, ptr(residual),
                            ptr(y), ptr(fq_out), ptr(row_exp), ptr(w.shift), ptr(flag.t), _stream(x_fq))
    check(st, "vh_gemv_mx8")
    return fq_out if mode == _lib.GEMV_SWIGLU else y


class KiviDesc(ctypes.Structure):
    """``vh_kivi_desc``."""

    _fields_ = [
        ("qkv", ctypes.c_void_p), ("qkv_ld", ctypes.c_int64),
        ("rope", ctypes.c_void_p), ("max_pos", ctypes.c_int64),
        ("main", ctypes.c_void_p), ("group_cap", ctypes.c_int64),
        ("kr", ctypes.c_void_p), ("vr", ctypes.c_void_p),
        ("state", ctypes.c_void_p),
        ("batch", ctypes.c_int64), ("nkv", ctypes.c_int64), ("nq", ctypes.c_int64), ("head_dim", ctypes.c_int64),
        ("softmax_scale", ctypes.c_float),
        ("part", ctypes.c_void_p), ("part_floats", ctypes.c_int64),
        ("attn", ctypes.c_void_p), ("attn_fq", ctypes.c_void_p), ("flag", ctypes.c_void_p),
        ("advance", ctypes.c_int32),
        ("scale_fmt", _lib.Format), ("code_fmt", _lib.Format),
    ]


def _vp(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


RES_CAP = _lib.KIVI_RES_CAP
GROUPS_PER_SPLIT = 16  # groups one attention workgroup streams


class KiviCache:
    """A KIVI KV cache for ``batch x nkv`` sequences with room for
    ``capacity`` tokens: a quantized main part in the attention layout
    (whole groups of 32 tokens) and a ``RES_CAP``-slot full-precision
    residual window holding the chunk being filled (the split cache of
    ``codegen/transform/quant_folding.py:1025-1120``).  The state the kernels
    use -- tokens in the main part, residual slots filled -- lives in device
    memory (``state``); ``n_main`` / ``n_res`` mirror it on the host, advanced
    by the same rule without a device read."""

    def __init__(self, batch: int, nkv: int, capacity: int, device):
        if capacity % KIVI_GROUP or capacity < RES_CAP:
            raise ValueError(f"KiviCache: capacity must be a multiple of 32 and at least {RES_CAP}")
        self.batch, self.nkv, self.capacity = batch, nkv, capacity
        self.P = batch * nkv
        self.group_cap = capacity // KIVI_GROUP
        self.n_main = self.n_res = 0
        bf = torch.bfloat16
        # one 3072-byte block per 32 tokens: key / value codes, key / value scale + zero point
        self.main = torch.zeros(self.P * self.group_cap * 3072, dtype=torch.uint8, device=device)
        self.kr = torch.zeros(self.P, RES_CAP, HEAD_DIM, dtype=bf, device=device)
        self.vr = torch.zeros(self.P, RES_CAP, HEAD_DIM, dtype=bf, device=device)
        self.state = torch.zeros(4, dtype=torch.int32, device=device)
        # the KIVI specs' maps (uint2 codes, fp16_e5m10 scale / zero point), for the device fold
        self.code_map = formats.quantization_map("uint2", device)
        self.scale_map = formats.quantization_map("fp16_e5m10", device)
        self.code_fmt = formats.classify(self.code_map).fmt
        self.scale_fmt = formats.classify(self.scale_map).fmt

    @property
    def position(self) -> int:
        """The position of the next step's token."""
        return self.n_main + self.n_res

    @classmethod
    def from_bf16(cls, k_main: torch.Tensor, v_main: torch.Tensor, k_res: torch.Tensor, v_res: torch.Tensor,
                  capacity: Optional[int] = None):
        """Quantize ``[batch, nkv, T, 128]`` keys / values with the KIVI specs
        (``quantize_affine`` on the GPU) and bake them; the residual tokens
        ``[batch, nkv, n, 128]`` fill the first n slots.  ``capacity``
        (default: T plus two chunks) bounds the tokens the cache can grow to.
        Returns the cache and the reference-form ``(scale, zero_point,
        codes)`` of keys and values."""
        B, nkv, T, D = k_main.shape
        if D != HEAD_DIM:
            raise ValueError(f"KiviCache: head_dim must be {HEAD_DIM}")
        dev = k_main.device
        c = cls(B, nkv, capacity if capacity is not None else T + 2 * RES_CAP, dev)
        kq = vq = None
        if T:
            kq = _quantize_affine_cuda(k_main, c.code_map, [-2], KIVI_GROUP, 0.0, 3.0, c.scale_map)
            vq = _quantize_affine_cuda(v_main, c.code_map, [-1], KIVI_GROUP, 0.0, 3.0, c.scale_map)
            c.load_main(kq, vq)
        c.load_residual(k_res, v_res)
        return c, kq, vq

    def load_main(self, kq, vq) -> None:
        """Bake reference-form ``quantize_affine`` outputs (keys grouped along
        tokens, values along channels) of T tokens as the main cache."""
        ks, kz, kcode = kq
        vs, vz, vcode = vq
        P = self.P
        T = kcode.numel() // (P * HEAD_DIM)
        if T % KIVI_GROUP or T + RES_CAP > self.capacity:
            raise ValueError(f"KiviCache: {T} main tokens (a multiple of 32) plus a chunk must fit the capacity "
                             f"{self.capacity}")
        self.n_main = T
        self._sync_state()
        if T == 0:
            return
        kc8 = kcode.reshape(P, T, HEAD_DIM).to(torch.uint8).contiguous()
        vc8 = vcode.reshape(P, T, HEAD_DIM).to(torch.uint8).contiguous()
        ks_, kz_ = ks.reshape(P, T // KIVI_GROUP, HEAD_DIM).contiguous(), kz.reshape(P, T // KIVI_GROUP, HEAD_DIM).contiguous()
        vs_, vz_ = vs.reshape(P, T, 4).contiguous(), vz.reshape(P, T, 4).contiguous()
        for t in (ks_, kz_, vs_, vz_):
            if t.dtype != torch.bfloat16:
                raise TypeError("KiviCache: scales / zero points must be bfloat16")
        st = load().vh_kivi_bake(ptr(kc8), ptr(ks_), ptr(kz_), ptr(vc8), ptr(vs_), ptr(vz_), P, T, self.group_cap, 0,
                                 ptr(self.main), _stream(kc8))
        check(st, "vh_kivi_bake")

    def load_residual(self, k_res: torch.Tensor, v_res: torch.Tensor) -> None:
        n = k_res.shape[2]
        if n >= RES_CAP:
            raise ValueError(f"KiviCache: the residual window holds at most {RES_CAP - 1} tokens before a step")
        self.n_res = n
        self._sync_state()
        if n == 0:
            return
        k = k_res.reshape(self.P, n, HEAD_DIM).bfloat16().contiguous()
        v = v_res.reshape(self.P, n, HEAD_DIM).bfloat16().contiguous()
        st = load().vh_kivi_bake_residual(ptr(k), ptr(v), self.P, n, ptr(self.kr), ptr(self.vr), _stream(k))
        check(st, "vh_kivi_bake_residual")

    def _sync_state(self) -> None:
        self.state.copy_(torch.tensor([self.n_main, self.n_res, 0, 0], dtype=torch.int32))

    def advance_host(self) -> None:
        """Move the host mirror past one step, as an advancing
        ``vh_kivi_attention`` moves the device state: a step that fills the
        last residual slot folds the chunk into the main cache."""
        if self.n_res + 1 == RES_CAP:
            if self.n_main + RES_CAP <= self.capacity:
                self.n_main += RES_CAP
                self.n_res = 0
        else:
            self.n_res += 1

    def device_state(self):
        """``(n_main, n_res)`` read from the device (synchronising)."""
        v = self.state.tolist()
        return int(v[0]), int(v[1])

    def residual_tokens(self, n: int):
        """The first n residual keys / values as ``[batch, nkv, n, 128]`` bf16."""
        k = self.kr[:, :n].reshape(self.batch, self.nkv, n, HEAD_DIM)
        v = self.vr[:, :n].reshape(self.batch, self.nkv, n, HEAD_DIM)
        return k, v

    def splits_cap(self) -> int:
        return -(-self.group_cap // GROUPS_PER_SPLIT)

    def part_floats(self) -> int:
        """The attention workspace in floats: per split and the residual
        window a (max, sum) per head, per split a share of the output, and
        the bf16 scores of every position."""
        def up4(v):
            return -(-v // 4) * 4
        S, T = self.splits_cap(), self.group_cap * KIVI_GROUP + RES_CAP
        return up4(self.P * (S + 1) * GQA * 2) + up4(self.P * S * GQA * HEAD_DIM) + up4(self.P * GQA * T // 2)


def kivi_attention(qkv: torch.Tensor, cache: KiviCache, rope: torch.Tensor, nq: int, flag: ErrorFlag,
                   part: Optional[torch.Tensor] = None, attn: Optional[torch.Tensor] = None,
                   attn_fq: Optional[torch.Tensor] = None, advance: bool = False) -> torch.Tensor:
    """Attention of this step's queries over the cache at the cache's own
    position (RoPE from ``rope`` [2, max_pos, 128] applied to q and the new
    key inside; the new key / value enter residual slot ``n_res``).  With
    ``advance`` the cache moves past the step's token on the device (folding
    a completed residual chunk into the main cache), and its host mirror
    with it.  Returns the fp16 fake quantization of the attention output;
    ``attn`` receives the bf16 output."""
    B = cache.batch
    dev = qkv.device
    if part is None:
        part = torch.empty(cache.part_floats(), dtype=torch.float32, device=dev)
    if attn_fq is None:
        attn_fq = torch.empty(B, nq * HEAD_DIM, dtype=torch.float16, device=dev)
    d = KiviDesc(qkv=qkv.data_ptr(), qkv_ld=qkv.stride(0), rope=rope.data_ptr(), max_pos=rope.shape[1],
                 main=cache.main.data_ptr(), group_cap=cache.group_cap, kr=cache.kr.data_ptr(),
                 vr=cache.vr.data_ptr(), state=cache.state.data_ptr(), batch=B, nkv=cache.nkv, nq=nq,
                 head_dim=HEAD_DIM, softmax_scale=HEAD_DIM ** -0.5, part=part.data_ptr(), part_floats=part.numel(),
                 attn=_vp(attn), attn_fq=attn_fq.data_ptr(), flag=flag.t.data_ptr(), advance=1 if advance else 0,
                 scale_fmt=cache.scale_fmt, code_fmt=cache.code_fmt)
    st = load().vh_kivi_attention(ctypes.byref(d), _stream(qkv))
    check(st, "vh_kivi_attention")
    if advance:
        cache.advance_host()
    return attn_fq


def rope_tables(max_pos: int, theta: float, device) -> torch.Tensor:
    """bf16 cos / sin tables ``[2, max_pos, 128]`` (``LlamaRotaryEmbedding``,
    default RoPE): layer constants, computed once in float32 on the CPU (so
    they do not depend on the device's transcendental functions) and copied
    to ``device``."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, HEAD_DIM, 2, dtype=torch.int64).float() / HEAD_DIM))
    freqs = torch.arange(max_pos).float()[:, None] * inv_freq[None, :]
    emb = torch.cat((freqs, freqs), dim=-1)
    return torch.stack((emb.cos(), emb.sin())).bfloat16().contiguous().to(device)


class DecoderLayer:
    """A Llama-architecture decoder layer with MX-int8 linears, baked for the
    GPU decode step.  ``weights``: bf16 tensors ``ln1, wq, wk, wv, wo, ln2,
    wg, wu, wd`` (nn.Linear layout ``[out, in]``)."""

    def __init__(self, weights: Dict[str, torch.Tensor], n_heads: int, n_kv_heads: int, eps: float,
                 rope_theta: float, max_batch: int, max_pos: int):
        w = weights
        dev = w["wq"].device
        self.nq, self.nkv, self.eps = n_heads, n_kv_heads, eps
        self.hidden = w["wq"].shape[1]
        self.ln1, self.ln2 = w["ln1"].contiguous(), w["ln2"].contiguous()
        self.qkv = quantize_mx8_weight(torch.cat((w["wq"], w["wk"], w["wv"])).contiguous())
        self.o = quantize_mx8_weight(w["wo"].contiguous())
        self.gate_up = quantize_mx8_weight(torch.cat((w["wg"], w["wu"])).contiguous(), paired=True)
        self.down = quantize_mx8_weight(w["wd"].contiguous())
        self.rope = rope_tables(max_pos, rope_theta, dev)
        self.flag = ErrorFlag(dev)
        H, F, B = self.hidden, self.gate_up.n_out, max_batch
        f16, bf = torch.float16, torch.bfloat16
        self.buf = {
            "fq1": torch.empty(B, H, dtype=f16, device=dev),
            "qkv": torch.empty(B, self.qkv.n_out, dtype=bf, device=dev),
            "attn": torch.empty(B, n_heads * HEAD_DIM, dtype=bf, device=dev),
            "attn_fq": torch.empty(B, n_heads * HEAD_DIM, dtype=f16, device=dev),
            "x1": torch.empty(B, H, dtype=bf, device=dev),
            "fq3": torch.empty(B, H, dtype=f16, device=dev),
            "act": torch.empty(B, F, dtype=bf, device=dev),
            "act_fq": torch.empty(B, F, dtype=f16, device=dev),
            "out": torch.empty(B, H, dtype=bf, device=dev),
        }
        self.part = None

    def stages(self, x: torch.Tensor, cache: KiviCache, advance: bool = True):
        """The step's launches as ``(name, fn)`` pairs, in order.  The step's
        position is the cache's (read on the device); with ``advance`` the
        attention also moves the cache past the step's token (folding a
        completed residual chunk into the main cache)."""
        B = x.shape[0]
        if B != cache.batch:
            raise ValueError(f"DecoderLayer: batch {B} does not match the cache's {cache.batch}")
        b = {k: v[:B] for k, v in self.buf.items()}
        if self.part is None or self.part.numel() < cache.part_floats():
            self.part = torch.empty(cache.part_floats(), dtype=torch.float32, device=x.device)
        f = self.flag
        out = [
            ("rmsnorm_1", lambda: rmsnorm_mx8(x, self.ln1, self.eps, f, fq=b["fq1"])),
            ("qkv_proj", lambda: gemv_mx8(b["fq1"], self.qkv, f, _lib.GEMV_STORE, y=b["qkv"])),
            ("attention", lambda: kivi_attention(b["qkv"], cache, self.rope, self.nq, f, part=self.part,
                                                 attn=b["attn"], attn_fq=b["attn_fq"], advance=advance)),
            ("o_proj", lambda: gemv_mx8(b["attn_fq"], self.o, f, _lib.GEMV_RESIDUAL, residual=x, y=b["x1"])),
            ("rmsnorm_2", lambda: rmsnorm_mx8(b["x1"], self.ln2, self.eps, f, fq=b["fq3"])),
            ("gate_up_proj", lambda: gemv_mx8(b["fq3"], self.gate_up, f, _lib.GEMV_SWIGLU, y=b["act"],
                                              fq_out=b["act_fq"])),
            ("down_proj", lambda: gemv_mx8(b["act_fq"], self.down, f, _lib.GEMV_RESIDUAL, residual=b["x1"],
                                           y=b["out"])),
        ]
        return out

    def safe_stages(self, x: torch.Tensor, cache: KiviCache, advance: bool, flag: ErrorFlag):
        """The step with each linear's input taken from its bf16 form as exact
        fp16 rows rebased to the row's largest block exponent
        (``gemm.quantize_mx8_f16``; the GEMV multiplies each row's sums back),
        in place of the fake-quantized fp16 operand, whose blocks must stay in
        the fp16 range: any activation magnitude, at the cost of a quantize
        launch per linear (and allocations, so not for graph capture).  The
        kernels whose fp16 operands it does not use report into ``flag``."""
        from . import gemm

        B = x.shape[0]
        b = {k: v[:B] for k, v in self.buf.items()}
        if "h1" not in self.buf:
            H = self.hidden
            self.buf["h1"] = torch.empty(self.buf["out"].shape[0], H, dtype=torch.bfloat16, device=x.device)
            self.buf["h2"] = torch.empty_like(self.buf["h1"])
        h1, h2 = self.buf["h1"][:B], self.buf["h2"][:B]
        f = self.flag

        def lin(inp, w, mode, **kw):
            x16, ex = gemm.quantize_mx8_f16(inp)
            return gemv_mx8(x16, w, flag if mode == _lib.GEMV_SWIGLU else f, mode, row_exp=ex, **kw)

        return [
            ("rmsnorm_1", lambda: rmsnorm_mx8(x, self.ln1, self.eps, flag, fq=b["fq1"], h_out=h1)),
            ("qkv_proj", lambda: lin(h1, self.qkv, _lib.GEMV_STORE, y=b["qkv"])),
            ("attention", lambda: kivi_attention(b["qkv"], cache, self.rope, self.nq, flag, part=self.part,
                                                 attn=b["attn"], attn_fq=b["attn_fq"], advance=advance)),
            ("o_proj", lambda: lin(b["attn"], self.o, _lib.GEMV_RESIDUAL, residual=x, y=b["x1"])),
            ("rmsnorm_2", lambda: rmsnorm_mx8(b["x1"], self.ln2, self.eps, flag, fq=b["fq3"], h_out=h2)),
            ("gate_up_proj", lambda: lin(h2, self.gate_up, _lib.GEMV_SWIGLU, y=b["act"], fq_out=b["act_fq"])),
            ("down_proj", lambda: lin(b["act"], self.down, _lib.GEMV_RESIDUAL, residual=b["x1"], y=b["out"])),
        ]

    def step_checked(self, x: torch.Tensor, cache: KiviCache, advance: bool = True) -> torch.Tensor:
        """``step``, then a synchronising look at the flag: when an activation
        block left the fp16 range of the GEMV operand, the cache state is put
        back and the step runs again through ``safe_stages`` (the cache bytes
        the first run wrote past the state -- the new token's residual slot, a
        folded chunk -- are written again); every other error raises, as
        ``ErrorFlag.check`` does."""
        state0, host0 = cache.state.clone(), (cache.n_main, cache.n_res)
        out = self.step(x, cache, advance)
        v = int(self.flag.t.item())
        if v & _lib.DECODE_ERR_FP16_RANGE:
            self.flag.t.fill_(v & ~_lib.DECODE_ERR_FP16_RANGE)
            cache.state.copy_(state0)
            cache.n_main, cache.n_res = host0
            side = ErrorFlag(x.device)
            self.stages(x, cache)  # sizes the attention workspace
            for _, fn in self.safe_stages(x, cache, advance, side):
                fn()
            sv = int(side.t.item()) & ~_lib.DECODE_ERR_FP16_RANGE
            if sv:
                self.flag.t.bitwise_or_(sv)
        self.flag.check()
        return out

    def step(self, x: torch.Tensor, cache: KiviCache, advance: bool = True) -> torch.Tensor:
        """One decode step of ``x [B, hidden]`` (bf16) at the cache's position;
        returns the layer output (a view of an internal buffer).  Nothing
        synchronises: read ``self.flag.check()`` to learn of data the kernels
        could not represent."""
        for _, fn in self.stages(x, cache, advance):
            fn()
        return self.buf["out"][: x.shape[0]]

    def capture(self, x: torch.Tensor, cache: KiviCache, warmup: int = 0) -> "torch.cuda.CUDAGraph":
        """A HIP graph of one whole step (the cache advance included) reading
        ``x`` and the cache state from device memory, so each ``replay()`` is
        the next decode step; call ``cache.advance_host()`` after each replay
        to keep the host mirror.  ``warmup`` eager steps run first (they
        advance the cache)."""
        for _ in range(warmup):
            self.step(x, cache)
        self.stages(x, cache)  # allocates the attention workspace outside the capture
        g = torch.cuda.CUDAGraph()
        n_main, n_res = cache.n_main, cache.n_res
        with torch.cuda.graph(g):
            for _, fn in self.stages(x, cache):
                fn()
        # capture ran the host bookkeeping once without device work
        cache.n_main, cache.n_res = n_main, n_res
        return g

    def stage_bytes(self, batch: int, cache: KiviCache) -> Dict[str, int]:
        """Algorithmic HBM bytes of each stage: weights (one code byte per
        weight, one exponent byte per 16), the KIVI cache read, activations."""
        H, B = self.hidden, batch
        w = lambda m: m.codes.numel() + m.hb.numel()
        qkv_n, F = self.qkv.n_out, self.gate_up.n_out
        G = cache.n_main // KIVI_GROUP
        kv = cache.P * (cache.n_main * HEAD_DIM // 4 * 2 + G * HEAD_DIM * 4 + cache.n_main * 4 * 4)
        kv += cache.P * (cache.n_res + 1) * HEAD_DIM * 2 * 2
        return {
            "rmsnorm_1": B * H * 4 + H * 2,
            "qkv_proj": w(self.qkv) + B * H * 2 + B * qkv_n * 2,
            "attention": kv + B * qkv_n * 2 + B * self.nq * HEAD_DIM * 4,
            "o_proj": w(self.o) + B * H * 2 * 3,
            "rmsnorm_2": B * H * 4 + H * 2,
            "gate_up_proj": w(self.gate_up) + B * H * 2 + B * F * 4,
            "down_proj": w(self.down) + B * F * 2 + B * H * 4,
        }
