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
    """The device int32 the decode kernels OR ``DECODE_ERR_*`` bits into."""

    def __init__(self, device):
        self.t = torch.zeros(1, dtype=torch.int32, device=device)

    def check(self) -> None:
        """Synchronising check: raise if a kernel flagged unrepresentable data."""
        v = int(self.t.item())
        if v:
            what = []
            if v & _lib.DECODE_ERR_FP16_RANGE:
                what.append("an activation block exceeds the fp16 range of the GEMV operand")
            if v & _lib.DECODE_ERR_WEIGHT_RANGE:
                what.append("a weight block exponent is outside [-24, 5]")
            raise RuntimeError("voyager_amd decode: " + "; ".join(what))


class MX8Weight(NamedTuple):
    codes: torch.Tensor  # uint8, baked GEMV layout
    hb: torch.Tensor     # uint8, baked fp16 exponent bytes
    n_out: int           # output columns (gate/up pairs count once when paired)
    K: int
    paired: bool


def bake_mx8(codes: torch.Tensor, scale: torch.Tensor, bias: int, paired: bool = False) -> MX8Weight:
    """Bake packed MX-int8 weights ``[N, K]`` (codes one int8 per byte, scales
    as biased exponent bytes, as ``packed.quantize_mx_packed`` returns them)."""
    N, K = codes.shape
    if codes.dtype != torch.uint8 or scale.dtype != torch.uint8:
        raise TypeError("bake_mx8: codes and scales must be uint8")
    wc = torch.empty(N * K, dtype=torch.uint8, device=codes.device)
    wh = torch.empty(N * K // MX_BLOCK, dtype=torch.uint8, device=codes.device)
    flag = ErrorFlag(codes.device)
    st = load().vh_mx8_bake(ptr(codes.contiguous()), ptr(scale.contiguous()), int(bias), N, K, 1 if paired else 0,
                            ptr(wc), ptr(wh), ptr(flag.t), _stream(codes))
    check(st, "vh_mx8_bake")
    flag.check()
    return MX8Weight(wc, wh, N // 2 if paired else N, K, paired)


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
             fq_out: Optional[torch.Tensor] = None, tiles_per_block: int = 0):
    """``linear_mx`` of fake-quantized activations and baked weights.  STORE /
    RESIDUAL return ``y`` (bf16); SWIGLU returns the fp16 fake quantization
    of ``silu(gate) * up`` (and fills ``y`` with the bf16 product if given)."""
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
                            ptr(y), ptr(fq_out), ptr(flag.t), _stream(x_fq))
    check(st, "vh_gemv_mx8")
    return fq_out if mode == _lib.GEMV_SWIGLU else y


class KiviDesc(ctypes.Structure):
    """``vh_kivi_desc``."""

    _fields_ = [
        ("qkv", ctypes.c_void_p), ("qkv_ld", ctypes.c_int64),
        ("cos", ctypes.c_void_p), ("sin", ctypes.c_void_p),
        ("main", ctypes.c_void_p),
        ("kr", ctypes.c_void_p), ("vr", ctypes.c_void_p),
        ("batch", ctypes.c_int64), ("nkv", ctypes.c_int64), ("nq", ctypes.c_int64), ("head_dim", ctypes.c_int64),
        ("n_main", ctypes.c_int64), ("n_res", ctypes.c_int64),
        ("softmax_scale", ctypes.c_float),
        ("part", ctypes.c_void_p), ("part_floats", ctypes.c_int64),
        ("attn", ctypes.c_void_p), ("attn_fq", ctypes.c_void_p), ("flag", ctypes.c_void_p),
    ]


def _vp(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


class KiviCache:
    """A KIVI KV cache for ``batch x nkv`` sequences: the quantized main part
    (``n_main`` tokens, a multiple of 32) in the attention layout and a
    ``VH_KIVI_RES_CAP``-slot full-precision residual window holding
    ``n_res`` tokens."""

    def __init__(self, batch: int, nkv: int, n_main: int, device):
        if n_main % KIVI_GROUP:
            raise ValueError("KiviCache: n_main must be a multiple of 32")
        self.batch, self.nkv, self.n_main, self.n_res = batch, nkv, n_main, 0
        P = batch * nkv
        self.P = P
        G = n_main // KIVI_GROUP
        bf = torch.bfloat16
        # one 3072-byte block per 32 tokens: key / value codes, key / value scale + zero point
        self.main = torch.zeros(P * G * 3072, dtype=torch.uint8, device=device)
        cap = _lib.KIVI_RES_CAP
        self.kr = torch.zeros(P, cap, HEAD_DIM, dtype=bf, device=device)
        self.vr = torch.zeros(P, cap, HEAD_DIM, dtype=bf, device=device)

    @classmethod
    def from_bf16(cls, k_main: torch.Tensor, v_main: torch.Tensor, k_res: torch.Tensor, v_res: torch.Tensor):
        """Quantize ``[batch, nkv, T, 128]`` keys / values with the KIVI specs
        (``quantize_affine`` on the GPU) and bake them; the residual tokens
        ``[batch, nkv, n, 128]`` fill the first n slots.  Returns the cache and
        the reference-form ``(scale, zero_point, codes)`` of keys and values."""
        B, nkv, T, D = k_main.shape
        if D != HEAD_DIM:
            raise ValueError(f"KiviCache: head_dim must be {HEAD_DIM}")
        dev = k_main.device
        c = cls(B, nkv, T, dev)
        kq = vq = None
        if T:
            qtab = formats.quantization_map("uint2", dev)
            stab = formats.quantization_map("fp16_e5m10", dev)
            kq = _quantize_affine_cuda(k_main, qtab, [-2], KIVI_GROUP, 0.0, 3.0, stab)
            vq = _quantize_affine_cuda(v_main, qtab, [-1], KIVI_GROUP, 0.0, 3.0, stab)
            c.load_main(kq, vq)
        c.load_residual(k_res, v_res)
        return c, kq, vq

    def load_main(self, kq, vq) -> None:
        """Bake reference-form ``quantize_affine`` outputs (keys grouped along
        tokens, values along channels) into the main cache."""
        ks, kz, kcode = kq
        vs, vz, vcode = vq
        P, T = self.P, self.n_main
        if T == 0:
            return
        kc8 = kcode.reshape(P, T, HEAD_DIM).to(torch.uint8).contiguous()
        vc8 = vcode.reshape(P, T, HEAD_DIM).to(torch.uint8).contiguous()
        ks_, kz_ = ks.reshape(P, T // KIVI_GROUP, HEAD_DIM).contiguous(), kz.reshape(P, T // KIVI_GROUP, HEAD_DIM).contiguous()
        vs_, vz_ = vs.reshape(P, T, 4).contiguous(), vz.reshape(P, T, 4).contiguous()
        for t in (ks_, kz_, vs_, vz_):
            if t.dtype != torch.bfloat16:
                raise TypeError("KiviCache: scales / zero points must be bfloat16")
        st = load().vh_kivi_bake(ptr(kc8), ptr(ks_), ptr(kz_), ptr(vc8), ptr(vs_), ptr(vz_), P, T, ptr(self.main),
                                 _stream(kc8))
        check(st, "vh_kivi_bake")

    def load_residual(self, k_res: torch.Tensor, v_res: torch.Tensor) -> None:
        n = k_res.shape[2]
        if n >= _lib.KIVI_RES_CAP:
            raise ValueError("KiviCache: the residual window holds at most 127 tokens before a step")
        self.n_res = n
        if n == 0:
            return
        k = k_res.reshape(self.P, n, HEAD_DIM).bfloat16().contiguous()
        v = v_res.reshape(self.P, n, HEAD_DIM).bfloat16().contiguous()
        st = load().vh_kivi_bake_residual(ptr(k), ptr(v), self.P, n, ptr(self.kr), ptr(self.vr), _stream(k))
        check(st, "vh_kivi_bake_residual")

    def residual_tokens(self, n: int):
        """The first n residual keys / values as ``[batch, nkv, n, 128]`` bf16."""
        k = self.kr[:, :n].reshape(self.batch, self.nkv, n, HEAD_DIM)
        v = self.vr[:, :n].reshape(self.batch, self.nkv, n, HEAD_DIM)
        return k, v


def part_floats(batch: int, nkv: int, n_main: int) -> int:
    splits = -(-(n_main // KIVI_GROUP) // 16)
    return max(1, batch * nkv * splits * GQA * (HEAD_DIM + 2))


def kivi_attention(qkv: torch.Tensor, cache: KiviCache, cos: torch.Tensor, sin: torch.Tensor, nq: int,
                   flag: ErrorFlag, part: Optional[torch.Tensor] = None, attn: Optional[torch.Tensor] = None,
                   attn_fq: Optional[torch.Tensor] = None, advance: bool = True) -> torch.Tensor:
    """Attention of this step's queries over the cache (RoPE applied to q and
    the new key inside; the new key / value enter residual slot ``n_res``).
    Returns the fp16 fake quantization of the attention output; ``attn``
    receives the bf16 output."""
    B = cache.batch
    dev = qkv.device
    if part is None:
        part = torch.empty(part_floats(B, cache.nkv, cache.n_main), dtype=torch.float32, device=dev)
    if attn_fq is None:
        attn_fq = torch.empty(B, nq * HEAD_DIM, dtype=torch.float16, device=dev)
    d = KiviDesc(qkv=qkv.data_ptr(), qkv_ld=qkv.stride(0), cos=cos.data_ptr(), sin=sin.data_ptr(),
                 main=_vp(cache.main) if cache.n_main else None, kr=_vp(cache.kr), vr=_vp(cache.vr), batch=B, nkv=cache.nkv, nq=nq, head_dim=HEAD_DIM,
                 n_main=cache.n_main, n_res=cache.n_res, softmax_scale=HEAD_DIM ** -0.5, part=part.data_ptr(),
                 part_floats=part.numel(), attn=_vp(attn), attn_fq=attn_fq.data_ptr(), flag=flag.t.data_ptr())
    st = load().vh_kivi_attention(ctypes.byref(d), _stream(qkv))
    check(st, "vh_kivi_attention")
    if advance:
        cache.n_res += 1
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

    def stages(self, x: torch.Tensor, cache: KiviCache, pos: int):
        """The step's launches as ``(name, fn)`` pairs, in order (the cache's
        residual count is not advanced by them)."""
        B = x.shape[0]
        b = {k: v[:B] for k, v in self.buf.items()}
        if self.part is None or self.part.numel() < part_floats(B, cache.nkv, cache.n_main):
            self.part = torch.empty(part_floats(B, cache.nkv, cache.n_main), dtype=torch.float32, device=x.device)
        f = self.flag
        return [
            ("rmsnorm_1", lambda: rmsnorm_mx8(x, self.ln1, self.eps, f, fq=b["fq1"])),
            ("qkv_proj", lambda: gemv_mx8(b["fq1"], self.qkv, f, _lib.GEMV_STORE, y=b["qkv"])),
            ("attention", lambda: kivi_attention(b["qkv"], cache, self.rope[0, pos], self.rope[1, pos], self.nq, f,
                                                 part=self.part, attn=b["attn"], attn_fq=b["attn_fq"],
                                                 advance=False)),
            ("o_proj", lambda: gemv_mx8(b["attn_fq"], self.o, f, _lib.GEMV_RESIDUAL, residual=x, y=b["x1"])),
            ("rmsnorm_2", lambda: rmsnorm_mx8(b["x1"], self.ln2, self.eps, f, fq=b["fq3"])),
            ("gate_up_proj", lambda: gemv_mx8(b["fq3"], self.gate_up, f, _lib.GEMV_SWIGLU, y=b["act"],
                                              fq_out=b["act_fq"])),
            ("down_proj", lambda: gemv_mx8(b["act_fq"], self.down, f, _lib.GEMV_RESIDUAL, residual=b["x1"],
                                           y=b["out"])),
        ]

    def step(self, x: torch.Tensor, cache: KiviCache, pos: int, advance: bool = True) -> torch.Tensor:
        """One decode step of ``x [B, hidden]`` (bf16) at position ``pos``;
        returns the layer output (a view of an internal buffer).  With
        ``advance`` the cache's residual count moves past this step's token."""
        for _, fn in self.stages(x, cache, pos):
            fn()
        if advance:
            cache.n_res += 1
        return self.buf["out"][: x.shape[0]]

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
