"""Run a converted Voyager graph's quantized GEMMs on the packed MI355X path.

The reference's GPU backend (``backend/gpu/__init__.py:102-285``) takes the
graph ``convert_pt2e`` produces and swaps each FP8 linear for a real FP8 GEMM
on FP8 codes (``find_sites`` / ``lower`` / ``check_sites``), leaving every
other node as written.  This module does the same for the formats the HIP
library runs packed:

* ``fp8``    -- ``quantize(x, s_x, qmap=fp8_e4m3)`` -> ``aten.linear`` with
  constant E4M3-grid weights -> ``dequantize(., s)`` with one scale (or no
  dequantize: a direct cast, unit scale).  One cast to E4M3 bytes
  (``vh_quantize``) and the FP8 GEMM with the round-scale epilogue.
* ``posit8`` -- ``quantize(x, s_x, qmap=posit8)`` -> ``aten.linear`` with
  posit-grid weights, no dequantize (``quantize_pt2e.py:557-561``): the
  quantize as written (posit values in bf16) and the bf16 GEMM on the
  graph's own weight.  At the shapes a posit8 site has (compute-bound), a
  decode of packed posit bytes per call costs more than it saves.
* ``mxint8`` -- ``quantize_mx(x, int8, [-1], bs, 127, pot)`` ->
  ``linear_mx``: int8 codes plus scale bytes and the MX-int8 GEMM.
* ``mxnf4``  -- ``quantize_mx(x, lut4_to_int6 index, [-1], 64, 31,
  scale_qmap=fp8_e5m3)`` -> ``linear_mx`` with codebook entries: at most 16
  activation rows run the weight-streaming GEMV on nibble-packed weights,
  more the prefill GEMM on the same baked bytes.

Each site's weights are packed once at ``lower`` time and their reference-form
copies dropped where no other node reads them.  NVFP4 needs CUDA (as the
reference reports on ROCm).
"""

import functools
import operator
from dataclasses import dataclass, field
from types import SimpleNamespace
from typing import Callable, Dict, List, Optional, Tuple

import torch
from torch.fx import GraphModule, Interpreter, Node

from . import formats, gemm, packed
from ._lib import FMT_HW_E4M3, FMT_INT, FMT_MINIFLOAT, FMT_POSIT

__all__ = ["check_sites", "find_sites", "fp8_unsupported", "lower", "nvfp4_unsupported"]

LINEAR = torch.ops.aten.linear.default
MATMUL = torch.ops.aten.matmul.default


@functools.lru_cache(maxsize=None)
def _q():
    """The ``quantized_ops`` overloads a converted graph calls, looked up on
    first use: the namespace is defined by ``voyager_amd.library`` or by the
    reference (``ops/quantized.py:97``), whichever the caller loaded, and
    importing this module needs neither."""
    try:
        q = torch.ops.quantized_ops
        t = SimpleNamespace(quantize=q.quantize.default, dequantize=q.dequantize.default,
                            quantize_mx=q.quantize_mx.default, linear_mx=q.linear_mx.default,
                            matmul_mx=q.matmul_mx.default)
    except (AttributeError, RuntimeError) as e:
        raise RuntimeError("voyager_amd.lower needs the quantized_ops namespace: import voyager_amd.library "
                           "(or load the reference's voyager_compiler.ops) first") from e
    t.gemm_targets = (LINEAR, MATMUL, t.linear_mx, t.matmul_mx)
    return t

# K in multiples of 16 for the FP8 and posit8 GEMMs (16-byte operand rows).
GEMM_ALIGNMENT = 16


def fp8_unsupported(device: torch.device) -> Optional[str]:
    """Why ``device`` has no FP8 GEMM on Voyager's fp8_e4m3 grid, or None
    (``backend/gpu/__init__.py:59-72``)."""
    if device.type != "cuda":
        return f"{device} is not a GPU"
    arch = torch.cuda.get_device_properties(device).gcnArchName
    if "gfx950" not in arch:
        return f"{arch} is not gfx950 (the library is built for MI355X only)"
    return None


def nvfp4_unsupported(device: torch.device) -> Optional[str]:
    """Why ``device`` has no NVFP4 GEMM (``backend/gpu/__init__.py:75-87``)."""
    if device.type != "cuda":
        return f"{device} is not a GPU"
    return "NVFP4 GEMMs need CUDA"


@dataclass
class Site:
    """One quantized GEMM of a converted graph the packed path runs.

    Attributes:
        kind: ``"fp8"``, ``"posit8"``, ``"mxint8"`` or ``"mxnf4"``.
        gemm: The ``aten.linear`` or ``linear_mx``.
        output: The node holding the site's result: the ``dequantize`` after
            an FP8 linear, else ``gemm``.
        quantize: The activation's ``quantize`` / ``quantize_mx`` (other
            sites may share it).
        weight: The weight codes (``get_attr``), ``[N, K]``.
        weight_scale: ``linear_mx``'s weight scales (``get_attr``), or None.
        out_scale: The FP8 ``dequantize`` scale (``get_attr``), or None.
        bias: ``linear_mx``'s bias (``get_attr``), or None.
        consts: Node arguments of the site that stay (tables, codebooks).
    """

    kind: str
    gemm: Node
    output: Node
    quantize: Node
    weight: Node
    weight_scale: Optional[Node] = None
    out_scale: Optional[Node] = None
    bias: Optional[Node] = None
    consts: Dict[str, Node] = field(default_factory=dict)


def _arg(node: Node, index: int, name: str, default=None):
    """Argument ``index`` / keyword ``name`` of ``node``."""
    if len(node.args) > index:
        return node.args[index]
    return node.kwargs.get(name, default)


def _attr(model: GraphModule, node) -> Optional[torch.Tensor]:
    """The tensor a ``get_attr`` node reads, or None."""
    if not isinstance(node, Node) or node.op != "get_attr":
        return None
    obj = model
    for part in node.target.split("."):
        obj = getattr(obj, part)
    return obj


def _classify(model: GraphModule, node) -> Optional[formats.Classified]:
    t = _attr(model, node)
    if t is None or t.dim() != 1 or t.numel() != formats.QMAP_SIZE or t.device.type != "cuda":
        return None
    try:
        return formats.classify(t)
    except Exception:  # a table no closed form reproduces: not a packed format
        return None


def _plain_quantize(node: Node) -> Optional[str]:
    """Why ``node`` is not ``quantize(x, scale, qmap=...)`` against one
    scale, or None."""
    if node.op != "call_function" or node.target is not _q().quantize:
        return "input is not quantized"
    for i, name in ((2, "zero_point"), (3, "axes"), (4, "block_size"), (6, "output_code"), (7, "seed")):
        if _arg(node, i, name) is not None:
            return "input quantize is not a plain scale"
    return None


def _match_linear(model: GraphModule, linear: Node) -> "Site | str":
    x, weight = linear.args[0], linear.args[1]
    if not isinstance(x, Node):
        return "input is not quantized"
    why = _plain_quantize(x)
    if why:
        return why
    if _arg(linear, 2, "bias") is not None:
        return "bias is not lowered"
    scale = _attr(model, x.args[1])
    if scale is None or scale.numel() != 1 or scale.dtype is not torch.bfloat16:
        return "input scale is not a per-tensor bfloat16 constant"
    c = _classify(model, _arg(x, 5, "qmap"))
    if c is None:
        return "input format has no packed form"
    w = _attr(model, weight)
    if w is None:
        return "weight is not a constant"
    if w.dim() != 2 or w.dtype is not torch.bfloat16 or w.shape[1] % GEMM_ALIGNMENT:
        return f"weight {tuple(w.shape)} is not bfloat16 [N, K] with K a multiple of {GEMM_ALIGNMENT}"
    x_val = x.args[0].meta.get("val") if isinstance(x.args[0], Node) else None
    if x_val is not None and x_val.dtype is not torch.bfloat16:
        return "input is not bfloat16"
    users = list(linear.users)
    if c.fmt.kind == FMT_MINIFLOAT and c.fmt.flags & FMT_HW_E4M3:
        output, out_scale = linear, None
        if any(u.target is _q().dequantize for u in users):
            if len(users) != 1:
                return "output dequantize is not its only user"
            output = users[0]
            for i, name in ((2, "zero_point"), (3, "axes"), (4, "block_size"), (6, "output_qmap")):
                if _arg(output, i, name) is not None:
                    return "output dequantize is not a plain scale"
            s = _attr(model, output.args[1])
            if s is None or s.numel() != 1:
                return "output scale is not a per-tensor constant"
            if s.dtype not in (torch.bfloat16, torch.float32):
                # the GEMM epilogue reads its scale as bf16 or float32
                return f"output scale is {s.dtype}, not bfloat16 or float32"
            out_scale = output.args[1]
        return Site("fp8", linear, output, x, weight, out_scale=out_scale,
                    consts={"scale": x.args[1], "qmap": _arg(x, 5, "qmap")})
    if c.fmt.kind == FMT_POSIT and c.fmt.p0 == 8:
        if any(u.target is _q().dequantize for u in users):
            return "a posit8 linear with a dequantize is not lowered"
        return Site("posit8", linear, linear, x, weight, consts={"scale": x.args[1], "qmap": _arg(x, 5, "qmap")})
    return "input format has no packed GEMM"


def _match_linear_mx(model: GraphModule, linear: Node) -> "Site | str":
    codes, weight = linear.args[0], linear.args[1]
    if not (isinstance(codes, Node) and codes.target is operator.getitem and codes.args[1] == 1):
        return "input is not quantized"
    quantize = codes.args[0]
    if quantize.target is not _q().quantize_mx:
        return "input is not quantized"
    scale = linear.kwargs.get("input_scale")
    if not (isinstance(scale, Node) and scale.target is operator.getitem and scale.args == (quantize, 0)):
        return "input scale is not its quantize_mx's"
    for name in ("alpha", "A_data", "A_indices", "A_indptr"):
        if linear.kwargs.get(name) is not None:
            return f"{name} is not lowered"
    if linear.kwargs.get("layout", gemm.LINEAR_LAYOUT) != gemm.LINEAR_LAYOUT or linear.kwargs.get("out_dtype"):
        return "layout or out_dtype is not the default"
    if _arg(quantize, 8, "seed") is not None or _arg(quantize, 9, "global_scale") is not None:
        return "input quantize_mx has a seed or a global scale"
    axes, bs, qmax = _arg(quantize, 2, "axes"), _arg(quantize, 3, "block_size"), _arg(quantize, 4, "quant_max")
    pot = _arg(quantize, 5, "force_scale_power_of_two", False)
    if list(axes) != [-1] or linear.kwargs.get("block_size") != bs:
        return "input is not in blocks along K"
    w, ws = _attr(model, weight), _attr(model, linear.kwargs.get("weight_scale"))
    if w is None or ws is None:
        return "weight is not a constant"
    if w.dim() != 2 or w.dtype is not torch.bfloat16 or ws.shape != (w.shape[0], w.shape[1] // bs):
        return "weight is not bfloat16 [N, K] with [N, K / block_size] scales"
    bias = _arg(linear, 2, "bias")
    if bias is not None and _attr(model, bias) is None:
        return "bias is not a constant"
    c = _classify(model, _arg(quantize, 1, "qmap"))
    if c is None:
        return "input format has no packed form"
    consts = {"qmap": _arg(quantize, 1, "qmap")}
    if c.fmt.kind == FMT_INT and (c.fmt.p0, c.fmt.p1) == (-128, 127) and pot and qmax == 127.0:
        if _arg(quantize, 6, "scale_qmap") is not None or linear.kwargs.get("input_code") is not None:
            return "an MX-int8 input with a scale map or codebook is not lowered"
        if bs < 16 or bs & (bs - 1) or w.shape[1] % 64:
            return "MX-int8 needs power-of-two blocks >= 16 and K a multiple of 64"
        return Site("mxint8", linear, linear, quantize, weight, weight_scale=linear.kwargs["weight_scale"], bias=bias,
                    consts=consts)
    sq = _classify(model, _arg(quantize, 6, "scale_qmap"))
    entries = _attr(model, linear.kwargs.get("weight_code"))
    if (c.index_table and sq is not None and bs == 64 and qmax == 31.0 and not pot and entries is not None
            and entries.numel() == 16 and linear.kwargs.get("input_code") is not None):
        if bias is not None:
            return "an MX-NF4 linear with a bias is not lowered"
        if w.shape[0] % 16 or w.shape[1] > 16384:
            return "MX-NF4 needs N a multiple of 16 and K <= 16384"
        consts.update(scale_qmap=_arg(quantize, 6, "scale_qmap"), output_code=_arg(quantize, 7, "output_code"),
                      input_code=linear.kwargs["input_code"], weight_code=linear.kwargs["weight_code"])
        return Site("mxnf4", linear, linear, quantize, weight, weight_scale=linear.kwargs["weight_scale"],
                    consts=consts)
    return "input format has no packed GEMM"


def match_site(model: GraphModule, node: Node) -> "Site | str":
    """The site ``node`` (a GEMM) heads, or why it is not one."""
    if node.target is LINEAR:
        return _match_linear(model, node)
    if node.target is _q().linear_mx:
        return _match_linear_mx(model, node)
    return f"{node.target} is not lowered"


def find_sites(model: GraphModule) -> Tuple[List[Site], Dict[str, str]]:
    """The sites of a converted graph its GPU runs packed
    (``backend/gpu/__init__.py:102-131``).

    Returns:
        ``(sites, skipped)``: the sites in graph order, and per other GEMM
        node, by name, why it is not one or why the GPU cannot run it.
    """
    sites, skipped = [], {}
    buffers = list(model.buffers())
    device = buffers[0].device if buffers else torch.device("cpu")
    reason = fp8_unsupported(device)
    for node in model.graph.nodes:
        if node.op != "call_function" or node.target not in _q().gemm_targets:
            continue
        if reason is not None:
            skipped[node.name] = reason
            continue
        site = match_site(model, node)
        if isinstance(site, str):
            skipped[node.name] = site
        else:
            sites.append(site)
    return sites, skipped


# ------------------------------------------------------------------ kernels
# The functions a lowered graph calls (``call_function`` targets).

def _rows(x: torch.Tensor) -> torch.Tensor:
    return x.reshape(-1, x.shape[-1]).contiguous()


def lowered_fp8_linear(x, x_scale, qmap, w_bytes, out_scale):
    """quantize(x, x_scale, qmap=e4m3) -> linear -> dequantize(., out_scale)
    on E4M3 bytes."""
    xq = packed.quantize_packed(_rows(x), x_scale, qmap)
    y = gemm.linear_fp8(xq, w_bytes, out_scale)
    return y.reshape(*x.shape[:-1], w_bytes.shape[0])


def lowered_posit8_linear(x, x_scale, qmap, w):
    """quantize(x, x_scale, qmap=posit8) -> linear: the quantize's posit
    values in bf16 and the bf16 GEMM against the posit-grid weight."""
    xq = torch.ops.quantized_ops.quantize(_rows(x), x_scale, qmap=qmap)
    y = gemm.gemm_bf16(xq, w, torch.bfloat16)
    return y.reshape(*x.shape[:-1], w.shape[0])


def lowered_mxint8_linear(x, qmap, w_codes, w_scale, w_bias, block_size: int, bias=None):
    """quantize_mx(x, int8, [-1], bs, 127, pot) -> linear_mx on int8 codes
    and scale bytes."""
    px = packed.quantize_mx_packed(_rows(x), qmap, [-1], block_size, 127.0, True)
    y = gemm.linear_mxint8(px.codes, px.scale, w_codes, w_scale, block_size, px.bias, w_bias, bias=bias)
    return y.reshape(*x.shape[:-1], w_codes.shape[0])


def lowered_mxnf4_linear(x, index, scale_qmap, w_packed, w_scale_bytes, levels: Tuple[int, ...], N: int):
    """quantize_mx(x, lut4_to_int6, [-1], 64, 31, fp8_e5m3) -> linear_mx on
    the weight baked once for the GEMV: the GEMV for up to 16 rows, the
    prefill GEMM on the same baked bytes for more (both decode each operand
    to the reference's bf16(level * scale)).  ``levels`` are the codebook's
    16 int8 levels, read from ``weight_code`` once when the graph is lowered,
    so no call copies device memory to the host (a lowered graph can be
    captured in a HIP graph)."""
    xr = _rows(x)
    K = xr.shape[1]
    sc = formats.classify(scale_qmap)
    wt = gemm.NF4Weight(w_packed, w_scale_bytes, sc, bytes(levels), N, K)
    y = gemm.linear_nf4(xr, wt, index, scale_qmap)
    return y.reshape(*x.shape[:-1], N)


# ------------------------------------------------------------------ baking

def _bake_fp8(w: torch.Tensor) -> torch.Tensor:
    b = w.to(torch.float8_e4m3fn)
    if not torch.equal(b.to(w.dtype), w):
        raise ValueError("weight values off the fp8_e4m3 grid")
    return b.view(torch.uint8).contiguous()


def _bake_mxint8(w: torch.Tensor, ws: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor, int]:
    codes = w.float()
    if not torch.equal(codes, codes.round()) or codes.min() < -128 or codes.max() > 127:
        raise ValueError("MX-int8 weight codes are not integers in [-128, 127]")
    s = ws.float()
    e = torch.log2(s)
    if not (torch.equal(e, e.round()) and bool((s > 0).all())):
        raise ValueError("MX-int8 weight scales are not powers of two")
    bias = packed.pot_bias(127.0)
    sb = e.round().to(torch.int32) + bias
    if sb.min() < 0 or sb.max() > 254:
        raise ValueError("MX-int8 weight scale exponents out of the byte range")
    return codes.to(torch.int8).view(torch.uint8).contiguous(), sb.to(torch.uint8).contiguous(), bias


def _bake_mxnf4(w: torch.Tensor, ws: torch.Tensor, scale_qmap: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    idx = w.float()
    if not torch.equal(idx, idx.round()) or idx.min() < 0 or idx.max() > 15:
        raise ValueError("MX-NF4 weight codes are not indices in [0, 15]")
    N, K = w.shape
    codes = idx.to(torch.uint8).contiguous()
    out = torch.empty(N * K // 2, dtype=torch.uint8, device=w.device)
    import ctypes

    from ._lib import check, load, stream_of

    st = load().vh_pack_nf4(ctypes.c_void_p(codes.data_ptr()), N, K, ctypes.c_void_p(out.data_ptr()),
                            ctypes.c_void_p(stream_of(w)))
    check(st, "vh_pack_nf4")
    one = torch.ones((), dtype=torch.bfloat16, device=w.device)
    sbytes = packed.quantize_packed(ws.contiguous(), one, scale_qmap)
    if not torch.equal(packed.unpack_codes(sbytes, scale_qmap), ws):
        raise ValueError("MX-NF4 weight scales off the scale map's grid")
    return out, gemm.nf4_tile_scales(sbytes.reshape(N, K // 64))


# ------------------------------------------------------------------ rewrite

def _const(model: GraphModule, graph, name: str, value: torch.Tensor) -> Node:
    base, i = name, 0
    while hasattr(model, name):
        i += 1
        name = f"{base}_{i}"
    model.register_buffer(name, value)
    return graph.get_attr(name)


def _insert(model: GraphModule, site: Site) -> Node:
    graph = model.graph
    w = _attr(model, site.weight)
    x = site.quantize.args[0]
    k = site.consts
    name = site.gemm.name
    with graph.inserting_before(site.output):
        if site.kind == "fp8":
            wb = _const(model, graph, f"{name}_fp8_weight", _bake_fp8(w))
            if site.out_scale is None:
                one = torch.ones((), dtype=torch.bfloat16, device=w.device)
                s = _const(model, graph, f"{name}_fp8_scale", one)
            else:
                s = site.out_scale
            return graph.call_function(lowered_fp8_linear, (x, k["scale"], k["qmap"], wb, s))
        if site.kind == "posit8":
            return graph.call_function(lowered_posit8_linear, (x, k["scale"], k["qmap"], site.weight))
        ws = _attr(model, site.weight_scale)
        if site.kind == "mxint8":
            codes, sbytes, bias_w = _bake_mxint8(w, ws)
            wc = _const(model, graph, f"{name}_mxint8_weight", codes)
            sc = _const(model, graph, f"{name}_mxint8_scale", sbytes)
            bs = _arg(site.quantize, 3, "block_size")
            return graph.call_function(lowered_mxint8_linear, (x, k["qmap"], wc, sc, bias_w, bs, site.bias))
        wp, sb = _bake_mxnf4(w, ws, _attr(model, k["scale_qmap"]))
        wpn = _const(model, graph, f"{name}_nf4_weight", wp)
        sbn = _const(model, graph, f"{name}_nf4_scale", sb)
        levels = tuple(gemm._levels_of(_attr(model, k["weight_code"])))
        return graph.call_function(lowered_mxnf4_linear,
                                   (x, k["qmap"], k["scale_qmap"], wpn, sbn, levels, int(w.shape[0])))


def _erase_unused(model: GraphModule, nodes: List[Node]) -> None:
    """Erase each of ``nodes`` left with no users and no side effect, then
    likewise their inputs, and the attribute behind each constant no other
    node reads (``backend/gpu/__init__.py:139-154``)."""
    graph = model.graph
    pending, erased = list(nodes), set()
    while pending:
        node = pending.pop()
        if node in erased or node.users or node.op in ("placeholder", "output") or node.is_impure():
            continue
        pending.extend(node.all_input_nodes)
        graph.erase_node(node)
        erased.add(node)
        if node.op == "get_attr" and not any(n.op == "get_attr" and n.target == node.target for n in graph.nodes):
            owner, _, attr = node.target.rpartition(".")
            delattr(model.get_submodule(owner) if owner else model, attr)


def lower(model: GraphModule) -> Dict[str, str]:
    """Swap each site of a converted graph for its packed kernel, in place
    (``backend/gpu/__init__.py:245-285``).

    Returns:
        Per GEMM node, by name: the site kind it now runs as, or why it was
        left as it is.
    """
    sites, report = find_sites(model)
    if not sites:
        return report
    graph = model.graph
    unused: List[Node] = []
    for site in sites:
        new = _insert(model, site)
        report[site.gemm.name] = site.kind
        site.output.replace_all_uses_with(new)
        replaced = dict.fromkeys((site.output, site.gemm))
        for node in replaced:
            unused.extend(n for n in node.all_input_nodes if n not in replaced)
            graph.erase_node(node)
    _erase_unused(model, unused)
    graph.lint()
    model.recompile()
    return report


class _SiteCheck(Interpreter):
    """Runs a converted graph and, beside each site, its packed kernel on the
    activation the site reads (``backend/gpu/__init__.py:288-381``)."""

    def __init__(self, model: GraphModule, sites: List[Site]):
        # values stay in the environment: a site reads its activation after
        # the graph's last use of it
        super().__init__(model, garbage_collect_values=False)
        self.sites = {site.output: site for site in sites}
        self.results = {}

    def run_node(self, node: Node):
        result = super().run_node(node)
        site = self.sites.get(node)
        if site is not None:
            real = self._packed(site)
            ref = result.float()
            err = (real.float() - ref).abs().max() / ref.abs().max().clamp_min(1e-30)
            self.results[site.gemm.name] = {"kind": site.kind, "error": float(err)}
        return result

    def _packed(self, site: Site) -> torch.Tensor:
        m, env, k = self.module, self.env, site.consts
        x = env[site.quantize.args[0]]
        w = _attr(m, site.weight)
        if site.kind == "fp8":
            s = env[site.out_scale] if site.out_scale is not None else torch.ones((), dtype=torch.bfloat16,
                                                                                 device=x.device)
            return lowered_fp8_linear(x, env[k["scale"]], env[k["qmap"]], _bake_fp8(w), s)
        if site.kind == "posit8":
            qmap = env[k["qmap"]]
            return lowered_posit8_linear(x, env[k["scale"]], qmap, w)
        ws = _attr(m, site.weight_scale)
        if site.kind == "mxint8":
            codes, sbytes, bias_w = _bake_mxint8(w, ws)
            bias = env[site.bias] if site.bias is not None else None
            return lowered_mxint8_linear(x, env[k["qmap"]], codes, sbytes, bias_w,
                                         _arg(site.quantize, 3, "block_size"), bias)
        wp, sb = _bake_mxnf4(w, ws, env[k["scale_qmap"]])
        return lowered_mxnf4_linear(x, env[k["qmap"]], env[k["scale_qmap"]], wp, sb,
                                    tuple(gemm._levels_of(env[k["weight_code"]])), int(w.shape[0]))


def check_sites(model: GraphModule, args, kwargs=None):
    """Run a converted graph (before ``lower``) and each site's packed kernel
    on the activation its quantize reads (``backend/gpu/__init__.py:384-408``).

    Returns:
        ``(results, output)``: per site, by GEMM name, its kind and the
        largest output difference over the largest output magnitude
        (``error``); and the graph's output.
    """
    sites, _ = find_sites(model)
    checker = _SiteCheck(model, sites)
    flat = list(args) + list((kwargs or {}).values())
    output = checker.run(*flat)
    return checker.results, output
