"""A converted model for the lowering tests (test infrastructure).

``TinyLlama`` is a small Llama-style decoder stack (RMSNorm, grouped-query
attention, SwiGLU MLP) exported with ``torch.export`` to an aten graph, the
form ``prepare_pt2e`` / ``convert_pt2e`` work on.  ``convert`` then lays out
its linears the way ``convert_pt2e`` does for the two formats the GPU lowers
packed (``quantization/quantize_pt2e.py:538-600``):

* ``fp8``: ``quantize(x, s_x, qmap=fp8_e4m3)`` -> ``aten.linear`` with the
  weight already on the E4M3 grid -> ``dequantize(y, s_x * s_w)``, scales the
  amax observer's ``bf16(amax / 448)`` (``quantize_pt2e.py:609-613``);
* ``mxint8``: ``quantize_mx(x, int8, [-1], 16, 127, True)`` ->
  ``linear_mx(codes, w_codes, bias, input_scale=..., weight_scale=...,
  block_size=16)`` with the weight's codes and scales baked.

``OracleRun`` executes any such graph on the CPU with every
``quantized_ops`` node calling the oracle function of the same name, so a
GPU run of the same graph, lowered or not, has an independent reference.
"""

import operator

import torch
import torch.nn.functional as F

from oracle import ops as O
from oracle import tables as T

Q = torch.ops.quantized_ops


class TinyLlama(torch.nn.Module):
    def __init__(self, hidden=256, heads=4, kv_heads=2, intermediate=512, layers=2, seq=16, seed=0):
        super().__init__()
        g = torch.Generator().manual_seed(seed)
        self.h, self.nh, self.nkv, self.hd, self.L = hidden, heads, kv_heads, hidden // heads, layers

        def w(n, k):
            return (torch.randn(n, k, generator=g) / k**0.5).bfloat16()

        for i in range(layers):
            self.register_buffer(f"ln1_{i}", (1 + 0.1 * torch.randn(hidden, generator=g)).bfloat16())
            self.register_buffer(f"ln2_{i}", (1 + 0.1 * torch.randn(hidden, generator=g)).bfloat16())
            self.register_buffer(f"wq_{i}", w(hidden, hidden))
            self.register_buffer(f"wk_{i}", w(kv_heads * self.hd, hidden))
            self.register_buffer(f"wv_{i}", w(kv_heads * self.hd, hidden))
            self.register_buffer(f"wo_{i}", w(hidden, hidden))
            self.register_buffer(f"wg_{i}", w(intermediate, hidden))
            self.register_buffer(f"wu_{i}", w(intermediate, hidden))
            self.register_buffer(f"wd_{i}", w(hidden, intermediate))
        mask = torch.full((seq, seq), float("-inf")).triu(1)
        self.register_buffer("mask", mask)

    @staticmethod
    def _rms(x, w):
        xf = x.float()
        return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-5)).to(x.dtype) * w

    def forward(self, x):
        B, S, H = x.shape
        for i in range(self.L):
            p = lambda n: getattr(self, f"{n}_{i}")  # noqa: E731
            h = self._rms(x, p("ln1"))
            q = F.linear(h, p("wq")).view(B, S, self.nh, self.hd).transpose(1, 2)
            k = F.linear(h, p("wk")).view(B, S, self.nkv, self.hd).transpose(1, 2)
            v = F.linear(h, p("wv")).view(B, S, self.nkv, self.hd).transpose(1, 2)
            k = k.repeat_interleave(self.nh // self.nkv, dim=1)
            v = v.repeat_interleave(self.nh // self.nkv, dim=1)
            # attention in float32 (no bfloat16 batched products)
            s = torch.matmul(q.float(), k.float().transpose(-1, -2).contiguous()) * self.hd**-0.5
            a = torch.matmul(torch.softmax(s + self.mask, dim=-1), v.float().contiguous())
            a = a.to(torch.bfloat16).transpose(1, 2).reshape(B, S, H)
            x = x + F.linear(a, p("wo"))
            h = self._rms(x, p("ln2"))
            x = x + F.linear(F.silu(F.linear(h, p("wg"))) * F.linear(h, p("wu")), p("wd"))
        return x


def export(model, x):
    """The aten graph of ``model`` (``torch.export``), as a GraphModule,
    without export's tensor-metadata assertions (they pin the device the
    graph was traced on)."""
    gm = torch.export.export(model, (x,)).module()
    for n in list(gm.graph.nodes):
        if n.op == "call_function" and n.target is torch.ops.aten._assert_tensor_metadata.default:
            gm.graph.erase_node(n)
    gm.recompile()
    return gm


class _Record(torch.fx.Interpreter):
    """Runs a graph, keeping each linear's input (calibration)."""

    def __init__(self, gm):
        super().__init__(gm)
        self.inputs = {}

    def run_node(self, n):
        out = super().run_node(n)
        if n.op == "call_function" and n.target is torch.ops.aten.linear.default:
            self.inputs[n.name] = self.env[n.args[0]]
        return out


def _amax_scale(t):
    a = torch.amax(torch.abs(t))
    return (a / 448.0).to(torch.bfloat16) if a > 0 else torch.ones((), dtype=torch.bfloat16)


def _const(gm, name, value):
    gm.register_buffer(name, value)
    return name


def convert(gm, x, mode_of):
    """Converts every ``aten.linear`` of ``gm`` (calibrated on ``x``): the
    format of the linear whose weight is the buffer ``name`` is
    ``mode_of(name)``, ``"fp8"``, ``"mxint8"`` or None (left in bf16).
    Returns {linear node name: mode}."""
    rec = _Record(gm)
    rec.run(x)
    fp8, ident, i8 = T.quantization_map("fp8_e4m3"), T.quantization_map(None), T.quantization_map("int8")
    graph = gm.graph
    done = {}
    qmap_fp8 = _const(gm, "cv_fp8", fp8)
    qmap_id = _const(gm, "cv_ident", ident)
    qmap_i8 = _const(gm, "cv_int8", i8)
    for n in list(graph.nodes):
        if n.op != "call_function" or n.target is not torch.ops.aten.linear.default:
            continue
        xn, wn = n.args[0], n.args[1]
        wname = wn.target if wn.op == "get_attr" else None
        mode = mode_of(wname) if wname else None
        if mode is None:
            continue
        w = getattr(gm, wname)
        tag = n.name
        with graph.inserting_before(n):
            if mode == "fp8":
                sx, sw = _amax_scale(rec.inputs[tag]), _amax_scale(w)
                wq = O.quantize(w, sw, qmap=fp8)
                sxn = graph.get_attr(_const(gm, f"cv_{tag}_sx", sx))
                qn = graph.call_function(Q.quantize.default, (xn, sxn, None, None, None, graph.get_attr(qmap_fp8)))
                wqn = graph.get_attr(_const(gm, f"cv_{tag}_wq", wq))
                lin = graph.call_function(torch.ops.aten.linear.default, (qn, wqn))
                sn = graph.get_attr(_const(gm, f"cv_{tag}_s", sx * sw))
                out = graph.call_function(Q.dequantize.default, (lin, sn, None, None, None, graph.get_attr(qmap_id)))
            elif mode == "mxint8":
                sw, cw = O.quantize_mx(w, i8, [-1], 16, 127.0, True)
                qn = graph.call_function(Q.quantize_mx.default, (xn, graph.get_attr(qmap_i8), [-1], 16, 127.0, True))
                codes = graph.call_function(operator.getitem, (qn, 1))
                scale = graph.call_function(operator.getitem, (qn, 0))
                out = graph.call_function(
                    Q.linear_mx.default,
                    (codes, graph.get_attr(_const(gm, f"cv_{tag}_wc", cw))),
                    {"input_scale": scale, "weight_scale": graph.get_attr(_const(gm, f"cv_{tag}_ws", sw)),
                     "block_size": 16})
            else:
                raise ValueError(mode)
        n.replace_all_uses_with(out)
        graph.erase_node(n)
        done[tag] = mode
    graph.eliminate_dead_code()
    graph.lint()
    gm.recompile()
    return done


class OracleRun(torch.fx.Interpreter):
    """A graph on the CPU with each ``quantized_ops`` node run by the oracle."""

    def call_function(self, target, args, kwargs):
        if isinstance(target, torch._ops.OpOverload) and target.namespace == "quantized_ops":
            return getattr(O, target._schema.name.split("::")[1])(*args, **kwargs)
        return super().call_function(target, args, kwargs)
