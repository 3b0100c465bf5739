"""voyager_amd.lower on graphs laid out as convert_pt2e leaves them: each
site kind is checked with check_sites, lowered, and its output compared with
the same converted graph run by the oracle on the CPU (1e-2
max-abs-normalized, the GEMM tolerance)."""

import copy

import pytest
import torch

import voyager_amd.library  # noqa: F401  (defines quantized_ops)
from convert_helpers import OracleRun
from helpers import max_rel_err
from oracle import ops as O
from oracle import tables as T

pytestmark = pytest.mark.gpu

Q = torch.ops.quantized_ops
TOL = 1e-2


def _rand(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).bfloat16()


class _Fp8Linear(torch.nn.Module):
    def __init__(self, sx, wq, s, qmap, ident, dequant=True):
        super().__init__()
        self.register_buffer("sx", sx)
        self.register_buffer("wq", wq)
        self.register_buffer("s", s)
        self.register_buffer("qmap", qmap)
        self.register_buffer("ident", ident)
        self.dequant = dequant

    def forward(self, x):
        xq = Q.quantize.default(x, self.sx, None, None, None, self.qmap)
        y = torch.ops.aten.linear.default(xq, self.wq)
        if self.dequant:
            y = Q.dequantize.default(y, self.s, None, None, None, self.ident)
        return y


class _MxLinear(torch.nn.Module):
    def __init__(self, qmap, w, ws, bs, qmax, pot, bias=None, scale_qmap=None, output_code=None, entries=None):
        super().__init__()
        self.register_buffer("qmap", qmap)
        self.register_buffer("w", w)
        self.register_buffer("ws", ws)
        self.register_buffer("bias", bias)
        self.register_buffer("sq", scale_qmap)
        self.register_buffer("oc", output_code)
        self.register_buffer("entries", entries)
        self.bs, self.qmax, self.pot = bs, qmax, pot

    def forward(self, x):
        q = Q.quantize_mx.default(x, self.qmap, [-1], self.bs, self.qmax, self.pot, self.sq, self.oc)
        return Q.linear_mx.default(q[1], self.w, self.bias, input_scale=q[0], weight_scale=self.ws,
                                   block_size=self.bs, input_code=self.entries, weight_code=self.entries)


def _kinds(gm):
    return [n.target for n in gm.graph.nodes if n.op == "call_function"]


def _check_and_lower(gm, x, kind):
    """Checks the site, lowers it, and compares both the converted graph on
    the GPU and the lowered one with the same graph run by the oracle on the
    CPU."""
    from voyager_amd import lower

    exp = OracleRun(copy.deepcopy(gm).cpu()).run(x.cpu())
    ref = gm(x)
    assert max_rel_err(ref, exp) < TOL
    results, out = lower.check_sites(gm, (x,))
    assert torch.equal(out, ref)
    (res,) = results.values()
    assert res["kind"] == kind and res["error"] < TOL, res
    report = lower.lower(gm)
    assert kind in report.values(), report
    targets = _kinds(gm)
    assert torch.ops.aten.linear.default not in targets and Q.linear_mx.default not in targets
    got = gm(x)
    assert got.shape == ref.shape and got.dtype == ref.dtype
    assert max_rel_err(got, exp) < TOL
    assert max_rel_err(got, ref) < TOL
    return report


@pytest.mark.parametrize("dequant", [True, False])
def test_lower_fp8_linear(dequant):
    tab = T.quantization_map("fp8_e4m3")
    x, w = _rand((3, 40, 256), 1), _rand((128, 256), 2, 0.02)
    sx = O.per_tensor_scale(x, 448.0)
    sw = O.per_tensor_scale(w, 448.0) if dequant else torch.tensor(1.0, dtype=torch.bfloat16)
    wq = O.quantize(w, sw, qmap=tab)
    m = _Fp8Linear(sx, wq, sx * sw, tab, T.quantization_map(None), dequant)
    gm = torch.fx.symbolic_trace(m).cuda()
    report = _check_and_lower(gm, x.cuda(), "fp8")
    assert Q.quantize.default not in _kinds(gm) and not hasattr(gm, "wq")
    assert list(report.values()) == ["fp8"]


def test_lower_posit8_linear():
    tab = T.quantization_map("posit8_1")
    one = torch.tensor(1.0, dtype=torch.bfloat16)
    x, w = _rand((64, 512), 3, 2.0), _rand((256, 512), 4, 0.02)
    wq = O.quantize(w, one, qmap=tab)
    gm = torch.fx.symbolic_trace(_Fp8Linear(one, wq, one, tab, tab, dequant=False)).cuda()
    _check_and_lower(gm, x.cuda(), "posit8")


@pytest.mark.parametrize("with_bias", [False, True])
def test_lower_mxint8_linear(with_bias):
    tab = T.quantization_map("int8")
    x, w = _rand((2, 24, 512), 5), _rand((192, 512), 6, 0.02)
    sw, cw = O.quantize_mx(w, tab, [-1], 16, 127.0, True)
    bias = _rand((192,), 7) if with_bias else None
    gm = torch.fx.symbolic_trace(_MxLinear(tab, cw, sw, 16, 127.0, True, bias)).cuda()
    _check_and_lower(gm, x.cuda(), "mxint8")


@pytest.mark.parametrize("M", [1, 32])
def test_lower_mxnf4_linear(M):
    """M = 1 runs the GEMV on nibble-packed weights, M = 32 the prefill GEMM
    on the same baked bytes."""
    vt = T.quantization_map("lut4_to_int6")
    index, entries, mid = T.codebook_index_table(vt)
    stab = T.quantization_map("fp8_e5m3")
    x, w = _rand((M, 1024), 8), _rand((256, 1024), 9, 0.02)
    sw, cw = O.quantize_mx(w, index, [-1], 64, 31.0, False, stab)
    m = _MxLinear(index, cw, sw, 64, 31.0, False, scale_qmap=stab, output_code=mid, entries=entries)
    gm = torch.fx.symbolic_trace(m).cuda()
    _check_and_lower(gm, x.cuda(), "mxnf4")


def test_lower_reports_unmatched_sites():
    """A linear with a bias, and a per-channel FP8 dequantize, stay as they
    are, with the reason."""
    from voyager_amd import lower

    tab = T.quantization_map("fp8_e4m3")
    x, w = _rand((16, 64), 10), _rand((32, 64), 11, 0.02)
    sx = O.per_tensor_scale(x, 448.0)
    wq = O.quantize(w, O.per_tensor_scale(w, 448.0), qmap=tab)

    class M(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.register_buffer("sx", sx)
            self.register_buffer("wq", wq)
            self.register_buffer("b", _rand((32,), 12))
            self.register_buffer("qmap", tab)

        def forward(self, x):
            xq = Q.quantize.default(x, self.sx, None, None, None, self.qmap)
            return torch.ops.aten.linear.default(xq, self.wq, self.b)

    gm = torch.fx.symbolic_trace(M()).cuda()
    ref = gm(x.cuda())
    report = lower.lower(gm)
    assert list(report.values()) == ["bias is not lowered"]
    assert torch.equal(gm(x.cuda()), ref)


def test_lowered_graph_replays_under_hip_graph_capture():
    """A lowered graph with all four site kinds, captured in a HIP graph
    after one eager run: every replay (with eager work and synchronisation
    between them) equals the eager result bit for bit."""
    from voyager_amd import lower

    f8, p8, i8 = T.quantization_map("fp8_e4m3"), T.quantization_map("posit8_1"), T.quantization_map("int8")
    vt = T.quantization_map("lut4_to_int6")
    index, entries, mid = T.codebook_index_table(vt)
    stab = T.quantization_map("fp8_e5m3")
    one = torch.tensor(1.0, dtype=torch.bfloat16)
    x = _rand((8, 256), 20)
    w1, w2, w3, w4 = (_rand((256, 256), 21 + i, 0.02) for i in range(4))
    sx = O.per_tensor_scale(x, 448.0)
    sw1 = O.per_tensor_scale(w1, 448.0)
    wq1 = O.quantize(w1, sw1, qmap=f8)
    wq2 = O.quantize(w2, one, qmap=p8)
    s3, c3 = O.quantize_mx(w3, i8, [-1], 16, 127.0, True)
    s4, c4 = O.quantize_mx(w4, index, [-1], 64, 31.0, False, stab)

    class M(torch.nn.Module):
        def __init__(self):
            super().__init__()
            for name, t in dict(sx=sx, s=sx * sw1, one=one, wq1=wq1, wq2=wq2, c3=c3, s3=s3, c4=c4, s4=s4, f8=f8,
                                p8=p8, i8=i8, ident=T.quantization_map(None), index=index, entries=entries, mid=mid,
                                stab=stab).items():
                self.register_buffer(name, t)

        def forward(self, x):
            a = Q.dequantize.default(
                torch.ops.aten.linear.default(Q.quantize.default(x, self.sx, None, None, None, self.f8), self.wq1),
                self.s, None, None, None, self.ident)
            b = torch.ops.aten.linear.default(Q.quantize.default(a, self.one, None, None, None, self.p8), self.wq2)
            q = Q.quantize_mx.default(b, self.i8, [-1], 16, 127.0, True)
            c = Q.linear_mx.default(q[1], self.c3, input_scale=q[0], weight_scale=self.s3, block_size=16)
            r = Q.quantize_mx.default(c, self.index, [-1], 64, 31.0, False, self.stab, self.mid)
            return Q.linear_mx.default(r[1], self.c4, input_scale=r[0], weight_scale=self.s4, block_size=64,
                                       input_code=self.entries, weight_code=self.entries)

    gm = torch.fx.symbolic_trace(M()).cuda()
    xd = x.cuda()
    ref = gm(xd)
    report = lower.lower(gm)
    assert sorted(report.values()) == ["fp8", "mxint8", "mxnf4", "posit8"], report
    eager = gm(xd)
    assert max_rel_err(eager, ref) < 0.05
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        gm(xd)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = gm(xd)
    for _ in range(3):
        torch.randn(1 << 16, device="cuda").sum()  # eager work between replays
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
