"""voyager_amd.lower without a GPU: sites of a graph whose constants are on
the CPU are reported with the reason, as the reference's find_sites reports
a device it cannot run (backend/gpu/__init__.py:102-131)."""

import torch

import voyager_amd.library  # noqa: F401  (defines quantized_ops)
from voyager_amd import lower
from oracle import tables as T

Q = torch.ops.quantized_ops


class _Site(torch.nn.Module):
    def __init__(self):
        super().__init__()
        g = torch.Generator().manual_seed(0)
        self.register_buffer("sx", torch.tensor(0.01, dtype=torch.bfloat16))
        self.register_buffer("wq", (torch.randn(32, 64, generator=g) * 0.02).bfloat16())
        self.register_buffer("qmap", T.quantization_map("fp8_e4m3"))

    def forward(self, x):
        xq = Q.quantize.default(x, self.sx, None, None, None, self.qmap)
        return torch.ops.aten.linear.default(xq, self.wq)


def test_cpu_graph_sites_are_reported_not_lowered():
    gm = torch.fx.symbolic_trace(_Site())
    before = [n.target for n in gm.graph.nodes]
    sites, skipped = lower.find_sites(gm)
    assert sites == [] and list(skipped.values()) == ["cpu is not a GPU"]
    assert list(lower.lower(gm).values()) == ["cpu is not a GPU"]
    assert [n.target for n in gm.graph.nodes] == before


def test_unsupported_device_reasons():
    cpu = torch.device("cpu")
    assert lower.fp8_unsupported(cpu) == "cpu is not a GPU"
    assert lower.nvfp4_unsupported(cpu) == "cpu is not a GPU"


def test_bias_operand_keeps_bf16_and_float32():
    """The GEMM epilogues widen a bf16 bias exactly, so the host passes bf16
    and float32 biases through as they are (no conversion launch) and
    converts any other dtype to float32."""
    from voyager_amd import gemm

    assert gemm._bias_operand(None) is None
    for dt in (torch.bfloat16, torch.float32):
        b = torch.randn(12).to(dt)
        assert gemm._bias_operand(b) is b
    strided = torch.randn(12, 2).bfloat16()[:, 0]
    out = gemm._bias_operand(strided)
    assert out.dtype == torch.bfloat16 and out.is_contiguous() and torch.equal(out, strided)
    for dt in (torch.float16, torch.float64):
        b = torch.randn(12).to(dt)
        out = gemm._bias_operand(b)
        assert out.dtype == torch.float32 and torch.equal(out, b.float())


def test_lower_imports_alone_and_names_what_it_needs():
    """``import voyager_amd.lower`` works in a fresh interpreter where no
    quantized_ops namespace is defined; matching a graph then says which
    import defines it, and works once ``voyager_amd.library`` is loaded."""
    import os
    import subprocess
    import sys

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    code = """
import torch
from voyager_amd import lower

class M(torch.nn.Module):
    def forward(self, x):
        return torch.ops.aten.linear.default(x, x)

gm = torch.fx.symbolic_trace(M())
try:
    lower.find_sites(gm)
except RuntimeError as e:
    assert "import voyager_amd.library" in str(e), e
else:
    raise AssertionError("no error without the namespace")
import voyager_amd.library  # noqa: F401
sites, skipped = lower.find_sites(gm)
assert sites == [] and list(skipped.values()) == ["cpu is not a GPU"], skipped
print("ok")
"""
    env = dict(os.environ, PYTHONPATH=os.pathsep.join([root, os.path.join(root, "voyager-compiler-2_amd")]))
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, env=env, timeout=300)
    assert r.returncode == 0 and r.stdout.strip().endswith("ok"), r.stderr[-2000:]
