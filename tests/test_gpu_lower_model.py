"""A whole converted model through ``voyager_amd.lower``: a two-layer
Llama-style stack exported to an aten graph, its fourteen linears converted
as ``convert_pt2e`` lays them out (FP8 per-tensor, MX-int8, or both), then
run on the GPU as converted and as lowered, each against the same graph run
by the oracle on the CPU (``backend/gpu/__init__.py:102-408`` is the
reference's lowering of a converted model)."""

import pytest
import torch

import voyager_amd.library  # noqa: F401  (defines quantized_ops)
from convert_helpers import OracleRun, TinyLlama, convert, export
from helpers import max_rel_err

pytestmark = pytest.mark.gpu

TOL = 1e-2
MLP = ("wg", "wu", "wd")


def _mode(mix):
    if mix == "mixed":
        return lambda name: "mxint8" if name.split("_")[0] in MLP else "fp8"
    return lambda name: mix


@pytest.mark.parametrize("mix", ["fp8", "mxint8", "mixed"])
def test_converted_model_lowered_against_oracle(mix):
    from voyager_amd import lower

    print(f"converted TinyLlama, {mix}", flush=True)
    x = torch.randn(2, 16, 256, generator=torch.Generator().manual_seed(5)).bfloat16()
    gm = export(TinyLlama(seed=1), x)
    done = convert(gm, x, _mode(mix))
    assert len(done) == 14
    exp = OracleRun(gm).run(x)
    gm = gm.cuda()
    xd = x.cuda()
    # The converted graph on the GPU is the oracle's, bit for bit, and every
    # site's packed kernel on that graph's own activation is within 1e-2 of
    # the site (the reference's own lowering check, per site on identical
    # inputs: backend/gpu/__init__.py:288-408).
    results, ref = lower.check_sites(gm, (xd,))
    assert torch.equal(ref.cpu(), exp)
    assert sorted(r["kind"] for r in results.values()) == sorted(done.values())
    assert all(r["error"] < TOL for r in results.values()), results
    report = lower.lower(gm)
    kinds = sorted(v for v in report.values() if v in ("fp8", "mxint8"))
    assert kinds == sorted(done.values()), report
    # what is left unlowered is the attention's float32 matmuls
    assert all(v in ("fp8", "mxint8") or "matmul" in k or "matmul" in v for k, v in report.items()), report
    got = gm(xd)
    err = max_rel_err(got, exp)
    print(f"{mix}: lowered end to end {err:.2e} against the oracle; sites "
          f"{max(r['error'] for r in results.values()):.2e} at most", flush=True)
    if mix == "mxint8":
        # the MX-int8 GEMM decodes both operands exactly and its float32
        # sums of these products come out as the reference's
        assert torch.equal(got.cpu(), exp)
    else:
        # Each FP8 GEMM is within 1e-2 on its own (above); end to end, the
        # next layer's E4M3 quantize turns a one-ulp bf16 difference of an
        # activation into a whole E4M3 step (1/8 relative) of that element,
        # so over two layers the output moves 1.4e-2 (mixed) to 2.2e-2 (all
        # FP8) from the oracle's.
        assert err < 3e-2


def test_lowered_model_replays_under_hip_graph_capture():
    """The lowered model captured after one eager run: three replays with
    eager work between them each equal the eager result."""
    from voyager_amd import lower

    x = torch.randn(2, 16, 256, generator=torch.Generator().manual_seed(6)).bfloat16()
    gm = export(TinyLlama(seed=2), x)
    convert(gm, x, _mode("mixed"))
    gm = gm.cuda()
    lower.lower(gm)
    xd = x.cuda()
    eager = gm(xd)
    static_in = xd.clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        gm(static_in)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = gm(static_in)
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        gm(xd)  # eager work between replays
        torch.cuda.synchronize()
