"""Benchmark of the quantized-operator hot path on one MI355X.

Workload: FP8 E4M3 per-tensor symmetric
quantization + GEMM at Llama-3.1-8B prefill projection shapes, M = 2048 tokens
and (K, N) in {(4096, 4096), (4096, 1024), (4096, 14336), (14336, 4096)}.
One step runs, for every shape, what a lowered graph runs
(quantization/quantize_pt2e.py:538-600): quantize the bf16 activations with
their calibrated scale to E4M3 bytes, then the FP8 GEMM whose epilogue applies
the dequantize by the bf16 scale product.  Weights are quantized once before
timing (the reference bakes them at convert).  Inputs are synthetic (seeded
N(0,1) activations, N(0,0.02) weights) and resident in HBM.

Prints ONE JSON line.  `value` = GEMM TFLOP/s over the whole step (the four
GEMMs' 2*M*N*K, divided by the step time, which includes the quantize
kernels).  `roofline` is for the dominant kernel (the fp8 GEMM), timed with
HIP events on the launch stream around each GEMM of 20 more steps right after
the timed region (in the step's own thermal and cache state); beside it,
`rotated` (the GEMMs alone, operands rotated over more than 512 MB) and
`warm` (the same operands replayed, Infinity-Cache resident).  `quantize`
is reported the same ways plus `ceiling`, the quantize's access pattern
without its arithmetic.  `cpu_baseline` times the CPU oracle (the
reference's op sequence in eager PyTorch) on a bounded sample.  `configs`
carries configs 1, 3, 4 and 5
as `--config N` measures them (value, roofline, CPU baseline on a shorter
sample); `--headline-only` leaves them out.

Options: --gpus N (1 only), --steps K, --warmup W, --no-cpu (skip the CPU
baseline), --copy-calibration BYTES (run only a plain device copy, for
rocprofv3 counter calibration), --profile-steps K (config 2's setup, then
only W warm-up and K timed step replays: a kernel trace of the timed steps
themselves), --profile-shapes R (run only, shape by shape
in SHAPES order, R quantize launches then R GEMM launches, eagerly: dispatch
order names the shape in a rocprofv3 counter run; with --config 3, R
linear_nf4 calls at M = 1 then M = 16 per shape), --calibrate (run only
the reference points: plain device copies and the vendor GEMMs at the
config-2 shapes), --outliers (the outlier (CSR) path: the filter's
bandwidth and the config-1 linear with its outlier stream).
"""

import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "voyager-compiler-2_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import torch  # noqa: E402

M = 2048
SHAPES = [(4096, 4096), (4096, 1024), (4096, 14336), (14336, 4096)]
HBM_PEAK_GBS = 8000.0
FP8_PEAK_TFLOPS = 5000.0
METRIC = "quantized GEMM TFLOPS + quantize GB/s, % of MI355X roofline, 1 GPU"
PROFILE_TRAFFIC = os.path.join(ROOT, "profiles", "fp8_gemm_cfg2_traffic.json")


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def make_inputs(device):
    """Seeded synthetic inputs generated on the CPU, then copied (so the CPU
    baseline sees the same values)."""
    data = []
    for i, (K, N) in enumerate(SHAPES):
        g = torch.Generator().manual_seed(100 + i)
        x = torch.randn(M, K, generator=g).bfloat16()
        w = (torch.randn(N, K, generator=g) * 0.02).bfloat16()
        data.append((x, w))
    return data


def amax_scale(t: torch.Tensor) -> torch.Tensor:
    """bf16(amax / 448) as the amax observer computes a calibrated scale."""
    a = torch.amax(torch.abs(t))
    return (a / 448.0).to(t.dtype) if a > 0 else torch.ones((), dtype=t.dtype, device=t.device)


def capture(fn):
    """A HIP graph of ``fn``'s launches (run once eagerly first, on a side
    stream, so tables are classified and allocations exist before capture)."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


def stream_2to1(x, out):
    """vh_stream_2to1 of a bf16 tensor's bytes into ``out`` (half of them)."""
    from voyager_amd import _lib

    st = _lib.load().vh_stream_2to1(ctypes.c_void_p(x.data_ptr()), x.numel() // 8, ctypes.c_void_p(out.data_ptr()),
                                    ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    _lib.check(st, "vh_stream_2to1")


def time_graph(g, reps, warm_s=0.5):
    """Average ms of one replay, from HIP events on the current stream, after
    replaying for ``warm_s`` seconds: the clock settles under a sustained
    load, and a short window would time its transient instead."""
    t_end = time.perf_counter() + warm_s
    g.replay()
    torch.cuda.synchronize()
    while time.perf_counter() < t_end:
        g.replay()
        torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(reps):
        g.replay()
    t1.record()
    torch.cuda.synchronize()
    return t0.elapsed_time(t1) / reps


MALL_BYTES = 256 << 20


def gpu_bench(args):
    import voyager_amd.library  # noqa: F401  (defines quantized_ops)
    from voyager_amd import formats, gemm, packed
    from voyager_amd.ops import _elementwise

    dev = torch.device("cuda:0")
    tab = formats.quantization_map("fp8_e4m3", dev)
    fmt = formats.classify(tab).fmt
    cpu_data = make_inputs(dev)
    layers = []
    for x, w in cpu_data:
        xd, wd = x.to(dev), w.to(dev)
        sx, sw = amax_scale(xd), amax_scale(wd)
        s = (sx * sw).contiguous()
        wq = packed.quantize_packed(wd, sw, tab)  # baked once, as convert does
        y = torch.empty(M, wd.shape[0], dtype=torch.bfloat16, device=dev)
        layers.append(dict(x=xd, sx=sx, s=s, wq=wq, y=y, K=xd.shape[1], N=wd.shape[0]))
        del wd
    torch.cuda.synchronize()

    def quantize(x, sx):
        # quantize(x, sx, qmap=fp8_e4m3) with one-byte codes
        return _elementwise("quantize", x, sx, None, None, torch.bfloat16, fmt, None, torch.uint8)

    def step():
        for L in layers:
            L["xq"] = quantize(L["x"], L["sx"])
            gemm.linear_fp8(L["xq"], L["wq"], L["s"], out=L["y"])

    g_step = capture(step)
    if args.profile_steps:
        # only the timed region's replays, for a kernel trace of the steps themselves
        for _ in range(args.warmup):
            g_step.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.profile_steps):
            g_step.replay()
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) * 1e3 / args.profile_steps
        return {"profile_steps": args.profile_steps, "warmup": args.warmup, "ms_per_step": round(ms, 4)}, None

    # Per-kernel average launch durations (HIP events around graph replays of
    # back-to-back launches), measured first: they also bring the GPU to the
    # clock it holds under sustained load before the steps are timed.
    # Quantize inputs rotate over more than the 256 MB Infinity Cache so HBM,
    # not the cache, serves them.
    R = 10
    g_ms, q_ms, c_ms = [], [], []
    for L in layers:
        gg = capture(lambda L=L: [gemm.linear_fp8(L["xq"], L["wq"], L["s"], out=L["y"]) for _ in range(R)])
        g_ms.append(time_graph(gg, 5) / R)
        nbuf = max(2, -(-2 * MALL_BYTES // (M * L["K"] * 2)))
        xs = [L["x"].clone() for _ in range(nbuf)]
        outs = {}
        gq = capture(lambda xs=xs: [outs.__setitem__(i, quantize(xb, L["sx"])) for i, xb in enumerate(xs)])
        q_ms.append(time_graph(gq, 5) / nbuf)
        # the same inputs through the quantize's access pattern with no
        # arithmetic (vh_stream_2to1): the ceiling that pattern reaches here
        oc = [torch.empty(M * L["K"], dtype=torch.uint8, device=dev) for _ in range(nbuf)]
        gs = capture(lambda xs=xs, oc=oc: [stream_2to1(xb, ob) for xb, ob in zip(xs, oc)])
        c_ms.append(time_graph(gs, 5) / nbuf)
        del xs, gq, gg, oc, gs
    torch.cuda.synchronize()

    # The same GEMMs with their operands rotated over more than twice the
    # Infinity Cache, as a step meets them: a step moves ~400 MB, so every
    # operand was last touched a whole step earlier and comes from HBM.
    gc_ms = []
    for L in layers:
        nbuf = max(2, -(-2 * MALL_BYTES // (L["xq"].numel() + L["wq"].numel())))
        ops = [(L["xq"].clone(), L["wq"].clone()) for _ in range(nbuf)]
        gg = capture(lambda ops=ops, L=L: [gemm.linear_fp8(a, b, L["s"], out=L["y"]) for a, b in ops])
        gc_ms.append(time_graph(gg, 3) / nbuf)
        del ops, gg
    torch.cuda.synchronize()

    for _ in range(args.warmup):
        g_step.replay()
    torch.cuda.synchronize()
    # Timed region: K whole steps, bracketed by synchronisation.
    t0 = time.perf_counter()
    for _ in range(args.steps):
        g_step.replay()
    torch.cuda.synchronize()
    ms_per_step = (time.perf_counter() - t0) * 1e3 / args.steps

    # In-step kernel durations, right after the timed region and in the same
    # thermal state: S more steps launched eagerly behind three graph replays
    # (so the launches queue ahead of the GPU and no kernel waits for its
    # launch), with a HIP event between consecutive kernels on the launch
    # stream.  The GEMMs meet their operands as in the timed steps (the
    # activation codes just written, the weight last read a step earlier).
    S = 20
    nk = 2 * len(layers)
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(nk + 1)] for _ in range(S)]
    for _ in range(3):
        g_step.replay()
    for e in ev:
        e[0].record()
        for i, L in enumerate(layers):
            L["xq"] = quantize(L["x"], L["sx"])
            e[2 * i + 1].record()
            gemm.linear_fp8(L["xq"], L["wq"], L["s"], out=L["y"])
            e[2 * i + 2].record()
    torch.cuda.synchronize()

    def med(v):
        v = sorted(v)
        return v[len(v) // 2]

    in_q = [med([e[2 * i].elapsed_time(e[2 * i + 1]) for e in ev]) for i in range(len(layers))]
    in_g = [med([e[2 * i + 1].elapsed_time(e[2 * i + 2]) for e in ev]) for i in range(len(layers))]

    flops = [2.0 * M * L["N"] * L["K"] for L in layers]
    qbytes = [M * L["K"] * 3.0 for L in layers]  # bf16 in + 1-byte codes out
    total_flops = sum(flops)
    value = total_flops / (ms_per_step * 1e-3) / 1e12
    gemm_tflops = total_flops / (sum(g_ms) * 1e-3) / 1e12
    cold_tflops = total_flops / (sum(gc_ms) * 1e-3) / 1e12
    step_tflops = total_flops / (sum(in_g) * 1e-3) / 1e12
    q_gbs = sum(qbytes) / (sum(q_ms) * 1e-3) / 1e9
    c_gbs = sum(qbytes) / (sum(c_ms) * 1e-3) / 1e9
    step_q_gbs = sum(qbytes) / (sum(in_q) * 1e-3) / 1e9
    per_shape = []
    for i, L in enumerate(layers):
        per_shape.append({
            "K": L["K"], "N": L["N"],
            "gemm_us": round(g_ms[i] * 1e3, 2), "gemm_tflops": round(flops[i] / (g_ms[i] * 1e-3) / 1e12, 1),
            "gemm_rotated_us": round(gc_ms[i] * 1e3, 2),
            "gemm_rotated_tflops": round(flops[i] / (gc_ms[i] * 1e-3) / 1e12, 1),
            "gemm_in_step_us": round(in_g[i] * 1e3, 2), "quantize_in_step_us": round(in_q[i] * 1e3, 2),
            "quantize_us": round(q_ms[i] * 1e3, 2), "stream_2to1_us": round(c_ms[i] * 1e3, 2),
            "quantize_gbs": round(qbytes[i] / (q_ms[i] * 1e-3) / 1e9, 1),
        })
    traffic = None
    if os.path.exists(PROFILE_TRAFFIC):
        with open(PROFILE_TRAFFIC) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")
    res = {
        "value": value, "ms_per_step": ms_per_step,
        "roofline": {"bound": "mfma", "achieved": round(step_tflops, 1), "peak": FP8_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(step_tflops / FP8_PEAK_TFLOPS, 4), "traffic": traffic,
                     "durations": f"in the step: median over {S} steps of the HIP-event time around each GEMM "
                                  "launch, right after the timed region",
                     "rotated": {"achieved": round(cold_tflops, 1), "frac": round(cold_tflops / FP8_PEAK_TFLOPS, 4),
                                 "operands": "GEMMs alone, operands rotated over > 2 x 256 MB (HBM)"},
                     "warm": {"achieved": round(gemm_tflops, 1), "frac": round(gemm_tflops / FP8_PEAK_TFLOPS, 4),
                              "operands": "GEMMs alone, the same operands replayed 10 times (Infinity-Cache warm)"}},
        "quantize": {"achieved": round(step_q_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(step_q_gbs / HBM_PEAK_GBS, 4), "durations": "in the step, as the GEMMs",
                     "rotated": {"achieved": round(q_gbs, 1), "frac": round(q_gbs / HBM_PEAK_GBS, 4),
                                 "operands": "quantizes alone, inputs rotated over > 2 x 256 MB"},
                     "ceiling": {"achieved": round(c_gbs, 1), "frac": round(c_gbs / HBM_PEAK_GBS, 4),
                                 "quantize_frac_of_ceiling": round(q_gbs / c_gbs, 4),
                                 "kernel": "vh_stream_2to1: the quantize's loads and stores (same workgroup "
                                           "shape, runs and cache hints) with no arithmetic, same rotated inputs"}},
        "per_shape": per_shape,
    }
    return res, cpu_data


# The configs' quantization specs, in the reference's spec-string grammar
# (quantization/qspec.py), parsed by the same rules the compiler uses.
CFG1_SPEC = "int8,qs=microscaling,bs=16,pot=1"
CFG3_SPEC = "lut4_to_int6,qs=microscaling,bs=64,scale=fp8_e5m3"


def bench_config1(args, cpu_budget_s=0.0):
    """Config 1: MXINT8 linear, X [256,4096] (0.1% outliers x20, seed 0), W
    [4096,4096] N(0,0.02); int8 bs=16 pot scales.  Step = quantize_mx(X) to
    packed codes + scale bytes, then the packed MX-int8 GEMM."""
    import voyager_amd.library  # noqa: F401  (defines quantized_ops)
    from voyager_amd import formats, gemm, packed

    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(0)
    x = torch.randn(256, 4096, generator=g)
    x = torch.where(torch.rand(256, 4096, generator=g) < 0.001, x * 20, x).bfloat16()
    w = (torch.randn(4096, 4096, generator=g) * 0.02).bfloat16()
    sp = formats.parse_spec(CFG1_SPEC)
    bs, qmax, pot = sp["block_size"], sp["quant_max"], sp["power_2_scale"]
    tab = formats.quantization_map(sp["dtype"], dev)
    xd, wd = x.to(dev), w.to(dev)
    pw = packed.quantize_mx_packed(wd, tab, [-1], bs, qmax, pot)
    st = {}

    def quant():
        st["px"] = packed.quantize_mx_packed(xd, tab, [-1], bs, qmax, pot)

    def mm():
        px = st["px"]
        st["y"] = gemm.linear_mxint8(px.codes, px.scale, pw.codes, pw.scale, bs, px.bias, pw.bias)

    def step():
        quant()
        mm()

    # the step as it runs: quantize_mx of X to exact fp16 rows and the fp16
    # GEMM on the weight baked once (gemm.linear_mx8_f16); the packed-code
    # kernel is timed beside it
    bw = gemm.bake_mx8_f16(pw.codes.view(torch.int8), pw.scale, pw.bias)

    def quant16():
        st["x16"] = gemm.quantize_mx8_f16(xd)

    def mm16():
        st["y"] = gemm.linear_mx8_f16(*st["x16"], bw)

    def step16():
        quant16()
        mm16()

    gq = capture(lambda: [quant16() for _ in range(20)])
    q_ms = time_graph(gq, 5) / 20
    gm = capture(lambda: [mm16() for _ in range(20)])
    g_ms = time_graph(gm, 5) / 20
    gqp = capture(lambda: [quant() for _ in range(20)])
    qp_ms = time_graph(gqp, 5) / 20
    gmp = capture(lambda: [mm() for _ in range(20)])
    gp_ms = time_graph(gmp, 5) / 20
    # eight steps per graph replay, as a model's graph would hold many: a
    # replay of a two-kernel graph carries ~4 us of launch cost of its own
    # (30.1 us per step at one step per replay, 25.8 at eight)
    per = 8
    gs = capture(lambda: [step16() for _ in range(per)])
    for _ in range(-(-args.warmup // per)):
        gs.replay()
    torch.cuda.synchronize()
    ms = time_graph(gs, -(-max(args.steps, 24) // per), warm_s=0.0) / per
    flops = 2.0 * 256 * 4096 * 4096
    qbytes = 256 * 4096 * 3 + 256 * 256  # bf16 in, int8 codes + scale bytes out
    gbytes = 256 * 4096 + 256 * 256 + 4096 * 4096 + 4096 * 256 + 256 * 4096 * 2
    # prefill: the same weight against X [2048, 4096] (the GEMM alone): the
    # packed linear (at this size both operands rebased to exact fp16 rows
    # per call, then the fp16 GEMM) and the fp16 GEMM on the weight baked once
    xp = torch.randn(2048, 4096, generator=torch.Generator().manual_seed(1)).bfloat16().to(dev)
    pxp = packed.quantize_mx_packed(xp, tab, [-1], bs, qmax, pot)
    gp = capture(lambda: [gemm.linear_mxint8(pxp.codes, pxp.scale, pw.codes, pw.scale, bs, pxp.bias, pw.bias)
                          for _ in range(10)])
    p_ms = time_graph(gp, 5) / 10
    p_flops = 2.0 * 2048 * 4096 * 4096
    p_tf = p_flops / (p_ms * 1e-3) / 1e12
    xp16 = gemm.quantize_mx8_f16(xp)
    gp16 = capture(lambda: [gemm.linear_mx8_f16(*xp16, bw) for _ in range(10)])
    p16_ms = time_graph(gp16, 5) / 10
    p_tf = max(p_tf, p_flops / (p16_ms * 1e-3) / 1e12)
    cpu = None
    if cpu_budget_s > 0:
        cpu = cpu_config1(x, w, cpu_budget_s)
    g_gbs = gbytes / (g_ms * 1e-3) / 1e9
    return {"metric": "MXINT8 linear TFLOP/s (config 1)", "value": round(flops / (ms * 1e-3) / 1e12, 2),
            "unit": "TFLOP/s", "ms_per_step": round(ms, 4),
            "roofline": {"bound": "hbm", "achieved": round(g_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(g_gbs / HBM_PEAK_GBS, 4), "traffic": None,
                         "note": "the GEMM at M = 256 (arithmetic intensity 408 FLOP/B, under the ridge): "
                                 "algorithmic bytes (int8 codes, scale bytes, bf16 out) / its duration"},
            "cpu_baseline": cpu,
            "gemm": {"us": round(g_ms * 1e3, 2), "TFLOP/s": round(flops / (g_ms * 1e-3) / 1e12, 1),
                     "GB/s": round(gbytes / (g_ms * 1e-3) / 1e9, 1),
                     "roofline_us": round(max(flops / 2.5e15, gbytes / 8e12) * 1e6, 2),
                     "note": "the weight baked once as exact fp16 rows (code * 2**(e - E_row)), an fp16 direct-to-LDS "
                             "GEMM (2.5 PF MFMA) on 64 x 64 tiles (256 workgroups of two waves, eight stages in flight, "
                             "K unsplit) whose epilogue applies 2**(E_row + E_col)"},
            "quantize_mx": {"us": round(q_ms * 1e3, 2), "GB/s": round(qbytes / (q_ms * 1e-3) / 1e9, 1),
                            "note": "quantize_mx of X written as exact fp16 rows and their exponents"},
            "packed": {"gemm_us": round(gp_ms * 1e3, 2), "quantize_us": round(qp_ms * 1e3, 2),
                       "note": "k_gemm_mxi8 on int8 codes + scale bytes (codes decoded to bf16 in staging, K split 4)"},
            "prefill_gemm": {"M": 2048, "us": round(min(p_ms, p16_ms) * 1e3, 2), "TFLOP/s": round(p_tf, 1),
                             "packed_us": round(p_ms * 1e3, 2), "f16_us": round(p16_ms * 1e3, 2),
                             "note": "packed_us: gemm.linear_mxint8 on the packed codes, which at this size rebases "
                                     "both operands to exact fp16 rows per call; f16_us: the fp16 GEMM on the "
                                     "weight baked once",
                             "mfma": "v_mfma_f32_32x32x16_f16 / _bf16 (2.5 PF dense)", "frac_of_mfma": round(p_tf / 2500.0, 4),
                             "frac_of_int8_peak": round(p_tf / 5000.0, 4)},
            "config": {"workload": "cfg1: MXINT8 bs=16 pot, X[256,4096] . W[4096,4096]^T"}}


def bench_outliers(args):
    """The outlier (CSR) path, not a headline config: (1) vh_filter_outlier
    on a [2048, 14336] prefill activation with config 1's outlier pattern
    (0.1% of entries x20), inputs rotated over > 256 MB; (2) the config-1
    linear as a converted graph with an outlier spec runs it:
    quantize_mx_outlier (threshold 5, a 1% stream) + linear_mx with the CSR
    term, against quantize_mx + linear_mx without it; the spmm_csr of the
    stream with the decoded weight alone; the oracle's step on the host."""
    import voyager_amd.library  # noqa: F401  (defines quantized_ops)
    from voyager_amd import formats, sparse

    Q = torch.ops.quantized_ops
    dev = torch.device("cuda:0")

    def outlier_input(rows, cols, seed):
        g = torch.Generator().manual_seed(seed)
        x = torch.randn(rows, cols, generator=g)
        return torch.where(torch.rand(rows, cols, generator=g) < 0.001, x * 20, x).bfloat16(), g

    # (1) the filter, HBM-bound
    R, C = 2048, 14336
    xf, _ = outlier_input(R, C, 0)
    nbuf = max(2, -(-2 * MALL_BYTES // (R * C * 2)))
    xs = [xf.to(dev) for _ in range(nbuf)]
    gf = capture(lambda: [sparse.filter_outlier(x, 5.0, 0.01) for x in xs])
    f_ms = time_graph(gf, 5) / nbuf
    cap = int(R * C * 0.01)
    nnz = int(sparse.filter_outlier(xs[0], 5.0, 0.01)[2][-1])
    fbytes = R * C * 2 * 2 + cap * 6 + (R + 1) * 4
    del gf, xs

    # (2) the config-1 linear with the outlier stream
    x, g = outlier_input(256, 4096, 0)
    w = (torch.randn(4096, 4096, generator=g) * 0.02).bfloat16()
    tab = formats.quantization_map("int8", dev)
    xd, wdev = x.to(dev), w.to(dev)
    ws, wc = Q.quantize_mx(wdev, tab, [-1], 16, 127.0, True)
    st = {}

    def with_csr():
        d, i, p, s_, c_ = Q.quantize_mx_outlier(xd, tab, [-1], 16, 127.0, True, threshold=5.0, max_pct=0.01)
        st["csr"] = (d, i, p)
        st["y"] = Q.linear_mx(c_, wc, input_scale=s_, weight_scale=ws, block_size=16, A_data=d, A_indices=i,
                              A_indptr=p)

    def without():
        s_, c_ = Q.quantize_mx(xd, tab, [-1], 16, 127.0, True)
        st["y0"] = Q.linear_mx(c_, wc, input_scale=s_, weight_scale=ws, block_size=16)

    g1 = capture(lambda: [with_csr() for _ in range(10)])
    t_csr = time_graph(g1, 5) / 10
    g0 = capture(lambda: [without() for _ in range(10)])
    t_plain = time_graph(g0, 5) / 10
    wdec = Q.dequantize_mx(wc, ws, 16)
    base = torch.zeros(256, 4096, dtype=torch.float32, device=dev)
    d, i, p = st["csr"]
    gs = capture(lambda: [sparse.spmm_into(d, i, p, wdec, "kc", torch.bfloat16, base=base) for _ in range(10)])
    t_spmm = time_graph(gs, 5) / 10
    nnz1 = int(p[-1])
    res = {"metric": "outlier (CSR) path: filter GB/s, step us", "unit": "us",
           "filter": {"shape": [R, C], "stored_outliers": nnz, "capacity": cap, "us": round(f_ms * 1e3, 2),
                      "GB/s": round(fbytes / (f_ms * 1e-3) / 1e9, 1),
                      "hbm_frac": round(fbytes / (f_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 3),
                      "bytes": fbytes, "note": "x read + inliers written + capacity slots (6 B) + row pointers"},
           "cfg1_step": {"with_csr_us": round(t_csr * 1e3, 2), "without_us": round(t_plain * 1e3, 2),
                         "stored_outliers": nnz1, "spmm_us": round(t_spmm * 1e3, 2),
                         "note": "ref-form ops as a converted graph runs them: quantize_mx_outlier + linear_mx "
                                 "(decode + bf16 GEMM to fp32 + CSR product added before the bf16 rounding)"},
           "config": {"workload": "outliers: cfg1 X[256,4096] (0.1% x20) . W[4096,4096]^T, threshold 5, "
                                  "1% stream; filter on X[2048,14336]"}}
    if not args.no_cpu:
        from oracle import ops as O  # the CPU baseline only

        tabc = tab.cpu()
        wsc, wcc = O.quantize_mx(w, tabc, [-1], 16, 127.0, True)
        times = []
        t_start = time.perf_counter()
        while time.perf_counter() - t_start < 10.0 or len(times) < 3:
            t0 = time.perf_counter()
            dd, ii, pp, sc, cc = O.quantize_mx_outlier(x, tabc, [-1], 16, 127.0, True, threshold=5.0, max_pct=0.01)
            O.linear_mx(cc, wcc, input_scale=sc, weight_scale=wsc, block_size=16, A_data=dd, A_indices=ii,
                        A_indptr=pp)
            times.append(time.perf_counter() - t0)
        times.sort()
        res["cpu_baseline"] = {"us": round(times[len(times) // 2] * 1e6, 1), "cores": torch.get_num_threads(),
                               "kind": "port", "sample": f"{len(times)} cfg1 outlier steps of the oracle, median"}
    return res


def bench_config3(args, cpu_budget_s=0.0):
    """Config 3: MXNF4 decode linear at M in {1, 16} over the four Llama-3.1-8B
    projections; weights baked once, rotated over > 256 MB."""
    import voyager_amd.library  # noqa: F401  (defines quantized_ops)
    from voyager_amd import formats, gemm

    dev = torch.device("cuda:0")
    sp = formats.parse_spec(CFG3_SPEC)
    index, entries, mid = formats.codebook_tables(sp["dtype"], dev)
    stab = formats.quantization_map(sp["scale_dtype"], dev)
    res = {}
    tot_b, tot_t = 0.0, 0.0
    for i, (K, N) in enumerate(SHAPES):
        g = torch.Generator().manual_seed(1)
        w = (torch.randn(N, K, generator=g) * 0.02).bfloat16().to(dev)
        wb = gemm.bake_nf4_weight(w, index, stab, entries)
        del w
        wbytes = N * K // 2 + N * K // 64
        nw = max(2, -(-2 * MALL_BYTES // wbytes))
        ws = [gemm.NF4Weight(wb.packed.clone(), wb.scale.clone(), wb.scale_fmt, wb.levels, N, K)
              for _ in range(nw)]
        for M in (1, 16):
            x = torch.randn(M, K, generator=torch.Generator().manual_seed(0)).bfloat16().to(dev)
            gg = capture(lambda: [gemm.linear_nf4(x, wi, index, stab) for wi in ws])
            ms = time_graph(gg, 5) / nw
            b = wbytes + M * K * 2 + M * N * 2
            res[f"M{M}_K{K}_N{N}"] = {"us": round(ms * 1e3, 2), "GB/s": round(b / (ms * 1e-3) / 1e9, 1),
                                      "roofline_us": round(b / 8e12 * 1e6, 2)}
            tot_b += b
            tot_t += ms
        del ws
    gbs = tot_b / (tot_t * 1e-3) / 1e9
    # prefill: the same format at M = 2048 (the lowered site's quantize_mx of
    # the activations, then vh_gemm_nf4 on the GEMV's baked weight bytes)
    from voyager_amd import packed
    prefill = {}
    for K, N in ((4096, 4096), (4096, 14336)):
        w = (torch.randn(N, K, generator=torch.Generator().manual_seed(1)) * 0.02).bfloat16().to(dev)
        wb = gemm.bake_nf4_weight(w, index, stab, entries)
        x = torch.randn(2048, K, generator=torch.Generator().manual_seed(0)).bfloat16().to(dev)
        px = packed.quantize_mx_packed(x, index, [-1], 64, 31.0, False, stab)
        gq = capture(lambda: [packed.quantize_mx_packed(x, index, [-1], 64, 31.0, False, stab) for _ in range(10)])
        q_ms = time_graph(gq, 5) / 10
        gg = capture(lambda: [gemm.gemm_nf4_packed(px, wb) for _ in range(10)])
        g_ms = time_graph(gg, 5) / 10
        gf = capture(lambda: [gemm.gemm_nf4_packed(px, wb, two_pass=False) for _ in range(10)])
        f_ms = time_graph(gf, 5) / 10
        gd = capture(lambda: [gemm.nf4_decode_bf16(px, wb) for _ in range(10)])
        d_ms = time_graph(gd, 5) / 10
        tf = 2 * 2048 * N * K / (g_ms * 1e-3) / 1e12
        prefill[f"M2048_K{K}_N{N}"] = {"gemm_us": round(g_ms * 1e3, 2), "TFLOP/s": round(tf, 1),
                                       "frac_of_mfma": round(tf / 2500.0, 4), "decode_us": round(d_ms * 1e3, 2),
                                       "fused_us": round(f_ms * 1e3, 2), "quantize_us": round(q_ms * 1e3, 2)}
        del w, wb, x, px, gq, gg, gf, gd
    cpu = cpu_config3(cpu_budget_s) if cpu_budget_s > 0 else None
    return {"metric": "MXNF4 decode linear GB/s (config 3)", "value": round(gbs, 1),
            "unit": "GB/s", "frac_of_hbm": round(gbs / HBM_PEAK_GBS, 4),
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                         "note": "the eight decode linears (weights rotated over > 512 MB): algorithmic bytes "
                                 "(4-bit codes, scale bytes, bf16 activations and outputs) / their durations"},
            "per_shape": res, "cpu_baseline": cpu,
            "prefill_gemm": {"shapes": prefill, "mfma": "v_mfma_f32_32x32x16_bf16 (2.5 PF dense)",
                             "note": "at M = 2048 both operands decoded once to bf16(level * scale) "
                                     "(vh_nf4_decode_bf16, decode_us) and multiplied by the bf16 GEMM, float32 "
                                     "accumulation (gemm_us, both); fused_us = vh_gemm_nf4, which decodes them "
                                     "while staging; quantize_us = the activation's quantize_mx"},
            "config": {"workload": "cfg3: lut4_to_int6 bs=64 fp8_e5m3 scales, M in {1,16}"}}


def bench_config4(args, cpu_budget_s=0.0):
    """Config 4: posit8 (es=1) quantize / dequantize of a 64M-element bf16
    tensor N(0,4), and the posit8 GEMM 2048x4096x4096."""
    import voyager_amd.library  # noqa: F401  (defines quantized_ops)
    from voyager_amd import formats, gemm, packed

    dev = torch.device("cuda:0")
    tab = formats.quantization_map("posit8_1", dev)
    one = torch.ones((), dtype=torch.bfloat16, device=dev)
    g = torch.Generator().manual_seed(0)
    n = 1 << 26
    t = (torch.randn(n, generator=g) * 2).bfloat16().to(dev)
    # Inputs rotate over more than twice the 256 MB Infinity Cache, so HBM,
    # not the cache, serves every launch (as for config 2's quantize).
    nbuf = max(2, -(-2 * MALL_BYTES // (n * 2)))
    ts = [t] + [t.clone() for _ in range(nbuf - 1)]
    cs = [packed.quantize_packed(tb, one, tab) for tb in ts]
    st = {}
    gq = capture(lambda: [st.__setitem__(i, packed.quantize_packed(tb, one, tab)) for i, tb in enumerate(ts)])
    q_ms = time_graph(gq, 5) / nbuf
    gr = capture(lambda: [st.__setitem__(i, torch.ops.quantized_ops.quantize(tb, one, qmap=tab)) for i, tb in enumerate(ts)])
    r_ms = time_graph(gr, 5) / nbuf
    gd = capture(lambda: [st.__setitem__(i, packed.unpack_codes(c, tab)) for i, c in enumerate(cs)])
    d_ms = time_graph(gd, 5) / nbuf
    del ts, cs, st, gq, gr, gd
    x = torch.randn(2048, 4096, generator=torch.Generator().manual_seed(1)).bfloat16().to(dev)
    w = (torch.randn(4096, 4096, generator=torch.Generator().manual_seed(2)) * 0.02).bfloat16().to(dev)
    cx, cw = packed.quantize_packed(x, one, tab), packed.quantize_packed(w, one, tab)
    lut = gemm.posit8_lut(tab)
    gm = capture(lambda: [gemm.linear_posit8(cx, cw, lut) for _ in range(10)])
    g_ms = time_graph(gm, 5) / 10
    # the lowered posit8 site: the activation's quantize as written (posit
    # values in bf16) and the bf16 GEMM on the posit-grid weight
    xq = torch.ops.quantized_ops.quantize(x, one, qmap=tab)
    wq = torch.ops.quantized_ops.quantize(w, one, qmap=tab)
    gl = capture(lambda: [gemm.gemm_bf16(xq, wq, torch.bfloat16) for _ in range(10)])
    l_ms = time_graph(gl, 5) / 10
    flops = 2.0 * 2048 * 4096 * 4096
    q_gbs = n * 3 / (q_ms * 1e-3) / 1e9
    cpu = cpu_config4(cpu_budget_s) if cpu_budget_s > 0 else None
    return {"metric": "posit8 quantize GB/s + posit8 GEMM TFLOP/s (config 4)",
            "value": round(q_gbs, 1), "unit": "GB/s",
            "roofline": {"bound": "hbm", "achieved": round(q_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(q_gbs / HBM_PEAK_GBS, 4), "traffic": None,
                         "note": "the packed posit8 quantize of the 64M-element tensor (bf16 in, one byte out)"},
            "cpu_baseline": cpu,
            "quantize_packed": {"us": round(q_ms * 1e3, 2), "GB/s": round(n * 3 / (q_ms * 1e-3) / 1e9, 1)},
            "quantize_ref_form": {"us": round(r_ms * 1e3, 2), "GB/s": round(n * 4 / (r_ms * 1e-3) / 1e9, 1)},
            "dequantize_packed": {"us": round(d_ms * 1e3, 2), "GB/s": round(n * 3 / (d_ms * 1e-3) / 1e9, 1)},
            "gemm": {"us": round(l_ms * 1e3, 2), "TFLOP/s": round(flops / (l_ms * 1e-3) / 1e12, 1),
                     "peak_TFLOP/s": 2500.0, "frac": round(flops / (l_ms * 1e-3) / 2.5e15, 4),
                     "note": "the lowered posit8 linear: bf16 direct-to-LDS GEMM of the activation's posit values "
                             "(its quantize, timed above as quantize_ref_form) and the posit-grid weight"},
            "gemm_packed": {"us": round(g_ms * 1e3, 2), "TFLOP/s": round(flops / (g_ms * 1e-3) / 1e12, 1),
                            "note": "both operands as posit bytes, decoded to bf16 through a 256-entry table each "
                                    "call, then the same GEMM (decode included in the time)"},
            "config": {"workload": "cfg4: posit8_1, 64M-element tensor (inputs rotated over 2x the Infinity Cache); "
                                   "GEMM M=2048 K=N=4096"}}


# Config 5's layer: Llama-3.1-8B's architecture (hidden 4096, 32 query / 8 kv
# heads of 128, MLP 14336, RMSNorm eps 1e-5, RoPE theta 5e5).
CFG5 = dict(hidden=4096, n_heads=32, n_kv_heads=8, intermediate=14336, eps=1e-5, rope_theta=5e5)


def cfg5_weights(seed):
    """A random-init layer in bf16, drawn from one generator in this order:
    ln1 = 1 + 0.1 N(0,1) (so the RMSNorm gain is exercised), wq, wk, wv, wo
    ~ N(0, 0.02), ln2, wg, wu, wd ([out, in], nn.Linear layout)."""
    g = torch.Generator().manual_seed(seed)
    H, F = CFG5["hidden"], CFG5["intermediate"]
    q, kv = CFG5["n_heads"] * 128, CFG5["n_kv_heads"] * 128

    def w(n, k):
        return (torch.randn(n, k, generator=g) * 0.02).bfloat16()

    return {
        "ln1": (1 + 0.1 * torch.randn(H, generator=g)).bfloat16(),
        "wq": w(q, H), "wk": w(kv, H), "wv": w(kv, H), "wo": w(H, q),
        "ln2": (1 + 0.1 * torch.randn(H, generator=g)).bfloat16(),
        "wg": w(F, H), "wu": w(F, H), "wd": w(H, F),
    }


def bench_config5(args, cpu_budget_s=10.0):
    """Config 5: one random-init Llama-3.1-8B-architecture decoder layer, decode
    at batch 8 over a 4096-token context.  Two such layers (weights and KIVI
    caches) run in turn, layer 0's output feeding layer 1, as consecutive
    layers of a model do, so neither fits the 256 MB Infinity Cache.

    The step is timed as it runs in a decode loop: one HIP graph of 128
    consecutive steps of both layers, each step advancing its cache on the
    device, from position 4032 (3968 tokens in the 2-bit main cache, 64 in
    the residual window) to 4159, so every step attends to 4033-4160 tokens
    (4096 on average) and each cache folds one completed 128-token chunk into
    its main cache on the way; the graph restores both states first, so it
    replays the same 128 steps.  ``us_per_step`` is one replay over 256.
    ``per_stage`` times each stage alone at position 4095 without the
    advance (a breakdown, not the step)."""
    import voyager_amd.library  # noqa: F401  (defines quantized_ops)
    from voyager_amd import decode

    dev = torch.device("cuda:0")
    B, n_main, n_res0, steps = 8, 3968, 64, 128
    cap = 4096 + decode.RES_CAP
    nkv = CFG5["n_kv_heads"]
    layers, caches, kvq, ws = [], [], [], []
    for li in range(2):
        w = cfg5_weights(li)
        g = torch.Generator().manual_seed(100 + li)
        k_main, v_main = (torch.randn(B, nkv, n_main, 128, generator=g).bfloat16() for _ in range(2))
        k_res, v_res = (torch.randn(B, nkv, 127, 128, generator=g).bfloat16() for _ in range(2))
        wd = {k: v.to(dev) for k, v in w.items()}
        layer = decode.DecoderLayer(wd, CFG5["n_heads"], nkv, CFG5["eps"], CFG5["rope_theta"], max_batch=B,
                                    max_pos=cap)
        cache, kq, vq = decode.KiviCache.from_bf16(k_main.to(dev), v_main.to(dev), k_res.to(dev), v_res.to(dev),
                                                   capacity=cap)
        layers.append(layer)
        caches.append(cache)
        kvq.append((kq, vq, k_res, v_res))
        ws.append((w, wd))
    x0 = torch.randn(B, CFG5["hidden"], generator=torch.Generator().manual_seed(7)).bfloat16().to(dev)
    xs = [x0, layers[0].buf["out"][:B]]
    sbytes = layers[0].stage_bytes(B, caches[0])  # at position 4095: 3968 main tokens, 127 residual
    total_b = sum(sbytes.values())
    torch.cuda.synchronize()

    # per-stage breakdown at position 4095, no advance
    stage_lists = [l.stages(x, c, advance=False) for l, c, x in zip(layers, caches, xs)]
    names = [n for n, _ in stage_lists[0]]
    reps = 10
    per = {}
    for i, name in enumerate(names):
        gi = capture(lambda: [st[i][1]() for _ in range(reps) for st in stage_lists])
        ms = time_graph(gi, 5) / (2 * reps)
        per[name] = {"us": round(ms * 1e3, 2), "GB/s": round(sbytes[name] / (ms * 1e-3) / 1e9, 1)}
    del gi

    # the decode loop: 128 advancing steps of both layers per replay
    state0 = torch.tensor([n_main, n_res0, 0, 0], dtype=torch.int32, device=dev)

    def window():
        for c in caches:
            c.state.copy_(state0)
        for _ in range(steps):
            for l, c, x in zip(layers, caches, xs):
                l.step(x, c, advance=True)

    gw = capture(window)
    for _ in range(max(1, args.warmup // 10)):
        gw.replay()
    torch.cuda.synchronize()
    step_ms = time_graph(gw, 3) / (2 * steps)
    for l, c in zip(layers, caches):
        l.flag.check()
        if c.device_state() != (4096, 64):
            raise RuntimeError(f"config 5: the decode loop ended at {c.device_state()}, not (4096, 64)")
    gbs = total_b / (step_ms * 1e-3) / 1e9
    dom = max(("gate_up_proj", "down_proj", "qkv_proj", "o_proj", "attention"), key=lambda n: sbytes[n])
    d_gbs = per[dom]["GB/s"]
    cpu = None
    if cpu_budget_s > 0:
        cpu = cpu_config5(ws[0], kvq[0], layers[0], n_main, cpu_budget_s)
        cpu["value"] = round(total_b / (cpu["ms_per_step"] * 1e-3) / 1e9, 3)
    return {"metric": "MX-int8 / KIVI decoder-layer decode step, HBM GB/s (config 5)",
            "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "higher_is_better": True,
            "us_per_step": round(step_ms * 1e3, 2), "roofline_us": round(total_b / 8e12 * 1e6, 2),
            "frac_of_hbm": round(gbs / HBM_PEAK_GBS, 4), "algorithmic_bytes": total_b,
            "dtype": "int8 codes / 2-bit KIVI, fp32 accumulate", "data": "synthetic (random-init layers, seeded)",
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                         "note": "the whole step (algorithmic bytes at context 4096 / step time)",
                         "dominant_kernel": {"stage": dom, "achieved": d_gbs, "frac": round(d_gbs / HBM_PEAK_GBS, 4)}},
            "per_stage": per, "stage_bytes": sbytes, "cpu_baseline": cpu,
            "timing": f"{steps} consecutive advancing steps of 2 layers per graph replay (one fold each), "
                      "positions 4032-4159",
            "config": {"workload": "cfg5: Llama-3.1-8B-arch decoder layer, decode, batch 8, ctx 4096, MXINT8 bs=16 "
                                   "linears, KIVI 2-bit K/V (group 32, fp16 scale/zero), 128-token residual"}}


def cpu_config5(w, kvq, layer, n_main, budget_s):
    """The oracle layer (eager torch, the reference's op sequence) on the
    host, at position 4095 over the same layer's weights and cache: the
    MX-int8 weight codes and the KIVI codes are the GPU's reference-form
    outputs of the same quantize ops, moved to the host."""
    from oracle import decode as D  # the CPU baseline only
    from voyager_amd import formats

    kq, vq, k_res, v_res = kvq
    tab = formats.quantization_map("int8", "cuda:0")
    mx = {}
    for k in ("wq", "wk", "wv", "wo", "wg", "wu", "wd"):
        sc, cd = torch.ops.quantized_ops.quantize_mx(w[1][k], tab, [-1], 16, 127.0, True)
        mx[k] = (cd.cpu(), sc.cpu())
    k_past = torch.cat((D.kivi_dequantize(kq[2].cpu(), kq[0].cpu(), kq[1].cpu(), -2), k_res), dim=2)
    v_past = torch.cat((D.kivi_dequantize(vq[2].cpu(), vq[0].cpu(), vq[1].cpu(), -1), v_res), dim=2)
    cfg = D.Config()
    x = torch.randn(k_past.shape[0], cfg.hidden, generator=torch.Generator().manual_seed(7)).bfloat16()
    cos, sin = D.rope_cos_sin(torch.tensor([n_main + 127]), 128, cfg.rope_theta)
    med, n, el = _time_cpu(lambda: D.decode_layer(x, w[0], k_past, v_past, cos, sin, cfg, mx=mx),
                           torch.get_num_threads(), budget_s, min_runs=3)
    return {"unit": "GB/s", "cores": torch.get_num_threads(), "kind": "port", "ms_per_step": round(med * 1e3, 1),
            "cpu_model": cpu_model(),
            "sample": f"{n} decode steps of the oracle layer at position 4095 (eager torch, the reference's op "
                      f"sequence), median, {el:.1f} s"}


def cpu_config1(x, w, budget_s):
    """The oracle's config-1 step on the host: quantize_mx of X, then
    linear_mx against the weight quantized once (as baked)."""
    from oracle import ops as O  # the CPU baseline only
    from oracle import tables as T

    tab = T.quantization_map("int8")
    ws, wc = O.quantize_mx(w, tab, [-1], 16, 127.0, True)

    def step():
        sx, cx = O.quantize_mx(x, tab, [-1], 16, 127.0, True)
        O.linear_mx(cx, wc, input_scale=sx, weight_scale=ws, block_size=16)

    med, n, el = _time_cpu(step, torch.get_num_threads(), budget_s, min_runs=3)
    flops = 2.0 * 256 * 4096 * 4096
    return {"value": round(flops / med / 1e12, 4), "unit": "TFLOP/s", "cores": torch.get_num_threads(),
            "kind": "port", "cpu_model": cpu_model(),
            "sample": f"{n} whole config-1 steps (quantize_mx + linear_mx, 256x4096x4096) of the oracle, "
                      f"median {med * 1e3:.1f} ms, {el:.1f} s"}


def cpu_config3(budget_s):
    """The oracle's config-3 linears on the host (quantize_mx of x, then
    linear_mx against the weight quantized once) for the two K = 4096, N <=
    4096 shapes at M = 1 and 16: a bounded sample of the eight (the two
    larger weights take the oracle several seconds each just to quantize)."""
    from oracle import ops as O  # the CPU baseline only
    from oracle import tables as T

    index, entries, mid = T.codebook_index_table(T.quantization_map("lut4_to_int6"))
    stab = T.quantization_map("fp8_e5m3")
    work, nbytes = [], 0
    for K, N in [(4096, 4096), (4096, 1024)]:
        w = (torch.randn(N, K, generator=torch.Generator().manual_seed(1)) * 0.02).bfloat16()
        sw, cw = O.quantize_mx(w, index, [-1], 64, 31.0, False, stab)
        for M in (1, 16):
            x = torch.randn(M, K, generator=torch.Generator().manual_seed(0)).bfloat16()
            work.append((x, cw, sw))
            nbytes += N * K // 2 + N * K // 64 + M * K * 2 + M * N * 2

    def step():
        for x, cw, sw in work:
            sx, cx = O.quantize_mx(x, index, [-1], 64, 31.0, False, stab, mid)
            O.linear_mx(cx, cw, input_scale=sx, weight_scale=sw, block_size=64, input_code=entries,
                        weight_code=entries)

    med, n, el = _time_cpu(step, torch.get_num_threads(), budget_s, min_runs=3)
    return {"value": round(nbytes / med / 1e9, 3), "unit": "GB/s", "cores": torch.get_num_threads(),
            "kind": "port", "cpu_model": cpu_model(),
            "sample": f"{n} passes over the (K, N) = (4096, 4096), (4096, 1024) linears at M = 1 and 16 "
                      f"(quantize_mx + linear_mx, the GPU's algorithmic bytes), median {med * 1e3:.1f} ms, "
                      f"{el:.1f} s"}


def cpu_config4(budget_s):
    """The oracle's posit8 quantize on the host over an 8M-element sample of
    config 4's N(0, 4) tensor (the reference form it computes: bf16 in, bf16
    out, 4 bytes an element)."""
    from oracle import ops as O  # the CPU baseline only
    from oracle import tables as T

    tab = T.quantization_map("posit8_1")
    one = torch.ones((), dtype=torch.bfloat16)
    n = 1 << 23
    t = (torch.randn(n, generator=torch.Generator().manual_seed(0)) * 2).bfloat16()
    med, runs, el = _time_cpu(lambda: O.quantize(t, one, qmap=tab), torch.get_num_threads(), budget_s,
                              min_runs=3)
    return {"value": round(n * 4 / med / 1e9, 3), "unit": "GB/s", "cores": torch.get_num_threads(),
            "kind": "port", "cpu_model": cpu_model(),
            "sample": f"{runs} quantize calls of the oracle (posit8_1, reference form) over the first 8M elements "
                      f"of the tensor, median {med * 1e3:.1f} ms, {el:.1f} s"}


def summary(res):
    """The fields of a config's measurement the headline line carries."""
    rl = res.get("roofline") or {}
    out = {"metric": res.get("metric"), "value": res.get("value"), "unit": res.get("unit"),
           "roofline": {k: rl.get(k) for k in ("bound", "achieved", "peak", "unit", "frac")},
           "cpu_baseline": res.get("cpu_baseline")}
    for k in ("us_per_step", "ms_per_step"):
        if k in res:
            out[k] = res[k]
    if "gemm" in res and "frac" in res["gemm"]:
        out["gemm"] = {k: res["gemm"].get(k) for k in ("us", "TFLOP/s", "frac")}
    if "prefill_gemm" in res:
        pg = res["prefill_gemm"]
        out["prefill_gemm"] = pg["shapes"] if "shapes" in pg else {k: pg.get(k) for k in ("us", "TFLOP/s", "frac_of_mfma")}
    out["workload"] = (res.get("config") or {}).get("workload")
    return out


def cpu_model() -> str:
    """The host CPU's model name (``/proc/cpuinfo``), as lscpu reports it."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _time_cpu(step, threads, budget_s, min_runs=5):
    """Median wall time of ``step`` on ``threads`` torch CPU threads after one
    warm-up run: at least ``min_runs`` runs, more while within ``budget_s``."""
    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        step()
        times = []
        t_start = time.perf_counter()
        while len(times) < min_runs or time.perf_counter() - t_start < budget_s:
            t0 = time.perf_counter()
            step()
            times.append(time.perf_counter() - t0)
        times.sort()
        return times[len(times) // 2], len(times), time.perf_counter() - t_start
    finally:
        torch.set_num_threads(prev)


def cpu_baseline(cpu_data, budget_s=10.0):
    """The reference's CPU op sequence (the oracle) on the host: whole
    config-2 steps (per shape: quantize X with its calibrated scale, linear,
    dequantize by the scale product; weights quantized once, as baked), on
    every host core and on one thread (the reference's own ``--debug``
    setting); median step time of each."""
    from oracle import ops as O
    from oracle import tables as T

    tab = T.quantization_map("fp8_e4m3")
    ident = T.quantization_map(None)
    prep = []
    for x, w in cpu_data:
        sx = O.per_tensor_scale(x, 448.0)
        sw = O.per_tensor_scale(w, 448.0)
        prep.append((x, sx, O.quantize(w, sw, qmap=tab), sx * sw))

    def step():
        for x, sx, wq, s in prep:
            xq = O.quantize(x, sx, qmap=tab)
            O.dequantize(O.linear(xq, wq), s, input_qmap=ident)

    flops = sum(2.0 * x.shape[0] * wq.shape[0] * wq.shape[1] for x, _, wq, _ in prep)
    cores = torch.get_num_threads()  # the job's share (OMP_NUM_THREADS), not every core of the host
    med, n, el = _time_cpu(step, cores, budget_s)
    med1, n1, el1 = _time_cpu(step, 1, budget_s)
    return {"value": round(flops / med / 1e12, 4), "unit": "TFLOP/s", "cores": cores, "kind": "port",
            "cpu_model": cpu_model(), "os_cpu_count": os.cpu_count(),
            "sample": f"{n} whole config-2 steps (4 shapes, M=2048) of the oracle's quantize + linear + "
                      f"dequantize, median {med * 1e3:.1f} ms, torch CPU threads={cores}, {el:.1f} s",
            "one_thread": {"value": round(flops / med1 / 1e12, 4), "unit": "TFLOP/s", "cores": 1,
                           "sample": f"{n1} whole config-2 steps on 1 thread (the reference's --debug "
                                     f"setting), median {med1 * 1e3:.1f} ms, {el1:.1f} s"}}


def copy_calibration(nbytes: int):
    """A plain device copy of known size, for scaling rocprofv3 byte counters."""
    a = torch.empty(nbytes, dtype=torch.uint8, device="cuda:0").fill_(1)
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    for _ in range(5):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes": nbytes, "launches": 5}))


def calibrate():
    """Reference points on the box, not this build's kernels: a plain device
    copy at three sizes (buffers rotated over 1 GiB, so the Infinity Cache
    cannot serve them) and the vendor GEMMs (hipBLASLt FP8 through
    ``torch._scaled_mm``, torch's bf16 ``linear``) at the config-2 shapes,
    each from graph replays timed with HIP events."""
    dev = torch.device("cuda:0")
    out = {}
    for mb in (16, 64, 256):
        n = mb << 20
        nb = max(2, (1 << 30) // n)
        src = [torch.ones(n, dtype=torch.uint8, device=dev) for _ in range(nb)]
        dst = [torch.empty(n, dtype=torch.uint8, device=dev) for _ in range(nb)]
        g = capture(lambda: [d.copy_(s_) for d, s_ in zip(dst, src)])
        out[f"copy_{mb}MB_GBs"] = round(2 * n * nb / time_graph(g, 5) / 1e6, 1)
        del g, src, dst
        log(f"calibrate: copy {mb} MB done")
    one = torch.ones((), device=dev)
    for K, N in SHAPES:
        gen = torch.Generator().manual_seed(7)
        a = torch.randn(M, K, generator=gen).to(dev).to(torch.float8_e4m3fn)
        b = torch.randn(N, K, generator=gen).to(dev).to(torch.float8_e4m3fn)
        flop = 2.0 * M * N * K
        g = capture(lambda: [torch._scaled_mm(a, b.t(), scale_a=one, scale_b=one, out_dtype=torch.bfloat16)
                             for _ in range(10)])
        out[f"hipblaslt_fp8_{M}x{K}x{N}_TFLOPs"] = round(flop / (time_graph(g, 5) / 10) / 1e9, 1)
        ab, bb = a.to(torch.bfloat16), b.to(torch.bfloat16)
        g = capture(lambda: [torch.nn.functional.linear(ab, bb) for _ in range(10)])
        out[f"torch_bf16_{M}x{K}x{N}_TFLOPs"] = round(flop / (time_graph(g, 5) / 10) / 1e9, 1)
        del g
        log(f"calibrate: GEMMs (K, N) = ({K}, {N}) done")
    print(json.dumps(out), flush=True)


def profile_shapes(reps: int, config: int = 2):
    """The config-2 kernels shape by shape, for rocprofv3 counter runs (with
    --config 3: config 3's linear_nf4 calls, M = 1 then M = 16 per shape)."""
    import voyager_amd.library  # noqa: F401  (defines quantized_ops)
    from voyager_amd import formats, gemm, packed
    from voyager_amd.ops import _elementwise

    dev = torch.device("cuda:0")
    if config == 3:
        sp = formats.parse_spec(CFG3_SPEC)
        index, entries, _ = formats.codebook_tables(sp["dtype"], dev)
        stab = formats.quantization_map(sp["scale_dtype"], dev)
        for i, (K, N) in enumerate(SHAPES):
            g = torch.Generator().manual_seed(1)
            wb = gemm.bake_nf4_weight((torch.randn(N, K, generator=g) * 0.02).bfloat16().to(dev), index, stab,
                                      entries)
            for rows in (1, 16):
                x = torch.randn(rows, K, generator=torch.Generator().manual_seed(0)).bfloat16().to(dev)
                torch.cuda.synchronize()
                for _ in range(reps):
                    gemm.linear_nf4(x, wb, index, stab)
                torch.cuda.synchronize()
            log(f"profile-shapes: shape {i} (K, N) = {SHAPES[i]} done")
        print(json.dumps({"profile_shapes": SHAPES, "M": [1, 16], "reps": reps}))
        return
    tab = formats.quantization_map("fp8_e4m3", dev)
    fmt = formats.classify(tab).fmt
    for i, (x, w) in enumerate(make_inputs(dev)):
        xd, wd = x.to(dev), w.to(dev)
        sx, sw = amax_scale(xd), amax_scale(wd)
        s = (sx * sw).contiguous()
        wq = packed.quantize_packed(wd, sw, tab)
        y = torch.empty(M, wd.shape[0], dtype=torch.bfloat16, device=dev)
        torch.cuda.synchronize()
        for _ in range(reps):
            xq = _elementwise("quantize", xd, sx, None, None, torch.bfloat16, fmt, None, torch.uint8)
        for _ in range(reps):
            gemm.linear_fp8(xq, wq, s, out=y)
        torch.cuda.synchronize()
        log(f"profile-shapes: shape {i} (K, N) = {SHAPES[i]} done")
    print(json.dumps({"profile_shapes": SHAPES, "reps": reps}))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--copy-calibration", type=int, default=0)
    ap.add_argument("--profile-shapes", type=int, default=0)
    ap.add_argument("--profile-steps", type=int, default=0)
    ap.add_argument("--calibrate", action="store_true")
    ap.add_argument("--outliers", action="store_true")
    ap.add_argument("--headline-only", action="store_true", help="config 2 alone, without the other configs")
    ap.add_argument("--config", type=int, default=2,
                    help="2 (default): the headline line; 1, 3, 4, 5: that config's measurements")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(the kernels run one GPU's share; sharding across GPUs is designed, not built)", file=sys.stderr)
        sys.exit(2)
    if args.copy_calibration:
        copy_calibration(args.copy_calibration)
        return
    if args.profile_shapes:
        profile_shapes(args.profile_shapes, args.config)
        return
    if args.calibrate:
        calibrate()
        return
    if args.outliers:
        print(json.dumps(bench_outliers(args)), flush=True)
        return
    fns = {1: bench_config1, 3: bench_config3, 4: bench_config4, 5: bench_config5}
    if args.config in fns:
        print(json.dumps(fns[args.config](args, 0.0 if args.no_cpu else 10.0)), flush=True)
        return
    res, cpu_data = gpu_bench(args)
    if args.profile_steps:
        print(json.dumps(res), flush=True)
        return
    cpu = None if args.no_cpu else cpu_baseline(cpu_data)
    # the other configs, each as `--config N` measures it, with a shorter CPU sample
    configs = {}
    if not args.headline_only:
        for n, fn in fns.items():
            t0 = time.perf_counter()
            try:
                configs[str(n)] = summary(fn(args, 0.0 if args.no_cpu else 4.0))
            except Exception as e:  # one config's failure must not lose the line
                configs[str(n)] = {"error": f"{type(e).__name__}: {e}"}
            log(f"bench: config {n} done in {time.perf_counter() - t0:.1f} s")
            torch.cuda.empty_cache()
    line = {
        "metric": METRIC,
        "value": round(res["value"], 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(res["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8_e4m3",
        "data": "synthetic",
        "config": {"workload": "cfg2: fp8_e4m3 per-tensor quantize + linear, M=2048, (K,N) in "
                               "{(4096,4096),(4096,1024),(4096,14336),(14336,4096)}",
                   "tokens": M, "shapes": SHAPES, "parallelism": "none (1 GPU)"},
        "roofline": res["roofline"],
        "quantize": res["quantize"],
        "per_shape": res["per_shape"],
        "cpu_baseline": cpu,
        "configs": configs,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
