"""The decoder-layer decode step (config 5) on the GPU against the oracle:
MX-int8 GEMV (exact products, fp32 accumulation), RMSNorm + MX-int8 fake
quantization, KIVI attention and the whole layer."""

import pytest
import torch

import voyager_amd.library  # noqa: F401  (defines quantized_ops)
from helpers import assert_within_bf16_ulps, max_rel_err
from oracle import decode as D
from voyager_amd import _lib, decode

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def _mx_ref(w_gpu):
    """Reference-form MX-int8 (scale, codes) of a GPU weight, by the
    parity-tested GPU quantize_mx, on the CPU."""
    tab = decode.formats.quantization_map("int8", DEV)
    s, c = torch.ops.quantized_ops.quantize_mx(w_gpu, tab, [-1], 16, 127.0, True)
    return c.cpu(), s.cpu()


@pytest.mark.parametrize("M", [1, 8, 16])
@pytest.mark.parametrize("K,N", [(4096, 6144), (14336, 4096), (256, 48), (768, 4096)])
def test_gemv_mx8_store(M, K, N):
    g = _gen(K + N + M)
    x = (torch.randn(M, K, generator=g) * 2).bfloat16()
    w = (torch.randn(N, K, generator=g) * 0.02).bfloat16()
    wg = w.to(DEV)
    cw, sw = _mx_ref(wg)
    if N * K <= 4096 * 4096:
        sw0, cw0 = D.mx8_quantize(w)
        assert torch.equal(cw0, cw) and torch.equal(sw0, sw)
    exp = D.mx8_linear(x, cw, sw)
    flag = decode.ErrorFlag(DEV)
    wt = decode.quantize_mx8_weight(wg)
    xq = D.mx8_fake_quant(x)
    fq = xq.half().to(DEV)
    ref64, abs64 = _ref64(xq, cw, sw)
    for tpb in (1, 2) if (N // 16) % 2 == 0 else (1,):
        got = decode.gemv_mx8(fq, wt, flag, tiles_per_block=tpb)
        assert got.dtype == torch.bfloat16 and list(got.shape) == [M, N]
        assert max_rel_err(got, exp) < 1e-2, tpb
        # exact products and float32 accumulation: the bf16 rounding of the exact sum
        assert_within_bf16_ulps(got, ref64, 1.0, 2.0**-14 * abs64, f"tiles_per_block={tpb}")
    flag.check()


def _ref64(xq, cw, sw):
    """float64 x_fq @ (codes * scale)^T and the sum of |terms| per output."""
    wd = D.O.dequantize_mx_parts(cw, sw, None, 16).double()
    x64 = xq.double()
    return x64 @ wd.T, x64.abs() @ wd.abs().T


def test_gemv_mx8_residual_and_zero_blocks():
    g = _gen(7)
    M, K, N = 8, 1024, 512
    x = torch.randn(M, K, generator=g).bfloat16()
    w = (torch.randn(N, K, generator=g) * 0.02).bfloat16()
    w[3, 64:128] = 0  # all-zero blocks bake with any exponent
    w[:, 512:528] = 0
    r = torch.randn(M, N, generator=g).bfloat16()
    cw, sw = _mx_ref(w.to(DEV))
    exp = (D.mx8_linear(x, cw, sw) + r)
    flag = decode.ErrorFlag(DEV)
    wt = decode.quantize_mx8_weight(w.to(DEV))
    xq = D.mx8_fake_quant(x)
    got = decode.gemv_mx8(xq.half().to(DEV), wt, flag, _lib.GEMV_RESIDUAL, residual=r.to(DEV))
    assert max_rel_err(got, exp) < 1e-2
    # bf16(bf16(exact sum) + r): within one ulp of each rounding
    ref64, abs64 = _ref64(xq, cw, sw)
    lin = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
    lin = decode.gemv_mx8(xq.half().to(DEV), wt, flag, y=lin)
    assert_within_bf16_ulps(lin, ref64, 1.0, 2.0**-14 * abs64, "linear part")
    assert torch.equal(got.cpu(), (lin.cpu() + r))
    flag.check()


def test_gemv_mx8_weight_range_error():
    w = torch.zeros(16, 256, dtype=torch.bfloat16, device=DEV)
    w[0, 0] = 2.0**-40  # block exponent -46: not representable in the fp16 operand
    tab = decode.formats.quantization_map("int8", DEV)
    p = decode.packed.quantize_mx_packed(w, tab, [-1], 16, 127.0, True)
    with pytest.raises(RuntimeError, match="weight block exponent"):
        decode.bake_mx8(p.codes, p.scale, p.bias, rebase=False)


@pytest.mark.parametrize("M", [1, 8])
def test_gemv_mx8_rebased_weight_rows(M):
    """Rows whose block exponents leave the fp16 operand's [-24, 5] bake
    rebased to their largest (any magnitude), the others as before: tiny,
    huge and mixed rows against the reference's linear_mx, and within one
    bf16 ulp of the float64 product (blocks within 29 binades of their row's
    largest, so nothing is flushed)."""
    g = _gen(21 + M)
    K, N = 512, 64
    x = torch.randn(M, K, generator=g).bfloat16()
    w = (torch.randn(N, K, generator=g) * 0.02).bfloat16()
    w[0] *= 2.0**-40                     # every block near 2**-52
    w[1] *= 2.0**20                      # every block near 2**14
    w[2, :256] *= 2.0**-25               # a row spanning 25 binades
    w[3, 96:112] = 2.0**-100             # one tiny block in a normal row: the row is rebased, the block flushed
    wg = w.to(DEV)
    cw, sw = _mx_ref(wg)
    exp = D.mx8_linear(x, cw, sw)
    flag = decode.ErrorFlag(DEV)
    wt = decode.quantize_mx8_weight(wg)
    assert wt.shift is not None
    shift = wt.shift.cpu()
    assert int(shift[4:].abs().sum()) == 0 and all(int(shift[i]) != 0 for i in range(4))
    xq = D.mx8_fake_quant(x)
    got = decode.gemv_mx8(xq.half().to(DEV), wt, flag)
    flag.check()
    assert max_rel_err(got[:, 4:], exp[:, 4:]) < 1e-2
    ref64, abs64 = _ref64(xq, cw, sw)
    # the rebased rows: exact products, float32 sums, one rounding (row 3's
    # flushed block is 2**-88 of its others, far under one ulp)
    for n in range(4):
        assert_within_bf16_ulps(got[:, n], ref64[:, n], 1.0, 2.0**-14 * abs64[:, n], f"row {n}")
    assert_within_bf16_ulps(got[:, 4:], ref64[:, 4:], 1.0, 2.0**-14 * abs64[:, 4:], "rows in range")


def test_step_checked_reruns_activation_overflow():
    """A layer whose RMSNorm gain pushes its normed activations past the fp16
    range of the GEMV operand: the fast step flags it, step_checked puts the
    cache back and reruns the step on rebased rows, and the result matches
    the oracle layer (which has no such range) within 1e-2; the cache ends
    one position on, as after any step."""
    cfg = D.Config(hidden=512, n_heads=4, n_kv_heads=1, head_dim=128, intermediate=1024)
    w = D.random_layer(cfg, seed=5)
    w["ln1"] = (w["ln1"].float() * 3.0e4).bfloat16()  # |h1| up to ~1e5
    wd = {k: v.to(DEV) for k, v in w.items()}
    mx = {k: _mx_ref(wd[k]) for k in ("wq", "wk", "wv", "wo", "wg", "wu", "wd")}
    layer = decode.DecoderLayer(wd, cfg.n_heads, cfg.n_kv_heads, cfg.eps, cfg.rope_theta, max_batch=2, max_pos=1024)
    g = _gen(6)
    B, n_main, n_res = 2, 256, 40
    k_main, v_main = (torch.randn(B, 1, n_main, 128, generator=g).bfloat16() for _ in range(2))
    k_res, v_res = (torch.randn(B, 1, n_res, 128, generator=g).bfloat16() for _ in range(2))
    x = torch.randn(B, cfg.hidden, generator=g).bfloat16()
    cache, kq, vq = decode.KiviCache.from_bf16(k_main.to(DEV), v_main.to(DEV), k_res.to(DEV), v_res.to(DEV),
                                               capacity=512)
    k_past = torch.cat((D.kivi_dequantize(kq[2].cpu(), kq[0].cpu(), kq[1].cpu(), -2), k_res), dim=2)
    v_past = torch.cat((D.kivi_dequantize(vq[2].cpu(), vq[0].cpu(), vq[1].cpu(), -1), v_res), dim=2)
    cos, sin = D.rope_cos_sin(torch.tensor([n_main + n_res]), 128, cfg.rope_theta)
    exp = D.decode_layer(x, w, k_past, v_past, cos, sin, cfg, mx=mx)
    assert float(exp["h1"].float().abs().max()) > 65504  # the fast path's operand cannot hold it
    # the fast step alone flags it
    state0 = cache.state.clone()
    layer.step(x.to(DEV), cache, advance=False)
    with pytest.raises(RuntimeError, match="fp16 range"):
        layer.flag.check()
    cache.state.copy_(state0)
    out = layer.step_checked(x.to(DEV), cache)
    torch.cuda.synchronize()
    err = max_rel_err(out, exp["out"])
    print(f"step_checked after an fp16-range overflow: {err:.5f} vs the oracle", flush=True)
    assert err < 1e-2
    assert cache.device_state() == (n_main, n_res + 1) == (cache.n_main, cache.n_res)
    kr, vr = cache.residual_tokens(n_res + 1)
    assert torch.equal(kr[:, :, n_res:].cpu(), exp["k"]) or max_rel_err(kr[:, :, n_res:], exp["k"]) < 1e-2


@pytest.mark.parametrize("M", [1, 8])
def test_gemv_mx8_swiglu(M):
    g = _gen(11 + M)
    K, F = 1024, 768
    x = torch.randn(M, K, generator=g).bfloat16()
    wg_, wu_ = (torch.randn(F, K, generator=g) * 0.05).bfloat16(), (torch.randn(F, K, generator=g) * 0.05).bfloat16()
    cg, sg = _mx_ref(wg_.to(DEV))
    cu, su = _mx_ref(wu_.to(DEV))
    act = torch.nn.functional.silu(D.mx8_linear(x, cg, sg)) * D.mx8_linear(x, cu, su)
    flag = decode.ErrorFlag(DEV)
    wt = decode.quantize_mx8_weight(torch.cat((wg_, wu_)).to(DEV), paired=True)
    y = torch.empty(M, F, dtype=torch.bfloat16, device=DEV)
    fq = decode.gemv_mx8(D.mx8_fake_quant(x).half().to(DEV), wt, flag, _lib.GEMV_SWIGLU, y=y)
    assert max_rel_err(y, act) < 1e-2
    # the fake quantization is the oracle's quantize_mx of the kernel's own product, bit for bit
    assert torch.equal(fq.cpu(), D.mx8_fake_quant(y.cpu()).half())
    flag.check()


@pytest.mark.parametrize("M,H", [(8, 4096), (3, 14336), (1, 256)])
def test_rmsnorm_mx8(M, H):
    g = _gen(H + M)
    x = (torch.randn(M, H, generator=g) * 3).bfloat16()
    w = (1 + 0.1 * torch.randn(H, generator=g)).bfloat16()
    exp = D.rms_norm(x, w, 1e-5)
    flag = decode.ErrorFlag(DEV)
    h = torch.empty(M, H, dtype=torch.bfloat16, device=DEV)
    fq = decode.rmsnorm_mx8(x.to(DEV), w.to(DEV), 1e-5, flag, h_out=h)
    hc = h.cpu()
    # the row sum of squares is accumulated in another order: at most one bf16 ulp apart
    diff = (hc.view(torch.int16).int() - exp.view(torch.int16).int()).abs()
    assert int(diff.max()) <= 1 and float((diff > 0).float().mean()) < 0.01
    assert torch.equal(fq.cpu(), D.mx8_fake_quant(hc).half())
    flag.check()


def test_fq_range_flag():
    # one nonzero element: rsqrt(mean(x**2)) = 16, so the normed value is
    # 16 * 8192 = 2**17 and its block's fake-quantized values exceed fp16
    x = torch.zeros(1, 256, dtype=torch.bfloat16)
    x[0, 0] = 1.0
    flag = decode.ErrorFlag(DEV)
    decode.rmsnorm_mx8(x.to(DEV), torch.full((256,), 8192.0, dtype=torch.bfloat16, device=DEV), 1e-5, flag)
    with pytest.raises(RuntimeError, match="fp16 range"):
        flag.check()


def _attention_case(B, nkv, n_main, n_res, seed):
    g = _gen(seed)
    nq = 4 * nkv
    qkv = torch.randn(B, (nq + 2 * nkv) * 128, generator=g).bfloat16()
    k_main = torch.randn(B, nkv, n_main, 128, generator=g).bfloat16()
    v_main = torch.randn(B, nkv, n_main, 128, generator=g).bfloat16()
    k_res = torch.randn(B, nkv, n_res, 128, generator=g).bfloat16()
    v_res = torch.randn(B, nkv, n_res, 128, generator=g).bfloat16()
    return nq, qkv, k_main, v_main, k_res, v_res


def _expected_attention(nq, nkv, qkv, k_deq, v_deq, k_res, v_res, cos, sin):
    B = qkv.shape[0]
    q = qkv[:, : nq * 128].view(B, 1, nq, 128).transpose(1, 2)
    k = qkv[:, nq * 128:(nq + nkv) * 128].view(B, 1, nkv, 128).transpose(1, 2)
    v = qkv[:, (nq + nkv) * 128:].view(B, 1, nkv, 128).transpose(1, 2)
    c, s = cos[:, None, None, :], sin[:, None, None, :]
    q, k = D.apply_rope(q, c, s), D.apply_rope(k, c, s)
    keys = torch.cat((k_deq, k_res, k), dim=2)
    values = torch.cat((v_deq, v_res, v), dim=2)
    exp = D.eager_attention(q, keys, values, 128 ** -0.5).reshape(B, nq * 128)
    # the same attention in float64 (no bf16 rounding after the dequantize)
    grp = nq // nkv
    K64, V64 = keys.double().repeat_interleave(grp, 1), values.double().repeat_interleave(grp, 1)
    w64 = torch.softmax((q.double() @ K64.transpose(2, 3)) * 128 ** -0.5, dim=-1)
    exp64 = (w64 @ V64).transpose(1, 2).reshape(B, nq * 128)
    return exp, exp64, k, v


ROPE = {}


def _ulp_stats(got, exp):
    """The fraction of bf16 outputs that differ from ``exp`` and the largest
    difference in ulps among those not near zero (|exp| above 1/64 of its
    largest magnitude, where a difference in summation order cannot cancel
    to a few ulps of a tiny value)."""
    g, e = got.detach().cpu(), exp.detach().cpu()
    gi, ei = g.view(torch.int16).int(), e.view(torch.int16).int()
    differ = gi != ei
    big = e.float().abs() > e.float().abs().max() / 64
    same_sign = (g.float() * e.float()) > 0
    d = (gi - ei).abs()[big & same_sign]
    return float(differ.float().mean()), int(d.max()) if d.numel() else 0


def _rope(max_pos=8192, theta=5e5):
    key = (max_pos, theta)
    if key not in ROPE:
        ROPE[key] = decode.rope_tables(max_pos, theta, DEV)
    return ROPE[key]


@pytest.mark.parametrize("B,nkv,n_main,n_res", [(2, 2, 96, 5), (1, 1, 0, 0), (2, 1, 544, 127), (1, 2, 512, 31),
                                                (8, 8, 3968, 127)])
def test_kivi_attention(B, nkv, n_main, n_res):
    nq, qkv, k_main, v_main, k_res, v_res = _attention_case(B, nkv, n_main, n_res, 100 + n_main + n_res)
    cache, kq, vq = decode.KiviCache.from_bf16(k_main.to(DEV), v_main.to(DEV), k_res.to(DEV), v_res.to(DEV))
    if n_main:
        if B * nkv * n_main <= 64 * 1024:
            ks, kz, kc = D.kivi_quantize(k_main, -2)
            assert torch.equal(kc, kq[2].cpu()) and torch.equal(ks, kq[0].cpu()) and torch.equal(kz, kq[1].cpu())
        k_deq = D.kivi_dequantize(kq[2].cpu(), kq[0].cpu(), kq[1].cpu(), -2)
        v_deq = D.kivi_dequantize(vq[2].cpu(), vq[0].cpu(), vq[1].cpu(), -1)
    else:
        k_deq = v_deq = torch.zeros(B, nkv, 0, 128, dtype=torch.bfloat16)
    pos = n_main + n_res
    assert cache.position == pos and cache.device_state() == (n_main, n_res)
    cos, sin = D.rope_cos_sin(torch.tensor([pos]), 128, 5e5)
    rope = _rope()
    assert torch.equal(rope[0, pos].cpu(), cos[0]) and torch.equal(rope[1, pos].cpu(), sin[0])
    exp, exp64, k_new, v_new = _expected_attention(nq, nkv, qkv, k_deq, v_deq, k_res, v_res, cos, sin)
    flag = decode.ErrorFlag(DEV)
    attn = torch.empty(B, nq * 128, dtype=torch.bfloat16, device=DEV)
    fq = decode.kivi_attention(qkv.to(DEV), cache, rope, nq, flag, attn=attn)
    # Keys and values are dequantized with the reference's bf16 roundings,
    # and every score and probability is rounded where its eager chain rounds
    # it, so the kernels follow that chain -- itself up to ~1.5%
    # (max-abs-normalized) from float64 at these lengths -- to summation
    # order: almost every output is the chain's bf16 value bit for bit
    err = max_rel_err(attn, exp)
    frac, ulps = _ulp_stats(attn, exp)
    print(f"attention B={B} nkv={nkv} n_main={n_main} n_res={n_res}: {err:.5f} vs the eager chain "
          f"({frac:.4%} of outputs differ, by at most {ulps} ulp), {max_rel_err(exp, exp64):.5f} eager chain "
          f"vs float64", flush=True)
    assert err < 5e-3 and frac < 0.01
    assert torch.equal(fq.cpu(), D.mx8_fake_quant(attn.cpu()).half())
    # the step's key (after RoPE) and value landed in the residual window; the state is not advanced
    kr, vr = cache.residual_tokens(n_res + 1)
    assert torch.equal(kr[:, :, :n_res].cpu(), k_res) and torch.equal(vr[:, :, :n_res].cpu(), v_res)
    assert torch.equal(kr[:, :, n_res:].cpu(), k_new) and torch.equal(vr[:, :, n_res:].cpu(), v_new)
    assert cache.device_state() == (n_main, n_res)
    flag.check()


def _bake_chunk(cache, k, v, g0):
    """The main-cache bytes of groups [g0, g0 + 4): the oracle's
    quantize_affine of a 128-token chunk ``[B, nkv, 128, 128]`` baked by
    vh_kivi_bake into a fresh cache of the same capacity."""
    ks, kz, kc = D.kivi_quantize(k, -2)
    vs, vz, vc = D.kivi_quantize(v, -1)
    P, T = cache.P, k.shape[2]
    fresh = torch.zeros_like(cache.main)
    args = [t.to(DEV).contiguous() for t in (kc.to(torch.uint8), ks, kz, vc.to(torch.uint8), vs, vz)]
    st = _lib.load().vh_kivi_bake(*[t.data_ptr() for t in args[:6]], P, T, cache.group_cap, g0, fresh.data_ptr(),
                                  torch.cuda.current_stream().cuda_stream)
    _lib.check(st, "vh_kivi_bake")
    return _groups(fresh, cache, g0, T // 32)


def _groups(main, cache, g0, n):
    m = main.view(cache.P, cache.group_cap, 3072)
    return m[:, g0:g0 + n].cpu()


def test_kivi_fold_is_the_reference_chunk_store():
    """A step that fills the residual's last slot: the advance quantizes the
    128 residual tokens (quantize_affine, KIVI specs) into the next four
    main-cache groups -- bytes identical to baking the oracle's quantization
    of the same chunk -- and restarts the residual; the next step's
    attention reads the chunk from the main cache."""
    B, nkv, n_main, n_res = 2, 2, 96, 127
    nq, qkv, k_main, v_main, k_res, v_res = _attention_case(B, nkv, n_main, n_res, 7)
    cache, _, _ = decode.KiviCache.from_bf16(k_main.to(DEV), v_main.to(DEV), k_res.to(DEV), v_res.to(DEV),
                                             capacity=512)
    rope, flag = _rope(), decode.ErrorFlag(DEV)
    before = cache.main.clone()
    decode.kivi_attention(qkv.to(DEV), cache, rope, nq, flag, advance=True)
    chunk_k, chunk_v = (t.cpu() for t in cache.residual_tokens(128))
    assert cache.device_state() == (n_main + 128, 0) == (cache.n_main, cache.n_res)
    g0 = n_main // 32
    assert torch.equal(_groups(cache.main, cache, g0, 4), _bake_chunk(cache, chunk_k, chunk_v, g0))
    assert torch.equal(_groups(cache.main, cache, 0, g0), _groups(before, cache, 0, g0))
    # an advance that completes nothing only counts the slot
    qkv2 = torch.randn(B, (nq + 2 * nkv) * 128, generator=_gen(8)).bfloat16()
    decode.kivi_attention(qkv2.to(DEV), cache, rope, nq, flag, advance=True)
    assert cache.device_state() == (n_main + 128, 1)
    flag.check()


def test_kivi_full_cache_is_flagged():
    B, nkv, n_main, n_res = 1, 1, 128, 127
    nq, qkv, k_main, v_main, k_res, v_res = _attention_case(B, nkv, n_main, n_res, 9)
    cache, _, _ = decode.KiviCache.from_bf16(k_main.to(DEV), v_main.to(DEV), k_res.to(DEV), v_res.to(DEV),
                                             capacity=256)
    rope, flag = _rope(), decode.ErrorFlag(DEV)
    decode.kivi_attention(qkv.to(DEV), cache, rope, nq, flag, advance=True)
    assert cache.device_state() == (256, 0)
    flag.check()
    for _ in range(127):
        decode.kivi_attention(qkv.to(DEV), cache, rope, nq, flag, advance=True)
    assert cache.device_state() == (256, 127)
    flag.check()
    # the next step completes a chunk the full main cache cannot take
    decode.kivi_attention(qkv.to(DEV), cache, rope, nq, flag, advance=True)
    assert cache.device_state() == (256, 127) == (cache.n_main, cache.n_res)
    with pytest.raises(RuntimeError, match="no room"):
        flag.check()
    flag.check()  # cleared by the check


def test_decode_layer_cfg5():
    """Config 5: one random-init Llama-3.1-8B-architecture layer, decode at
    batch 8 over a 4096-token context (3968 KIVI tokens + 127 residual +
    this step's), every linear MX-int8 bs=16, against the oracle layer on the
    same quantized weights and cache."""
    cfg = D.Config()
    w = D.random_layer(cfg, seed=0)
    wd = {k: v.to(DEV) for k, v in w.items()}
    mx = {k: _mx_ref(wd[k]) for k in ("wq", "wk", "wv", "wo", "wg", "wu", "wd")}
    layer = decode.DecoderLayer(wd, cfg.n_heads, cfg.n_kv_heads, cfg.eps, cfg.rope_theta, max_batch=8, max_pos=4096)
    g = _gen(1)
    B, n_main, n_res = 8, 3968, 127
    k_main = torch.randn(B, 8, n_main, 128, generator=g).bfloat16()
    v_main = torch.randn(B, 8, n_main, 128, generator=g).bfloat16()
    k_res = torch.randn(B, 8, n_res, 128, generator=g).bfloat16()
    v_res = torch.randn(B, 8, n_res, 128, generator=g).bfloat16()
    x = torch.randn(B, cfg.hidden, generator=g).bfloat16()
    cache, kq, vq = decode.KiviCache.from_bf16(k_main.to(DEV), v_main.to(DEV), k_res.to(DEV), v_res.to(DEV),
                                               capacity=4096)
    k_past = torch.cat((D.kivi_dequantize(kq[2].cpu(), kq[0].cpu(), kq[1].cpu(), -2), k_res), dim=2)
    v_past = torch.cat((D.kivi_dequantize(vq[2].cpu(), vq[0].cpu(), vq[1].cpu(), -1), v_res), dim=2)
    pos = n_main + n_res
    cos, sin = D.rope_cos_sin(torch.tensor([pos]), 128, cfg.rope_theta)
    assert torch.equal(layer.rope[0, pos].cpu(), cos[0]) and torch.equal(layer.rope[1, pos].cpu(), sin[0])
    exp = D.decode_layer(x, w, k_past, v_past, cos, sin, cfg, mx=mx)
    out = layer.step(x.to(DEV), cache)
    torch.cuda.synchronize()
    layer.flag.check()
    # the step filled the residual's last slot: its chunk was folded
    assert cache.device_state() == (4096, 0)
    b = {k: v[:B] for k, v in layer.buf.items()}
    # Every quantized stage is the reference op sequence bit for bit when fed
    # the oracle's own inputs (isolating it from upstream differences):
    assert torch.equal(b["qkv"].cpu(), torch.cat([D.mx8_linear(exp["h1"], *mx[k]) for k in ("wq", "wk", "wv")], -1))
    f = decode.ErrorFlag(DEV)
    o = decode.gemv_mx8(D.mx8_fake_quant(exp["attn"]).half().to(DEV), layer.o, f, _lib.GEMV_RESIDUAL,
                        residual=x.to(DEV))
    assert torch.equal(o.cpu(), exp["x1"])
    act = torch.empty(B, cfg.intermediate, dtype=torch.bfloat16, device=DEV)
    decode.gemv_mx8(D.mx8_fake_quant(exp["h2"]).half().to(DEV), layer.gate_up, f, _lib.GEMV_SWIGLU, y=act)
    assert torch.equal(act.cpu(), exp["act"])
    d = decode.gemv_mx8(D.mx8_fake_quant(exp["act"]).half().to(DEV), layer.down, f, _lib.GEMV_RESIDUAL,
                        residual=exp["x1"].to(DEV))
    assert torch.equal(d.cpu(), exp["out"])
    f.check()
    # Stage by stage on the GPU's own intermediates: the attention within
    # 1e-2 of the eager chain on the GPU's q / k / v, and each later stage
    # equal to the oracle's op sequence applied to the GPU's own input.
    g_attn, g_x1, g_act = (b[k].cpu() for k in ("attn", "x1", "act"))
    g_out = out.cpu()
    assert max_rel_err(g_attn, exp["attn"]) < 1e-2
    assert torch.equal(g_x1, x + D.mx8_linear(g_attn, *mx["wo"]))
    h2 = D.rms_norm(g_x1, w["ln2"], cfg.eps)
    act_ref = torch.nn.functional.silu(D.mx8_linear(h2, *mx["wg"])) * D.mx8_linear(h2, *mx["wu"])
    assert max_rel_err(g_act, act_ref) < 1e-2  # the RMSNorm's row sum is accumulated in another order
    assert torch.equal(g_out, g_x1 + D.mx8_linear(g_act, *mx["wd"]))
    # End to end, the attention's remaining ulp differences (summation
    # order) pass through the MX re-quantization of x1 and act: in the
    # reference's own pipeline, moving 0.05% of the attention outputs by one
    # ulp already moves the layer output 0.6-0.8% (tests/test_oracle_decode.py)
    errs = {k: max_rel_err(b[k], exp[k]) for k in ("attn", "x1", "act")}
    errs["out"] = max_rel_err(out, exp["out"])
    frac, ulps = _ulp_stats(b["attn"], exp["attn"])
    print("cfg5 max-abs-normalized errors vs the oracle:", errs,
          f"attention outputs differing: {frac:.4%} (at most {ulps} ulp)", flush=True)
    assert frac < 0.01
    assert all(v < 1e-2 for v in errs.values()), errs


def test_decode_replay_crosses_folds():
    """A captured decode step replayed 160 times (positions 356..515 of a
    small layer): each replay is the next step -- the position, the residual
    slot and the fold of a completed chunk come from device state -- and
    matches the oracle layer over the reference's split cache (within 1e-2),
    each fold storing the bytes the reference's chunk store gives."""
    cfg = D.Config(hidden=512, n_heads=4, n_kv_heads=1, head_dim=128, intermediate=1024)
    w = D.random_layer(cfg, seed=3)
    wd = {k: v.to(DEV) for k, v in w.items()}
    mx = {k: _mx_ref(wd[k]) for k in ("wq", "wk", "wv", "wo", "wg", "wu", "wd")}
    B, n_main, n_res, steps = 2, 256, 100, 160
    layer = decode.DecoderLayer(wd, cfg.n_heads, cfg.n_kv_heads, cfg.eps, cfg.rope_theta, max_batch=B,
                                max_pos=1024)
    g = _gen(4)
    k_main, v_main = torch.randn(B, 1, n_main, 128, generator=g).bfloat16(), torch.randn(B, 1, n_main, 128,
                                                                                          generator=g).bfloat16()
    k_res, v_res = torch.randn(B, 1, n_res, 128, generator=g).bfloat16(), torch.randn(B, 1, n_res, 128,
                                                                                       generator=g).bfloat16()
    xs = torch.randn(steps, B, cfg.hidden, generator=g).bfloat16()
    cache, _, _ = decode.KiviCache.from_bf16(k_main.to(DEV), v_main.to(DEV), k_res.to(DEV), v_res.to(DEV),
                                             capacity=768)
    ref = D.KiviCacheRef(k_main, v_main, k_res, v_res)
    x_dev = torch.empty(B, cfg.hidden, dtype=torch.bfloat16, device=DEV)
    x_dev.copy_(xs[0])
    graph = layer.capture(x_dev, cache)
    worst = 0.0
    folds = 0
    for s in range(steps):
        x_dev.copy_(xs[s])
        fold_now = cache.n_res == 127
        if fold_now:
            chunk = None  # the residual's 128 tokens after this step's append, read below
        graph.replay()
        cache.advance_host()
        torch.cuda.synchronize()
        pos = ref.position
        cos, sin = D.rope_cos_sin(torch.tensor([pos]), 128, cfg.rope_theta)
        k_past, v_past = ref.past()
        exp = D.decode_layer(xs[s], w, k_past, v_past, cos, sin, cfg, mx=mx)
        out = layer.buf["out"][:B].cpu()
        err = max_rel_err(out, exp["out"])
        worst = max(worst, err)
        assert err < 1e-2, (s, pos, err)
        folded = ref.append(exp["k"], exp["v"])
        assert folded == fold_now, s
        if folded:
            folds += 1
            g0 = (ref.n_main - 128) // 32
            chunk_k, chunk_v = (t.cpu() for t in cache.residual_tokens(128))
            assert torch.equal(_groups(cache.main, cache, g0, 4), _bake_chunk(cache, chunk_k, chunk_v, g0)), s
        assert cache.device_state() == (ref.n_main, ref.position - ref.n_main) == (cache.n_main, cache.n_res)
    print(f"replay: {steps} steps, {folds} folds, worst max-abs-normalized error {worst:.5f}", flush=True)
    assert folds == 2
    layer.flag.check()
