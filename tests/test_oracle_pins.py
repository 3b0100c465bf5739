"""Pins of the CPU oracle against what the mathematics fixes.

Every check here computes the expected answer a different way than the oracle
does (enumerated grids and nearest-value search, textbook posit rounding,
published NormalFloat constants, exact rational arithmetic, float64 numpy),
so that a dropped term, a wrong sign or an off-by-one in the oracle fails.
"""

import math
from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import ops as O
from oracle import qspec as Q
from oracle import tables as T

ALL = T.all_bf16()
ALLF = ALL.double().numpy()
FIN = np.isfinite(ALLF)


def _same_values(oracle_tab: torch.Tensor, expect: np.ndarray, mask=None):
    got = oracle_tab.float().numpy().astype(np.float64)
    both_nan = np.isnan(got) & np.isnan(expect)
    ok = (got == expect) | both_nan
    if mask is not None:
        ok = ok | ~mask
    bad = np.flatnonzero(~ok)
    assert bad.size == 0, f"{bad.size} entries differ, first at pattern {hex(bad[0])}: " \
        f"input {ALLF[bad[0]]!r} oracle {got[bad[0]]!r} expected {expect[bad[0]]!r}"


# ------------------------------------------------------------------ spec grammar
def test_spec_ranges():
    assert Q.int_range("int8") == (-128, 127)
    assert Q.int_range("uint2") == (0, 3)
    assert Q.float_format("fp8_e4m3").max_norm == 448
    assert Q.float_format("fp8_e4m3_ieee").max_norm == 240
    e5m3 = Q.float_format("fp8_e5m3")
    assert e5m3.max_norm == 61440 and not e5m3.signed and e5m3.ieee
    assert Q.float_format("fp16_e5m10").max_norm == 65504
    assert Q.quant_min_max("lut4_to_int6") == (-31, 31)
    assert Q.quant_min_max("posit8_1") == (-4096, 4096)


# ------------------------------------------------------------------ int tables
@pytest.mark.parametrize("dtype,lo,hi", [("int8", -128, 127), ("uint2", 0, 3), ("int6", -32, 31), ("uint8", 0, 255)])
def test_int_table(dtype, lo, hi):
    expect = np.clip(np.round(ALLF), lo, hi)  # numpy rounds half to even
    _same_values(T.quantization_map(dtype), expect)


# ------------------------------------------------------------------ minifloats
def _grid(ebits, mbits, max_norm):
    """Non-negative values of a minifloat, ascending, enumerated from fields."""
    emin = 2 - 2 ** (ebits - 1)
    vals = [m * 2.0 ** (emin - mbits) for m in range(0, 2**mbits)]  # subnormals and zero
    e = emin
    while True:
        row = [(2**mbits + m) * 2.0 ** (e - mbits) for m in range(2**mbits)]
        vals += [v for v in row if v <= max_norm]
        if row[-1] >= max_norm:
            break
        e += 1
    return np.array(sorted(set(vals)))


def _nearest_even(v, grid):
    """Round |v| to the grid: nearest, ties to the even grid index (the even
    mantissa), saturating at the top."""
    a = np.abs(v)
    i = np.clip(np.searchsorted(grid, a), 1, len(grid) - 1)
    lo, hi = grid[i - 1], grid[i]
    pick_hi = (hi - a < a - lo) | ((hi - a == a - lo) & (i % 2 == 0))
    r = np.where(pick_hi, hi, lo)
    r = np.where(a >= grid[-1], grid[-1], r)
    r = np.where(np.isnan(a), np.nan, r)
    return np.copysign(r, v)


@pytest.mark.parametrize("dtype", ["fp8_e4m3", "fp8_e5m3", "fp16_e5m10", "fp8_e5m2", "fp6_e2m3", "fp4_e2m1"])
def test_minifloat_table(dtype):
    f = Q.float_format(dtype)
    grid = _grid(f.ebits, f.mbits, f.max_norm)
    v = ALLF.copy() if f.signed else np.abs(ALLF)
    cm = torch.tensor(f.max_norm).bfloat16().item()
    v = np.clip(v, -cm, cm)
    r = _nearest_even(v, grid)
    r = np.minimum(r, f.max_norm)
    expect = torch.from_numpy(r.astype(np.float32)).bfloat16().double().numpy()
    _same_values(T.quantization_map(dtype), expect)


def test_fp8_e4m3_matches_torch_cast():
    v = torch.clamp(ALL.float(), -448, 448)
    expect = v.to(torch.float8_e4m3fn).float().numpy().astype(np.float64)
    _same_values(T.quantization_map("fp8_e4m3"), expect)


def test_fp16_matches_torch_cast():
    v = torch.clamp(ALL.float(), -65504, 65504)
    expect = v.half().float().bfloat16().double().numpy()
    _same_values(T.quantization_map("fp16_e5m10"), expect)


# ------------------------------------------------------------------ posit8
def _posit_decode(code, n, es):
    if code == 0:
        return 0.0
    if code == 1 << (n - 1):
        return math.nan
    neg = code >> (n - 1)
    if neg:
        code = (-code) & ((1 << n) - 1)
    bits = [(code >> i) & 1 for i in range(n - 2, -1, -1)]
    first, run = bits[0], 0
    while run < len(bits) and bits[run] == first:
        run += 1
    k = run - 1 if first else -run
    rest = bits[run + 1:]
    e = 0
    for j in range(es):
        e = (e << 1) | (rest[j] if j < len(rest) else 0)
    fr = rest[es:]
    f = sum(b * 2.0 ** -(j + 1) for j, b in enumerate(fr))
    val = 2.0 ** (k * 2**es + e) * (1 + f)
    return -val if neg else val


def _posit_round(x, n, es):
    """Textbook posit rounding: write the exact value's regime, exponent and
    fraction as one bit string, keep n-1 bits, round half to even on the
    dropped bits; saturate at maxpos and never round a nonzero to zero."""
    if x == 0:
        return 0.0
    a = abs(x)
    m, ex = math.frexp(a)  # a = m * 2**ex, m in [0.5, 1)
    s = ex - 1
    frac = Fraction(m) * 2 - 1  # in [0, 1)
    k, e = divmod(s, 2**es)
    useed_bits = []
    if k >= 0:
        useed_bits = [1] * (k + 1) + [0]
    else:
        useed_bits = [0] * (-k) + [1]
    ebits = [(e >> (es - 1 - j)) & 1 for j in range(es)]
    # Fraction bits: exact, 40 are plenty for a bf16 input.
    fbits = []
    f = frac
    for _ in range(40):
        f *= 2
        fbits.append(int(f >= 1))
        if f >= 1:
            f -= 1
    body = useed_bits + ebits + fbits
    keep, drop = body[: n - 1], body[n - 1:]
    kept = 0
    for b in keep:
        kept = (kept << 1) | b
    kept <<= max(0, n - 1 - len(keep))
    guard = drop[0] if drop else 0
    sticky = any(drop[1:]) or f != 0
    if guard and (sticky or (kept & 1)):
        kept += 1
    maxcode = (1 << (n - 1)) - 1
    kept = min(max(kept, 1), maxcode)
    v = _posit_decode(kept, n, es)
    return -v if x < 0 else v


def test_posit8_table_matches_textbook_rounding_above_minpos():
    n, es = 8, 1
    minpos = 2.0 ** -12
    tab = T.quantization_map("posit8_1").float().numpy()
    bad = []
    for i in range(0, 65536, 1):
        v = ALLF[i]
        if not np.isfinite(v):
            assert np.isnan(tab[i])
            continue
        if abs(v) < 2.0**-13:
            # The reference flushes below 2**floor(-(n-1)*2**es + 2**(es-1)).
            assert tab[i] == 0.0
            continue
        exp = _posit_round(v, n, es)
        if tab[i] != exp:
            bad.append((hex(i), v, tab[i], exp))
    assert not bad, f"{len(bad)} mismatches, e.g. {bad[:5]}"
    # The values themselves are the 255 finite posit8 levels.
    lv = T.table_levels(T.quantization_map("posit8_1")).numpy()
    codes = [c for c in range(256) if c != 128]
    assert sorted(set(_posit_decode(c, n, es) for c in codes)) == sorted(lv.tolist())
    assert lv.min() == -4096 and lv.max() == 4096 and np.min(np.abs(lv[lv != 0])) == minpos


# ------------------------------------------------------------------ NormalFloat codebook
NF4_PUBLISHED = [-1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
                 -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
                 0.07958029955625534, 0.16093020141124725, 0.24611230194568634, 0.33791524171829224,
                 0.44070982933044434, 0.5626170039176941, 0.7229568362236023, 1.0]


def test_nf4_levels_match_published_constants():
    np.testing.assert_allclose(T.normal_map(4).numpy(), NF4_PUBLISHED, atol=2e-7)


def test_lut4_to_int6_table():
    levels = np.round(np.array(NF4_PUBLISHED) * 31)
    assert levels.tolist() == [-31, -22, -16, -12, -9, -6, -3, 0, 2, 5, 8, 10, 14, 17, 22, 31]
    v = np.clip(ALLF, levels[0], levels[-1])
    v = np.where(np.isnan(v), levels[0], v)  # argmin over NaN distances picks index 0
    d = np.abs(v[:, None] - levels[None, :])
    idx = np.argmin(d, axis=1)  # numpy argmin also keeps the first on ties
    _same_values(T.quantization_map("lut4_to_int6"), levels[idx])
    index, entries, mid = T.codebook_index_table(T.quantization_map("lut4_to_int6"))
    assert entries.float().tolist() == levels.tolist()
    np.testing.assert_array_equal(index.numpy(), idx)
    np.testing.assert_array_equal(mid.float().numpy(), (levels[1:] + levels[:-1]) / 2)


# ------------------------------------------------------------------ arithmetic of the ops
def _bf16_round_exact(fr: Fraction) -> float:
    """Round an exact rational to bfloat16, half to even (normal range)."""
    if fr == 0:
        return 0.0
    s = -1 if fr < 0 else 1
    a = abs(fr)
    e = math.floor(math.log2(a))
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    q = a / (Fraction(2) ** (e - 7))
    r = math.floor(q)
    rem = q - r
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and r % 2 == 1):
        r += 1
    return s * float(r * Fraction(2) ** (e - 7))


def test_bf16_division_is_true_division_rne():
    g = torch.Generator().manual_seed(3)
    x = (torch.randn(4000, generator=g) * 10).bfloat16()
    s = (torch.rand(4000, generator=g) * 5 + 0.1).bfloat16()
    got = O.quantize(x, s).float().numpy()
    for i in range(4000):
        exp = _bf16_round_exact(Fraction(x[i].item()) / Fraction(s[i].item()))
        assert got[i] == exp, (x[i].item(), s[i].item(), got[i], exp)


def test_scalar_division_of_amax():
    # amax / quant_max with a Python float divisor: true division, RNE to bf16.
    g = torch.Generator().manual_seed(4)
    a = (torch.rand(3000, generator=g) * 100).bfloat16()
    got = (a / 31.0).float().numpy()
    for i in range(3000):
        assert got[i] == _bf16_round_exact(Fraction(a[i].item()) / 31)


def test_shared_exponent_is_exponent_field():
    pos = ALL[(ALL.float() > 0) & torch.isfinite(ALL.float())]
    e = O.shared_exponents(pos.view(-1, 1), [1]).view(-1).float().numpy()
    expect = np.array([math.frexp(v)[1] - 1 for v in pos.float().tolist()])
    np.testing.assert_array_equal(e, expect)
    z = O.shared_exponents(torch.zeros(1, 1, dtype=torch.bfloat16), [1])
    assert z.item() == -126


@pytest.mark.parametrize("block,expect", [
    ([1.0], 2.0**-6),
    ([127.0, -3.0], 1.0),
    ([-128.0], 2.0),
    ([0.0, 0.0], 2.0**-132),
    ([float("nan"), 1.0], 1.0),
    ([float("inf"), 1.0], float("inf")),
    ([2.0**-127], 2.0**-133),
    ([2.0**-128], 1.0),  # 2**-134 rounds to zero in bfloat16, then becomes 1
    ([3.0e38], 2.0**121),
])
def test_pot_scale_cases(block, expect):
    x = torch.tensor(block + [0.0] * (16 - len(block)), dtype=torch.bfloat16).view(1, 16)
    s = O.calculate_mx_qparam(x, [-1], 16, 127.0, True)
    assert s.item() == expect or (math.isinf(expect) and math.isinf(s.item()))


def test_quantize_mx_int8_against_float64():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(64, 256, generator=g)
    x = torch.where(torch.rand(64, 256, generator=g) < 0.01, x * 20, x).bfloat16()
    table = T.quantization_map("int8")
    s, c = O.quantize_mx(x, table, [-1], 16, 127.0, True)
    xf = x.double().numpy().reshape(64, 16, 16)
    amax = np.abs(xf).max(axis=2)
    e = np.floor(np.log2(np.where(amax == 0, 2.0**-126, amax))) - 6
    sc = 2.0**e
    np.testing.assert_array_equal(s.double().numpy(), sc)
    q = xf / sc[:, :, None]
    codes = np.clip(np.round(q), -128, 127).reshape(64, 256)
    np.testing.assert_array_equal(c.double().numpy(), codes)
    # dequantize(quantize(x)) is the fake-quant round trip
    dq = O.dequantize_mx(c, s, 16)
    np.testing.assert_array_equal(dq.double().numpy(), (codes.reshape(64, 16, 16) * sc[:, :, None]).reshape(64, 256))


def test_quantize_mx_nf4_against_pinned_tables():
    g = torch.Generator().manual_seed(1)
    x = (torch.randn(8, 256, generator=g) * 0.02).bfloat16()
    vt = T.quantization_map("lut4_to_int6")
    index, entries, mid = T.codebook_index_table(vt)
    stab = T.quantization_map("fp8_e5m3")
    s, c = O.quantize_mx(x, index, [-1], 64, 31.0, False, stab, mid)
    # scale: e5m3 grid value nearest bf16(amax / 31)
    f = Q.float_format("fp8_e5m3")
    grid = _grid(f.ebits, f.mbits, f.max_norm)
    amax = x.float().abs().view(8, 4, 64).amax(-1)
    ratio = (amax / 31).bfloat16().double().numpy()
    sc = _nearest_even(ratio, grid)
    sc = np.where(sc > 0, sc, 1.0)
    np.testing.assert_array_equal(s.double().numpy(), sc)
    levels = np.array([-31, -22, -16, -12, -9, -6, -3, 0, 2, 5, 8, 10, 14, 17, 22, 31], dtype=np.float64)
    q = (x.float().view(8, 4, 64) / torch.from_numpy(sc).float()[:, :, None]).bfloat16().double().numpy()
    q = np.clip(q, -31, 31)
    idx = np.argmin(np.abs(q[..., None] - levels), axis=-1).reshape(8, 256)
    np.testing.assert_array_equal(c.double().numpy(), idx)


def test_quantize_affine_hand_cases():
    tab = T.quantization_map("uint2")
    x = torch.tensor([[0.0, 1.0, 2.0, 3.0], [-1.0, 1.0, 0.0, 0.5]], dtype=torch.bfloat16)
    s, z, v = O.quantize_affine(x, tab, [-1], 4, 0.0, 3.0)
    assert s.view(-1).tolist() == [1.0, pytest.approx(2 / 3, rel=1e-2)]
    assert z.view(-1)[0].item() == 0.0
    assert v[0].tolist() == [0.0, 1.0, 2.0, 3.0]
    # row 2: scale = bf16(2/3); zp = 1/scale; codes = round(x/scale + zp)
    sc = torch.tensor(2 / 3).bfloat16().item()
    zp = torch.tensor(1 / sc).bfloat16().item()
    exp = [min(3, max(0, round(torch.tensor(torch.tensor(xx / sc).bfloat16().item() + zp).bfloat16().item())))
           for xx in [-1.0, 1.0, 0.0, 0.5]]
    assert v[1].tolist() == exp
    # A constant block: scale 1, zero point -min + qmin
    c = torch.full((1, 4), 2.5, dtype=torch.bfloat16)
    s, z, v = O.quantize_affine(c, tab, [-1], 4, 0.0, 3.0)
    assert s.item() == 1.0 and z.item() == -2.5 and v.view(-1).tolist() == [0.0] * 4


def test_linear_mx_against_float64_matmul():
    g = torch.Generator().manual_seed(2)
    x = torch.randn(32, 128, generator=g).bfloat16()
    w = (torch.randn(48, 128, generator=g) * 0.02).bfloat16()
    t = T.quantization_map("int8")
    sx, cx = O.quantize_mx(x, t, [-1], 16, 127.0, True)
    sw, cw = O.quantize_mx(w, t, [-1], 16, 127.0, True)
    y = O.linear_mx(cx, cw, input_scale=sx, weight_scale=sw, block_size=16)
    xd = (cx.double().view(32, 8, 16) * sx.double()[:, :, None]).view(32, 128).numpy()
    wd = (cw.double().view(48, 8, 16) * sw.double()[:, :, None]).view(48, 128).numpy()
    ref = xd @ wd.T
    err = np.abs(y.double().numpy() - ref).max() / np.abs(ref).max()
    assert y.dtype == torch.bfloat16 and err < 1e-2


# ------------------------------------------------------------ decoder layer
def _hf_layer(cfg, weights):
    from transformers import LlamaConfig
    from transformers.models.llama.modeling_llama import LlamaDecoderLayer, LlamaRotaryEmbedding

    hc = LlamaConfig(hidden_size=cfg.hidden, num_attention_heads=cfg.n_heads, num_key_value_heads=cfg.n_kv_heads,
                     head_dim=cfg.head_dim, intermediate_size=cfg.intermediate, rope_theta=cfg.rope_theta,
                     rms_norm_eps=cfg.eps, max_position_embeddings=4096)
    hc._attn_implementation = "eager"
    layer = LlamaDecoderLayer(hc, layer_idx=0).to(torch.bfloat16).eval()
    names = {"input_layernorm.weight": "ln1", "post_attention_layernorm.weight": "ln2",
             "self_attn.q_proj.weight": "wq", "self_attn.k_proj.weight": "wk", "self_attn.v_proj.weight": "wv",
             "self_attn.o_proj.weight": "wo", "mlp.gate_proj.weight": "wg", "mlp.up_proj.weight": "wu",
             "mlp.down_proj.weight": "wd"}
    state = {k: weights[v] for k, v in names.items()}
    layer.load_state_dict(state, strict=True)
    return layer, LlamaRotaryEmbedding(hc)


def test_decode_layer_matches_transformers():
    """With plain bf16 linears and an unquantized cache, the oracle's decode
    step is transformers' LlamaDecoderLayer (eager attention, default RoPE)
    bit for bit -- the reference's pinned dependency (pyproject.toml:37)."""
    from transformers.cache_utils import DynamicCache

    from oracle import decode as D

    cfg = D.Config(hidden=256, n_heads=8, n_kv_heads=2, head_dim=32, intermediate=512)
    w = D.random_layer(cfg, seed=3)
    layer, rotary = _hf_layer(cfg, w)
    g = torch.Generator().manual_seed(4)
    B, T = 3, 45
    x = torch.randn(B, cfg.hidden, generator=g).bfloat16()
    k_past = torch.randn(B, cfg.n_kv_heads, T, cfg.head_dim, generator=g).bfloat16()
    v_past = torch.randn(B, cfg.n_kv_heads, T, cfg.head_dim, generator=g).bfloat16()
    cos, sin = D.rope_cos_sin(torch.tensor([T]), cfg.head_dim, cfg.rope_theta)
    ours = D.decode_layer(x, w, k_past, v_past, cos, sin, cfg)["out"]
    pos = torch.full((B, 1), T, dtype=torch.long)
    pe = rotary(x[:, None, :], pos)
    assert torch.equal(pe[0][0, 0], cos[0]) and torch.equal(pe[1][0, 0], sin[0])
    cache = DynamicCache()
    cache.update(k_past.clone(), v_past.clone(), 0)
    with torch.no_grad():
        ref = layer(x[:, None, :], attention_mask=None, position_ids=pos, past_key_values=cache, use_cache=True,
                    position_embeddings=pe)
    ref = ref[0] if isinstance(ref, tuple) else ref
    assert torch.equal(ours, ref.reshape(B, cfg.hidden))


def test_kivi_round_trip_float64():
    """quantize_affine + dequantize with the KIVI spec (uint2, group 32,
    fp16 scale / zero point) against the affine formula in float64: codes are
    round-half-even((x - min) / s) clamped to [0, 3] with s = fp16((max - min) / 3)
    and zp = fp16(-min / s), and the round trip is (code - zp) * s."""
    import numpy as np

    from oracle import decode as D

    g = torch.Generator().manual_seed(5)
    x = (torch.randn(2, 3, 64, 64, generator=g) * 2).bfloat16()
    for axis in (-2, -1):
        s, z, c = D.kivi_quantize(x, axis)
        xr = x.float().numpy()
        if axis == -2:
            blk = xr.reshape(2, 3, 2, 32, 64)
            lo, hi = blk.min(axis=3), blk.max(axis=3)
            rep = lambda a: np.repeat(a, 32, axis=2)
        else:
            blk = xr.reshape(2, 3, 64, 2, 32)
            lo, hi = blk.min(axis=4), blk.max(axis=4)
            rep = lambda a: np.repeat(a, 32, axis=3)
        bf = lambda a: torch.from_numpy(np.asarray(a, dtype=np.float32)).bfloat16().float().numpy()
        sc = bf(bf(hi - lo) / 3.0)
        sc = np.where(sc > 0, sc, 1.0).astype(np.float32)
        sc = bf(sc.astype(np.float16).astype(np.float32))
        zp = bf(bf(bf(-lo) / sc))
        zp = bf(zp.astype(np.float16).astype(np.float32))
        assert np.array_equal(s.float().numpy(), sc)
        assert np.array_equal(z.float().numpy(), zp)
        q = bf(bf(xr / rep(sc)) + rep(zp))
        codes = np.clip(np.round(q), 0, 3)
        assert np.array_equal(c.float().numpy(), codes)
        deq = D.kivi_dequantize(c, s, z, axis).double().numpy()
        ref = bf(bf(codes - rep(zp)) * rep(sc))
        assert np.allclose(deq, ref, rtol=0, atol=0)


def test_nvfp4_global_scale_round_trip():
    """The NVFP4 branch of quantize_mx / dequantize_mx (a 0-d global scale
    divided out of the block scale before its E4M3 map and multiplied back
    into the elements' divisor and into the dequantized values), pinned by
    what the two-level scheme guarantees rather than by its formula: with a
    global scale far from 1, the returned block scales lie on the E4M3 grid
    and near amax / 6 / gs, every code lies on the E2M1 grid, and the round
    trip recovers each element to within half an E2M1 step at that block's
    scale (or saturates at 6 steps) -- dropping gs from the divisor, from the
    scale or from the dequantize misses all of these by the factor gs."""
    g = torch.Generator().manual_seed(41)
    x = (torch.randn(32, 128, generator=g) * torch.exp(torch.randn(32, 1, generator=g) * 2) * 5e4).bfloat16()
    fp4, e4m3 = T.quantization_map("fp4_e2m1"), T.quantization_map("fp8_e4m3")
    gs = (x.float().abs().amax() / (6.0 * 448.0)).to(torch.float32)
    assert gs > 10.0  # far from 1
    scale, codes = O.quantize_mx(x, fp4, [-1], 16, 6.0, False, e4m3, None, None, gs)
    grid4 = {v * s for v in (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0) for s in (1.0, -1.0)}
    assert set(codes.float().unique().tolist()) <= grid4
    e4 = set(e4m3.float().unique().tolist())
    assert set(scale.float().unique().tolist()) <= e4
    xb = x.float().view(32, 8, 16)
    amax = xb.abs().amax(-1)
    s = scale.float()
    # the E4M3 rounding of amax / 6 / gs (relative step 2**-3; subnormal scales excluded)
    ref = amax / 6.0 / gs
    big = ref > 2.0**-6
    assert torch.all((s[big] - ref[big]).abs() <= ref[big] * 2.0**-3)
    back = O.dequantize_mx(codes, scale, 16, None, gs).float().view(32, 8, 16)
    step = s.unsqueeze(-1) * gs  # one unit of E2M1 at this block's scale
    err = (back - xb).abs()
    # nearest E2M1 value: within a half of the local gap (gap 2 between 4 and 6), or saturation at 6
    tol = torch.where(xb.abs() > 6 * step, xb.abs() - 6 * step, step) + step * 2.0**-6
    assert torch.all(err[big.unsqueeze(-1).expand_as(err)] <= tol[big.unsqueeze(-1).expand_as(tol)])
