"""Shared test helpers."""

import torch


def assert_same_bits(got: torch.Tensor, exp: torch.Tensor, what: str = ""):
    """Bit-identical tensors, any NaN matching any NaN (the reference's NaN
    payloads depend on which of its CPU code paths produced them)."""
    got = got.detach().cpu()
    exp = exp.detach().cpu()
    assert got.dtype == exp.dtype, f"{what}: dtype {got.dtype} != {exp.dtype}"
    assert list(got.shape) == list(exp.shape), f"{what}: shape {list(got.shape)} != {list(exp.shape)}"
    if got.dtype.is_floating_point:
        ib = {2: torch.int16, 4: torch.int32, 8: torch.int64}[got.element_size()]
        same = (got.contiguous().view(ib) == exp.contiguous().view(ib)) | (torch.isnan(got) & torch.isnan(exp))
    else:
        same = got == exp
    if not bool(same.all()):
        bad = (~same).nonzero()
        i = tuple(bad[0].tolist())
        raise AssertionError(f"{what}: {bad.shape[0]} of {same.numel()} elements differ; first at {i}: "
                             f"got {got[i].item()!r} expected {exp[i].item()!r}")


def max_rel_err(got: torch.Tensor, ref: torch.Tensor) -> float:
    """max |got - ref| / max |ref| (the reference's GEMM check metric,
    backend/gpu/__init__.py:372-376)."""
    g = got.detach().double().cpu()
    r = ref.detach().double().cpu()
    return float((g - r).abs().max() / r.abs().max().clamp_min(1e-30))


def assert_within_bf16_ulps(got, ref64, ulps=1.0, atol=None, what=""):
    """Each bf16 element of ``got`` within ``ulps`` bf16 ulps of the float64
    reference ``ref64`` (the ulp of |ref| in bf16), plus ``atol`` (a tensor or
    scalar: the float32 accumulation error allowance where terms cancel)."""
    g = got.detach().cpu().double()
    r = ref64.detach().cpu().double()
    mag = r.abs().clamp_min(2.0**-126)
    ulp = torch.pow(2.0, torch.floor(torch.log2(mag)) - 7)
    lim = ulps * ulp + (0.0 if atol is None else atol)
    bad = (g - r).abs() > lim
    assert not bool(bad.any()), f"{what}: {int(bad.sum())} elements beyond {ulps} bf16 ulp(s)"
