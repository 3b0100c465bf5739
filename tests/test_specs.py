"""``formats.parse_spec`` / ``quant_min_max`` (``quantization/qspec.py:87-273``)
on the spec strings the reference's configs and tests use.

The implied ranges are pinned by what the formats fix, not by the code:
int8 spans [-128, 127], uint2 [0, 3], E4M3 tops out at 448 and E5M2 at
57344, the OCP FP4 E2M1 grid at 6, posit8 with es = 1 at
useed**(n - 2) = 4**6, and a LUT takes its entries' range (int6: 31)."""

import pytest

from voyager_amd import formats


@pytest.mark.parametrize("dtype, lo, hi", [
    ("int8", -128, 127), ("int6", -32, 31), ("uint2", 0, 3), ("uint4", 0, 15), ("int1", -1, 0),
    ("fp8_e4m3", -448.0, 448.0), ("fp8_e5m2", -57344.0, 57344.0), ("fp4_e2m1", -6.0, 6.0),
    ("posit8_1", -4096, 4096), ("lut4_to_int6", -31, 31), ("lut4", -1, 1),
])
def test_quant_min_max(dtype, lo, hi):
    assert formats.quant_min_max(dtype) == (lo, hi)


def test_parse_spec_fields_and_implied_range():
    sp = formats.parse_spec("int8,qs=microscaling,bs=16,pot=1")
    assert sp == {"dtype": "int8", "qscheme": "microscaling", "block_size": 16, "power_2_scale": True,
                  "quant_min": -128.0, "quant_max": 127.0}
    sp = formats.parse_spec("lut4_to_int6,qs=microscaling,bs=64,scale=fp8_e5m3")
    assert (sp["quant_max"], sp["scale_dtype"], sp["block_size"]) == (31.0, "fp8_e5m3", 64)
    # an explicit bound wins over the implied one; the symmetric schemes get a history length
    sp = formats.parse_spec("fp8_e4m3,qs=microscaling,bs=32,pot=1,qmax=240")
    assert sp["quant_max"] == 240.0 and sp["quant_min"] == -448.0
    assert formats.parse_spec("fp8_e4m3,qs=per_tensor_symmetric")["amax_history_len"] == 64
    assert formats.parse_spec("fp8_e5m2,qs=per_tensor_symmetric,ahl=16")["amax_history_len"] == 16
    # tuples inside parentheses stay one field
    sp = formats.parse_spec("int6,qs=microscaling,bs=32,ax=(-2,-1),scale=fp8_e5m3")
    assert sp["ch_axis"] == (-2, -1) and sp["block_size"] == 32
    sp = formats.parse_spec("uint2,qs=group_wise_affine,bs=32,ax=-2,scale=fp16_e5m10")
    assert (sp["quant_min"], sp["quant_max"], sp["ch_axis"]) == (0.0, 3.0, -2)
    # no qscheme: nothing implied
    assert formats.parse_spec("fp8_e4m3") == {"dtype": "fp8_e4m3"}


@pytest.mark.parametrize("bad", ["", "int8,qs", "int8,foo=1", "int8,qs=per_block", "int8,pot=2"])
def test_parse_spec_rejects(bad):
    with pytest.raises(ValueError):
        formats.parse_spec(bad)
