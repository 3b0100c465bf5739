"""CPU oracle for the quantized-operator path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU with eager PyTorch ops, the algorithm of the
reference's ``quantized_ops`` operators (``src/voyager_compiler/ops/quantized.py``,
``ops/layout.py``, ``quantization/mx_utils.py``, ``quantization/qspec.py``,
``quantization/dtypes/*.py`` and ``quantization/fake_quantize.py:68-160``).
Each function cites the reference lines it follows.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it, and only as the checker (or the timed CPU
baseline).  The product package (``voyager_amd``) never imports it: its ops
run only through the HIP library and raise when that library is missing.

Parity pins (each checked in ``tests/test_oracle_pins.py``):

* tables (``tables.py``): int tables against round-half-even + clip in
  numpy; minifloat tables against an exhaustive nearest-value search over the
  format's enumerated grid in float64 and, for ``fp8_e4m3`` and
  ``fp16_e5m10``, against torch's own ``float8_e4m3fn`` / ``float16`` casts;
  posit8 against a textbook posit decoder with rounding in the encoding domain
  (plus the reference's documented flush below ``2**-13``); NormalFloat levels
  against the published QLoRA NF4 constants; ``lut4_to_int6`` index tables
  against nearest-level search in exact arithmetic with ties to the lower
  index.
* ``calculate_mx_qparam`` / ``quantize_mx``: the shared exponent against the
  bf16 exponent field, scales against closed forms, hand-computed blocks
  (all-zero, NaN, Inf, tiny) and the invariant that dequantizing the codes
  equals the fake-quant round trip computed independently in float64.
* ``quantize_affine``: hand-computed blocks and a float64 restatement.
* GEMMs (``linear``/``linear_mx``/``matmul_mx``): float64 numpy matmul of
  the decoded operands.
* Outliers (``filter_outlier``, ``quantize_mx_outlier``, ``slice_csr_tensor``,
  ``spmm_csr`` and the CSR term of ``linear_mx``/``matmul_mx``; checked in
  ``tests/test_oracle_outliers.py``): the CSR against a brute-force
  row-major scan in plain Python (slot order, capacity cut, row-pointer
  clamp, padding), dense reconstruction (CSR + inliers == input), the
  threshold compared after rounding to the input dtype, slices against
  slices of the dense matrix, and the products against float64 numpy
  matmul of the densified CSR.
"""
