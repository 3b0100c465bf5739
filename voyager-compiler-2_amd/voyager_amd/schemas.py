"""Schema strings of the ``quantized_ops`` operators, byte for byte the
reference's (``src/voyager_compiler/ops/quantized.py:147, 449-453, 518-522,
651-658, 596-603, 742-748, 822-832, 958-962, 1070-1075, 1118-1121,
1160-1166, 1218-1222, 1286-1289, 1396-1402, 1493-1497, 1567-1571``;
``ops/layout.py:176-181, 221-228, 294-303``), so graphs the reference's
convert emits resolve against them unchanged.  Importing this module
registers nothing.
"""

import torch

LINEAR_LAYOUT = "xc,kc->xk"
MATMUL_LAYOUT = "xc,ck->xk"

SCHEMAS = {
    "vmap": "vmap(Tensor self, Tensor other) -> Tensor",
    "quantize": (
        "quantize(Tensor input, Tensor scale, Tensor? zero_point=None, "
        "SymInt[]? axes=None, int? block_size=None, Tensor? qmap=None, "
        "Tensor? output_code=None, Tensor? seed=None) -> Tensor"
    ),
    "dequantize": (
        "dequantize(Tensor input, Tensor scale, Tensor? zero_point=None, "
        "SymInt[]? axes=None, int? block_size=None, Tensor? input_qmap=None, "
        "Tensor? output_qmap=None) -> Tensor"
    ),
    "linear_mx": (
        "linear_mx(Tensor input, Tensor weight, Tensor? bias=None, *, "
        "Tensor? input_scale=None, Tensor? weight_scale=None, "
        "int? block_size=None, Tensor? input_code=None, Tensor? weight_code=None, "
        "Tensor? alpha=None, Tensor? A_data=None, Tensor? A_indices=None, "
        f'Tensor? A_indptr=None, str layout="{LINEAR_LAYOUT}", '
        "ScalarType? out_dtype=None) -> Tensor"
    ),
    "matmul_mx": (
        "matmul_mx(Tensor self, Tensor other, *, Tensor? input_scale=None, "
        "Tensor? weight_scale=None, int? block_size=None, Tensor? input_code=None, "
        "Tensor? weight_code=None, Tensor? alpha=None, Tensor? A_data=None, "
        "Tensor? A_indices=None, Tensor? A_indptr=None, "
        f'str layout="{MATMUL_LAYOUT}", ScalarType? out_dtype=None) -> Tensor'
    ),
    "calculate_mx_qparam": (
        "calculate_mx_qparam(Tensor self, SymInt[] axes, int block_size, "
        "float quant_max, bool force_scale_power_of_two=False, "
        "Tensor scale_qmap=None, Tensor? global_scale=None) -> Tensor"
    ),
    "quantize_mx": (
        "quantize_mx(Tensor self, Tensor qmap, SymInt[] axes, int block_size, "
        "float quant_max, bool force_scale_power_of_two=False, "
        "Tensor scale_qmap=None, Tensor output_code=None, Tensor? seed=None, "
        "Tensor? global_scale=None) -> (Tensor, Tensor)"
    ),
    "dequantize_mx": (
        "dequantize_mx(Tensor self, Tensor scale, int block_size, "
        "Tensor? code=None, Tensor? global_scale=None) -> Tensor"
    ),
    "quantize_affine": (
        "quantize_affine(Tensor self, Tensor qmap, SymInt[] axes, int block_size, "
        "float quant_min, float quant_max, Tensor scale_qmap=None) "
        "-> (Tensor, Tensor, Tensor)"
    ),
    "linear": (
        "linear(Tensor input, Tensor weight, Tensor? bias=None, *, "
        f'str layout="{LINEAR_LAYOUT}", ScalarType? out_dtype=None) -> Tensor'
    ),
    "matmul": (
        f'matmul(Tensor self, Tensor other, *, str layout="{MATMUL_LAYOUT}", '
        "ScalarType? out_dtype=None) -> Tensor"
    ),
    "conv2d": (
        "conv2d(Tensor input, Tensor weight, Tensor? bias=None, "
        "SymInt[2] stride=[1, 1], SymInt[2] padding=[0, 0], "
        "SymInt[2] dilation=[1, 1], SymInt groups=1, *, "
        'str layout="nchw", ScalarType? out_dtype=None) '
        "-> Tensor"
    ),
    "conv2d_mx": (
        "conv2d_mx(Tensor input, Tensor weight, Tensor? bias=None, "
        "SymInt[2] stride=1, SymInt[2] padding=0, SymInt[2] dilation=1, "
        "SymInt groups=1, *, Tensor? input_scale=None, Tensor? weight_scale=None, "
        "int? block_size=None, Tensor? input_code=None, "
        'Tensor? weight_code=None, str layout="nchw", '
        "ScalarType? out_dtype=None) -> Tensor"
    ),
    "filter_outlier": (
        "filter_outlier(Tensor input, float threshold, float max_pct=0.01) "
        "-> (Tensor, Tensor, Tensor, Tensor)"
    ),
    "quantize_mx_outlier": (
        "quantize_mx_outlier(Tensor self, Tensor qmap, SymInt[] axes, "
        "int block_size, float quant_max, bool force_scale_power_of_two=False, "
        "Tensor scale_qmap=None, Tensor output_code=None, float? threshold=None, "
        "float max_pct=0.01, SymInt indptr_offset=0) "
        "-> (Tensor, Tensor, Tensor, Tensor, Tensor)"
    ),
    "slice_csr_tensor": (
        "slice_csr_tensor(Tensor data, Tensor indices, Tensor indptr, int dim=0, "
        "SymInt? start=None, SymInt? end=None, float size_factor=1.0) "
        "-> (Tensor, Tensor, Tensor)"
    ),
    "spmm_csr": (
        "spmm_csr(Tensor data, Tensor indices, Tensor indptr, Tensor B, "
        "Tensor? B_scale=None, Tensor? B_code=None, int? block_size=None, "
        'str weight_layout="kc", *, ScalarType? out_dtype=None) -> Tensor'
    ),
}

# Ops the package registers as torch restatements (no HIP kernel of their
# own beyond the quantized ops they call), so converted graphs that use them
# load and run on the GPU.
TWIN_SCHEMAS = {
    "sdpa_mx": (
        "sdpa_mx(Tensor query, Tensor key, Tensor value, Tensor? attn_mask=None, "
        "float dropout_p=0., bool is_causal=False, Tensor? query_residual=None, "
        "Tensor? key_residual=None, Tensor? value_residual=None, "
        "Tensor? residual_mask=None, *, float? scale=None, "
        "bool enable_gqa=False, Tensor? query_scale=None, Tensor? key_scale=None, "
        "Tensor? value_scale=None, int? block_size=None, Tensor? input_code=None, "
        "Tensor? weight_code=None, Tensor? probs_qmap=None, "
        "float? probs_quant_max=None, Tensor? probs_scale_qmap=None, "
        "Tensor? probs_code=None, bool force_scale_power_of_two=False) -> Tensor"
    ),
    "quantize_mx_transpose": (
        "quantize_mx_transpose(Tensor self, Tensor qmap, int block_size, "
        "float quant_max, bool force_scale_power_of_two=False, "
        "Tensor scale_qmap=None, Tensor output_code=None, Tensor? seed=None, "
        "Tensor? global_scale=None, Tensor? transpose_seed=None, "
        "Tensor? transpose_global_scale=None, Tensor? hadamard=None) "
        "-> (Tensor, Tensor, Tensor, Tensor)"
    ),
    "sdpa_kmajor": (
        "sdpa_kmajor(Tensor query, Tensor key, Tensor value, "
        "Tensor? attn_mask=None, float dropout_p=0.0, bool is_causal=False, *, "
        "float? scale=None, bool enable_gqa=False, bool transpose_output=False) "
        "-> Tensor"
    ),
    "rms_norm_kmajor": "rms_norm_kmajor(Tensor input, Tensor? weight=None, float? eps=None) -> Tensor",
}

#: The aten pools whose NHWC twins join the namespace under aten's own name
#: and schema (``ops/layout.py:127-168``).
NHWC_POOLS = (
    torch.ops.aten.max_pool2d.default,
    torch.ops.aten.avg_pool2d.default,
    torch.ops.aten.adaptive_avg_pool2d.default,
    torch.ops.aten._adaptive_avg_pool2d.default,
)


def pool_schema(aten_op) -> str:
    """The twin's schema: aten's, without the namespace."""
    return str(aten_op._schema).split("::", 1)[1]


def all_schemas():
    """Every schema the standalone namespace defines, in definition order."""
    out = dict(SCHEMAS)
    out.update(TWIN_SCHEMAS)
    for op in NHWC_POOLS:
        out[op._schema.name.split("::")[1]] = pool_schema(op)
    return out
