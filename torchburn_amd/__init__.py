"""torchburn_amd: TorchBurn's quantized decode hot path, rebuilt for AMD MI355X (gfx950).

The compute lives in libtbhip.so (hand-written HIP kernels behind a C ABI,
include/tbhip.h).  This package is the host-side mirror of the reference's
Python operator API (python/torchburn/quantization.py): same names, argument
meaning and error behaviour.
"""
from ._lib import UnsupportedOpError
from .decoder import RustQwenDecoder, create_rust_qwen_decoder
from .sampling import sample_logits, sample_uniform
from .quantization import (
    QuantizedLinear,
    fused_attention_step,
    fused_attention_step_w4a32,
    fused_attention_step_w8a32,
    fused_transformer_layer_step,
    fused_transformer_layer_step_w4a32,
    fused_swiglu_mlp,
    fused_swiglu_mlp_w4a32,
    fused_swiglu_mlp_batched,
    fused_swiglu_mlp_batched_w4a32,
    fused_swiglu_mlp_w8a32,
    dequantize_int4_grouped_v2,
    pack_rows_w4a32_group64_v1_to_v2,
    quantize_model,
    quantize_weight_int4,
    quantize_weight_int4_grouped,
    quantize_weight_int4_grouped_v2,
    quantize_weight_int8,
    set_vnni_semantics,
    release_stream_workspace,
    unpack_rows_w4a32_group64_v2_to_v1,
    w4a32_grouped_linear,
    w4a32_grouped_linear_residual,
    w4a32_grouped_linear_v2,
    w4a32_linear,
    w8a32_linear,
)
from .decoder import rotary_tables_f32

__all__ = [
    "RustQwenDecoder",
    "create_rust_qwen_decoder",
    "fused_swiglu_mlp_w8a32",
    "w8a32_linear",
    "UnsupportedOpError",
    "QuantizedLinear",
    "fused_attention_step",
    "fused_attention_step_w4a32",
    "fused_attention_step_w8a32",
    "fused_transformer_layer_step",
    "fused_transformer_layer_step_w4a32",
    "fused_swiglu_mlp",
    "fused_swiglu_mlp_w4a32",
    "fused_swiglu_mlp_batched",
    "fused_swiglu_mlp_batched_w4a32",
    "quantize_model",
    "quantize_weight_int4",
    "quantize_weight_int4_grouped",
    "quantize_weight_int8",
    "w4a32_grouped_linear",
    "w4a32_grouped_linear_residual",
    "w4a32_grouped_linear_v2",
    "w4a32_linear",
    "rotary_tables_f32",
    "quantize_weight_int4_grouped_v2",
    "dequantize_int4_grouped_v2",
    "pack_rows_w4a32_group64_v1_to_v2",
    "set_vnni_semantics",
    "release_stream_workspace",
    "unpack_rows_w4a32_group64_v2_to_v1",
    "sample_logits",
    "sample_uniform",
]
