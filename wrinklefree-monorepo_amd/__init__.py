"""MI355X-native (gfx950) ternary BitLinear hot path: I2_S W2A8 pack, fused RMSNorm + int8 quant,
decode GEMV and int8-MFMA prefill GEMM behind a C ABI (include/wfbitnet.h).

The directory name is not a Python identifier; entry points load it under the module name
``wrinklefree_monorepo_amd`` (see ``__graft_entry__.load_package``).
"""

from ._lib import LIB_PATH, available as library_available
from .ops import (
    QK_I2_S,
    absmean_scale,
    bitnet_gemm,
    bitnet_gemv,
    bitnet_linear,
    bitnet_linear_argmax,
    bitnet_linear_glu,
    bitnet_linear_residual,
    bitnet_linear_segmented,
    bitnet_mlp_forward,
    bitnet_qkv_forward,
    check_kernel_available,
    convert_hf_offline_i2s,
    glu_rmsnorm_quantize_i8,
    gqa_decode_attention,
    gqa_prefill_attention,
    lm_head_argmax,
    pack_ternary_i2s,
    quantize_activations_i8,
    quantize_activations_i8_per_token,
    rmsnorm_linear,
    rmsnorm_linear_glu,
    rmsnorm_linear_glu_supported,
    rmsnorm_linear_preferred,
    rmsnorm_linear_supported,
    rmsnorm_quantize_i8,
    rope_tables,
    unpack_i2s,
)
from . import engine, model, sglbitnt
from .engine import NativeEngine
from .sglbitnt import SGLBitNetFile, write_sglbitnt
from .bitlinear import (
    BitLinear,
    BitNetLinearMethod,
    BitNetLinearNative,
    SubLNBitLinear,
    convert_linear_to_bitlinear,
    patch_model_with_native_kernels,
    set_lambda_source,
)

__all__ = [
    "LIB_PATH", "library_available", "QK_I2_S", "absmean_scale", "bitnet_gemm", "bitnet_gemv", "bitnet_linear",
    "bitnet_linear_argmax", "bitnet_linear_glu", "bitnet_linear_residual", "bitnet_linear_segmented", "bitnet_mlp_forward", "bitnet_qkv_forward", "check_kernel_available", "convert_hf_offline_i2s",
    "glu_rmsnorm_quantize_i8", "gqa_decode_attention", "gqa_prefill_attention", "lm_head_argmax", "pack_ternary_i2s",
    "quantize_activations_i8", "quantize_activations_i8_per_token", "rmsnorm_linear", "rmsnorm_linear_glu", "rmsnorm_linear_glu_supported", "rmsnorm_linear_preferred", "rmsnorm_linear_supported",
    "rmsnorm_quantize_i8", "rope_tables", "unpack_i2s",
    "BitLinear", "BitNetLinearMethod", "BitNetLinearNative", "SubLNBitLinear", "convert_linear_to_bitlinear",
    "patch_model_with_native_kernels", "set_lambda_source", "engine", "NativeEngine", "model", "sglbitnt", "SGLBitNetFile", "write_sglbitnt",
]
