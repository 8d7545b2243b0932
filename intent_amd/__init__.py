"""intent_amd — MI355X-native (gfx950) quantized-contraction hot path of IntentDSL.

Operator surface (same names and behaviour as the reference's
``intent.compile`` / ``CompiledArtifact``):

    import intent_amd as intent
    art = intent.compile(intent.weight_only_int4_asym_matmul, target=intent.MI355XTarget())
    y = art.run(x, packed, scales, zeros)          # allocates the Out buffer
    art(x, packed, scales, zeros, y)               # explicit outputs
    op = art.as_torch_op("mylib::w4a16")           # torch custom op

Every definition is backed by hand-written HIP kernels in
``intent_amd/_lib/libintent_amd.so`` (C ABI: ``include/intent_amd.h``).
"""
from .artifact import CompiledArtifact
from .compiler import CompileOptions, MI355XTarget, compile
from .definitions import (
    ALL_DEFINITIONS,
    KernelDefinition,
    bitnet_int2_matmul,
    block_scaled_matmul,
    scaled_fp8_matmul,
    scaled_fp8_splitk_matmul,
    deepgemm_fp8_2xacc,
    fp8_e4m3_matmul,
    fp8_e5m2_matmul,
    dequant_bf16_fp4_matmul,
    weight_only_int4_matmul,
    quantized_gemm,
    gemm,
    bf16_gemm,
    nvfp4_quantize,
    ragged_grouped_gemm,
    ragged_grouped_gemm_bf16,
    routed_expert_projection_bf16,
    bf16_groupwise_fp8_quantize,
    f32_groupwise_fp8_quantize,
    per_token_int8_quantize,
    bf16_per_token_int8_quantize,
    gemm_i8,
    gemm_i8_nt,
    moe_align_block_size,
    moe_combine,
    moe_down_w4,
    moe_expert_ffn,
    moe_expert_ffn_w4,
    moe_gate_up_w4,
    moe_route_topk,
    q4_k_q8_k_dot,
    q8_k_quantize,
    quantized_projection,
    w4a8_packed_matmul,
    w8a8_scaled_matmul,
    weight_only_int4_asym_matmul,
    weight_only_int8_matmul,
)
from .errors import CompilationStageError, LanguageUseError, NativeLibraryError
from .interface import DType, PublicInterface, ScalarParameter, ViewKind, ViewParameter


def kernel(function=None):
    """The reference's ``@intent.kernel`` compiles arbitrary DSL functions; this
    build only ships the fixed quantized-contraction definitions."""
    raise NotImplementedError("intent_amd compiles only its fixed quantized-contraction definitions "
                              f"({', '.join(d.name for d in ALL_DEFINITIONS)})")


__all__ = [
    "ALL_DEFINITIONS", "CompilationStageError", "bitnet_int2_matmul", "block_scaled_matmul", "scaled_fp8_matmul", "scaled_fp8_splitk_matmul", "deepgemm_fp8_2xacc", "fp8_e4m3_matmul", "fp8_e5m2_matmul", "dequant_bf16_fp4_matmul", "weight_only_int4_matmul", "quantized_gemm", "gemm", "bf16_gemm", "nvfp4_quantize", "ragged_grouped_gemm", "ragged_grouped_gemm_bf16", "routed_expert_projection_bf16", "gemm_i8", "w4a8_packed_matmul", "bf16_groupwise_fp8_quantize", "f32_groupwise_fp8_quantize", "per_token_int8_quantize", "bf16_per_token_int8_quantize", "CompileOptions", "CompiledArtifact", "DType", "KernelDefinition",
    "LanguageUseError", "MI355XTarget", "NativeLibraryError", "PublicInterface", "ScalarParameter", "ViewKind",
    "ViewParameter", "compile", "gemm_i8_nt", "kernel", "moe_align_block_size", "moe_combine", "moe_down_w4",
    "moe_expert_ffn", "moe_expert_ffn_w4", "moe_gate_up_w4", "moe_route_topk", "q4_k_q8_k_dot", "q8_k_quantize",
    "quantized_projection", "w8a8_scaled_matmul", "weight_only_int4_asym_matmul",
    "weight_only_int8_matmul",
]
