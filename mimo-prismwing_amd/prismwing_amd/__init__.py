"""MI355X (gfx950) block-scaled FP8 projection and routed-MoE path.

Host-side mirror of the reference's WideMetalMoeRuntime (src/wide_metal_moe.rs:113-1315) over the
C ABI of include/pwfp8.h. Names and argument meanings follow the reference: ``compile`` /
``compile_with_fused_gate_up``, ``execute_fp8_linear``, ``execute`` / ``execute_fused_gate_up``,
``WideExpertBinding`` (expert, positions, route_weights, gate, up, down) and the routing helpers
of src/text_endpoint.rs:4342-4473. Errors raise ``PwError`` (the reference returns Err(String)).
"""
from ._abi import (DTYPE_BF16, DTYPE_F32, DTYPE_F32_RAW, FLAG_QUANT_NONFINITE, FLAG_ROUND_NONFINITE, FLAG_ROUTE,
                   FLAG_SCHEDULE, FLAG_SWIGLU_NONFINITE, LAYOUT_FULL_QKV_TP4,
                   LAYOUT_PLAIN, LAYOUT_SWA_QKV_TP4, MODE_A, MODE_B, PwError, lib)
from .runtime import (ExpertBank, Projection, Safetensors, WideExpertBinding, WideLinearExecution,
                      WideMoeExecution, WideMoeRuntime, full_qkv_scale_row, full_qkv_source_row,
                      noaux_routes, route_from_logits, swa_qkv_source_row, topk_unsorted)

__all__ = [
    "DTYPE_BF16", "DTYPE_F32", "DTYPE_F32_RAW", "FLAG_QUANT_NONFINITE", "FLAG_ROUND_NONFINITE", "FLAG_ROUTE",
    "FLAG_SCHEDULE", "FLAG_SWIGLU_NONFINITE", "LAYOUT_FULL_QKV_TP4",
    "LAYOUT_PLAIN", "LAYOUT_SWA_QKV_TP4",
    "MODE_A", "MODE_B", "PwError", "lib", "ExpertBank", "Projection", "Safetensors", "WideExpertBinding",
    "WideLinearExecution", "WideMoeExecution", "WideMoeRuntime", "full_qkv_scale_row",
    "full_qkv_source_row", "noaux_routes", "route_from_logits", "swa_qkv_source_row",
    "topk_unsorted",
]
