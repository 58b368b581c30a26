"""MI355X-native quantized linear path of Viper (gfx950 HIP kernels behind a C ABI).

Compute goes through ``viper_amd/lib/libviper_qlinear.so`` (include/viper_qlinear.h);
there is no CPU fallback.
"""
from .qlinear import (GROUP, MAX_M, Prologue, QType, QuantizedWeight, ScaleEnc, Status, StatusCode,  # noqa: F401
                      check_quantizer, is_lossless, lib, linear, linear_fused2, linear_fused2_prequantized, linear_m1,
                      linear_m1_swiglu, linear_partials, linear_prequantized, packed_bytes, qtype_name, quantize_act,
                      linear_bf16, rmsnorm_quantize, sampling_greedy, greedy_workspace_bytes, swiglu_quantize,
                      workspace_bytes, workspace_layout, frag_bytes, rmsnorm_quantize_frag, swiglu_quantize_frag,
                      linear_prequantized_frag, linear_fused2_prequantized_frag, frag_workspace_bytes)
