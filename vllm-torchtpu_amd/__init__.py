"""MI355X-native Ragged Paged Attention for the vllm-torchtpu attention path.

Public API mirrors src/vllm_torchtpu/kernels/ragged_paged_attention/v3/kernel.py
of the reference; the compute is the gfx950 HIP library librpa_hip.so.
"""

from .quantization import quantize_kv, static_per_tensor_quantize_tensor
from .rpa import (
    RpaCase,
    dynamic_validate_inputs,
    get_kv_cache_shape,
    merge_attn_results,
    merge_attn_states,
    merge_kv,
    ragged_paged_attention,
    ragged_paged_attention_bundled,
    rpa_kv_cache_update,
    static_validate_inputs,
)
from .rpa_hd64 import (
    dynamic_validate_inputs_hd64,
    get_kv_cache_shape_hd64,
    merge_kv_hd64,
    ragged_paged_attention_hd64,
    static_validate_inputs_hd64,
)
from .util import align_to, cdiv, get_dtype_packing, next_power_of_2

__all__ = [
    "RpaCase",
    "align_to",
    "cdiv",
    "dynamic_validate_inputs",
    "dynamic_validate_inputs_hd64",
    "get_dtype_packing",
    "get_kv_cache_shape",
    "get_kv_cache_shape_hd64",
    "merge_attn_results",
    "merge_attn_states",
    "merge_kv",
    "merge_kv_hd64",
    "next_power_of_2",
    "quantize_kv",
    "ragged_paged_attention",
    "ragged_paged_attention_bundled",
    "ragged_paged_attention_hd64",
    "rpa_kv_cache_update",
    "static_per_tensor_quantize_tensor",
    "static_validate_inputs",
    "static_validate_inputs_hd64",
]
