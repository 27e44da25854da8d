"""Static per-tensor KV quantisation, the fp8 producer in front of RPA
(reference src/vllm_torchtpu/layers/core/quantization.py:73-103)."""

from __future__ import annotations

import torch


def static_per_tensor_quantize_tensor(tensor: torch.Tensor, quant_dtype: torch.dtype,
                                      scale: float) -> torch.Tensor:
    """clamp(x.f32 / scale, finfo.min, finfo.max).to(quant_dtype) (quantization.py:73-88)."""
    if scale == 0.0:
        raise ValueError("Quantization scale must be non-zero.")
    info = (torch.finfo(quant_dtype) if quant_dtype.is_floating_point
            else torch.iinfo(quant_dtype))
    return torch.clamp(tensor.to(torch.float32) / scale, info.min, info.max).to(quant_dtype)


def quantize_kv(quant_dtype: torch.dtype, key: torch.Tensor, value: torch.Tensor | None = None,
                k_scale: float = 1.0, v_scale: float = 1.0):
    """Quantise key (and value) with per-tensor scales (quantization.py:91-103)."""
    key = static_per_tensor_quantize_tensor(key, quant_dtype, k_scale)
    if value is None:
        return key, None
    return key, static_per_tensor_quantize_tensor(value, quant_dtype, v_scale)
