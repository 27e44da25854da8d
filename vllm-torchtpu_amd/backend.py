"""Attention-backend glue: the vLLM-facing layer above ragged_paged_attention.

Mirrors the reference's `PallasAttentionBackend` / `PallasAttentionBackendImpl`
(src/vllm_torchtpu/layers/adapter/attention.py, "attention.py" below) and its
metadata contract (`AttentionMetadata`, layers/core/attention_metadata.py:84-94)
for the RPA path only.  vLLM itself is not a dependency: the classes keep the
reference's names, method signatures, policies and error conditions so a
caller (or a thin registration shim in a vLLM install) can use them as it uses
the reference's, and the compute goes to this package's HIP library.

What is mirrored:
  * cache geometry: `get_kv_cache_shape` (the "auto" placeholder probe,
    attention.py:617-656), `get_kv_cache_page_size_bytes` (:658-677),
    `get_kv_cache_stride_order` (:704-709);
  * page-size policy `get_page_size` (:733-758);
  * the metadata contract: seq_lens, block_tables (flat, max_num_seqs *
    pages_per_seq), query_start_loc, request_distribution;
  * `forward` (attention.py:1464-1698): 2-D or 3-D q/k/v, KV-shared layers
    (no key/value: the cache is read with skip_kv_update), head-dim padding
    into a wider pool page (`kv_page_head_padding`, :215-247), fp8
    quantize-on-write with the layer's k/v scales (:1560-1569), the output
    buffer written in place, the profiling call with an empty cache;
  * the per-configuration kernel registry (`_build_rpa_kernel`, :971-1193): one
    cached callable per (window, scales, skip_kv_update, decode_query_size) so
    a compiled graph reuses it;
  * `decode_query_size` (K + 1 query tokens per decode sequence under
    speculative decoding, :1706-1712), here a constructor keyword.

Two cache layouts, as in the reference (attention.py:617-656): head_size 64
uses the packed layout of ragged_paged_attention_hd64 (K|V of a head in one
128-wide row) and the hd64 kernel, the only one that takes attention sinks
(layers/core/attention_interface.py:418-436); every other head size uses
K and V interleaved per head with head_dim padded to a multiple of 128.

Deliberate differences:
  * `get_max_num_seqs*` report the batch the fused kernels plan in LDS
    (2048 sequences); the reference's figure is a TPU SMEM budget.
  * DCP/PCP sharding and the bundled (block-major) pool are not routed here
    (the bundled cache has its own entry point, `ragged_paged_attention_bundled`).
"""

from __future__ import annotations

import dataclasses
import math
from typing import Any

import torch

from . import rpa as _rpa
from . import rpa_hd64 as _rpa_hd64
from .quantization import quantize_kv
from .util import cdiv, next_power_of_2

# attention.py:144-154 (the entries this backend supports).
STR_DTYPE_TO_TORCH_DTYPE = {
    "half": torch.half,
    "bfloat16": torch.bfloat16,
    "bf16": torch.bfloat16,
    "float": torch.float,
    "fp8": torch.float8_e4m3fn,
    "fp8_e4m3": torch.float8_e4m3fn,
    "fp8_e5m2": torch.float8_e5m2,
}

HEAD_SIZE_ALIGNMENT = 128

# The largest max_num_seqs the decode and prefill kernels plan in LDS.
MAX_PLANNED_SEQS = 2048

DECODER = "decoder"


def is_fp8_kv_cache_dtype(cache_dtype_str: str) -> bool:
    """attention.py:157-158."""
    return cache_dtype_str.lower().strip() in frozenset(("fp8", "fp8_e4m3", "fp8_e5m2"))


def resolve_kv_cache_dtype(cache_dtype: str | torch.dtype) -> torch.dtype:
    """attention.py:161-173: a concrete dtype for a cache dtype string."""
    if isinstance(cache_dtype, torch.dtype):
        return cache_dtype
    normalized = cache_dtype.lower().strip()
    if normalized == "auto":
        raise ValueError(
            "cache_dtype='auto' must be resolved to a concrete torch.dtype "
            "before calling get_kv_cache_shape.")
    dtype = STR_DTYPE_TO_TORCH_DTYPE.get(normalized)
    if dtype is None:
        raise ValueError(f"Unsupported KV cache dtype string: {cache_dtype}")
    return dtype


def kv_page_head_padding(pool_page: tuple[int, ...], native_page: tuple[int, ...],
                         pool_head_dim: int, head_size: int) -> int:
    """attention.py:215-247: zero padding to append to q/k/v so a layer writes
    into a pool page defined by another (wider) attention spec."""
    if pool_page == native_page or pool_head_dim <= head_size:
        return 0
    return pool_head_dim - head_size


@dataclasses.dataclass
class AttentionMetadata:
    """The RPA fields of the reference's AttentionMetadata
    (layers/core/attention_metadata.py:84-94)."""

    input_positions: torch.Tensor | None  # (padded_total_num_scheduled_tokens,)
    block_tables: torch.Tensor | None = None  # (max_num_seqs * max_num_blocks_per_req,)
    seq_lens: torch.Tensor | None = None  # (max_num_seqs,)
    query_start_loc: torch.Tensor | None = None  # (max_num_seqs + 1,)
    request_distribution: torch.Tensor | None = None  # (3,)


class RpaAttentionBackend:
    """Mirror of PallasAttentionBackend (attention.py:599-758)."""

    supported_kv_cache_dtypes = ["auto", "bfloat16", "fp8", "fp8_e4m3", "fp8_e5m2"]

    @staticmethod
    def get_name() -> str:
        return "FLASH_ATTN"

    @staticmethod
    def get_impl_cls() -> type["RpaAttentionBackendImpl"]:
        return RpaAttentionBackendImpl

    @staticmethod
    def get_kv_cache_shape(num_blocks: int, block_size: int, num_kv_heads: int,
                           head_size: int,
                           cache_dtype_str: str | torch.dtype = "auto") -> tuple[int, ...]:
        """[num_blocks, block_size, Kx2 / packing, packing, padded head size],
        Kx2 = num_kv_heads for head_size 64 (K|V packed along the row) and
        2 * num_kv_heads otherwise.  With "auto" (vLLM's offloading probe,
        which only looks for num_blocks at dim 0) the packing is left at 1, as
        the reference does."""
        padded = cdiv(head_size, HEAD_SIZE_ALIGNMENT) * HEAD_SIZE_ALIGNMENT
        use_hd64 = head_size == 64
        if isinstance(cache_dtype_str, str) and cache_dtype_str.lower().strip() == "auto":
            kx2 = num_kv_heads if use_hd64 else 2 * num_kv_heads
            return (num_blocks, block_size, kx2, 1, padded)
        kv_dtype = resolve_kv_cache_dtype(cache_dtype_str)
        if use_hd64:
            return tuple(_rpa_hd64.get_kv_cache_shape_hd64(num_blocks, block_size, num_kv_heads,
                                                           head_size, kv_dtype))
        return tuple(_rpa.get_kv_cache_shape(num_blocks, block_size, num_kv_heads, head_size,
                                             kv_dtype))

    @classmethod
    def get_kv_cache_page_size_bytes(cls, block_size: int, num_kv_heads: int, head_size: int,
                                     cache_dtype_str: str | torch.dtype = "auto") -> int:
        """One cache page in bytes, layout padding included (attention.py:658-677)."""
        dtype = resolve_kv_cache_dtype(cache_dtype_str)
        shape = cls.get_kv_cache_shape(1, block_size, num_kv_heads, head_size, dtype)
        return math.prod(shape) * torch.empty((), dtype=dtype).element_size()

    @staticmethod
    def swap_blocks(src_kv_cache, dst_kv_cache, src_to_dst) -> None:
        raise RuntimeError("swap_blocks is not used by the RPA backend.")

    @staticmethod
    def get_kv_cache_stride_order(include_num_layers_dimension: bool = False) -> tuple[int, ...]:
        if include_num_layers_dimension:
            return (1, 0, 2, 3, 4, 5)
        return (0, 1, 2, 3, 4)

    @staticmethod
    def get_max_num_seqs(model_len: int, page_size: int) -> int:
        return RpaAttentionBackend.get_max_num_seqs_for_pages(cdiv(model_len, page_size))

    @staticmethod
    def get_max_num_seqs_for_pages(pages_per_req: int) -> int:
        if pages_per_req <= 0:
            raise ValueError("pages_per_req must be positive")
        return MAX_PLANNED_SEQS

    @staticmethod
    def get_page_size(max_model_len: int) -> int:
        """attention.py:733-758: 128-token pages past 8192 tokens, else
        max_model_len / 16 rounded to a power of two within [16, 256].  (The
        reference takes a VllmConfig and reads model_config.max_model_len.)"""
        if max_model_len > 8192:
            return 128
        page_size = next_power_of_2(max_model_len) // 16
        if page_size <= 16:
            return 16
        if page_size >= 256:
            return 256
        return page_size


class RpaAttentionBackendImpl:
    """Mirror of PallasAttentionBackendImpl (attention.py:844-1698), RPA path."""

    def __init__(self, num_heads: int, head_size: int, scale: float, num_kv_heads: int,
                 alibi_slopes: list[float] | None, sliding_window: int | None,
                 kv_cache_dtype: str, logits_soft_cap: float | None = None,
                 attn_type: str = DECODER, kv_sharing_target_layer_name: str | None = None,
                 sinks: torch.Tensor | None = None, **kwargs: Any) -> None:
        self.num_heads = num_heads
        self.head_size = head_size
        self.scale = float(scale)
        self.num_kv_heads = num_kv_heads
        self.sliding_window = sliding_window
        self.logits_soft_cap = logits_soft_cap
        self.kv_sharing_target_layer_name = kv_sharing_target_layer_name
        self.use_causal_mask = kwargs.get("use_causal_mask", True)
        # Query tokens of a decode sequence: K + 1 under speculative decoding
        # (the reference reads speculative_config.num_speculative_tokens,
        # attention.py:1706-1712; head_dim 64 keeps 1).
        self.decode_query_size = int(kwargs.get("decode_query_size", 1))
        if head_size == 64:
            self.decode_query_size = 1
        if alibi_slopes is not None:
            raise NotImplementedError("Alibi slopes is not supported.")
        if attn_type != DECODER:
            raise NotImplementedError(
                "Encoder self-attention and encoder/decoder cross-attention are not "
                "implemented for RpaAttentionBackendImpl")
        if sinks is not None:  # attention.py:914-920
            assert sinks.shape[0] == num_heads, (
                "Sinks must have the same number of heads as the number of heads in the layer")
        self.sinks = sinks
        self.kv_cache_quantized_dtype = None
        if is_fp8_kv_cache_dtype(kv_cache_dtype):
            self.kv_cache_quantized_dtype = STR_DTYPE_TO_TORCH_DTYPE[
                kv_cache_dtype.lower().strip()]
        self._kernel_config_cache: dict = {}
        self._shared_kv_zeros: dict = {}

    def process_weights_after_loading(self, act_dtype: torch.dtype) -> None:
        """attention.py:1455-1463: the kernels take f32 sinks."""
        if self.sinks is not None:
            self.sinks = torch.nn.Parameter(self.sinks.to(torch.float32), requires_grad=False)

    def _build_rpa_kernel(self, q_scale: float | None, k_scale: float | None,
                          v_scale: float | None, skip_kv_update: bool = False):
        """One callable per kernel configuration, cached (attention.py:971-1193):
        kernel(kv_cache, query, key, value, seq_lens, block_tables,
        query_start_loc, request_distribution, sink) -> output, updating the
        cache in place."""
        key = (self.sliding_window, self.logits_soft_cap, q_scale, k_scale, v_scale,
               skip_kv_update, self.use_causal_mask, self.decode_query_size)
        fn = self._kernel_config_cache.get(key)
        if fn is not None:
            return fn

        def rpa_kernel_impl(kv_cache, query, key_t, value, seq_lens, block_tables,
                            query_start_loc, request_distribution, sink, out=None):
            # head_dim 64 goes to the hd64 kernel, strict window
            # (attention_interface.py:418-436); only it takes sinks.
            if query.shape[-1] == 64:
                out, _ = _rpa_hd64.ragged_paged_attention_hd64(
                    query, key_t, value, kv_cache, seq_lens, block_tables.reshape(-1),
                    query_start_loc, request_distribution,
                    None if sink is None else sink.detach().to(torch.float32).contiguous(),
                    sm_scale=self.scale, sliding_window=self.sliding_window,
                    strict_sliding_window=True, soft_cap=self.logits_soft_cap,
                    q_scale=q_scale, k_scale=k_scale, v_scale=v_scale,
                    skip_kv_update=skip_kv_update, use_causal_mask=self.use_causal_mask)
                return out
            if sink is not None:
                raise NotImplementedError(
                    "Attention sink support is only available when head_dim==64")
            out, _ = _rpa.ragged_paged_attention(
                query, key_t, value, kv_cache, seq_lens, block_tables.reshape(-1),
                query_start_loc, request_distribution, use_causal_mask=self.use_causal_mask,
                skip_kv_update=skip_kv_update, sm_scale=self.scale,
                sliding_window=self.sliding_window, soft_cap=self.logits_soft_cap,
                q_scale=q_scale, k_scale=k_scale, v_scale=v_scale,
                decode_query_size=self.decode_query_size, out=out)
            return out

        self._kernel_config_cache[key] = rpa_kernel_impl
        return rpa_kernel_impl

    def forward(self, layer: Any, query: torch.Tensor, key: torch.Tensor | None,
                value: torch.Tensor | None, kv_cache: torch.Tensor,
                attn_metadata: AttentionMetadata, output: torch.Tensor | None = None,
                output_scale: torch.Tensor | None = None,
                output_block_scale: torch.Tensor | None = None) -> torch.Tensor:
        """attention.py:1464-1698.  query [T, Hq, D] or [T, Hq * D]; key/value
        [T, Hkv, D] or [T, Hkv * D], or None for a KV-shared layer; kv_cache
        from get_kv_cache_shape.  Returns the output in query's layout and
        writes it into `output` when given."""
        if output_scale is not None or output_block_scale is not None:
            raise NotImplementedError(
                "fused output quantization is not yet supported for RpaAttentionBackendImpl")
        if kv_cache.numel() == 0:  # the memory-profiling call
            if output is None:
                output = torch.ones_like(query)
            return output
        query_dim = query.dim()
        if query_dim == 3:
            q_len, q_compute_dim = query.shape[0], query.shape[1] * query.shape[2]
        else:
            q_len, q_compute_dim = query.shape
        if key is None:
            # KV-shared layer: the cache already holds every key (read with
            # skip_kv_update); zeros only fill the operand slots, kept per
            # shape so no call allocates them again.
            assert value is None and self.kv_sharing_target_layer_name is not None
            zkey = (query.device, query.dtype, q_len)
            key = self._shared_kv_zeros.get(zkey)
            if key is None:
                key = query.new_zeros(q_len, self.num_kv_heads * self.head_size)
                self._shared_kv_zeros[zkey] = key
            value = key
        k_len = key.shape[0]
        k_compute_dim = key.shape[1] * key.shape[2] if key.dim() == 3 else key.shape[1]
        assert q_compute_dim == self.head_size * self.num_heads
        assert k_compute_dim == self.head_size * self.num_kv_heads
        query = query.reshape(q_len, self.num_heads, self.head_size)
        key = key.reshape(k_len, self.num_kv_heads, self.head_size)
        value = value.reshape(k_len, self.num_kv_heads, self.head_size)
        assert key.shape == value.shape

        native_page = tuple(RpaAttentionBackend.get_kv_cache_shape(
            1, 1, self.num_kv_heads, self.head_size, kv_cache.dtype)[2:])
        pad = kv_page_head_padding(tuple(kv_cache.shape[-3:]), native_page, kv_cache.shape[-1],
                                   self.head_size)
        if pad:
            query = torch.nn.functional.pad(query, (0, pad))
            key = torch.nn.functional.pad(key, (0, pad))
            value = torch.nn.functional.pad(value, (0, pad))
        k_scale = v_scale = None
        if self.kv_cache_quantized_dtype:
            k_scale = float(layer._k_scale_float)
            v_scale = float(layer._v_scale_float)
            if k_scale == 0.0 or v_scale == 0.0:
                raise ValueError("k_scale_float and v_scale_float must be non-zero")
            key, value = quantize_kv(self.kv_cache_quantized_dtype, key, value, k_scale, v_scale)
        skip_kv_update = self.kv_sharing_target_layer_name is not None
        kernel = self._build_rpa_kernel(None, k_scale, v_scale, skip_kv_update=skip_kv_update)
        # The kernels write [T, Hq, D] rows; when `output` has exactly that
        # memory layout (no head padding, contiguous, the q dtype) they write
        # into it directly instead of into a temporary that is then copied.
        direct = (output is not None and not pad and self.head_size != 64
                  and output.is_contiguous() and output.dtype == query.dtype
                  and output.numel() == query.numel() and output.device == query.device)
        outputs = kernel(kv_cache, query, key, value, attn_metadata.seq_lens,
                         attn_metadata.block_tables, attn_metadata.query_start_loc,
                         attn_metadata.request_distribution, self.sinks,
                         out=output.view(query.shape) if direct else None)
        if direct:
            return output
        if outputs.shape[-1] > self.head_size:
            outputs = outputs[..., :self.head_size]
        if query_dim == 2:
            outputs = outputs.reshape(q_len, self.num_heads * self.head_size)
        if output is not None:
            output.copy_(outputs)
        return outputs

