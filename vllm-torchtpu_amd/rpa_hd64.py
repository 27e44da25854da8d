"""Ragged paged attention for head_dim 64 with attention sinks: host-side mirror
of `src/vllm_torchtpu/kernels/ragged_paged_attention/v3/kernel_hd64.py`
("kernel_hd64.py" below) -- the same names, positional order, keyword names,
defaults and `ValueError` conditions.

The cache layout is the reference's packed one (kernel_hd64.py:246-261):
[P, page_size, align(Hkv, packing) / packing, packing, 128], each 128-wide row
holding K_h (64) then V_h (64).  Those are the same bytes as this library's
head-packed layout with a padded head_dim of 64 (combined head 2h = K_h,
2h + 1 = V_h), so the call views the cache that way (no copy) and runs the
same kernels (include/rpa.h, rpa_forward_ex) with the sink logits.

Deliberate differences (besides those of rpa.py):
  * strict_sliding_window=False lets the Pallas kernel keep keys outside the
    window that share a block with keys inside it; here every row is masked
    strictly, as the reference function (ref_ragged_paged_attention_hd64)
    does, whatever the flag says.
  * The block-size knobs are validated and otherwise ignored.
  * sliding_window with use_causal_mask=False masks keys j <= p - W of every
    row, as kernel_hd64.py:155-158 and :443-446 do (the v3 reference windows
    causal rows only); such calls run on the shape-generic kernels.
"""

from __future__ import annotations

import torch

from . import _native as N
from .rpa import _require_device, _rpa_forward_impl
from .util import align_to, cdiv, get_dtype_packing

__all__ = [
    "DEFAULT_MASK_VALUE",
    "get_kv_cache_shape_hd64",
    "merge_kv_hd64",
    "static_validate_inputs_hd64",
    "dynamic_validate_inputs_hd64",
    "ragged_paged_attention_hd64",
]

# kernel_hd64.py:36.
DEFAULT_MASK_VALUE = -0.7 * float(torch.finfo(torch.float32).max)


def get_kv_cache_shape_hd64(total_num_pages, page_size, actual_num_kv_heads, actual_head_dim,
                            kv_dtype):
    """kernel_hd64.py:246-261."""
    assert actual_head_dim == 64
    kv_packing = get_dtype_packing(kv_dtype)
    return (total_num_pages, page_size,
            align_to(actual_num_kv_heads, kv_packing) // kv_packing, kv_packing, 128)


def merge_kv_hd64(k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """Cache records for k/v rows (kernel_hd64.py:1018-1041): [K_h | V_h] per
    head, heads zero-padded to the packing."""
    assert k.shape == v.shape and k.dtype == v.dtype
    t, hkv, d = k.shape
    pack = get_dtype_packing(k.dtype)
    heads = align_to(hkv, pack)
    kv = torch.zeros((t, heads, 2 * d), dtype=k.dtype, device=k.device)
    kv[:, :hkv, :d] = k
    kv[:, :hkv, d:] = v
    return kv.reshape(t, heads // pack, pack, 2 * d)


def static_validate_inputs_hd64(queries, keys, values, kv_cache, kv_lens, page_indices,
                                cu_q_lens, distribution, attention_sink=None, *,
                                sm_scale=1.0, sliding_window=None, soft_cap=None,
                                mask_value=DEFAULT_MASK_VALUE, q_scale=None, k_scale=None,
                                v_scale=None, chunk_prefill_size=None,
                                num_kv_pages_per_block=None, num_queries_per_block=None,
                                vmem_limit_bytes=None, debug_mode=False):
    """kernel_hd64.py:1211-1316, raising ValueError."""
    q, k, v = queries, keys, values
    if not (q.dim() == k.dim() == v.dim() == 3):
        raise ValueError(f"Expected 3D array for {q.shape=}, {k.shape=}, {v.shape=}")
    if k.shape != v.shape:
        raise ValueError(f"Expected {k.shape=} to be equal to {v.shape=}")
    if not (q.shape[0] == k.shape[0] == v.shape[0]):
        raise ValueError(
            f"Expected {q.shape[0]=} to be equal to {k.shape[0]=} and {v.shape[0]=}")
    if not (q.shape[2] == k.shape[2] == v.shape[2]):
        raise ValueError(
            f"Expected {q.shape[2]=} to be equal to {k.shape[2]=} and {v.shape[2]=}")
    if attention_sink is not None:
        if attention_sink.shape[0] != q.shape[1]:
            raise ValueError(f"Expected {attention_sink.shape[0]=} to be equal to"
                             f" {q.shape[1]=} (num_q_heads).")
        if attention_sink.dtype != torch.float32:
            raise ValueError(f"Expected {attention_sink.dtype=} to be equal to torch.float32.")
    actual_head_dim = q.shape[2]
    if actual_head_dim != 64:
        raise ValueError(f"Expected {actual_head_dim=} to be 64.")
    actual_num_q_heads, actual_num_kv_heads = q.shape[1], k.shape[1]
    if actual_num_q_heads % actual_num_kv_heads != 0:
        raise ValueError(
            f"Expected {actual_num_q_heads=} to be divisible by {actual_num_kv_heads=}.")
    if kv_cache.dim() != 5:
        raise ValueError(f"Expected 5D kv_cache, got {tuple(kv_cache.shape)}")
    _, page_size, num_kv_heads_per_kv_packing, kv_packing, actual_head_dim_x2 = kv_cache.shape
    if actual_head_dim_x2 != 128:
        raise ValueError(f"Expected {actual_head_dim_x2=} is equal to 128")
    if not (kv_cache.dtype == k.dtype == v.dtype):
        raise ValueError(
            f"Expected {kv_cache.dtype=} to be equal to {k.dtype=} and {v.dtype=}.")
    if not kv_cache.dtype.is_floating_point:
        raise ValueError(f"Expected {kv_cache.dtype=} to be a floating point.")
    if kv_packing != get_dtype_packing(kv_cache.dtype):
        raise ValueError(f"{kv_packing=} does not match with {kv_cache.dtype=}")
    num_kv_heads = num_kv_heads_per_kv_packing * kv_packing
    if align_to(actual_num_kv_heads, kv_packing) != num_kv_heads:
        raise ValueError(f"Invalid {num_kv_heads=}, {actual_num_kv_heads=}, {kv_packing=}")
    if not (torch.int32 == kv_lens.dtype == page_indices.dtype == cu_q_lens.dtype
            == distribution.dtype):
        raise ValueError(
            f"Expected int32 dtype for {kv_lens.dtype=}, {page_indices.dtype=},"
            f" {cu_q_lens.dtype=}, {distribution.dtype=}")
    if not (kv_lens.dim() == page_indices.dim() == cu_q_lens.dim() == 1):
        raise ValueError(f"Expected 1D array for {kv_lens.shape=}, {page_indices.shape=},"
                         f" {cu_q_lens.shape=}")
    max_num_seqs = kv_lens.shape[0]
    num_page_indices = page_indices.shape[0]
    if num_page_indices % max_num_seqs != 0:
        raise ValueError(f"Expected {num_page_indices=} to be divisible by {max_num_seqs=}.")
    if tuple(cu_q_lens.shape) != (max_num_seqs + 1,):
        raise ValueError(f"Expected {cu_q_lens.shape=} to be ({max_num_seqs + 1},).")
    if tuple(distribution.shape) != (3,):
        raise ValueError(f"Expected {distribution.shape=} to be (3,).")
    if page_size % kv_packing != 0:
        raise ValueError(f"{page_size=} must be divisible by {kv_packing=}.")
    if sliding_window is not None and sliding_window <= 0:
        raise ValueError(f"{sliding_window=} must be positive.")
    if soft_cap is not None and soft_cap == 0.0:
        raise ValueError(f"{soft_cap=} must not be 0.0.")
    if chunk_prefill_size is not None and chunk_prefill_size <= 0:
        raise ValueError(f"{chunk_prefill_size=} must be positive.")
    if num_kv_pages_per_block is not None and num_kv_pages_per_block <= 0:
        raise ValueError(f"{num_kv_pages_per_block=} must be positive.")
    if num_queries_per_block is not None and num_queries_per_block <= 0:
        raise ValueError(f"{num_queries_per_block=} must be positive.")
    if vmem_limit_bytes is not None and vmem_limit_bytes <= 0:
        raise ValueError(f"{vmem_limit_bytes=} must be positive.")


def dynamic_validate_inputs_hd64(queries, keys, values, kv_cache, kv_lens, page_indices,
                                 cu_q_lens, distribution, attention_sink=None, **kwargs):
    """kernel_hd64.py:1121-1208 (reads the metadata back to the host)."""
    static_validate_inputs_hd64(queries, keys, values, kv_cache, kv_lens, page_indices,
                                cu_q_lens, distribution, attention_sink, **kwargs)
    max_num_tokens = queries.shape[0]
    total_num_pages, page_size = kv_cache.shape[0], kv_cache.shape[1]
    max_num_seqs = kv_lens.shape[0]
    pages_per_seq = page_indices.shape[0] // max_num_seqs
    i, j, k = (int(x) for x in distribution.cpu().tolist())
    if not (i <= j <= k):
        raise ValueError(f"Invalid distribution: {(i, j, k)=}")
    if k > max_num_seqs:
        raise ValueError(f"num_seqs={k} must be <= {max_num_seqs=}")
    cu = cu_q_lens.cpu().tolist()
    kvl = kv_lens.cpu().tolist()
    pi = page_indices.cpu().tolist()
    if cu[k] > max_num_tokens:
        raise ValueError(f"Total q tokens {cu[k]} must be <= {max_num_tokens=}.")
    for s in range(k):
        q_len, kv_len = cu[s + 1] - cu[s], kvl[s]
        if not (0 < q_len <= kv_len):
            raise ValueError(f"Require 0 < {q_len=} <= {kv_len=} at sequence {s}.")
        page_cnt = cdiv(kv_len, page_size)
        if page_cnt > pages_per_seq:
            raise ValueError(f"Require {page_cnt=} <= {pages_per_seq=} at sequence {s} where"
                             f" {kv_len=} and {page_size=}.")
        for pg in range(page_cnt):
            page_idx = pi[s * pages_per_seq + pg]
            if not (0 <= page_idx < total_num_pages):
                raise ValueError(f"Require 0 <= {page_idx=} < {total_num_pages=} at sequence"
                                 f" {s} where {kv_len=} and {page_size=}.")


def _as_head_packed(kv_cache: torch.Tensor) -> torch.Tensor:
    """The packed hd64 cache viewed as [P, ps, 2 * heads / packing, packing, 64]:
    combined head 2h = K_h, 2h + 1 = V_h (the same bytes)."""
    p, ps, hp, pack, _ = kv_cache.shape
    return kv_cache.view(p, ps, 2 * hp, pack, 64)


def _rpa_hd64_impl(queries: torch.Tensor, keys: torch.Tensor, values: torch.Tensor,
                   kv_cache: torch.Tensor, kv_lens: torch.Tensor, page_indices: torch.Tensor,
                   cu_q_lens: torch.Tensor, distribution: torch.Tensor,
                   attention_sink: torch.Tensor | None, use_causal_mask: bool,
                   skip_kv_update: bool, sm_scale: float, sliding_window: int, soft_cap: float,
                   has_soft_cap: bool, q_scale: float, k_scale: float,
                   v_scale: float) -> torch.Tensor:
    out = torch.empty(queries.shape, dtype=queries.dtype, device=queries.device)
    return _rpa_forward_impl(
        queries, keys, values, _as_head_packed(kv_cache), kv_lens, page_indices, cu_q_lens,
        distribution, out, use_causal_mask=use_causal_mask, skip_kv_update=skip_kv_update,
        sm_scale=sm_scale, sliding_window=sliding_window if sliding_window > 0 else None,
        soft_cap=soft_cap if has_soft_cap else None, q_scale=q_scale, k_scale=k_scale,
        v_scale=v_scale, attention_sink=attention_sink, window_all_rows=True)


@torch.library.custom_op("rpa_amd::ragged_paged_attention_hd64", mutates_args=("kv_cache",))
def _rpa_hd64_op(queries: torch.Tensor, keys: torch.Tensor, values: torch.Tensor,
                 kv_cache: torch.Tensor, kv_lens: torch.Tensor, page_indices: torch.Tensor,
                 cu_q_lens: torch.Tensor, distribution: torch.Tensor,
                 attention_sink: torch.Tensor | None, use_causal_mask: bool,
                 skip_kv_update: bool, sm_scale: float, sliding_window: int, soft_cap: float,
                 has_soft_cap: bool, q_scale: float, k_scale: float,
                 v_scale: float) -> torch.Tensor:
    return _rpa_hd64_impl(queries, keys, values, kv_cache, kv_lens, page_indices, cu_q_lens,
                          distribution, attention_sink, use_causal_mask, skip_kv_update,
                          sm_scale, sliding_window, soft_cap, has_soft_cap, q_scale, k_scale,
                          v_scale)


@_rpa_hd64_op.register_fake
def _(queries, keys, values, kv_cache, kv_lens, page_indices, cu_q_lens, distribution,
      attention_sink, use_causal_mask, skip_kv_update, sm_scale, sliding_window, soft_cap,
      has_soft_cap, q_scale, k_scale, v_scale):
    return torch.empty(queries.shape, dtype=queries.dtype, device=queries.device)


def ragged_paged_attention_hd64(
    queries: torch.Tensor,  # [max_num_tokens, actual_num_q_heads, 64]
    keys: torch.Tensor,  # [max_num_tokens, actual_num_kv_heads, 64]
    values: torch.Tensor,  # [max_num_tokens, actual_num_kv_heads, 64]
    # [total_num_pages, page_size, num_kv_heads // kv_packing, kv_packing, 128]
    kv_cache: torch.Tensor,
    kv_lens: torch.Tensor,  # i32[max_num_seqs]
    page_indices: torch.Tensor,  # i32[max_num_seqs * pages_per_seq]
    cu_q_lens: torch.Tensor,  # i32[max_num_seqs + 1]
    distribution: torch.Tensor,  # i32[3]
    attention_sink: torch.Tensor | None = None,  # f32[actual_num_q_heads]
    *,
    sm_scale: float = 1.0,
    sliding_window: int | None = None,
    strict_sliding_window: bool = True,
    soft_cap: float | None = None,
    mask_value: float = DEFAULT_MASK_VALUE,
    q_scale: float | None = None,
    k_scale: float | None = None,
    v_scale: float | None = None,
    chunk_prefill_size: int | None = None,
    num_kv_pages_per_block: int | None = None,
    num_queries_per_block: int | None = None,
    vmem_limit_bytes: int | None = None,
    debug_mode: bool = False,
    skip_kv_update: bool = False,
    use_causal_mask: bool = True,
):
    """Ragged paged attention for head_dim 64 with optional attention sinks
    (kernel_hd64.py:1377-1620).  Returns (out [max_num_tokens, Hq, 64] in the q
    dtype, kv_cache), the cache updated in place.  attention_sink[g] is a
    logit that joins q head g's softmax with value 0 (kernel_hd64.py:161-172)."""
    del strict_sliding_window, debug_mode
    static_validate_inputs_hd64(
        queries, keys, values, kv_cache, kv_lens, page_indices, cu_q_lens, distribution,
        attention_sink, sm_scale=sm_scale, sliding_window=sliding_window, soft_cap=soft_cap,
        mask_value=mask_value, q_scale=q_scale, k_scale=k_scale, v_scale=v_scale,
        chunk_prefill_size=chunk_prefill_size, num_kv_pages_per_block=num_kv_pages_per_block,
        num_queries_per_block=num_queries_per_block, vmem_limit_bytes=vmem_limit_bytes)
    if mask_value is not None and mask_value > -1e30:
        raise NotImplementedError(
            f"{mask_value=}: only mask values <= -1e30 (the default) are supported")
    _require_device(queries, keys, values, kv_cache)
    q = queries
    if q_scale is not None:  # kernel_hd64.py:126-133
        info = torch.finfo(kv_cache.dtype)
        q = torch.clamp(q / q_scale, min=info.min, max=info.max).to(kv_cache.dtype)
    sink = None if attention_sink is None else attention_sink.contiguous()
    if type(queries) is torch.Tensor and not torch.compiler.is_compiling():
        # Eager call on real tensors: the op's body without its dispatcher.
        out = _rpa_hd64_impl(
            q.contiguous(), keys.contiguous(), values.contiguous(), kv_cache, kv_lens,
            page_indices, cu_q_lens, distribution, sink, bool(use_causal_mask),
            bool(skip_kv_update), float(sm_scale),
            0 if sliding_window is None else int(sliding_window),
            0.0 if soft_cap is None else float(soft_cap), soft_cap is not None,
            1.0 if q_scale is None else float(q_scale), 1.0 if k_scale is None else float(k_scale),
            1.0 if v_scale is None else float(v_scale))
        return out, kv_cache
    out = torch.ops.rpa_amd.ragged_paged_attention_hd64(
        q.contiguous(), keys.contiguous(), values.contiguous(), kv_cache, kv_lens, page_indices,
        cu_q_lens, distribution, sink, bool(use_causal_mask), bool(skip_kv_update),
        float(sm_scale), 0 if sliding_window is None else int(sliding_window),
        0.0 if soft_cap is None else float(soft_cap), soft_cap is not None,
        1.0 if q_scale is None else float(q_scale), 1.0 if k_scale is None else float(k_scale),
        1.0 if v_scale is None else float(v_scale))
    return out, kv_cache


assert N.RPA_PATH_AUTO == 0  # the op always takes the automatic kernel choice
