"""Ragged Paged Attention on MI355X: host-side mirror of the reference API.

Mirrors `vllm_torchtpu.kernels.ragged_paged_attention.v3.kernel`
(reference file src/vllm_torchtpu/kernels/ragged_paged_attention/v3/kernel.py,
"kernel.py" below): same function names, positional order, keyword names and
defaults, same `ValueError` conditions.  The compute is the HIP library
`librpa_hip.so` (C ABI in include/rpa.h); this module only validates,
describes the call and passes device pointers plus the current HIP stream.

Deliberate differences from the Pallas entry point, each also recorded in
the design notes:
  * The cache is updated in place (the reference donates and aliases it,
    kernel.py:1631, :1908); the returned cache is the same tensor.
  * The output is a fresh [T, Hq, D] tensor in the q dtype (the reference
    aliases it to the donated q buffer, so rows past cu_q_lens[num_seqs] hold
    stale data there and undefined data here).
  * All sequences [0, distribution[2]) are computed, as in
    ref_ragged_paged_attention (kernel.py:143); the Pallas call skips the
    [distribution[0], distribution[1]) segment unless chunk_prefill_size is
    given (kernel.py:1958-1966).  The runner emits distribution[0] ==
    distribution[1], where both agree.
  * Accumulation is fp32 whatever out_dtype says (out_dtype selects the
    Pallas accumulator precision, kernel.py:1820-1829).
  * Tiling knobs (*_block_sizes, vmem_limit_bytes, chunk_prefill_size) are
    validated like the reference and otherwise ignored; debug_mode and the
    disable_* checks have no effect.
"""

from __future__ import annotations

import enum
import warnings
from typing import Any

import torch

from . import _native as N
from .util import align_to, cdiv, get_dtype_packing

__all__ = [
    "RpaCase",
    "get_kv_cache_shape",
    "merge_kv",
    "static_validate_inputs",
    "dynamic_validate_inputs",
    "ragged_paged_attention",
    "ragged_paged_attention_bundled",
    "rpa_kv_cache_update",
    "reserve_workspace",
    "merge_attn_results",
    "merge_attn_states",
]


class RpaCase(enum.Enum):
    """Segments of `distribution` (kernel.py:42-71)."""

    DECODE = 0
    PREFILL = 1
    MIXED = 2

    @property
    def symbol(self) -> str:
        return {RpaCase.DECODE: "d", RpaCase.PREFILL: "p", RpaCase.MIXED: "m"}[self]

    def get_range(self, distribution):
        assert tuple(distribution.shape) == (3,)
        if self == RpaCase.DECODE:
            return 0, distribution[0]
        if self == RpaCase.PREFILL:
            return distribution[0], distribution[1]
        return distribution[1], distribution[2]


def get_kv_cache_shape(total_num_pages, page_size, actual_num_kv_heads,
                       actual_head_dim, kv_dtype):
    """Paged cache shape (kernel.py:278-292):
    [P, page_size, align(2*Hkv, pack) // pack, pack, align(D, 128)]."""
    kv_packing = get_dtype_packing(kv_dtype)
    return (
        total_num_pages,
        page_size,
        align_to(actual_num_kv_heads * 2, kv_packing) // kv_packing,
        kv_packing,
        align_to(actual_head_dim, 128),
    )


def merge_kv(k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """Cache records for k/v rows (kernel.py:1140-1168): combined head 2h = K_h,
    2h+1 = V_h, zero padding of heads to the packing and dims to 128."""
    assert k.shape == v.shape and k.dtype == v.dtype
    t, hkv, d = k.shape
    pack = get_dtype_packing(k.dtype)
    hx2 = align_to(2 * hkv, pack)
    dp = align_to(d, 128)
    out = torch.zeros((t, hx2, dp), dtype=k.dtype, device=k.device)
    out[:, :2 * hkv, :d] = torch.cat([k, v], dim=-1).reshape(t, 2 * hkv, d)
    return out.reshape(t, hx2 // pack, pack, dp)


def static_validate_inputs(queries, keys, values, kv_cache, kv_lens, page_indices,
                           cu_q_lens, distribution, *, use_causal_mask=True,
                           skip_kv_mask=False, sm_scale=1.0, sliding_window=None,
                           soft_cap=None, out_dtype=None, mask_value=None,
                           q_scale=None, k_scale=None, v_scale=None,
                           chunk_prefill_size=None, d_block_sizes=None,
                           p_block_sizes=None, m_block_sizes=None,
                           vmem_limit_bytes=None):
    """Shape and dtype rules, raising ValueError (kernel.py:1366-1538)."""
    q, k, v = queries, keys, values
    if use_causal_mask and skip_kv_mask:
        raise ValueError("Can not skip kv mask when using causal mask.")
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
    actual_head_dim, actual_num_q_heads, actual_num_kv_heads = q.shape[2], q.shape[1], k.shape[1]
    if actual_num_q_heads % actual_num_kv_heads != 0:
        raise ValueError(
            f"Expected {actual_num_q_heads=} to be divisible by {actual_num_kv_heads=}.")
    expected = get_kv_cache_shape(kv_cache.shape[0], kv_cache.shape[1], actual_num_kv_heads,
                                  actual_head_dim, kv_cache.dtype)
    if tuple(kv_cache.shape) != tuple(expected):
        raise ValueError(f"Expected {kv_cache.shape=} to be equal to {expected=}")
    _, page_size, hx2_per_pack, kv_packing, head_dim = kv_cache.shape
    if head_dim != align_to(actual_head_dim, 128):
        raise ValueError(f"Expected {head_dim=} is equal to {align_to(actual_head_dim, 128)=}")
    if not (kv_cache.dtype == k.dtype == v.dtype):
        raise ValueError(
            f"Expected {kv_cache.dtype=} to be equal to {k.dtype=} and {v.dtype=}.")
    if not kv_cache.dtype.is_floating_point:
        raise ValueError(f"Expected {kv_cache.dtype=} to be a floating point.")
    if kv_packing != get_dtype_packing(kv_cache.dtype):
        raise ValueError(f"{kv_packing=} does not match with {kv_cache.dtype=}")
    hx2 = hx2_per_pack * kv_packing
    if hx2 % 2 != 0:
        raise ValueError(f"Combined KV heads must be divisible by 2, but got {hx2}")
    if hx2 % kv_packing != 0 or hx2 // 2 < actual_num_kv_heads:
        raise ValueError(f"Invalid {hx2=}, {actual_num_kv_heads=}, {kv_packing=}")
    if not (torch.int32 == kv_lens.dtype == page_indices.dtype == cu_q_lens.dtype
            == distribution.dtype):
        raise ValueError(
            f"Expected int32 dtype for {kv_lens.dtype=}, {page_indices.dtype=},"
            f" {cu_q_lens.dtype=}, {distribution.dtype=}")
    if not (kv_lens.dim() == page_indices.dim() == cu_q_lens.dim() == 1):
        raise ValueError(
            f"Expected 1D array for {kv_lens.shape=}, {page_indices.shape=},"
            f" {cu_q_lens.shape=}")
    max_num_seqs = kv_lens.shape[0]
    num_page_indices = page_indices.shape[0]
    if max_num_seqs == 0 or num_page_indices % max_num_seqs != 0:
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
    for block_sizes, prefix in ((d_block_sizes, "decode"), (p_block_sizes, "prefill"),
                                (m_block_sizes, "mixed")):
        if block_sizes is None:
            continue
        bq_sz, bkv_sz, bq_csz, bkv_csz = block_sizes
        if not (bq_csz > 0 and bq_sz % bq_csz == 0):
            raise ValueError(f"{prefix} {bq_csz=} and {bq_sz=} must satisfy "
                             "(0 < bq_csz and bq_sz % bq_csz == 0).")
        if not (bkv_csz > 0 and bkv_sz % bkv_csz == 0):
            raise ValueError(f"{prefix} {bkv_csz=} and {bkv_sz=} must satisfy "
                             "(0 < bkv_csz and bkv_sz % bkv_csz == 0).")
        if bkv_sz % page_size != 0:
            raise ValueError(f"{prefix} {bkv_sz=} must be divisible by {page_size=}.")
        if bkv_csz % page_size != 0:
            raise ValueError(f"{prefix} {bkv_csz=} must be divisible by {page_size=}.")
    if vmem_limit_bytes is not None and vmem_limit_bytes <= 0:
        raise ValueError(f"{vmem_limit_bytes=} must be positive.")


def dynamic_validate_inputs(queries, keys, values, kv_cache, kv_lens, page_indices,
                            cu_q_lens, distribution, **kwargs):
    """Metadata value rules (kernel.py:1273-1362).  Reads the metadata back to
    the host, so it synchronises; the reference likewise runs it only in its
    CPU reference path (kernel.py:103-122), never inside the kernel call."""
    static_validate_inputs(queries, keys, values, kv_cache, kv_lens, page_indices,
                           cu_q_lens, distribution, **kwargs)
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
        q_len = cu[s + 1] - cu[s]
        kv_len = kvl[s]
        if not (0 < q_len <= kv_len):
            raise ValueError(f"Require 0 < {q_len=} <= {kv_len=} at sequence {s}.")
        page_cnt = cdiv(kv_len, page_size)
        if page_cnt > pages_per_seq:
            raise ValueError(f"Require {page_cnt=} <= {pages_per_seq=} at sequence {s} where"
                             f" {kv_len=} and {page_size=}.")
        for p in range(page_cnt):
            page_idx = pi[s * pages_per_seq + p]
            if not (0 <= page_idx < total_num_pages):
                raise ValueError(f"Require 0 <= {page_idx=} < {total_num_pages=} at sequence"
                                 f" {s} where {kv_len=} and {page_size=}.")


# ---------------------------------------------------------------------------
# Descriptor + native call
# ---------------------------------------------------------------------------
def _make_desc(q, k, kv_cache, kv_lens, page_indices, out_dtype, *, use_causal_mask,
               skip_kv_update, sm_scale, sliding_window, soft_cap, q_scale, k_scale,
               v_scale, path=N.RPA_PATH_AUTO, decode_query_size=1,
               window_all_rows=False) -> N.RpaDesc:
    d = N.RpaDesc()
    d.abi_version = N.ABI_VERSION
    d.q_dtype = N.rpa_dtype(q.dtype)
    d.kv_dtype = N.rpa_dtype(kv_cache.dtype)
    d.out_dtype = N.rpa_dtype(out_dtype)
    d.max_num_tokens = q.shape[0]
    d.num_q_heads = q.shape[1]
    d.num_kv_heads = k.shape[1]
    d.head_dim = q.shape[2]
    d.head_dim_padded = kv_cache.shape[4]
    d.total_num_pages = kv_cache.shape[0]
    d.page_size = kv_cache.shape[1]
    d.kv_packing = kv_cache.shape[3]
    d.kv_heads_x2 = kv_cache.shape[2] * kv_cache.shape[3]
    d.max_num_seqs = kv_lens.shape[0]
    d.pages_per_seq = page_indices.shape[0] // kv_lens.shape[0]
    d.use_causal_mask = int(bool(use_causal_mask))
    d.skip_kv_update = int(bool(skip_kv_update))
    d.sliding_window = 0 if sliding_window is None else int(sliding_window)
    d.has_soft_cap = int(soft_cap is not None)
    d.soft_cap = float(soft_cap) if soft_cap is not None else 0.0
    d.sm_scale = float(sm_scale)
    d.q_scale = 1.0 if q_scale is None else float(q_scale)
    d.k_scale = 1.0 if k_scale is None else float(k_scale)
    d.v_scale = 1.0 if v_scale is None else float(v_scale)
    d.path = int(path)
    d.decode_query_size = int(decode_query_size)
    d.window_all_rows = int(bool(window_all_rows))
    return d


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _require_device(*tensors: torch.Tensor) -> torch.device:
    dev = tensors[0].device
    if dev.type != "cuda":
        raise RuntimeError(
            "ragged_paged_attention runs on the MI355X HIP library only; got tensors on "
            f"{dev} (there is no CPU path)")
    for t in tensors:
        if t.device != dev:
            raise ValueError(f"all tensors must be on {dev}, got {t.device}")
    return dev


# Per-device workspace (decode partials and work plan), grown on demand and
# kept.  Calls that share a device's workspace must be ordered on one stream
# (as vLLM's are).  A HIP graph captured over a call keeps that call's
# workspace pointer, so a workspace is never freed once handed out: a larger
# one replaces it for later calls and the old one stays alive in _RETIRED.
# Growing during a capture would allocate inside it, so that raises: reserve
# the largest workspace first (reserve_workspace, or one eager call of the
# largest shape, as vLLM's warm-up does).
_WORKSPACES: dict = {}
# Argument signatures (shapes, dtypes, scalars) that passed static_validate_inputs.
_VALIDATED: set = set()


def _hashable(x):
    return None if x is None else tuple(x)

_RETIRED: list = []
# Largest max_num_seqs the fast kernels' in-LDS plan holds (rpa_internal.h,
# kMaxDecodeSeqs); larger batches run on the shape-generic kernels.
MAX_FAST_SEQS = 2048
_WARNED_GENERIC = set()


def _ws_key(device: torch.device):
    if device.type == "cuda" and device.index is None:
        return (device.type, torch.cuda.current_device())
    return (device.type, device.index)


def reserve_workspace(device, nbytes: int) -> torch.Tensor:
    """Make the workspace of `device` at least `nbytes` (call before capturing
    graphs whose calls need more than eager calls so far did)."""
    return _workspace(torch.device(device), nbytes)


def _workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    key = _ws_key(device)
    buf = _WORKSPACES.get(key)
    if buf is None or buf.numel() < nbytes:
        if device.type == "cuda" and torch.cuda.is_current_stream_capturing():
            raise RuntimeError(
                f"the RPA workspace on {device} must grow to {nbytes} bytes during graph "
                "capture; reserve it first (vllm_torchtpu_amd.rpa.reserve_workspace, or one "
                "eager call of the largest shape before capturing)")
        if buf is not None:
            _RETIRED.append(buf)
        buf = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=device)
        _WORKSPACES[key] = buf
    return buf


def _rpa_forward_impl(queries, keys, values, kv_cache, kv_lens, page_indices, cu_q_lens,
                      distribution, out, *, use_causal_mask, skip_kv_update, sm_scale,
                      sliding_window, soft_cap, q_scale, k_scale, v_scale,
                      path=N.RPA_PATH_AUTO, workspace=None, lse=None, attention_sink=None,
                      decode_query_size=1, window_all_rows=False):
    L = N.lib()
    _require_device(queries, keys, values, kv_cache, kv_lens, page_indices, cu_q_lens,
                    distribution, out)
    for name, t in (("queries", queries), ("keys", keys), ("values", values),
                    ("kv_cache", kv_cache), ("kv_lens", kv_lens),
                    ("page_indices", page_indices), ("cu_q_lens", cu_q_lens),
                    ("distribution", distribution), ("out", out)):
        if not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous")
    desc = _make_desc(queries, keys, kv_cache, kv_lens, page_indices, out.dtype,
                      use_causal_mask=use_causal_mask, skip_kv_update=skip_kv_update,
                      sm_scale=sm_scale, sliding_window=sliding_window, soft_cap=soft_cap,
                      q_scale=q_scale, k_scale=k_scale, v_scale=v_scale, path=path,
                      decode_query_size=decode_query_size, window_all_rows=window_all_rows)
    N.check(L.rpa_validate_desc(desc), "rpa_validate_desc")
    if desc.max_num_seqs > MAX_FAST_SEQS and desc.max_num_seqs not in _WARNED_GENERIC:
        _WARNED_GENERIC.add(desc.max_num_seqs)
        warnings.warn(
            f"max_num_seqs={desc.max_num_seqs} exceeds {MAX_FAST_SEQS}, the most the decode and "
            "prefill kernels plan for: this call runs on the shape-generic kernels (correct, "
            "but not a fast path)", RuntimeWarning, stacklevel=3)
    with torch.cuda.device(queries.device):
        ws_bytes = int(L.rpa_workspace_size(desc))
        if workspace is None:
            workspace = _workspace(queries.device, ws_bytes)
        elif workspace.numel() < ws_bytes:
            raise ValueError(f"workspace has {workspace.numel()} bytes, needs {ws_bytes}")
        stream = torch.cuda.current_stream(queries.device).cuda_stream
        if lse is not None and (lse.dtype != torch.float32 or not lse.is_contiguous()
                                or lse.device != out.device
                                or tuple(lse.shape) != tuple(queries.shape[:2])):
            raise ValueError(f"lse must be a contiguous f32 {tuple(queries.shape[:2])} "
                             f"tensor on {out.device}")
        if attention_sink is not None and (
                attention_sink.dtype != torch.float32 or not attention_sink.is_contiguous()
                or attention_sink.device != out.device
                or tuple(attention_sink.shape) != (queries.shape[1],)):
            raise ValueError(f"attention_sink must be a contiguous f32 ({queries.shape[1]},) "
                             f"tensor on {out.device}")
        code = L.rpa_forward_ex(desc, _ptr(queries), _ptr(keys), _ptr(values), _ptr(kv_cache),
                                _ptr(kv_lens), _ptr(page_indices), _ptr(cu_q_lens),
                                _ptr(distribution), _ptr(out), _ptr(attention_sink), _ptr(lse),
                                _ptr(workspace), ws_bytes, stream)
    N.check(code, "rpa_forward")
    return out


# torch custom op: opaque to torch.compile, mutates the cache in place
# (mirrors the reference's torch-facing op, attention.py:1157-1189).
@torch.library.custom_op("rpa_amd::ragged_paged_attention", mutates_args=("kv_cache",))
def _rpa_op(queries: torch.Tensor, keys: torch.Tensor, values: torch.Tensor,
            kv_cache: torch.Tensor, kv_lens: torch.Tensor, page_indices: torch.Tensor,
            cu_q_lens: torch.Tensor, distribution: torch.Tensor, out_dtype: torch.dtype,
            use_causal_mask: bool, skip_kv_update: bool, sm_scale: float,
            sliding_window: int, soft_cap: float, has_soft_cap: bool, q_scale: float,
            k_scale: float, v_scale: float, path: int,
            decode_query_size: int) -> torch.Tensor:
    out = torch.empty(queries.shape, dtype=out_dtype, device=queries.device)
    return _rpa_forward_impl(
        queries, keys, values, kv_cache, kv_lens, page_indices, cu_q_lens, distribution, out,
        use_causal_mask=use_causal_mask, skip_kv_update=skip_kv_update, sm_scale=sm_scale,
        sliding_window=sliding_window if sliding_window > 0 else None,
        soft_cap=soft_cap if has_soft_cap else None, q_scale=q_scale, k_scale=k_scale,
        v_scale=v_scale, path=path, decode_query_size=decode_query_size)


@_rpa_op.register_fake
def _(queries, keys, values, kv_cache, kv_lens, page_indices, cu_q_lens, distribution,
      out_dtype, use_causal_mask, skip_kv_update, sm_scale, sliding_window, soft_cap,
      has_soft_cap, q_scale, k_scale, v_scale, path, decode_query_size):
    return torch.empty(queries.shape, dtype=out_dtype, device=queries.device)


# The same op with the LSE output (return_lse=True), as the batched RPA
# wrapper's return_lse (batched_rpa/wrapper.py:553, :610-623).
@torch.library.custom_op("rpa_amd::ragged_paged_attention_lse", mutates_args=("kv_cache",))
def _rpa_lse_op(queries: torch.Tensor, keys: torch.Tensor, values: torch.Tensor,
                kv_cache: torch.Tensor, kv_lens: torch.Tensor, page_indices: torch.Tensor,
                cu_q_lens: torch.Tensor, distribution: torch.Tensor, out_dtype: torch.dtype,
                use_causal_mask: bool, skip_kv_update: bool, sm_scale: float,
                sliding_window: int, soft_cap: float, has_soft_cap: bool, q_scale: float,
                k_scale: float, v_scale: float, path: int,
                decode_query_size: int) -> tuple[torch.Tensor, torch.Tensor]:
    out = torch.empty(queries.shape, dtype=out_dtype, device=queries.device)
    lse = torch.full(queries.shape[:2], float("-inf"), dtype=torch.float32,
                     device=queries.device)
    _rpa_forward_impl(
        queries, keys, values, kv_cache, kv_lens, page_indices, cu_q_lens, distribution, out,
        use_causal_mask=use_causal_mask, skip_kv_update=skip_kv_update, sm_scale=sm_scale,
        sliding_window=sliding_window if sliding_window > 0 else None,
        soft_cap=soft_cap if has_soft_cap else None, q_scale=q_scale, k_scale=k_scale,
        v_scale=v_scale, path=path, lse=lse, decode_query_size=decode_query_size)
    return out, lse


@_rpa_lse_op.register_fake
def _(queries, keys, values, kv_cache, kv_lens, page_indices, cu_q_lens, distribution,
      out_dtype, use_causal_mask, skip_kv_update, sm_scale, sliding_window, soft_cap,
      has_soft_cap, q_scale, k_scale, v_scale, path, decode_query_size):
    return (torch.empty(queries.shape, dtype=out_dtype, device=queries.device),
            torch.empty(queries.shape[:2], dtype=torch.float32, device=queries.device))


# The same op writing into a caller-provided output (the attention backend's
# `output` buffer): mutates kv_cache and out, returns nothing.
@torch.library.custom_op("rpa_amd::ragged_paged_attention_out", mutates_args=("kv_cache", "out"))
def _rpa_out_op(queries: torch.Tensor, keys: torch.Tensor, values: torch.Tensor,
                kv_cache: torch.Tensor, kv_lens: torch.Tensor, page_indices: torch.Tensor,
                cu_q_lens: torch.Tensor, distribution: torch.Tensor, out: torch.Tensor,
                use_causal_mask: bool, skip_kv_update: bool, sm_scale: float,
                sliding_window: int, soft_cap: float, has_soft_cap: bool, q_scale: float,
                k_scale: float, v_scale: float, path: int, decode_query_size: int) -> None:
    _rpa_forward_impl(
        queries, keys, values, kv_cache, kv_lens, page_indices, cu_q_lens, distribution, out,
        use_causal_mask=use_causal_mask, skip_kv_update=skip_kv_update, sm_scale=sm_scale,
        sliding_window=sliding_window if sliding_window > 0 else None,
        soft_cap=soft_cap if has_soft_cap else None, q_scale=q_scale, k_scale=k_scale,
        v_scale=v_scale, path=path, decode_query_size=decode_query_size)


@_rpa_out_op.register_fake
def _(queries, keys, values, kv_cache, kv_lens, page_indices, cu_q_lens, distribution, out,
      use_causal_mask, skip_kv_update, sm_scale, sliding_window, soft_cap, has_soft_cap,
      q_scale, k_scale, v_scale, path, decode_query_size):
    return None


def ragged_paged_attention(
    queries: torch.Tensor,  # [max_num_tokens, actual_num_q_heads, actual_head_dim]
    keys: torch.Tensor,  # [max_num_tokens, actual_num_kv_heads, actual_head_dim]
    values: torch.Tensor,  # [max_num_tokens, actual_num_kv_heads, actual_head_dim]
    # [total_num_pages, page_size, num_kv_heads_x2 // kv_packing, kv_packing, head_dim]
    kv_cache: torch.Tensor,
    kv_lens: torch.Tensor,  # i32[max_num_seqs]
    page_indices: torch.Tensor,  # i32[max_num_seqs * pages_per_seq]
    cu_q_lens: torch.Tensor,  # i32[max_num_seqs + 1]
    distribution: torch.Tensor,  # i32[3]
    *,
    use_causal_mask: bool = True,
    skip_kv_mask: bool = False,
    skip_kv_update: bool = False,
    sm_scale: float = 1.0,
    sliding_window: int | None = None,
    soft_cap: float | None = None,
    out_dtype: Any = None,
    mask_value: float | None = None,
    q_scale: float | None = None,
    k_scale: float | None = None,
    v_scale: float | None = None,
    chunk_prefill_size: int | None = None,
    d_block_sizes: tuple[int, int, int, int] | None = None,
    p_block_sizes: tuple[int, int, int, int] | None = None,
    m_block_sizes: tuple[int, int, int, int] | None = None,
    vmem_limit_bytes: int | None = None,
    debug_mode: bool = False,
    disable_bounds_checks: bool = True,
    disable_semaphore_checks: bool = True,
    return_lse: bool = False,
    decode_query_size: int = 1,
    out: torch.Tensor | None = None,
):
    """Ragged paged attention with mixed prefill and decode (kernel.py:1633-1984).

    Returns (out [max_num_tokens, Hq, D] in the q dtype, kv_cache).  kv_cache is
    updated in place with the new tokens' K/V (unless skip_kv_update) and
    returned.  Rows of `out` at or beyond cu_q_lens[distribution[2]] are not
    written.  See the module docstring for the deliberate differences.

    return_lse (an addition from the batched RPA wrapper, batched_rpa/
    wrapper.py:553, :610-623): also return lse, f32 [max_num_tokens, Hq], the
    natural-log log-sum-exp m + log(l) of each computed row's logits (after
    scaling and soft cap; -inf for a row without keys, and for rows past
    cu_q_lens[distribution[2]]) -- what merge_attn_results combines.

    decode_query_size (the batched wrapper's, batched_rpa/wrapper.py:549,
    :601-602): the largest number of query tokens of a decode sequence
    (speculative-decoding verify windows of K + 1 tokens).  Sequences with up to
    that many new tokens run on the decode kernel (while q_len * Hq/Hkv <= 16);
    the result does not depend on it.

    out (an addition for the attention backend, whose forward receives an
    output buffer): a contiguous [max_num_tokens, Hq, D] tensor in the q dtype
    on the same device; the rows are written there and `out` is returned.
    Not combinable with return_lse.
    """
    del debug_mode, disable_bounds_checks, disable_semaphore_checks
    # static_validate_inputs reads only shapes, dtypes and these scalars, so a
    # signature that passed once passes again (about 14 us a call on the host).
    sig = (tuple(queries.shape), tuple(keys.shape), tuple(values.shape),
           tuple(kv_cache.shape), tuple(kv_lens.shape), tuple(page_indices.shape),
           tuple(cu_q_lens.shape), tuple(distribution.shape), queries.dtype, keys.dtype,
           values.dtype, kv_cache.dtype, kv_lens.dtype, page_indices.dtype, cu_q_lens.dtype,
           distribution.dtype, bool(use_causal_mask), bool(skip_kv_mask), sliding_window,
           soft_cap, chunk_prefill_size, _hashable(d_block_sizes), _hashable(p_block_sizes),
           _hashable(m_block_sizes), vmem_limit_bytes)
    if sig not in _VALIDATED:
        static_validate_inputs(
            queries, keys, values, kv_cache, kv_lens, page_indices, cu_q_lens, distribution,
            use_causal_mask=use_causal_mask, skip_kv_mask=skip_kv_mask, sm_scale=sm_scale,
            sliding_window=sliding_window, soft_cap=soft_cap, out_dtype=out_dtype,
            mask_value=mask_value, q_scale=q_scale, k_scale=k_scale, v_scale=v_scale,
            chunk_prefill_size=chunk_prefill_size, d_block_sizes=d_block_sizes,
            p_block_sizes=p_block_sizes, m_block_sizes=m_block_sizes,
            vmem_limit_bytes=vmem_limit_bytes)
        if len(_VALIDATED) < 4096:
            _VALIDATED.add(sig)
    if int(decode_query_size) < 1:
        raise ValueError(f"{decode_query_size=} must be positive.")
    if mask_value is not None and mask_value > -1e30:
        # Masked logits are excluded with weight exactly 0; that equals the
        # reference only when exp(mask_value - rowmax) underflows.
        raise NotImplementedError(
            f"{mask_value=}: only mask values <= -1e30 (default finfo.min) are supported")
    result_dtype = queries.dtype
    q = queries
    if q_scale is not None:
        # kernel.py:176-183: q / q_scale in q's dtype, clip to the KV dtype range,
        # cast to the KV dtype; q_scale is multiplied back into the logits.
        info = torch.finfo(kv_cache.dtype)
        q = torch.clamp(q / q_scale, min=info.min, max=info.max).to(kv_cache.dtype)
    if out is not None:
        if return_lse:
            raise ValueError("out= and return_lse=True cannot be combined")
        if (out.dtype != result_dtype or tuple(out.shape) != tuple(queries.shape)
                or not out.is_contiguous() or out.device != queries.device):
            raise ValueError(f"out must be a contiguous {result_dtype} tensor of shape "
                             f"{tuple(queries.shape)} on {queries.device}")
        if type(queries) is torch.Tensor and not torch.compiler.is_compiling():
            _rpa_forward_impl(
                q.contiguous(), keys.contiguous(), values.contiguous(), kv_cache, kv_lens,
                page_indices, cu_q_lens, distribution, out,
                use_causal_mask=bool(use_causal_mask), skip_kv_update=bool(skip_kv_update),
                sm_scale=float(sm_scale),
                sliding_window=None if sliding_window is None else int(sliding_window),
                soft_cap=None if soft_cap is None else float(soft_cap),
                q_scale=1.0 if q_scale is None else float(q_scale),
                k_scale=1.0 if k_scale is None else float(k_scale),
                v_scale=1.0 if v_scale is None else float(v_scale), path=N.RPA_PATH_AUTO,
                decode_query_size=int(decode_query_size))
            return out, kv_cache
        torch.ops.rpa_amd.ragged_paged_attention_out(
            q.contiguous(), keys.contiguous(), values.contiguous(), kv_cache, kv_lens,
            page_indices, cu_q_lens, distribution, out, bool(use_causal_mask),
            bool(skip_kv_update), float(sm_scale),
            0 if sliding_window is None else int(sliding_window),
            0.0 if soft_cap is None else float(soft_cap), soft_cap is not None,
            1.0 if q_scale is None else float(q_scale), 1.0 if k_scale is None else float(k_scale),
            1.0 if v_scale is None else float(v_scale), N.RPA_PATH_AUTO, int(decode_query_size))
        return out, kv_cache
    if type(queries) is torch.Tensor and not torch.compiler.is_compiling():
        # Eager call on real tensors: the same work as the custom op's body without
        # its dispatcher (about 18 us a call on the host); under torch.compile,
        # export or fake tensors the op keeps the call opaque.
        res = torch.empty(queries.shape, dtype=result_dtype, device=queries.device)
        lse = None
        if return_lse:
            lse = torch.full(queries.shape[:2], float("-inf"), dtype=torch.float32,
                             device=queries.device)
        _rpa_forward_impl(
            q.contiguous(), keys.contiguous(), values.contiguous(), kv_cache, kv_lens,
            page_indices, cu_q_lens, distribution, res, use_causal_mask=bool(use_causal_mask),
            skip_kv_update=bool(skip_kv_update), sm_scale=float(sm_scale),
            sliding_window=None if sliding_window is None else int(sliding_window),
            soft_cap=None if soft_cap is None else float(soft_cap),
            q_scale=1.0 if q_scale is None else float(q_scale),
            k_scale=1.0 if k_scale is None else float(k_scale),
            v_scale=1.0 if v_scale is None else float(v_scale), path=N.RPA_PATH_AUTO,
            lse=lse, decode_query_size=int(decode_query_size))
        if return_lse:
            return res, kv_cache, lse
        return res, kv_cache
    op = (torch.ops.rpa_amd.ragged_paged_attention_lse if return_lse
          else torch.ops.rpa_amd.ragged_paged_attention)
    res = op(
        q.contiguous(), keys.contiguous(), values.contiguous(), kv_cache, kv_lens, page_indices,
        cu_q_lens, distribution, result_dtype, bool(use_causal_mask), bool(skip_kv_update),
        float(sm_scale), 0 if sliding_window is None else int(sliding_window),
        0.0 if soft_cap is None else float(soft_cap), soft_cap is not None,
        1.0 if q_scale is None else float(q_scale), 1.0 if k_scale is None else float(k_scale),
        1.0 if v_scale is None else float(v_scale), N.RPA_PATH_AUTO, int(decode_query_size))
    if return_lse:
        out, lse = res
        return out, kv_cache, lse
    return res, kv_cache


def merge_attn_states(outs: torch.Tensor, lses: torch.Tensor, out_dtype=torch.float32):
    """LSE-weighted merge of R partial attentions of the same rows.

    outs [R, ..., D] (bf16 or f32), lses [R, ...] (natural-log LSE, any float
    dtype; computed in f32) -> (out [..., D] in out_dtype, lse [...] f32).
    merge_attn_results (cp_attention.py:45-72) generalised to R partials, on
    the GPU (rpa_merge_attn_states in include/rpa.h): weights exp(lse_r - m)
    with m = max_r lse_r (a NaN lse propagates, as torch.maximum), NaN/inf
    partial outputs counted as 0, rows whose partials all have lse -inf give
    0 and lse -inf.  out_dtype defaults to f32, the reference's result dtype
    (its f32 weights promote bf16 partials); bf16 is also accepted.
    """
    if outs.dim() < 2 or lses.shape != outs.shape[:-1]:
        raise ValueError(f"outs {tuple(outs.shape)} and lses {tuple(lses.shape)} do not match")
    if not outs.is_cuda or lses.device != outs.device:
        raise RuntimeError("merge_attn_states: tensors must be on one GPU (no CPU fallback)")
    if out_dtype not in (torch.float32, torch.bfloat16):
        raise ValueError(f"out_dtype {out_dtype} is not supported (f32 or bf16)")
    parts, dim = outs.shape[0], outs.shape[-1]
    rows = outs[0].numel() // max(dim, 1)
    outs_c = outs.contiguous()
    lses_c = lses.to(torch.float32).contiguous()
    out = torch.empty(outs.shape[1:], dtype=out_dtype, device=outs.device)
    lse = torch.empty(lses.shape[1:], dtype=torch.float32, device=outs.device)
    L = N.lib()
    with torch.cuda.device(outs.device):
        stream = torch.cuda.current_stream(outs.device).cuda_stream
        code = L.rpa_merge_attn_states(parts, rows, dim, N.rpa_dtype(outs.dtype),
                                       N.rpa_dtype(out_dtype), _ptr(outs_c), _ptr(lses_c),
                                       _ptr(out), _ptr(lse), stream)
    N.check(code, "rpa_merge_attn_states")
    return out, lse


def merge_attn_results(out_a: torch.Tensor, lse_a: torch.Tensor, out_b: torch.Tensor,
                       lse_b: torch.Tensor):
    """Numerically stable LSE-weighted combination of two partial attentions
    (cp_attention.py:45-72): out [T, H, D], lse [T, H] (natural log) each;
    returns (combined_out f32, combined_lse f32), the reference's dtypes."""
    if out_a.shape != out_b.shape or lse_a.shape != lse_b.shape:
        raise ValueError("merge_attn_results: partials differ in shape")
    return merge_attn_states(torch.stack([out_a, out_b]),
                             torch.stack([lse_a.to(torch.float32), lse_b.to(torch.float32)]))


def ragged_paged_attention_bundled(queries, keys, values, kv_cache_bundle, layer_idx,
                                   kv_lens, page_indices, cu_q_lens, distribution, **kwargs):
    """RPA on a block-major multi-layer cache (kernel.py:2011-2061).

    kv_cache_bundle is [num_pages, num_layers, page_size, ...]; it is viewed as
    [num_pages * num_layers, page_size, ...] (no copy) and logical page p of
    layer l maps to flat page p * num_layers + l.  Updated in place.
    """
    num_blocks, num_layers = kv_cache_bundle.shape[0], kv_cache_bundle.shape[1]
    flat = kv_cache_bundle.view(num_blocks * num_layers, *kv_cache_bundle.shape[2:])
    flat_page_indices = (page_indices * num_layers + layer_idx).to(torch.int32)
    out, _ = ragged_paged_attention(queries, keys, values, flat, kv_lens, flat_page_indices,
                                    cu_q_lens, distribution, **kwargs)
    return out, kv_cache_bundle


def rpa_kv_cache_update(keys, values, kv_cache, kv_lens, page_indices, cu_q_lens,
                        distribution):
    """Only the cache write of an RPA call (kernel.py:652-715), in place."""
    L = N.lib()
    _require_device(keys, values, kv_cache, kv_lens, page_indices, cu_q_lens, distribution)
    desc = _make_desc(keys, keys, kv_cache, kv_lens, page_indices, torch.bfloat16,
                      use_causal_mask=True, skip_kv_update=False, sm_scale=1.0,
                      sliding_window=None, soft_cap=None, q_scale=None, k_scale=None,
                      v_scale=None)
    desc.q_dtype = desc.kv_dtype
    stream = torch.cuda.current_stream(keys.device).cuda_stream
    with torch.cuda.device(keys.device):
        code = L.rpa_kv_cache_update(desc, _ptr(keys), _ptr(values), _ptr(kv_cache),
                                     _ptr(kv_lens), _ptr(page_indices), _ptr(cu_q_lens),
                                     _ptr(distribution), stream)
    N.check(code, "rpa_kv_cache_update")
    return kv_cache
