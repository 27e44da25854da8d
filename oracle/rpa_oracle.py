"""CPU oracle for Ragged Paged Attention (RPA) -- TEST INFRASTRUCTURE ONLY.

This module restates, on the CPU, the reference algorithm of
`vllm_torchtpu.kernels.ragged_paged_attention.v3` (all citations below are
relative to the reference tree, "kernel.py" meaning
`src/vllm_torchtpu/kernels/ragged_paged_attention/v3/kernel.py`).  It is the
checker, never the product: only `tests/`, `__graft_entry__.smoke()` and the
`cpu_baseline` leg of `bench.py` may import it.  The product path
(`vllm_torchtpu_amd`) never imports it and fails loudly if its HIP library is
missing.

Functions and what pins each one (the tests live in
`tests/test_oracle_*.py`):

* `cdiv`, `align_to`, `get_dtype_packing`       -- util.py:20-35.
  Pinned by closed-form tests (packing = 32 // bits).
* `get_kv_cache_shape`                           -- kernel.py:278-292.
  Pinned by the geometry the reference's own layout tests assert
  (`tests/kernels/test_pipelined_dma_flag.py:160-195` shapes) and closed forms.
* `merge_kv`                                     -- kernel.py:1140-1168.
  Pinned bytewise against an explicit element loop (K at even, V at odd
  combined heads, zero padding).
* `quantize_kv`                                  -- layers/core/quantization.py:73-103.
  Pinned against exhaustive fp8 round-trip properties.
* `update_kv_cache_np`                           -- kernel.py:148-166 (the
  cache-write half of the reference), restated with integer numpy views so it
  is bit-exact.  Pinned by a brute-force per-element scatter and the
  skip_kv_update invariant (`tests/kernels/test_rpa_skip_kv_update.py:169-182`).
* `static_validate_inputs`, `dynamic_validate_inputs` -- kernel.py:1273-1538.
  Pinned by one table-driven test per `ValueError` condition.
* `merge_attn_results`                           -- layers/adapter/cp_attention.py:45-72;
  `merge_attn_states`, its R-partial generalisation.  Pinned by the split
  identity (attention over a key set equals the merge of the attentions over
  any partition of it, computed independently in fp64), closed forms (a
  partial with lse -inf drops out; equal lses average) and R = 2 agreement.
* `ref_ragged_paged_attention(..., return_lse=True)` -- the LSE is pinned
  against a per-element fp64 log-sum-exp loop and closed forms (one key:
  lse = its logit; constant logits c over n keys: c + log n).
* `ref_ragged_paged_attention(mode=...)`         -- kernel.py:74-214.
  - mode="fp32"/"fp64": the same algorithm with every intermediate kept in
    fp32/fp64 (the BASELINE tolerance target).  Pinned by a per-element
    brute-force loop in fp64, by `torch.nn.functional.scaled_dot_product_attention`
    on the cases that reduce to it (q_len == kv_len causal, decode), and by
    closed forms (kv_len = 1, constant V, soft_cap -> inf, window >= kv_len)
    and invariants (page permutation, sequence shuffle, NaN isolation).
  - mode="faithful": the reference's own cast points (scores cast to the
    output dtype before scaling, softmax in the output dtype, P cast to the
    value dtype, PV result in the value dtype).  Bit-level agreement with
    XLA:CPU's reduction order is **parity unpinned** (it needs JAX, which is
    not installable here); faithful mode is pinned only to tolerance against
    the fp64 mode.

The reference itself is JAX/Pallas (Python 3.12, jax 0.11.2) and cannot be
imported or built in this environment, so there is no `oracle/_ref`.
"""

from __future__ import annotations

import math
from typing import Any

import numpy as np
import torch

__all__ = [
    "cdiv",
    "align_to",
    "get_dtype_packing",
    "get_kv_cache_shape",
    "merge_kv",
    "quantize_kv",
    "update_kv_cache_np",
    "static_validate_inputs",
    "dynamic_validate_inputs",
    "ref_ragged_paged_attention",
    "merge_attn_results",
    "merge_attn_states",
    "get_kv_cache_shape_hd64",
    "merge_kv_hd64",
    "ref_ragged_paged_attention_hd64",
]


# --------------------------------------------------------------------------
# util.py:20-35
# --------------------------------------------------------------------------
def cdiv(a: int, b: int) -> int:
    """Ceiling division (util.py:20-22)."""
    assert b != 0
    return (a + b - 1) // b


def align_to(x: int, a: int) -> int:
    """Round x up to a multiple of a (util.py:25-26)."""
    return cdiv(x, a) * a


def get_dtype_packing(dtype: torch.dtype) -> int:
    """Elements per 32-bit word: 32 // bits (util.py:33-35)."""
    bits = torch.empty((), dtype=dtype).element_size() * 8
    return 32 // bits


# --------------------------------------------------------------------------
# kernel.py:278-292
# --------------------------------------------------------------------------
def get_kv_cache_shape(total_num_pages, page_size, actual_num_kv_heads,
                       actual_head_dim, kv_dtype):
    """[P, ps, align(2*Hkv, pack) // pack, pack, align(D, 128)] (kernel.py:278-292)."""
    kv_packing = get_dtype_packing(kv_dtype)
    return (
        total_num_pages,
        page_size,
        align_to(actual_num_kv_heads * 2, kv_packing) // kv_packing,
        kv_packing,
        align_to(actual_head_dim, 128),
    )


# --------------------------------------------------------------------------
# kernel.py:1140-1168
# --------------------------------------------------------------------------
def merge_kv(k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """Interleave K and V per head into cache records (kernel.py:1140-1168).

    Combined head c = 2*h + 0 holds K_h and c = 2*h + 1 holds V_h; the
    combined-head axis is zero-padded to a multiple of the packing and the
    last axis to a multiple of 128.
    """
    assert k.shape == v.shape and k.dtype == v.dtype
    t, hkv, d = k.shape
    pack = get_dtype_packing(k.dtype)
    hx2 = hkv * 2
    hx2_pad = align_to(hx2, pack)
    dp = align_to(d, 128)
    kv = torch.cat([k, v], dim=-1).reshape(t, hx2, d)
    out = torch.zeros((t, hx2_pad, dp), dtype=k.dtype)
    out[:, :hx2, :d] = kv
    return out.reshape(t, hx2_pad // pack, pack, dp)


# --------------------------------------------------------------------------
# layers/core/quantization.py:73-103
# --------------------------------------------------------------------------
def quantize_kv(quant_dtype, key, value=None, k_scale=1.0, v_scale=1.0):
    """clamp(x.f32 / scale, finfo.min, finfo.max).to(dtype) (quantization.py:73-103)."""

    def _q(x, scale):
        if scale == 0.0:
            raise ValueError("Quantization scale must be non-zero.")
        info = torch.finfo(quant_dtype)
        return torch.clamp(x.to(torch.float32) / scale, info.min,
                           info.max).to(quant_dtype)

    key = _q(key, k_scale)
    if value is None:
        return key, None
    return key, _q(value, v_scale)


# --------------------------------------------------------------------------
# Cache write, bit exact (kernel.py:148-166)
# --------------------------------------------------------------------------
def _int_view(t: torch.Tensor) -> np.ndarray:
    """Raw integer view of a tensor's bytes (no value conversion)."""
    itype = {1: torch.uint8, 2: torch.int16, 4: torch.int32, 8: torch.int64}[
        t.element_size()]
    return t.contiguous().view(itype).numpy()


def update_kv_cache_np(keys, values, kv_cache, kv_lens, page_indices,
                       cu_q_lens, distribution):
    """Return the cache after the reference's K/V write, computed bitwise.

    For each sequence i < distribution[2], the new tokens
    merge_kv(k, v)[cu_q_lens[i]:cu_q_lens[i+1]] land at logical positions
    [kv_len - q_len, kv_len), i.e. page page_indices[i*pps + j // ps], slot
    j % ps (kernel.py:148-166).  Every other byte is unchanged.  Works on
    integer views so the result is exact for any float dtype.
    """
    merged = _int_view(merge_kv(keys, values))
    cache = _int_view(kv_cache).copy()
    kv_lens = np.asarray(kv_lens, dtype=np.int64)
    page_indices = np.asarray(page_indices, dtype=np.int64)
    cu = np.asarray(cu_q_lens, dtype=np.int64)
    num_seqs = int(np.asarray(distribution)[2])
    page_size = cache.shape[1]
    pps = page_indices.shape[0] // kv_lens.shape[0]
    for i in range(num_seqs):
        q_start, q_end = int(cu[i]), int(cu[i + 1])
        q_len = q_end - q_start
        kv_len = int(kv_lens[i])
        for t in range(q_len):
            j = kv_len - q_len + t
            page = int(page_indices[i * pps + j // page_size])
            cache[page, j % page_size] = merged[q_start + t]
    return torch.from_numpy(cache).view(kv_cache.dtype)


# --------------------------------------------------------------------------
# kernel.py:1366-1538 and :1273-1362
# --------------------------------------------------------------------------
def static_validate_inputs(q, k, v, kv_cache, kv_lens, page_indices,
                           cu_q_lens, distribution, *, use_causal_mask=True,
                           skip_kv_mask=False, sliding_window=None,
                           soft_cap=None, chunk_prefill_size=None,
                           d_block_sizes=None, p_block_sizes=None,
                           m_block_sizes=None, vmem_limit_bytes=None,
                           **unused):
    """Shape/dtype checks raising ValueError (kernel.py:1366-1538)."""
    if use_causal_mask and skip_kv_mask:
        raise ValueError("Can not skip kv mask when using causal mask.")
    if not (q.dim() == k.dim() == v.dim() == 3):
        raise ValueError(f"Expected 3D array for {q.shape=}, {k.shape=}, {v.shape=}")
    if k.shape != v.shape:
        raise ValueError(f"Expected {k.shape=} to be equal to {v.shape=}")
    if not (q.shape[0] == k.shape[0] == v.shape[0]):
        raise ValueError("Expected equal token counts for q, k and v")
    if not (q.shape[2] == k.shape[2] == v.shape[2]):
        raise ValueError("Expected equal head_dim for q, k and v")
    d = q.shape[2]
    hq, hkv = q.shape[1], k.shape[1]
    if hq % hkv != 0:
        raise ValueError(f"Expected {hq=} to be divisible by {hkv=}.")
    expected = get_kv_cache_shape(kv_cache.shape[0], kv_cache.shape[1], hkv, d,
                                  kv_cache.dtype)
    if tuple(kv_cache.shape) != tuple(expected):
        raise ValueError(f"Expected {kv_cache.shape=} to be equal to {expected=}")
    _, page_size, hx2_per_pack, pack, head_dim = kv_cache.shape
    if head_dim != align_to(d, 128):
        raise ValueError(f"Expected {head_dim=} is equal to {align_to(d, 128)=}")
    if not (kv_cache.dtype == k.dtype == v.dtype):
        raise ValueError("Expected kv_cache, k and v dtypes to be equal.")
    if not kv_cache.dtype.is_floating_point:
        raise ValueError(f"Expected {kv_cache.dtype=} to be a floating point.")
    if pack != get_dtype_packing(kv_cache.dtype):
        raise ValueError(f"{pack=} does not match with {kv_cache.dtype=}")
    hx2 = hx2_per_pack * pack
    if hx2 % 2 != 0:
        raise ValueError(f"Combined KV heads must be divisible by 2, but got {hx2}")
    if hx2 % pack != 0 or hx2 // 2 < hkv:
        raise ValueError(f"Invalid {hx2=}, {hkv=}, {pack=}")
    if not (torch.int32 == kv_lens.dtype == page_indices.dtype == cu_q_lens.dtype
            == distribution.dtype):
        raise ValueError("Expected int32 dtype for the metadata arrays")
    if not (kv_lens.dim() == page_indices.dim() == cu_q_lens.dim() == 1):
        raise ValueError("Expected 1D metadata arrays")
    max_num_seqs = kv_lens.shape[0]
    if page_indices.shape[0] % max_num_seqs != 0:
        raise ValueError("Expected num_page_indices to be divisible by max_num_seqs.")
    if tuple(cu_q_lens.shape) != (max_num_seqs + 1,):
        raise ValueError(f"Expected {cu_q_lens.shape=} to be ({max_num_seqs + 1},).")
    if tuple(distribution.shape) != (3,):
        raise ValueError(f"Expected {distribution.shape=} to be (3,).")
    if page_size % pack != 0:
        raise ValueError(f"{page_size=} must be divisible by {pack=}.")
    if sliding_window is not None and sliding_window <= 0:
        raise ValueError(f"{sliding_window=} must be positive.")
    if soft_cap is not None and soft_cap == 0.0:
        raise ValueError(f"{soft_cap=} must not be 0.0.")
    if chunk_prefill_size is not None and chunk_prefill_size <= 0:
        raise ValueError(f"{chunk_prefill_size=} must be positive.")
    for bs, prefix in ((d_block_sizes, "decode"), (p_block_sizes, "prefill"),
                       (m_block_sizes, "mixed")):
        if bs is None:
            continue
        bq_sz, bkv_sz, bq_csz, bkv_csz = bs
        if not (bq_csz > 0 and bq_sz % bq_csz == 0):
            raise ValueError(f"{prefix} {bq_csz=} and {bq_sz=} invalid")
        if not (bkv_csz > 0 and bkv_sz % bkv_csz == 0):
            raise ValueError(f"{prefix} {bkv_csz=} and {bkv_sz=} invalid")
        if bkv_sz % page_size != 0:
            raise ValueError(f"{prefix} {bkv_sz=} must be divisible by {page_size=}.")
        if bkv_csz % page_size != 0:
            raise ValueError(f"{prefix} {bkv_csz=} must be divisible by {page_size=}.")
    if vmem_limit_bytes is not None and vmem_limit_bytes <= 0:
        raise ValueError(f"{vmem_limit_bytes=} must be positive.")


def dynamic_validate_inputs(q, k, v, kv_cache, kv_lens, page_indices, cu_q_lens,
                            distribution, **kw):
    """Value checks over the metadata (kernel.py:1273-1362)."""
    static_validate_inputs(q, k, v, kv_cache, kv_lens, page_indices, cu_q_lens,
                           distribution, **kw)
    max_num_tokens = q.shape[0]
    total_num_pages, page_size = kv_cache.shape[0], kv_cache.shape[1]
    max_num_seqs = kv_lens.shape[0]
    pps = page_indices.shape[0] // max_num_seqs
    dist = [int(x) for x in distribution.tolist()]
    i, j, n = dist
    if not (i <= j <= n):
        raise ValueError(f"Invalid distribution: {dist=}")
    if n > max_num_seqs:
        raise ValueError(f"num_seqs={n} must be <= {max_num_seqs=}")
    cu = cu_q_lens.tolist()
    kvl = kv_lens.tolist()
    pi = page_indices.tolist()
    if cu[n] > max_num_tokens:
        raise ValueError(f"Total q tokens {cu[n]} must be <= {max_num_tokens=}.")
    for s in range(n):
        q_len = cu[s + 1] - cu[s]
        kv_len = kvl[s]
        if not (0 < q_len <= kv_len):
            raise ValueError(f"Require 0 < {q_len=} <= {kv_len=} at sequence {s}.")
        page_cnt = cdiv(kv_len, page_size)
        if page_cnt > pps:
            raise ValueError(f"Require {page_cnt=} <= {pps=} at sequence {s}.")
        for p in range(page_cnt):
            page_idx = pi[s * pps + p]
            if not (0 <= page_idx < total_num_pages):
                raise ValueError(
                    f"Require 0 <= {page_idx=} < {total_num_pages=} at sequence {s}.")


# --------------------------------------------------------------------------
# kernel.py:74-214
# --------------------------------------------------------------------------
def _finfo_min(dtype):
    return float(torch.finfo(dtype).min)


def _softmax_faithful(x: torch.Tensor) -> torch.Tensor:
    """jax.nn.softmax op sequence on a low-precision tensor: every elementwise
    op rounds to x.dtype; the sum accumulates in fp32 and rounds once."""
    x_max = x.amax(dim=-1, keepdim=True)
    unnorm = torch.exp((x - x_max))  # both ops round to x.dtype
    denom = unnorm.to(torch.float32).sum(dim=-1, keepdim=True).to(x.dtype)
    return unnorm / denom


def ref_ragged_paged_attention(
    queries, keys, values, kv_cache, kv_lens, page_indices, cu_q_lens,
    distribution, *, use_causal_mask: bool = True, skip_kv_mask: bool = False,
    skip_kv_update: bool = False, sm_scale: float = 1.0,
    sliding_window: int | None = None, soft_cap: float | None = None,
    out_dtype: Any = None, mask_value: float | None = None,
    q_scale: float | None = None, k_scale: float | None = None,
    v_scale: float | None = None, mode: str = "faithful", validate: bool = True,
    return_lse: bool = False,
):
    """CPU restatement of ref_ragged_paged_attention (kernel.py:74-214).

    Returns (out [cu_q_lens[num_seqs], Hq, D], new_kv_cache), plus, with
    return_lse (fp32/fp64 modes), lse [cu_q_lens[num_seqs], Hq]: the
    natural-log log-sum-exp of each row's unmasked logits, the quantity the
    batched RPA wrapper returns (batched_rpa/wrapper.py:610-623,
    batched_rpa/kernel.py:116-124: m + log(l)).  `mode`:
      "faithful" -- the reference's cast points (kernel.py:185-209) in
                    torch's bf16/fp8 arithmetic.
      "fp32" / "fp64" -- identical algorithm, every intermediate in that
                    precision; out is returned in that precision.
    The cache write is always the bit-exact `update_kv_cache_np`.
    """
    assert mode in ("faithful", "fp32", "fp64")
    if out_dtype is None:  # kernel.py:97-98
        out_dtype = torch.float32 if queries.dtype == torch.float32 else torch.bfloat16
    if mask_value is None:  # kernel.py:100-102
        mask_value = _finfo_min(out_dtype)
    if validate:
        dynamic_validate_inputs(queries, keys, values, kv_cache, kv_lens,
                                page_indices, cu_q_lens, distribution,
                                use_causal_mask=use_causal_mask,
                                skip_kv_mask=skip_kv_mask,
                                sliding_window=sliding_window, soft_cap=soft_cap)
    d = queries.shape[2]
    hq = queries.shape[1]
    hkv = keys.shape[1]
    qpk = hq // hkv
    _, page_size, hx2_per_pack, pack, dp = kv_cache.shape
    hx2 = hx2_per_pack * pack
    max_num_seqs = kv_lens.shape[0]
    pps = page_indices.shape[0] // max_num_seqs
    num_seqs = int(distribution[2])

    kv_dtype = kv_cache.dtype
    # The cache is walked through an integer view so that gathers and
    # scatters move bits, never values (NaN payloads and -0.0 survive).
    work = torch.from_numpy(_int_view(kv_cache).copy())
    merged = torch.from_numpy(_int_view(merge_kv(keys, values)))

    acc_dtype = {"fp32": torch.float32, "fp64": torch.float64}.get(mode)
    assert not (return_lse and mode == "faithful"), "return_lse needs mode fp32 or fp64"
    outputs = []
    lses = []
    for i in range(num_seqs):
        q_start, q_end = int(cu_q_lens[i]), int(cu_q_lens[i + 1])
        q_len = q_end - q_start
        kv_len = int(kv_lens[i])
        idx = page_indices[i * pps:i * pps + cdiv(kv_len, page_size)].long()
        # Gather the logical pages from the cache as updated by the sequences
        # before this one (kernel.py:148-158), overlay the new tokens from the
        # k/v inputs and scatter them back (kernel.py:159-166).
        gathered = work[idx].reshape(-1, hx2_per_pack, pack, dp).clone()
        if not skip_kv_update:
            gathered[kv_len - q_len:kv_len] = merged[q_start:q_end]
            work[idx] = gathered.reshape(-1, page_size, hx2_per_pack, pack, dp)
        gathered = gathered.view(kv_dtype)
        kv = gathered.reshape(-1, hx2, dp)[:, :hkv * 2, :].reshape(-1, hkv, 2 * dp)
        k = kv[:kv_len, :, :dp][:, :, :d]
        v = kv[:kv_len, :, dp:][:, :, :d]
        k = k.repeat_interleave(qpk, dim=1)  # jnp.repeat, kernel.py:173-174
        v = v.repeat_interleave(qpk, dim=1)
        q = queries[q_start:q_end, :, :d]
        if q_scale is not None:  # kernel.py:176-183
            q = q / q_scale
            info = torch.finfo(k.dtype)
            q = torch.clamp(q, min=info.min, max=info.max)
            q = q.to(k.dtype)

        # Logical positions for the causal / window mask (kernel.py:196-204).
        q_pos = (kv_len - q_len) + torch.arange(q_len).view(1, q_len, 1)
        k_pos = torch.arange(kv_len).view(1, 1, kv_len)
        mask = None
        if use_causal_mask:
            mask = q_pos >= k_pos
            if sliding_window is not None:
                mask = mask & (q_pos < k_pos + sliding_window)

        if mode == "faithful":
            # einsum with f32 accumulation, cast to out_dtype (kernel.py:185-187)
            attn = torch.einsum("qhd,khd->hqk", q.to(torch.float32),
                                k.to(torch.float32)).to(out_dtype)
            attn = attn * sm_scale
            if k_scale is not None:
                attn = attn * k_scale
            if q_scale is not None:
                attn = attn * q_scale
            if soft_cap is not None:
                attn = soft_cap * torch.tanh(attn / soft_cap)
            if mask is not None:
                attn = torch.where(mask, attn,
                                   torch.tensor(mask_value, dtype=attn.dtype))
            p = _softmax_faithful(attn).to(v.dtype)  # kernel.py:205
            # einsum in the value dtype (f32 accumulate, one rounding)
            out = torch.einsum("hqk,khd->qhd", p.to(torch.float32),
                               v.to(torch.float32)).to(v.dtype).to(out_dtype)
            if v_scale is not None:
                out = out * v_scale
        else:
            attn = torch.einsum("qhd,khd->hqk", q.to(acc_dtype), k.to(acc_dtype))
            attn = attn * sm_scale
            if k_scale is not None:
                attn = attn * k_scale
            if q_scale is not None:
                attn = attn * q_scale
            if soft_cap is not None:
                attn = soft_cap * torch.tanh(attn / soft_cap)
            if return_lse:
                live = attn if mask is None else torch.where(
                    mask, attn, torch.tensor(float("-inf"), dtype=acc_dtype))
                lses.append(torch.logsumexp(live, dim=-1).transpose(0, 1))  # [q, h]
            if mask is not None:
                attn = torch.where(mask, attn,
                                   torch.tensor(mask_value, dtype=acc_dtype))
            p = torch.softmax(attn, dim=-1)
            out = torch.einsum("hqk,khd->qhd", p, v.to(acc_dtype))
            if v_scale is not None:
                out = out * v_scale
        outputs.append(out)

    if outputs:
        result = torch.cat(outputs, dim=0)
    else:
        rdt = out_dtype if mode == "faithful" else acc_dtype
        result = torch.empty((0, hq, d), dtype=rdt)
    if return_lse:
        lse = torch.cat(lses, dim=0) if lses else torch.empty((0, hq), dtype=acc_dtype)
        return result, work.view(kv_dtype), lse
    return result, work.view(kv_dtype)


def merge_attn_results(out_a, lse_a, out_b, lse_b):
    """Restates merge_attn_results (layers/adapter/cp_attention.py:45-72): the
    numerically stable LSE-weighted combination of two partial attentions,
    out [T, H, D] and lse [T, H] (natural log) each."""
    m = torch.maximum(lse_a, lse_b)
    m_finite = torch.isfinite(m)
    m_safe = torch.where(m_finite, m, torch.zeros_like(m))
    ea = torch.exp(lse_a - m_safe)
    eb = torch.exp(lse_b - m_safe)
    norm = ea + eb
    out_a = torch.nan_to_num(out_a, nan=0.0, posinf=0.0, neginf=0.0)
    out_b = torch.nan_to_num(out_b, nan=0.0, posinf=0.0, neginf=0.0)
    norm_safe = torch.where(norm > 0, norm, torch.ones_like(norm))
    out = (ea.unsqueeze(-1) * out_a + eb.unsqueeze(-1) * out_b) / norm_safe.unsqueeze(-1)
    lse_out = torch.where(m_finite, m + torch.log(norm_safe), m)
    return out, lse_out


def merge_attn_states(outs, lses):
    """merge_attn_results generalised to R partials: outs [R, ..., D], lses
    [R, ...]; the same max, finiteness, nan_to_num and zero-norm rules.  For
    R = 2 it equals merge_attn_results."""
    m = lses.max(dim=0).values
    m_finite = torch.isfinite(m)
    m_safe = torch.where(m_finite, m, torch.zeros_like(m))
    e = torch.exp(lses - m_safe.unsqueeze(0))
    norm = e.sum(dim=0)
    outs = torch.nan_to_num(outs, nan=0.0, posinf=0.0, neginf=0.0)
    norm_safe = torch.where(norm > 0, norm, torch.ones_like(norm))
    out = (e.unsqueeze(-1) * outs).sum(dim=0) / norm_safe.unsqueeze(-1)
    lse_out = torch.where(m_finite, m + torch.log(norm_safe), m)
    return out, lse_out


# --------------------------------------------------------------------------
# kernel_hd64.py (src/vllm_torchtpu/kernels/ragged_paged_attention/v3/
# kernel_hd64.py): head_dim 64, K|V of a head packed in one 128-wide row,
# optional attention sinks.
# --------------------------------------------------------------------------
def get_kv_cache_shape_hd64(total_num_pages, page_size, actual_num_kv_heads,
                            actual_head_dim, kv_dtype):
    """kernel_hd64.py:246-261."""
    assert actual_head_dim == 64
    pack = get_dtype_packing(kv_dtype)
    return (total_num_pages, page_size, align_to(actual_num_kv_heads, pack) // pack,
            pack, 128)


def merge_kv_hd64(k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """Cache records for k/v rows (kernel_hd64.py:1018-1041): head h's row is
    K_h (64 values) then V_h (64 values); heads are zero-padded to a multiple
    of the packing.  [T, align(Hkv, pack) / pack, pack, 128]."""
    assert k.shape == v.shape and k.dtype == v.dtype and k.shape[2] == 64
    t, hkv, _ = k.shape
    pack = get_dtype_packing(k.dtype)
    heads = align_to(hkv, pack)
    out = torch.zeros((t, heads, 128), dtype=k.dtype)
    out[:, :hkv] = torch.cat([k, v], dim=-1)
    return out.reshape(t, heads // pack, pack, 128)


def ref_ragged_paged_attention_hd64(
    queries, keys, values, kv_cache, kv_lens, page_indices, cu_q_lens, distribution,
    attention_sink=None, *, sm_scale: float = 1.0, sliding_window: int | None = None,
    soft_cap: float | None = None, mask_value: float | None = None,
    q_scale: float | None = None, k_scale: float | None = None,
    v_scale: float | None = None, skip_kv_update: bool = False,
    use_causal_mask: bool = True, mode: str = "fp32",
):
    """CPU restatement of ref_ragged_paged_attention_hd64 (kernel_hd64.py:43-183).

    Returns (out [cu_q_lens[num_seqs], Hq, 64], new_kv_cache).  Per sequence:
    the cache pages are gathered, the new [K|V] records overlaid at positions
    [kv_len - q_len, kv_len) and written back (:124-136); logits q . k scaled
    by sm_scale, k_scale, q_scale (:147-152), soft cap (:162-163), the mask --
    causal when use_causal_mask, and the window q_pos - W >= k_pos whether or
    not causal -- replaced by mask_value (:157-164); with attention_sink, the
    sink logit of each q head is prepended to every row before the softmax and
    its column dropped afterwards (:166-172): it adds to the denominator only.
    `mode`: "fp32"/"fp64" keep every intermediate in that precision (the
    tolerance target); "faithful" keeps the reference's cast points (f32
    logits and softmax, probabilities cast to the KV dtype, PV in the KV
    dtype, then the q dtype, then v_scale).
    """
    assert mode in ("faithful", "fp32", "fp64")
    if mask_value is None:  # kernel_hd64.py:65-66, :36
        mask_value = -0.7 * float(torch.finfo(torch.float32).max)
    d = queries.shape[2]
    assert d == 64
    hq, hkv = queries.shape[1], keys.shape[1]
    qpk = hq // hkv
    _, page_size, heads_per_pack, pack, width = kv_cache.shape
    assert width == 128
    heads = heads_per_pack * pack
    max_num_seqs = kv_lens.shape[0]
    pps = page_indices.shape[0] // max_num_seqs
    num_seqs = int(distribution[2])
    kv_dtype = kv_cache.dtype
    work = torch.from_numpy(_int_view(kv_cache).copy())
    merged = torch.from_numpy(_int_view(merge_kv_hd64(keys, values)))
    acc = {"fp32": torch.float32, "fp64": torch.float64, "faithful": torch.float32}[mode]
    outputs = []
    for i in range(num_seqs):
        q_start, q_end = int(cu_q_lens[i]), int(cu_q_lens[i + 1])
        q_len = q_end - q_start
        kv_len = int(kv_lens[i])
        assert kv_len - q_len >= 0
        idx = page_indices[i * pps:i * pps + cdiv(kv_len, page_size)].long()
        gathered = work[idx].reshape(-1, heads_per_pack, pack, 128).clone()
        if not skip_kv_update:
            gathered[kv_len - q_len:kv_len] = merged[q_start:q_end]
            work[idx] = gathered.reshape(-1, page_size, heads_per_pack, pack, 128)
        kv = gathered.view(kv_dtype).reshape(-1, heads, 128)[:kv_len, :hkv]
        kv = kv.repeat_interleave(qpk, dim=1)  # [kv_len, Hq, 128]
        q = queries[q_start:q_end]
        if q_scale is not None:  # kernel_hd64.py:137-144
            q = q / q_scale
            info = torch.finfo(kv_dtype)
            q = torch.clamp(q, min=info.min, max=info.max).to(kv_dtype)
        # q padded with 64 zeros meets only the K half of each row (:118, :146).
        attn = torch.einsum("qhd,khd->hqk", q.to(acc), kv[..., :64].to(acc))
        attn = attn * sm_scale
        if k_scale is not None:
            attn = attn * k_scale
        if q_scale is not None:
            attn = attn * q_scale
        q_pos = (kv_len - q_len) + torch.arange(q_len).view(1, q_len, 1)
        k_pos = torch.arange(kv_len).view(1, 1, kv_len)
        mask = (q_pos < k_pos) if use_causal_mask else torch.zeros((1, q_len, kv_len),
                                                                   dtype=torch.bool)
        if sliding_window is not None:
            mask = mask | (q_pos - sliding_window >= k_pos)
        if soft_cap is not None:
            attn = soft_cap * torch.tanh(attn / soft_cap)
        attn = torch.where(mask, torch.tensor(mask_value, dtype=acc), attn)
        if attention_sink is not None:
            sink = attention_sink.to(acc).view(hq, 1, 1).expand(hq, q_len, 1)
            attn = torch.softmax(torch.cat([sink, attn], dim=2), dim=-1)[..., 1:]
        else:
            attn = torch.softmax(attn, dim=-1)
        vals = kv[..., 64:]
        if mode == "faithful":
            p = attn.to(kv_dtype).to(torch.float32)
            out = torch.einsum("hqk,khd->qhd", p, vals.to(torch.float32)).to(kv_dtype)
            out = out.to(queries.dtype)
        else:
            out = torch.einsum("hqk,khd->qhd", attn, vals.to(acc))
        if v_scale is not None:
            out = out * v_scale
        outputs.append(out)
    if outputs:
        result = torch.cat(outputs, dim=0)
    else:
        result = torch.empty((0, hq, d), dtype=queries.dtype if mode == "faithful" else acc)
    return result, work.view(kv_dtype)


def _self_check():  # pragma: no cover - manual use
    print(get_kv_cache_shape(4, 16, 2, 128, torch.bfloat16), math.pi)
