"""Shared helpers for the RPA tests: an independent brute-force reference and
comparison utilities.  Test infrastructure only."""

from __future__ import annotations

import math

import numpy as np
import torch


# ---------------------------------------------------------------------------
# Number formats, written from their definitions (sign, exponent bits,
# mantissa bits, bias), for the q_scale branch of the brute force.  None of
# this calls torch's casts.
# ---------------------------------------------------------------------------
# (exponent bits, mantissa bits, bias, has_inf): OCP fp8 e4m3fn has no
# infinities and only S.1111.111 as NaN; e5m2 is IEEE-like.
_FP8_FORMATS = {"e4m3fn": (4, 3, 7, False), "e5m2": (5, 2, 15, True)}


def fp8_values(fmt: str) -> np.ndarray:
    """Every finite non-negative value of an fp8 format, ascending (codes
    0x00..0x7f minus NaN/inf), as float64."""
    eb, mb, bias, has_inf = _FP8_FORMATS[fmt]
    vals = []
    for code in range(1 << (eb + mb)):
        e, m = code >> mb, code & ((1 << mb) - 1)
        if e == (1 << eb) - 1 and (has_inf or m == (1 << mb) - 1):
            continue  # inf / NaN codes
        if e == 0:
            vals.append(m * 2.0 ** (1 - bias - mb))
        else:
            vals.append((1 + m / 2.0 ** mb) * 2.0 ** (e - bias))
    return np.array(vals)


def round_to_fp8(x: np.ndarray, fmt: str) -> np.ndarray:
    """Round-to-nearest, ties to the even code (= even mantissa LSB, since the
    codes are ordered like their magnitudes), of values within the format's
    range."""
    vals = fp8_values(fmt)
    a = np.abs(x)
    assert (a <= vals[-1]).all(), "value outside the fp8 range (clip first)"
    hi = np.searchsorted(vals, a, side="left")  # first value >= a
    hi = np.minimum(hi, len(vals) - 1)
    lo = np.maximum(hi - 1, 0)
    dlo, dhi = a - vals[lo], vals[hi] - a
    pick_hi = (dhi < dlo) | ((dhi == dlo) & (hi % 2 == 0))
    r = np.where(pick_hi, vals[hi], vals[lo])
    r = np.where(a == vals[hi], vals[hi], r)
    return np.sign(x) * r


def round_to_bf16(x: np.ndarray) -> np.ndarray:
    """float32 values -> nearest bf16 (ties to even), via the f32 bit pattern."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32).astype(np.float64)


def fmt_max(dtype: torch.dtype) -> float:
    """Largest finite value of a floating format, from its definition."""
    if dtype == torch.bfloat16:
        return (2.0 - 2.0 ** -7) * 2.0 ** 127
    if dtype == torch.float32:
        return (2.0 - 2.0 ** -23) * 2.0 ** 127
    return float(fp8_values({torch.float8_e4m3fn: "e4m3fn",
                             torch.float8_e5m2: "e5m2"}[dtype])[-1])


def quantize_q(q: torch.Tensor, q_scale: float, kv_dtype: torch.dtype) -> np.ndarray:
    """kernel.py:176-183 restated from the definitions: q / q_scale computed in
    q's dtype (an f32 quotient rounded to bf16 for a bf16 q), clipped to the
    KV dtype's finite range, then rounded to the KV dtype."""
    qf = q.to(torch.float64).numpy()
    quot = (qf.astype(np.float32) / np.float32(q_scale)).astype(np.float64)
    if q.dtype == torch.bfloat16:
        quot = round_to_bf16(quot)
    mx = fmt_max(kv_dtype)
    quot = np.clip(quot, -mx, mx)
    if kv_dtype == torch.bfloat16:
        return round_to_bf16(quot)
    if kv_dtype == torch.float32:
        return quot.astype(np.float32).astype(np.float64)
    return round_to_fp8(quot, {torch.float8_e4m3fn: "e4m3fn", torch.float8_e5m2: "e5m2"}[kv_dtype])


def brute_force_rpa(q, k, v, kv_cache, kv_lens, page_indices, cu_q_lens, distribution, *,
                    sm_scale=1.0, sliding_window=None, soft_cap=None, k_scale=None,
                    v_scale=None, q_scale=None, use_causal_mask=True, skip_kv_update=False,
                    return_lse=False, attention_sink=None, window_all_rows=False):
    """Per-element fp64 attention written directly from the semantic contract
    (positions, page table, K/V combined-head interleave), independent of the
    oracle's gather/einsum code.  Returns [num_tokens, Hq, D] float64 (and,
    with return_lse, the per-row log(sum_j exp(logit_j)) [num_tokens, Hq]).
    attention_sink [Hq]: one more term exp(sink) in each row's denominator.
    window_all_rows: without the causal mask, keys j <= pos - sliding_window are
    still excluded (the head_dim 64 contract, kernel_hd64.py:155-158); the v3
    contract windows causal rows only (kernel.py:196-204).
    q_scale (kernel.py:176-183): q is quantized by `quantize_q` and the logit
    multiplied by q_scale.
    A head_dim 64 packed cache is read through its view
    [P, ps, 2 * heads / pack, pack, 64] (K_h at combined head 2h, V_h at 2h + 1)."""
    Q = q.to(torch.float64).numpy() if q_scale is None else quantize_q(q, q_scale, kv_cache.dtype)
    K = k.to(torch.float64).numpy()
    V = v.to(torch.float64).numpy()
    C = kv_cache.to(torch.float64).numpy()
    _, ps, _, pack, _ = kv_cache.shape
    T, Hq, D = q.shape
    Hkv = k.shape[1]
    qpk = Hq // Hkv
    S = kv_lens.shape[0]
    pps = page_indices.shape[0] // S
    n = int(distribution[2])
    cu = [int(x) for x in cu_q_lens.tolist()]
    kvl = [int(x) for x in kv_lens.tolist()]
    pt = [int(x) for x in page_indices.tolist()]
    out = np.zeros((cu[n], Hq, D))
    lse = np.full((cu[n], Hq), -np.inf)
    for s in range(n):
        q0, ql, kl = cu[s], cu[s + 1] - cu[s], kvl[s]
        for i in range(ql):
            pos = kl - ql + i
            for gq in range(Hq):
                h = gq // qpk
                logits, vals = [], []
                for j in range(kl):
                    if skip_kv_update or j < kl - ql:
                        page, slot = pt[s * pps + j // ps], j % ps
                        kr = C[page, slot, (2 * h) // pack, (2 * h) % pack, :D]
                        vr = C[page, slot, (2 * h + 1) // pack, (2 * h + 1) % pack, :D]
                    else:
                        t = q0 + j - (kl - ql)
                        kr, vr = K[t, h], V[t, h]
                    if use_causal_mask:
                        if j > pos:
                            continue
                        if sliding_window is not None and j <= pos - sliding_window:
                            continue
                    elif window_all_rows and sliding_window is not None:
                        if j <= pos - sliding_window:
                            continue
                    x = float(np.dot(Q[q0 + i, gq], kr)) * sm_scale
                    if k_scale is not None:
                        x *= k_scale
                    if q_scale is not None:
                        x *= q_scale
                    if soft_cap is not None:
                        x = soft_cap * math.tanh(x / soft_cap)
                    logits.append(x)
                    vals.append(vr)
                m = max(logits)
                w = [math.exp(x - m) for x in logits]
                tot = sum(w)
                if attention_sink is not None:
                    tot += math.exp(float(attention_sink[gq]) - m)
                o = sum(wi * vi for wi, vi in zip(w, vals)) / tot
                if v_scale is not None:
                    o = o * v_scale
                out[q0 + i, gq] = o
                lse[q0 + i, gq] = m + math.log(tot)
    if return_lse:
        return torch.from_numpy(out), torch.from_numpy(lse)
    return torch.from_numpy(out)


def assert_close(actual, expected, atol, rtol, what=""):
    a = actual.to(torch.float64).cpu()
    e = expected.to(torch.float64).cpu()
    assert a.shape == e.shape, (a.shape, e.shape)
    err = (a - e).abs()
    bound = atol + rtol * e.abs()
    # NaN on one side only is a mismatch (err > bound is False for a NaN err), and
    # so is an infinity the other side does not share (the bound is infinite
    # there); NaN on both sides, or the same infinity, matches.
    inf = torch.isinf(a) | torch.isinf(e)
    bad = (err > bound) | (torch.isnan(a) != torch.isnan(e)) | (inf & (a != e))
    if bad.any():
        idx = bad.nonzero()[0].tolist()
        raise AssertionError(
            f"{what}: {int(bad.sum())}/{bad.numel()} elements out of tolerance "
            f"(atol={atol}, rtol={rtol}); max err {err.max().item():.4g}; first bad {idx}: "
            f"actual {a[tuple(idx)].item():.6g} expected {e[tuple(idx)].item():.6g}")


def bytes_equal(a: torch.Tensor, b: torch.Tensor) -> bool:
    """Bitwise equality of two tensors of the same dtype (NaN-safe)."""
    assert a.dtype == b.dtype and a.shape == b.shape
    itype = {1: torch.uint8, 2: torch.int16, 4: torch.int32, 8: torch.int64}[a.element_size()]
    return bool(torch.equal(a.contiguous().view(itype).cpu(), b.contiguous().view(itype).cpu()))


def bytes_diff(a: torch.Tensor, b: torch.Tensor, limit: int = 8) -> str:
    """Where two same-shaped tensors differ bitwise: count and the first
    `limit` indices with both values (for failure messages)."""
    itype = {1: torch.uint8, 2: torch.int16, 4: torch.int32, 8: torch.int64}[a.element_size()]
    ai = a.contiguous().view(itype).cpu()
    bi = b.contiguous().view(itype).cpu()
    bad = (ai != bi).nonzero()
    lines = [f"{bad.shape[0]} of {ai.numel()} elements differ"]
    for idx in bad[:limit].tolist():
        t = tuple(idx)
        lines.append(f"  at {t}: {int(ai[t]) & 0xff:#04x} vs {int(bi[t]) & 0xff:#04x}"
                     if a.element_size() == 1 else f"  at {t}: {int(ai[t])} vs {int(bi[t])}")
    return "\n".join(lines)
