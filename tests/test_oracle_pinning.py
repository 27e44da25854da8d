"""Pins the CPU oracle (oracle/rpa_oracle.py) before anything is compared to it.

Each oracle function is checked against something that does not share its
code: closed forms, a per-element brute force, torch's SDPA on the cases that
reduce to it, and invariants of the algorithm.  The case lists follow the
reference's own tests (tests/kernels/test_rpa_skip_kv_update.py:98-182,
tests/kernels/experimental/batched_rpa/correctness_test.py:472-986).
"""

import math

import numpy as np
import pytest
import torch

from oracle import rpa_oracle as O
from rpa_testlib import assert_close, brute_force_rpa, bytes_equal

import vllm_torchtpu_amd as R
import vllm_torchtpu_amd.workloads  # noqa: F401

BF16, E4M3, E5M2 = torch.bfloat16, torch.float8_e4m3fn, torch.float8_e5m2


def wl(seq_lens, hq, hkv, d, ps, **kw):
    return R.workloads.make_workload(seq_lens, hq, hkv, d, ps, **kw)


# ---------------------------------------------------------------------------
# util / layout (util.py:20-35, kernel.py:278-292, kernel.py:1140-1168)
# ---------------------------------------------------------------------------
def test_util_closed_forms():
    assert [O.cdiv(a, 16) for a in (0, 1, 16, 17, 32)] == [0, 1, 1, 2, 2]
    assert [O.align_to(a, 128) for a in (1, 80, 128, 129, 240)] == [128, 128, 128, 256, 256]
    assert O.get_dtype_packing(torch.float32) == 1
    assert O.get_dtype_packing(BF16) == 2
    assert O.get_dtype_packing(E4M3) == 4 and O.get_dtype_packing(E5M2) == 4


@pytest.mark.parametrize("hkv,d,dt,expect", [
    (2, 128, BF16, (7, 16, 2, 2, 128)),
    (8, 128, BF16, (7, 16, 8, 2, 128)),
    (1, 80, BF16, (7, 16, 1, 2, 128)),
    (1, 128, E4M3, (7, 16, 1, 4, 128)),   # 2 combined heads padded to 4
    (3, 240, E4M3, (7, 16, 2, 4, 256)),
    (3, 64, torch.float32, (7, 16, 6, 1, 128)),
])
def test_kv_cache_shape(hkv, d, dt, expect):
    assert O.get_kv_cache_shape(7, 16, hkv, d, dt) == expect
    assert R.get_kv_cache_shape(7, 16, hkv, d, dt) == expect


@pytest.mark.parametrize("dt", [BF16, E4M3, torch.float32])
@pytest.mark.parametrize("hkv,d", [(2, 128), (3, 80), (1, 240)])
def test_merge_kv_elementwise(dt, hkv, d):
    g = torch.Generator().manual_seed(3)
    k = torch.randn(5, hkv, d, generator=g).to(dt)
    v = torch.randn(5, hkv, d, generator=g).to(dt)
    m = O.merge_kv(k, v)
    pack = O.get_dtype_packing(dt)
    assert tuple(m.shape[1:]) == O.get_kv_cache_shape(1, 1, hkv, d, dt)[2:]
    mf = m.to(torch.float32)
    hx2, dp = m.shape[1] * pack, m.shape[3]
    for t in range(5):
        for c in range(hx2):
            row = mf[t, c // pack, c % pack]
            if c < 2 * hkv:
                src = (k if c % 2 == 0 else v)[t, c // 2].to(torch.float32)
                assert torch.equal(row[:d], src)
                assert torch.count_nonzero(row[d:]) == 0
            else:
                assert torch.count_nonzero(row) == 0
    assert bytes_equal(R.merge_kv(k, v), m)


# ---------------------------------------------------------------------------
# cache write, bit exact (kernel.py:148-166)
# ---------------------------------------------------------------------------
def _brute_force_cache(w):
    cache = w.kv_cache.clone()
    _, ps, _, pack, dp = cache.shape
    S = w.kv_lens.shape[0]
    pps = w.page_indices.shape[0] // S
    hkv, d = w.k.shape[1], w.k.shape[2]
    itype = {1: torch.uint8, 2: torch.int16, 4: torch.int32}[cache.element_size()]
    ci = cache.view(itype)
    ki, vi = w.k.contiguous().view(itype), w.v.contiguous().view(itype)
    for s in range(w.num_seqs):
        q0, q1 = int(w.cu_q_lens[s]), int(w.cu_q_lens[s + 1])
        kl = int(w.kv_lens[s])
        for t in range(q0, q1):
            j = kl - (q1 - q0) + (t - q0)
            page = int(w.page_indices[s * pps + j // ps])
            rec = ci[page, j % ps].reshape(-1, dp)
            rec.zero_()
            for h in range(hkv):
                rec[2 * h, :d] = ki[t, h]
                rec[2 * h + 1, :d] = vi[t, h]
    return cache


@pytest.mark.parametrize("dt", [BF16, E4M3, torch.float32])
def test_cache_update_bruteforce(dt):
    w = wl([(5, 18), (1, 33), (16, 48), (3, 3)], 6, 3, 80, 16, kv_dtype=dt, q_dtype=BF16,
           seed=7, k_scale=0.5 if dt == E4M3 else None, v_scale=0.5 if dt == E4M3 else None)
    expect = _brute_force_cache(w)
    got = O.update_kv_cache_np(w.k, w.v, w.kv_cache, w.kv_lens, w.page_indices, w.cu_q_lens,
                               w.distribution)
    assert bytes_equal(got, expect)
    _, cache2 = O.ref_ragged_paged_attention(*w.args(), mode="fp32", **w.kwargs)
    assert bytes_equal(cache2, expect)
    # Only the new tokens' records changed.
    changed = (got.view(-1, got.shape[2] * got.shape[3] * got.shape[4]).to(torch.float32) !=
               w.kv_cache.view(got.shape[0] * got.shape[1], -1).to(torch.float32)).any(dim=1)
    assert int(changed.sum()) <= sum(q for q, _ in w.seq_lens)


@pytest.mark.parametrize("kv_len,q_len,dist", [(48, 16, (0, 0, 1)), (33, 1, (1, 1, 1))])
def test_skip_kv_update_invariant(kv_len, q_len, dist):
    """test_rpa_skip_kv_update.py:98-182 restated on the oracle."""
    g = torch.Generator().manual_seed(0)
    hkv, hq, d, ps, P = 2, 4, 128, 16, 8

    def r(*s):
        return (torch.randn(*s, generator=g) * 0.5)

    tk, tv = r(kv_len, hkv, d), r(kv_len, hkv, d)
    query = r(q_len, hq, d).to(BF16)
    gk, gv = r(q_len, hkv, d).to(BF16), r(q_len, hkv, d).to(BF16)
    ck, cv = tk[kv_len - q_len:].to(BF16), tv[kv_len - q_len:].to(BF16)
    shape = O.get_kv_cache_shape(P, ps, hkv, d, BF16)
    cache = torch.zeros(shape, dtype=BF16)
    cache.view(P * ps, *shape[2:])[:kv_len] = O.merge_kv(tk.to(BF16), tv.to(BF16))
    meta = (torch.tensor([kv_len], dtype=torch.int32), torch.arange(P, dtype=torch.int32),
            torch.tensor([0, q_len], dtype=torch.int32), torch.tensor(dist, dtype=torch.int32))

    def run(keys, values, skip):
        return O.ref_ragged_paged_attention(query, keys, values, cache.clone(), *meta,
                                            sm_scale=d ** -0.5, skip_kv_update=skip,
                                            mode="fp32")

    oracle_out, _ = run(ck, cv, False)
    skip_out, skip_cache = run(gk, gv, True)
    bad_out, bad_cache = run(gk, gv, False)
    assert_close(skip_out, oracle_out, 1e-5, 0, "skip path")
    assert bytes_equal(skip_cache, cache)
    assert (bad_out - oracle_out).abs().max() > 1e-2
    assert (bad_cache.float() - cache.float()).abs().max() > 1e-2


# ---------------------------------------------------------------------------
# attention math (kernel.py:185-209)
# ---------------------------------------------------------------------------
BRUTE_CASES = [
    dict(seq_lens=[(5, 18), (1, 29), (12, 12)], hq=4, hkv=2, d=24, ps=16),
    dict(seq_lens=[(7, 20), (1, 9)], hq=6, hkv=3, d=16, ps=8, sliding_window=5),
    dict(seq_lens=[(4, 30)], hq=2, hkv=1, d=32, ps=4, soft_cap=3.0),
    dict(seq_lens=[(3, 11), (2, 2)], hq=4, hkv=4, d=8, ps=4, sliding_window=1),
    dict(seq_lens=[(6, 17), (1, 40)], hq=8, hkv=2, d=20, ps=16, sliding_window=8,
         soft_cap=5.0),
]


@pytest.mark.parametrize("case", range(len(BRUTE_CASES)))
@pytest.mark.parametrize("kv_dtype", [BF16, E4M3])
def test_oracle_vs_bruteforce(case, kv_dtype):
    c = dict(BRUTE_CASES[case])
    seq_lens, hq, hkv, d, ps = (c.pop(x) for x in ("seq_lens", "hq", "hkv", "d", "ps"))
    scales = dict(k_scale=0.75, v_scale=1.5) if kv_dtype == E4M3 else {}
    w = wl(seq_lens, hq, hkv, d, ps, kv_dtype=kv_dtype, seed=11 + case, **scales, **c)
    out, _ = O.ref_ragged_paged_attention(*w.args(), mode="fp64", **w.kwargs)
    bf = brute_force_rpa(*w.args(), **w.kwargs)
    assert_close(out, bf, 1e-10, 1e-10, "fp64 oracle vs brute force")
    out32, _ = O.ref_ragged_paged_attention(*w.args(), mode="fp32", **w.kwargs)
    assert_close(out32, bf, 1e-5, 1e-5, "fp32 oracle vs brute force")


def test_oracle_f16_vs_bruteforce():
    c = dict(BRUTE_CASES[4])
    seq_lens, hq, hkv, d, ps = (c.pop(x) for x in ("seq_lens", "hq", "hkv", "d", "ps"))
    w = wl(seq_lens, hq, hkv, d, ps, q_dtype=torch.float16, kv_dtype=torch.float16, seed=17,
           **c)
    out, cache = O.ref_ragged_paged_attention(*w.args(), mode="fp64", **w.kwargs)
    assert cache.dtype == torch.float16
    assert_close(out, brute_force_rpa(*w.args(), **w.kwargs), 1e-10, 1e-10, "f16")


def test_oracle_non_causal_vs_bruteforce():
    w = wl([(5, 18), (3, 7)], 4, 2, 32, 8, seed=5)
    out, _ = O.ref_ragged_paged_attention(*w.args(), mode="fp64", use_causal_mask=False,
                                          **w.kwargs)
    bf = brute_force_rpa(*w.args(), use_causal_mask=False, **w.kwargs)
    assert_close(out, bf, 1e-10, 1e-10)


# ---------------------------------------------------------------------------
# q_scale branch (kernel.py:176-183): q / q_scale, clip to the KV dtype's
# range, cast to the KV dtype; the logits are multiplied by q_scale.
# ---------------------------------------------------------------------------
def test_format_tables_from_definitions():
    """The brute force's own fp8 / bf16 rounding: closed forms of the formats,
    and agreement with torch's casts on random values (two independent
    implementations)."""
    from rpa_testlib import fp8_values, round_to_bf16, round_to_fp8

    e4 = fp8_values("e4m3fn")
    assert len(e4) == 127 and e4[-1] == 448.0 and e4[1] == 2.0 ** -9
    e5 = fp8_values("e5m2")
    assert len(e5) == 124 and e5[-1] == 57344.0 and e5[1] == 2.0 ** -16
    assert (np.diff(e4) > 0).all() and (np.diff(e5) > 0).all()
    g = torch.Generator().manual_seed(3)
    x = torch.randn(20000, generator=g, dtype=torch.float64) * 30
    for fmt, dt, mx in (("e4m3fn", E4M3, 448.0), ("e5m2", E5M2, 57344.0)):
        xc = x.clamp(-mx, mx)
        mine = round_to_fp8(xc.numpy(), fmt)
        theirs = xc.to(torch.float32).to(dt).to(torch.float64).numpy()
        assert np.array_equal(mine, theirs), fmt
    # Ties go to the even code: 1 + 2^-4 sits between 1 and 1.125 in e4m3fn.
    assert round_to_fp8(np.array([1.0625, 1.1875]), "e4m3fn").tolist() == [1.0, 1.25]
    xf = x.to(torch.float32)
    assert np.array_equal(round_to_bf16(xf.numpy()),
                          xf.to(BF16).to(torch.float64).numpy())


Q_SCALE_CASES = [
    (BF16, 0.37, 1.0),
    (E4M3, 0.5, 1.0),
    (E4M3, 0.004, 1.0),   # q / q_scale beyond 448 for |q| > 1.8: the clip matters
    (E5M2, 0.25, 1.0),
    (E4M3, 2.0, 40.0),    # large q: clipped after the division
]


@pytest.mark.parametrize("case", range(len(Q_SCALE_CASES)))
def test_oracle_q_scale_vs_bruteforce(case):
    kv_dtype, q_scale, q_mul = Q_SCALE_CASES[case]
    scales = dict(k_scale=0.75, v_scale=1.5) if kv_dtype != BF16 else {}
    w = wl([(5, 18), (1, 29), (7, 40)], 8, 2, 32, 16, kv_dtype=kv_dtype, seed=61 + case,
           q_scale=q_scale, **scales)
    w.q.mul_(q_mul)
    out, _ = O.ref_ragged_paged_attention(*w.args(), mode="fp64", **w.kwargs)
    bf = brute_force_rpa(*w.args(), **w.kwargs)
    assert_close(out, bf, 1e-10, 1e-10, "fp64 oracle vs brute force, q_scale")
    out32, _ = O.ref_ragged_paged_attention(*w.args(), mode="fp32", **w.kwargs)
    assert_close(out32, bf, 1e-5, 1e-5, "fp32 oracle vs brute force, q_scale")


@pytest.mark.parametrize("mistake", ["no_multiply_back", "no_clip", "no_cast"])
def test_q_scale_pin_catches_planted_mistakes(mistake):
    """Slips of the q_scale branch, planted in the oracle's inputs on the CPU,
    move its result far from the brute force (the pin above holds to 1e-10)."""
    from rpa_testlib import round_to_bf16

    kv_dtype, q_scale, q_mul = (E4M3, 0.004, 1.0) if mistake != "no_cast" else (E4M3, 0.5, 1.0)
    w = wl([(5, 18), (1, 29), (7, 40)], 8, 2, 32, 16, kv_dtype=kv_dtype, seed=71,
           q_scale=q_scale, k_scale=0.75, v_scale=1.5)
    w.q.mul_(q_mul)
    bf = brute_force_rpa(*w.args(), **w.kwargs)
    args, kw = list(w.args()), dict(w.kwargs)
    qd = torch.from_numpy(round_to_bf16((w.q.float() / q_scale).numpy()))
    if mistake == "no_multiply_back":
        # q quantized as the reference does, logits never multiplied by q_scale.
        args[0] = qd.clamp(-448, 448).to(E4M3).to(torch.float64)
        kw.pop("q_scale")
    elif mistake == "no_clip":
        # Out-of-range quotients left unclipped (carried at full precision).
        args[0] = qd.to(torch.float64)
        kw.pop("q_scale")
        kw["k_scale"] = kw["k_scale"] * q_scale
    else:
        # q never rounded to the KV dtype.
        args[0] = qd.to(torch.float64)
        kw.pop("q_scale")
        kw["k_scale"] = kw["k_scale"] * q_scale
    out, _ = O.ref_ragged_paged_attention(*args, mode="fp64", validate=False, **kw)
    n = bf.shape[0]
    assert (out[:n] - bf).abs().max().item() > 1e-3, mistake


def _sdpa(q, k, v, causal, scale):
    # q [L, H, D], k/v [S, H, D] -> [L, H, D], fp64
    o = torch.nn.functional.scaled_dot_product_attention(
        q.transpose(0, 1).double(), k.transpose(0, 1).double(), v.transpose(0, 1).double(),
        is_causal=causal, scale=scale)
    return o.transpose(0, 1)


@pytest.mark.parametrize("qpk", [1, 4])
def test_prefill_equals_causal_sdpa(qpk):
    """q_len == kv_len with no window/cap is causal SDPA on the new tokens."""
    hkv, d, L = 2, 64, 37
    w = wl([(L, L)], hkv * qpk, hkv, d, 16, seed=2)
    out, _ = O.ref_ragged_paged_attention(*w.args(), mode="fp64", **w.kwargs)
    k = w.k[:L].repeat_interleave(qpk, dim=1)
    v = w.v[:L].repeat_interleave(qpk, dim=1)
    ref = _sdpa(w.q[:L], k, v, True, d ** -0.5)
    assert_close(out, ref, 1e-10, 1e-10)


def test_decode_equals_unmasked_sdpa():
    hkv, qpk, d = 2, 4, 128
    w = wl([(1, 70), (1, 5)], hkv * qpk, hkv, d, 16, seed=4)
    out, cache = O.ref_ragged_paged_attention(*w.args(), mode="fp64", **w.kwargs)
    for s, (ql, kl) in enumerate(w.seq_lens):
        pages = w.page_indices[s * 5:s * 5 + O.cdiv(kl, 16)]
        S = w.kv_lens.shape[0]
        pps = w.page_indices.shape[0] // S
        pages = w.page_indices[s * pps:s * pps + O.cdiv(kl, 16)].long()
        rec = cache[pages].reshape(-1, 2 * hkv, d)[:kl]
        k = rec[:, 0::2].repeat_interleave(qpk, dim=1)
        v = rec[:, 1::2].repeat_interleave(qpk, dim=1)
        ref = _sdpa(w.q[s:s + 1], k, v, False, d ** -0.5)
        assert_close(out[s:s + 1], ref, 1e-10, 1e-10, f"seq {s}")


def test_closed_forms():
    d = 32
    # kv_len == 1: out = v0 * v_scale
    w = wl([(1, 1)], 4, 2, d, 16, seed=9, kv_dtype=E4M3, k_scale=2.0, v_scale=0.5)
    out, _ = O.ref_ragged_paged_attention(*w.args(), mode="fp64", **w.kwargs)
    expect = w.v[0].double().repeat_interleave(2, dim=0) * 0.5
    assert_close(out[0], expect, 1e-12, 0)
    # constant V everywhere -> out = that constant
    w = wl([(3, 20), (1, 9)], 4, 2, d, 8, seed=10)
    w.kv_cache.view(-1, d if d == 128 else 128)[:] = 0  # zero everything first
    cache = w.kv_cache.view(w.kv_cache.shape[0], w.kv_cache.shape[1], -1, 128)
    cache[:, :, 1::2, :d] = 0.375
    w.v[:] = 0.375
    out, _ = O.ref_ragged_paged_attention(*w.args(), mode="fp64", **w.kwargs)
    assert_close(out, torch.full_like(out, 0.375), 1e-12, 0)


def test_limits_reduce_to_plain():
    w = wl([(6, 40), (1, 17)], 4, 2, 64, 16, seed=12)
    base, _ = O.ref_ragged_paged_attention(*w.args(), mode="fp64", **w.kwargs)
    capped, _ = O.ref_ragged_paged_attention(*w.args(), mode="fp64", soft_cap=1e9, **w.kwargs)
    assert_close(capped, base, 1e-9, 1e-9, "soft_cap -> inf")
    wide, _ = O.ref_ragged_paged_attention(*w.args(), mode="fp64", sliding_window=40,
                                           **w.kwargs)
    assert_close(wide, base, 0, 0, "window >= kv_len")
    narrow, _ = O.ref_ragged_paged_attention(*w.args(), mode="fp64", sliding_window=39,
                                             **w.kwargs)
    assert (narrow - base).abs().max() > 0  # the window actually bites at 39


def test_page_permutation_invariance():
    w = wl([(5, 40), (1, 63), (9, 9)], 8, 2, 128, 16, seed=13)
    out, cache = O.ref_ragged_paged_attention(*w.args(), mode="fp64", **w.kwargs)
    P = w.kv_cache.shape[0]
    perm = torch.randperm(P, generator=torch.Generator().manual_seed(1))
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(P)
    cache_p = w.kv_cache[inv]            # physical page x moves to perm[x]
    table_p = perm[w.page_indices.long()].to(torch.int32)
    out2, cache2 = O.ref_ragged_paged_attention(w.q, w.k, w.v, cache_p, w.kv_lens, table_p,
                                                w.cu_q_lens, w.distribution, mode="fp64",
                                                **w.kwargs)
    assert_close(out2, out, 0, 0)
    assert bytes_equal(cache2[perm], cache)


def test_sequence_shuffle_invariance():
    seqs = [(5, 40), (1, 63), (9, 9), (2, 30)]
    w = wl(seqs, 4, 2, 64, 16, seed=14)
    out, _ = O.ref_ragged_paged_attention(*w.args(), mode="fp64", **w.kwargs)
    order = [2, 0, 3, 1]
    S = w.kv_lens.shape[0]
    pps = w.page_indices.shape[0] // S
    cu = w.cu_q_lens.tolist()
    rows = torch.cat([torch.arange(cu[s], cu[s + 1]) for s in order])
    q2, k2, v2 = w.q[rows], w.k[rows], w.v[rows]
    pt2 = torch.cat([w.page_indices[s * pps:(s + 1) * pps] for s in order])
    kvl2 = w.kv_lens[order]
    cu2 = torch.zeros(S + 1, dtype=torch.int32)
    cu2[1:] = torch.cumsum(torch.tensor([seqs[s][0] for s in order]), 0)
    out2, _ = O.ref_ragged_paged_attention(q2, k2, v2, w.kv_cache, kvl2, pt2, cu2,
                                           w.distribution, mode="fp64", **w.kwargs)
    assert_close(out2, out[rows], 0, 0)


def test_nan_poison_does_not_leak():
    """Unused rows/pages/table slots are NaN (correctness_test.py:280-323)."""
    w = wl([(5, 18), (1, 129), (3, 33)], 8, 2, 128, 16, seed=15, nan_fill=True,
           max_num_seqs=5, max_num_tokens=16)
    out, _ = O.ref_ragged_paged_attention(*w.args(), mode="fp32", **w.kwargs)
    assert torch.isfinite(out).all()


def test_faithful_mode_tolerance():
    """Faithful (bf16 cast points) vs fp64: inside the bf16 budget."""
    w = wl([(16, 100), (1, 300), (64, 64)], 8, 2, 128, 16, seed=16)
    f, _ = O.ref_ragged_paged_attention(*w.args(), mode="faithful", **w.kwargs)
    e, _ = O.ref_ragged_paged_attention(*w.args(), mode="fp64", **w.kwargs)
    assert f.dtype == BF16
    assert_close(f, e, 3e-2, 3e-2, "faithful vs fp64")


def test_quantize_kv():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(1000, generator=g) * 300
    for dt, rel in ((E4M3, 2 ** -4), (E5M2, 2 ** -3)):
        for scale in (0.5, 1.0, 1.7):
            qk, qv = O.quantize_kv(dt, x, x, scale, scale)
            assert qk.dtype == dt and qv.dtype == dt
            back = qk.to(torch.float32)
            clip = torch.clamp(x / scale, torch.finfo(dt).min, torch.finfo(dt).max)
            assert torch.isfinite(back).all()
            err = (back - clip).abs()
            assert bool((err <= rel * clip.abs() + 2 ** -9 + 1e-12).all())
            qk2, _ = R.quantize_kv(dt, x, None, scale)
            assert bytes_equal(qk2, qk)
    with pytest.raises(ValueError):
        O.quantize_kv(E4M3, x, x, 0.0, 1.0)


# ---------------------------------------------------------------------------
# validators (kernel.py:1273-1538)
# ---------------------------------------------------------------------------
def _valid():
    w = wl([(3, 20), (1, 9)], 4, 2, 128, 16, seed=1, max_num_seqs=3)
    return w


def _bad_cases():
    """(description, mutator) pairs; each must raise ValueError."""
    def mutate(**ch):
        def f(a):
            a = dict(a)
            a.update(ch)
            return a
        return f
    w = _valid()
    base = dict(zip(("queries", "keys", "values", "kv_cache", "kv_lens", "page_indices",
                     "cu_q_lens", "distribution"), w.args()))
    cases = [
        ("causal+skip_kv_mask", base, dict(skip_kv_mask=True)),
        ("q not 3d", dict(base, queries=w.q[:, :, None]), {}),
        ("k/v shape", dict(base, values=w.v[:, :1]), {}),
        ("token count", dict(base, keys=w.k[:-1], values=w.v[:-1]), {}),
        ("head dim", dict(base, keys=w.k[..., :64], values=w.v[..., :64]), {}),
        ("q heads % kv heads", dict(base, queries=w.q[:, :3]), {}),
        ("cache shape", dict(base, kv_cache=w.kv_cache[..., :64]), {}),
        ("kv dtype", dict(base, kv_cache=w.kv_cache.float()), {}),
        ("int32 metadata", dict(base, kv_lens=w.kv_lens.long()), {}),
        ("1d metadata", dict(base, page_indices=w.page_indices.view(3, -1)), {}),
        ("pps divisibility", dict(base, page_indices=w.page_indices[:-1]), {}),
        ("cu_q_lens shape", dict(base, cu_q_lens=w.cu_q_lens[:-1]), {}),
        ("distribution shape", dict(base, distribution=w.distribution[:2]), {}),
        ("window", base, dict(sliding_window=0)),
        ("soft cap", base, dict(soft_cap=0.0)),
        ("chunk prefill", base, dict(chunk_prefill_size=0)),
        ("block sizes", base, dict(d_block_sizes=(4, 32, 3, 16))),
        ("bkv % page", base, dict(m_block_sizes=(4, 24, 2, 8))),
        ("vmem", base, dict(vmem_limit_bytes=0)),
    ]
    return cases


@pytest.mark.parametrize("idx", range(len(_bad_cases())))
def test_static_validation_raises(idx):
    desc, args, kw = _bad_cases()[idx]
    with pytest.raises(ValueError):
        O.static_validate_inputs(*args.values(), **kw)
    with pytest.raises(ValueError):
        R.static_validate_inputs(*args.values(), **kw)


def _dyn_bad():
    w = _valid()
    out = []
    d = w.distribution.clone(); d[:] = torch.tensor([2, 1, 2]); out.append(("order", d, None, None, None))
    d = w.distribution.clone(); d[2] = 4; out.append(("num_seqs > max", d, None, None, None))
    kvl = w.kv_lens.clone(); kvl[1] = 0; out.append(("q_len > kv_len", None, kvl, None, None))
    kvl = w.kv_lens.clone(); kvl[0] = 10 ** 4; out.append(("too many pages", None, kvl, None, None))
    pt = w.page_indices.clone(); pt[0] = w.kv_cache.shape[0]; out.append(("page oob", None, None, pt, None))
    cu = w.cu_q_lens.clone(); cu[1] = cu[0]; out.append(("empty q", None, None, None, cu))
    return out


@pytest.mark.parametrize("idx", range(6))
def test_dynamic_validation_raises(idx):
    w = _valid()
    _, dist, kvl, pt, cu = _dyn_bad()[idx]
    args = [w.q, w.k, w.v, w.kv_cache, kvl if kvl is not None else w.kv_lens,
            pt if pt is not None else w.page_indices, cu if cu is not None else w.cu_q_lens,
            dist if dist is not None else w.distribution]
    with pytest.raises(ValueError):
        O.dynamic_validate_inputs(*args)
    with pytest.raises(ValueError):
        R.dynamic_validate_inputs(*args)
    O.dynamic_validate_inputs(*w.args())
    R.dynamic_validate_inputs(*w.args())


def test_algorithmic_bytes_formula():
    """Closed-form byte count on a hand-computed case."""
    import vllm_torchtpu_amd.workloads as WL

    kvl, cu = [100, 7], [0, 1, 4]
    b = WL.algorithmic_bytes(kvl, cu, 2, 8, 2, 128, 128, 16, 2, 2, 2)
    rec = 2 * 2 * 128 * 2
    expect = (100 + 7) * rec + 4 * rec + 4 * 8 * 128 * 4 + (7 + 1) * 4 + (3 * 2 + 4) * 4
    assert b == expect
    assert WL.algorithmic_bytes(kvl, cu, 2, 8, 2, 128, 128, 16, 2, 2, 2,
                                kv_write=False) == expect - 4 * rec
    # decode kernel: only sequence 0 (q_len 1) counts, q read only.
    assert WL.decode_kernel_bytes(kvl, cu, 2, 8, 2, 128, 128, 16, 2, 2) == \
        100 * rec + 8 * 128 * 2 + 7 * 4 + (3 * 2 + 4) * 4
    assert WL.algorithmic_flops(kvl, cu, 2, 8, 128) == 4 * 128 * 8 * (100 + 5 + 6 + 7)
    assert WL.prefill_flops(kvl, cu, 2, 8, 128) == 4 * 128 * 8 * (5 + 6 + 7)
    assert math.isclose(WL.algorithmic_flops([10], [0, 4], 1, 1, 1, sliding_window=8),
                        4 * (7 + 8 + 8 + 8))


# ---------------------------------------------------------------------------
# LSE output and the LSE merge (batched_rpa/wrapper.py:610-623,
# layers/adapter/cp_attention.py:45-72)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("case", range(len(BRUTE_CASES)))
def test_oracle_lse_vs_bruteforce(case):
    c = dict(BRUTE_CASES[case])
    seq_lens, hq, hkv, d, ps = (c.pop(x) for x in ("seq_lens", "hq", "hkv", "d", "ps"))
    w = wl(seq_lens, hq, hkv, d, ps, kv_dtype=E4M3, seed=31 + case, k_scale=0.75,
           v_scale=1.5, **c)
    out, _, lse = O.ref_ragged_paged_attention(*w.args(), mode="fp64", return_lse=True,
                                               **w.kwargs)
    bf_out, bf_lse = brute_force_rpa(*w.args(), return_lse=True, **w.kwargs)
    assert_close(out, bf_out, 1e-10, 1e-10, "out")
    assert_close(lse, bf_lse, 1e-10, 1e-10, "lse")


def test_lse_closed_forms():
    # One key: lse is that key's logit.
    w = wl([(1, 1)], 2, 1, 16, 16, seed=41)
    _, _, lse = O.ref_ragged_paged_attention(*w.args(), mode="fp64", return_lse=True,
                                             **w.kwargs)
    logit = (w.q[0].double() @ w.k[0, 0].double()) * w.kwargs["sm_scale"]
    assert_close(lse[0], logit, 1e-12, 0, "single key")
    # q = 0: every logit is 0, so lse = log(number of attended keys).
    w = wl([(3, 20), (1, 9)], 4, 2, 32, 8, seed=42, sliding_window=5)
    w.q.zero_()
    _, _, lse = O.ref_ragged_paged_attention(*w.args(), mode="fp64", return_lse=True,
                                             **w.kwargs)
    counts = torch.tensor([5.0, 5.0, 5.0, 5.0], dtype=torch.float64)  # window 5 everywhere
    assert_close(lse, counts.log().view(-1, 1).expand(4, 4), 1e-12, 0, "log n")


def _partial(q, k, v, idx, scale):
    """fp64 attention of q [H, D] over keys idx of k/v [n, D]: (out, lse)."""
    s = (q @ k[idx].T) * scale                      # [H, m]
    lse = torch.logsumexp(s, dim=-1)
    out = torch.softmax(s, dim=-1) @ v[idx]
    return out, lse


def test_merge_split_identity():
    """Attention over a key set equals the merge of the attentions over any
    partition of it: the identity context-parallel decoding relies on."""
    g = torch.Generator().manual_seed(43)
    H, D, n = 6, 32, 50
    q = torch.randn(H, D, generator=g, dtype=torch.float64)
    k = torch.randn(n, D, generator=g, dtype=torch.float64)
    v = torch.randn(n, D, generator=g, dtype=torch.float64)
    full_out, full_lse = _partial(q, k, v, torch.arange(n), 0.3)
    perm = torch.randperm(n, generator=g)
    a, b, c = perm[:7], perm[7:31], perm[31:]
    pa, pb, pc = (_partial(q, k, v, i, 0.3) for i in (a, b, c))
    out2, lse2 = O.merge_attn_results(*_partial(q, k, v, perm[:20], 0.3),
                                      *_partial(q, k, v, perm[20:], 0.3))
    assert_close(out2, full_out, 1e-12, 1e-12, "two-way")
    assert_close(lse2, full_lse, 1e-12, 1e-12, "two-way lse")
    out3, lse3 = O.merge_attn_states(torch.stack([pa[0], pb[0], pc[0]]),
                                     torch.stack([pa[1], pb[1], pc[1]]))
    assert_close(out3, full_out, 1e-12, 1e-12, "three-way")
    assert_close(lse3, full_lse, 1e-12, 1e-12, "three-way lse")
    # R = 2 of the generalisation is the reference function.
    o_s, l_s = O.merge_attn_states(torch.stack([pa[0], pb[0]]), torch.stack([pa[1], pb[1]]))
    o_r, l_r = O.merge_attn_results(pa[0], pa[1], pb[0], pb[1])
    assert torch.equal(o_s, o_r) and torch.equal(l_s, l_r)


def test_merge_closed_forms():
    g = torch.Generator().manual_seed(44)
    out_a = torch.randn(3, 2, 8, generator=g, dtype=torch.float64)
    lse_a = torch.randn(3, 2, generator=g, dtype=torch.float64)
    # A partial with lse -inf (no keys) drops out, even with a NaN output.
    out_b = torch.full_like(out_a, float("nan"))
    lse_b = torch.full_like(lse_a, float("-inf"))
    o, l = O.merge_attn_results(out_a, lse_a, out_b, lse_b)
    assert_close(o, out_a, 0, 0)
    assert_close(l, lse_a, 0, 0)
    # Equal lses average the outputs and add log 2.
    o, l = O.merge_attn_results(out_a, lse_a, -out_a, lse_a)
    assert_close(o, torch.zeros_like(o), 1e-15, 0)
    assert_close(l, lse_a + math.log(2.0), 1e-15, 1e-15)
    # Both partials empty: output 0, lse -inf.
    o, l = O.merge_attn_results(out_b, lse_b, out_b, lse_b)
    assert torch.equal(o, torch.zeros_like(o)) and bool(torch.isneginf(l).all())


def test_merge_nan_lse_propagates():
    """merge_attn_results takes the max with torch.maximum, which propagates a
    NaN lse (cp_attention.py:59): that row's output and lse are NaN; other
    rows are untouched."""
    out_a = torch.ones(3, 1, 4)
    out_b = torch.full((3, 1, 4), 2.0)
    lse_a = torch.tensor([[0.0], [float("nan")], [1.0]])
    lse_b = torch.tensor([[0.0], [0.0], [float("nan")]])
    o, l = O.merge_attn_results(out_a, lse_a, out_b, lse_b)
    assert torch.isnan(l[1:]).all() and torch.isnan(o[1:]).all()
    assert torch.allclose(o[0], torch.full((1, 4), 1.5)) and abs(float(l[0, 0]) - math.log(2)) < 1e-6
    o3, l3 = O.merge_attn_states(torch.stack([out_a, out_b]), torch.stack([lse_a, lse_b]))
    assert torch.equal(torch.isnan(o3), torch.isnan(o)) and torch.equal(torch.isnan(l3), torch.isnan(l))



def test_assert_close_flags_one_sided_nan():
    """The parity helper treats NaN on one side only as a mismatch (a NaN error
    compares false against any bound), NaN on both sides and equal infinities as
    matches."""
    one = torch.tensor([1.0, 2.0])
    with pytest.raises(AssertionError):
        assert_close(torch.tensor([float("nan"), 2.0]), one, 1e-2, 1e-2, "nan vs finite")
    with pytest.raises(AssertionError):
        assert_close(one, torch.tensor([1.0, float("nan")]), 1e-2, 1e-2, "finite vs nan")
    with pytest.raises(AssertionError):
        assert_close(torch.tensor([float("inf")]), torch.tensor([-float("inf")]), 1e-2, 1e-2)
    with pytest.raises(AssertionError):
        assert_close(torch.tensor([3.0]), torch.tensor([float("inf")]), 1e-2, 1e-2)
    assert_close(torch.tensor([float("nan"), float("inf")]),
                 torch.tensor([float("nan"), float("inf")]), 1e-2, 1e-2, "matching")
