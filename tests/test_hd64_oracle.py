"""Pins for the head_dim 64 oracle (ref_ragged_paged_attention_hd64,
kernel_hd64.py:43-183) and the hd64 host API: layout byte checks, agreement
with the (separately pinned) v3 oracle on the same logical K/V, a per-element
fp64 brute force with sinks, the closed form of a sink, and the validators'
ValueError table (kernel_hd64.py:1211-1316)."""

import math

import pytest
import torch

from oracle import rpa_oracle as O
from rpa_testlib import assert_close, brute_force_rpa, bytes_equal

import vllm_torchtpu_amd as R
import vllm_torchtpu_amd.workloads as W

BF16, E4M3, E5M2 = torch.bfloat16, torch.float8_e4m3fn, torch.float8_e5m2


def wl64(seq_lens, hq, hkv, ps, **kw):
    return W.make_workload(seq_lens, hq, hkv, 64, ps, layout="hd64", **kw)


def as_view(cache):
    """The hd64 cache as [P, ps, 2 * heads / pack, pack, 64] (K_h at combined
    head 2h, V_h at 2h + 1)."""
    p, ps, hp, pack, _ = cache.shape
    return cache.view(p, ps, 2 * hp, pack, 64)


def to_v3(cache, hkv):
    """The same logical K/V in the v3 layout (head_dim padded to 128)."""
    p, ps, hp, pack, _ = cache.shape
    rows = cache.reshape(p, ps, hp * pack, 128)[:, :, :hkv]
    v3 = torch.zeros(O.get_kv_cache_shape(p, ps, hkv, 64, cache.dtype), dtype=cache.dtype)
    flat = v3.view(p, ps, -1, 128)
    flat[:, :, 0:2 * hkv:2, :64] = rows[..., :64]
    flat[:, :, 1:2 * hkv:2, :64] = rows[..., 64:]
    return v3


@pytest.mark.parametrize("hkv,dt,expect", [
    (2, BF16, (9, 16, 1, 2, 128)),
    (1, BF16, (9, 16, 1, 2, 128)),   # one head padded to the packing
    (3, E4M3, (9, 16, 1, 4, 128)),
    (5, E5M2, (9, 16, 2, 4, 128)),
    (3, torch.float32, (9, 16, 3, 1, 128)),
])
def test_hd64_cache_shape(hkv, dt, expect):
    assert O.get_kv_cache_shape_hd64(9, 16, hkv, 64, dt) == expect
    assert R.get_kv_cache_shape_hd64(9, 16, hkv, 64, dt) == expect


@pytest.mark.parametrize("dt", [BF16, E4M3, torch.float32])
@pytest.mark.parametrize("hkv", [1, 2, 3])
def test_merge_kv_hd64_elementwise(dt, hkv):
    g = torch.Generator().manual_seed(4)
    k = torch.randn(5, hkv, 64, generator=g).to(dt)
    v = torch.randn(5, hkv, 64, generator=g).to(dt)
    m = O.merge_kv_hd64(k, v)
    pack = O.get_dtype_packing(dt)
    heads = O.align_to(hkv, pack)
    assert tuple(m.shape) == (5, heads // pack, pack, 128)
    rows = m.reshape(5, heads, 128)
    for t in range(5):
        for h in range(heads):
            for e in range(128):
                if h < hkv:
                    want = k[t, h, e] if e < 64 else v[t, h, e - 64]
                else:
                    want = torch.zeros((), dtype=dt)
                assert bytes_equal(rows[t, h, e], want)
    assert bytes_equal(R.merge_kv_hd64(k, v), m)


@pytest.mark.parametrize("dt", [BF16, E4M3])
@pytest.mark.parametrize("hkv,hq", [(2, 4), (1, 3), (3, 6)])
def test_hd64_matches_v3_oracle(dt, hkv, hq):
    """No sink: the hd64 oracle equals the v3 oracle on the same logical K/V,
    outputs (fp64) and the updated caches (bit exact, after relayout)."""
    scales = dict(k_scale=0.8, v_scale=1.3) if dt == E4M3 else {}
    w = wl64([(5, 18), (1, 29), (12, 12), (3, 40)], hq, hkv, 8, kv_dtype=dt, seed=31,
             sliding_window=9, soft_cap=4.0, **scales)
    out64, cache64 = O.ref_ragged_paged_attention_hd64(*w.args(), mode="fp64", **w.kwargs)
    v3 = to_v3(w.kv_cache, hkv)
    out3, cache3 = O.ref_ragged_paged_attention(w.q, w.k, w.v, v3, *w.args()[4:], mode="fp64",
                                                **w.kwargs)
    assert_close(out64, out3, 1e-12, 1e-12, "hd64 vs v3 oracle")
    assert bytes_equal(to_v3(cache64, hkv), cache3)
    # Padding heads of written records are zero, the rest of the cache is
    # unchanged: the byte diff is confined to the written slots.
    changed = (cache64.view(torch.uint8) != w.kv_cache.view(torch.uint8)).reshape(
        cache64.shape[0], cache64.shape[1], -1).any(-1)
    assert int(changed.sum()) <= w.num_tokens


@pytest.mark.parametrize("case", [
    dict(seq_lens=[(5, 18), (1, 29), (12, 12)], hq=4, hkv=2, ps=16),
    dict(seq_lens=[(7, 20), (1, 9)], hq=6, hkv=3, ps=8, sliding_window=5),
    dict(seq_lens=[(4, 30)], hq=2, hkv=1, ps=4, soft_cap=3.0),
])
@pytest.mark.parametrize("dt", [BF16, E4M3])
def test_hd64_sink_vs_bruteforce(case, dt):
    c = dict(case)
    seq_lens, hq, hkv, ps = (c.pop(x) for x in ("seq_lens", "hq", "hkv", "ps"))
    scales = dict(k_scale=0.75, v_scale=1.5) if dt == E4M3 else {}
    w = wl64(seq_lens, hq, hkv, ps, kv_dtype=dt, seed=7, **scales, **c)
    sink = torch.linspace(-2.0, 3.0, hq)
    out, _ = O.ref_ragged_paged_attention_hd64(*w.args(), sink, mode="fp64", **w.kwargs)
    bf = brute_force_rpa(w.q, w.k, w.v, as_view(w.kv_cache), *w.args()[4:],
                         attention_sink=sink, **w.kwargs)
    assert_close(out, bf, 1e-10, 1e-10, "hd64 oracle with sinks vs brute force")
    out32, _ = O.ref_ragged_paged_attention_hd64(*w.args(), sink, mode="fp32", **w.kwargs)
    assert_close(out32, bf, 1e-5, 1e-5, "fp32 mode")


@pytest.mark.parametrize("dt", [BF16, E4M3])
def test_hd64_noncausal_window_vs_bruteforce(dt):
    """kernel_hd64.py:155-158: without the causal mask the window still drops
    keys j <= pos - W of every row (future keys stay).  The brute force states
    that per element; a planted oracle that ignores the window (the v3 rule,
    kernel.py:196-204) must fail, and W >= kv_len is the unwindowed result."""
    scales = dict(k_scale=0.75, v_scale=1.5) if dt == E4M3 else {}
    w = wl64([(7, 20), (1, 9), (5, 5), (12, 40)], 4, 2, 8, kv_dtype=dt, seed=9, **scales)
    sink = torch.linspace(-1.0, 2.0, 4)
    kw = dict(w.kwargs)
    kw.pop("sliding_window", None)
    out, _ = O.ref_ragged_paged_attention_hd64(*w.args(), sink, mode="fp64",
                                               use_causal_mask=False, sliding_window=3, **kw)
    bf = brute_force_rpa(w.q, w.k, w.v, as_view(w.kv_cache), *w.args()[4:], attention_sink=sink,
                         use_causal_mask=False, sliding_window=3, window_all_rows=True, **kw)
    assert_close(out, bf, 1e-10, 1e-10, "hd64 non-causal window vs brute force")
    planted = brute_force_rpa(w.q, w.k, w.v, as_view(w.kv_cache), *w.args()[4:],
                              attention_sink=sink, use_causal_mask=False, sliding_window=3, **kw)
    assert (out - planted).abs().max().item() > 1e-3
    wide, _ = O.ref_ragged_paged_attention_hd64(*w.args(), sink, mode="fp64",
                                                use_causal_mask=False, sliding_window=40, **kw)
    none, _ = O.ref_ragged_paged_attention_hd64(*w.args(), sink, mode="fp64",
                                                use_causal_mask=False, **kw)
    assert_close(wide, none, 1e-12, 1e-12, "window >= kv_len")


def test_sink_closed_form():
    """A sink s scales each row by sigmoid(lse - s) = 1 / (1 + exp(s - lse)),
    lse from the v3 oracle (pinned separately); s = -inf is no sink; a huge s
    sends the row to 0."""
    hkv, hq = 2, 4
    w = wl64([(6, 25), (1, 40)], hq, hkv, 16, seed=12)
    sink = torch.tensor([-1.0, 0.5, 2.0, 7.0])
    out_s, _ = O.ref_ragged_paged_attention_hd64(*w.args(), sink, mode="fp64", **w.kwargs)
    v3 = to_v3(w.kv_cache, hkv)
    out, _, lse = O.ref_ragged_paged_attention(w.q, w.k, w.v, v3, *w.args()[4:], mode="fp64",
                                               return_lse=True, **w.kwargs)
    factor = 1.0 / (1.0 + torch.exp(sink.double().view(1, hq) - lse))
    assert_close(out_s, out * factor.unsqueeze(-1), 1e-12, 1e-12, "sink closed form")
    none_sink = torch.full((hq,), -math.inf)
    out_n, _ = O.ref_ragged_paged_attention_hd64(*w.args(), none_sink, mode="fp64", **w.kwargs)
    assert_close(out_n, out, 1e-12, 1e-12, "-inf sink")
    big, _ = O.ref_ragged_paged_attention_hd64(*w.args(), torch.full((hq,), 1e4), mode="fp64",
                                               **w.kwargs)
    assert big.abs().max().item() < 1e-300


def test_hd64_skip_kv_update_invariant():
    """kernel_hd64.py:127-136 / test_rpa_skip_kv_update.py:98-182: skip with
    garbage K/V equals the no-op rewrite, and the cache is unchanged."""
    w = wl64([(16, 48)], 4, 2, 16, seed=3)
    _, written = O.ref_ragged_paged_attention_hd64(*w.args(), mode="fp64", **w.kwargs)
    base = (w.q, w.k, w.v, written) + w.args()[4:]
    out_a, cache_a = O.ref_ragged_paged_attention_hd64(*base, mode="fp64", **w.kwargs)
    garbage = torch.randn_like(w.k.float()).to(w.k.dtype)
    out_b, cache_b = O.ref_ragged_paged_attention_hd64(w.q, garbage, garbage, written,
                                                       *w.args()[4:], mode="fp64",
                                                       skip_kv_update=True, **w.kwargs)
    assert_close(out_b, out_a, 0, 0)
    assert bytes_equal(cache_b, written) and bytes_equal(cache_a, written)


# ---------------------------------------------------------------------------
# host validation (kernel_hd64.py:1211-1316, :1121-1208)
# ---------------------------------------------------------------------------
def _valid():
    return wl64([(3, 10), (1, 20)], 4, 2, 16, seed=1, max_num_seqs=3)


def _bad():
    w = _valid()
    a = dict(zip(("queries", "keys", "values", "kv_cache", "kv_lens", "page_indices",
                  "cu_q_lens", "distribution"), w.args()))
    sink = torch.zeros(4)
    return [
        ("q not 3d", dict(a, queries=w.q[:, :, None]), {}),
        ("k/v shape", dict(a, values=w.v[:, :1]), {}),
        ("tokens", dict(a, keys=w.k[:-1], values=w.v[:-1]), {}),
        ("head dim", dict(a, queries=w.q[..., :32], keys=w.k[..., :32],
                          values=w.v[..., :32]), {}),
        ("sink heads", a, dict(attention_sink=torch.zeros(3))),
        ("sink dtype", a, dict(attention_sink=sink.to(BF16))),
        ("q % kv heads", dict(a, queries=w.q[:, :3]), {}),
        ("row width", dict(a, kv_cache=w.kv_cache[..., :64]), {}),
        ("kv dtype", dict(a, kv_cache=w.kv_cache.float()), {}),
        ("heads padding", dict(a, kv_cache=torch.cat([w.kv_cache] * 2, dim=2)), {}),
        ("int32 metadata", dict(a, kv_lens=w.kv_lens.long()), {}),
        ("pps divisibility", dict(a, page_indices=w.page_indices[:-1]), {}),
        ("cu shape", dict(a, cu_q_lens=w.cu_q_lens[:-1]), {}),
        ("distribution shape", dict(a, distribution=w.distribution[:2]), {}),
        ("window", a, dict(sliding_window=0)),
        ("soft cap", a, dict(soft_cap=0.0)),
        ("chunk", a, dict(chunk_prefill_size=0)),
        ("kv pages", a, dict(num_kv_pages_per_block=0)),
        ("queries", a, dict(num_queries_per_block=0)),
        ("vmem", a, dict(vmem_limit_bytes=0)),
    ]


@pytest.mark.parametrize("idx", range(len(_bad())))
def test_hd64_static_validation_raises(idx):
    _, args, kw = _bad()[idx]
    kw = dict(kw)
    sink = kw.pop("attention_sink", None)
    with pytest.raises(ValueError):
        R.static_validate_inputs_hd64(*args.values(), sink, **kw)


def test_hd64_validation_accepts_valid():
    w = _valid()
    R.static_validate_inputs_hd64(*w.args(), torch.zeros(4))
    R.dynamic_validate_inputs_hd64(*w.args(), torch.zeros(4))


@pytest.mark.parametrize("what", ["order", "num_seqs", "q_len", "pages", "page oob"])
def test_hd64_dynamic_validation_raises(what):
    w = _valid()
    dist, kvl, pt = w.distribution.clone(), w.kv_lens.clone(), w.page_indices.clone()
    if what == "order":
        dist[:] = torch.tensor([2, 1, 2])
    elif what == "num_seqs":
        dist[2] = 4
    elif what == "q_len":
        kvl[1] = 0
    elif what == "pages":
        kvl[0] = 10 ** 4
    else:
        pt[0] = w.kv_cache.shape[0]
    with pytest.raises(ValueError):
        R.dynamic_validate_inputs_hd64(w.q, w.k, w.v, w.kv_cache, kvl, pt, w.cu_q_lens, dist)


def test_hd64_requires_device():
    w = _valid()
    with pytest.raises(RuntimeError, match="no CPU path"):
        R.ragged_paged_attention_hd64(*w.args(), **w.kwargs)
    with pytest.raises(RuntimeError, match="no CPU path"):
        R.ragged_paged_attention_hd64(*w.args(), use_causal_mask=False, sliding_window=4,
                                      **w.kwargs)
