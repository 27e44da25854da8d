"""GPU parity for head_dim 64 with the packed K|V cache and attention sinks
(ragged_paged_attention_hd64, kernel_hd64.py:1377-1620) against the CPU oracle
ref_ragged_paged_attention_hd64 (kernel_hd64.py:43-183).

Bars as for the v3 path: cache bit exact; outputs within atol = rtol = 2e-2
(bf16 / f32 KV) or 5e-2 (fp8 KV) of the oracle's fp32 mode.  Cases follow the
reference's hd64 coverage (tests/kernels/test_rpa_skip_kv_update.py:98-182)
widened to decode, prefill and mixed batches, windows, soft caps, sinks on and
off, kv heads that are not a multiple of the packing, and fp8.
"""

import sys
from types import SimpleNamespace

import pytest
import torch

from oracle import rpa_oracle as O
from rpa_testlib import assert_close, bytes_diff, bytes_equal

import vllm_torchtpu_amd as R
import vllm_torchtpu_amd.workloads as W
from vllm_torchtpu_amd import _native as N
from vllm_torchtpu_amd import backend as B

pytestmark = pytest.mark.gpu

BF16, E4M3, E5M2 = torch.bfloat16, torch.float8_e4m3fn, torch.float8_e5m2
TOL = {BF16: 2e-2, E4M3: 5e-2, E5M2: 5e-2, torch.float32: 2e-2}

DECODE = [(1, k) for k in (18, 129, 597, 1, 64, 322, 4097, 181, 1107, 33, 31, 1229)]
PREFILL = [(5, 18), (15, 129), (120, 597), (100, 122), (21, 64), (251, 463), (3, 1229)]
MIXED = [(1, 900), (5, 18), (1, 129), (120, 597), (1, 10000), (32, 322), (1, 181),
         (99, 123), (1, 31), (117, 229)]


def _log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _sink(hq, seed=0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(hq, generator=g) * 2.0).to(torch.float32)


def _run(w, dev, sink, path=N.RPA_PATH_AUTO, **extra):
    kw = dict(w.kwargs)
    kw.update(extra)
    g = w.to(dev)
    s = None if sink is None else sink.to(dev)
    if path == N.RPA_PATH_AUTO:
        out, cache = R.ragged_paged_attention_hd64(*g.args(), s, **kw)
    else:
        out = torch.empty(g.q.shape, dtype=g.q.dtype, device=dev)
        p, ps, hp, pack, _ = g.kv_cache.shape
        R.rpa._rpa_forward_impl(
            g.q, g.k, g.v, g.kv_cache.view(p, ps, 2 * hp, pack, 64), g.kv_lens,
            g.page_indices, g.cu_q_lens, g.distribution, out,
            use_causal_mask=kw.get("use_causal_mask", True),
            skip_kv_update=kw.get("skip_kv_update", False), sm_scale=kw["sm_scale"],
            sliding_window=kw.get("sliding_window"), soft_cap=kw.get("soft_cap"),
            q_scale=kw.get("q_scale"), k_scale=kw.get("k_scale"), v_scale=kw.get("v_scale"),
            path=path, attention_sink=s)
        cache = g.kv_cache
    torch.cuda.synchronize()
    return out[:w.num_tokens].cpu(), cache.cpu()


def check(w, dev, sink=None, path=N.RPA_PATH_AUTO, **extra):
    _log(f"[hd64-gpu] case {w.name} seqs={w.seq_lens[:5]}{'...' if len(w.seq_lens) > 5 else ''}"
         f" q={tuple(w.q.shape)} cache={tuple(w.kv_cache.shape)} {w.kv_cache.dtype}"
         f" sink={sink is not None} path={path} extra={extra}")
    kw = dict(w.kwargs)
    kw.update(extra)
    exp_out, exp_cache = O.ref_ragged_paged_attention_hd64(*w.args(), sink, mode="fp32", **kw)
    out, cache = _run(w, dev, sink, path, **extra)
    tol = TOL[w.kv_cache.dtype]
    assert_close(out, exp_out, tol, tol, f"{w.name} output")
    assert bytes_equal(cache, exp_cache), (
        f"{w.name}: cache differs from the oracle: {bytes_diff(cache, exp_cache)}")


def wl64(seqs, hq, hkv, ps, name, seed=71, **kw):
    return W.make_workload(seqs, hq, hkv, 64, ps, layout="hd64", seed=seed, name=name, **kw)


@pytest.mark.parametrize("sinks", [False, True])
@pytest.mark.parametrize("heads", [(8, 2), (16, 1), (12, 3), (64, 8)])
def test_hd64_decode(gpu_device, heads, sinks):
    hq, hkv = heads
    w = wl64(DECODE, hq, hkv, 16, "hd64-decode", distribution=[12, 12, 12])
    check(w, gpu_device, _sink(hq) if sinks else None)


@pytest.mark.parametrize("sinks", [False, True])
@pytest.mark.parametrize("name,seqs", [("prefill", PREFILL), ("mixed", MIXED)])
def test_hd64_prefill_mixed(gpu_device, name, seqs, sinks):
    w = wl64(seqs, 16, 2, 16, f"hd64-{name}")
    check(w, gpu_device, _sink(16, 1) if sinks else None)


@pytest.mark.parametrize("path", [N.RPA_PATH_AUTO, N.RPA_PATH_GENERIC])
@pytest.mark.parametrize("window,cap", [(5, None), (128, None), (None, 30.0), (64, 20.0)])
def test_hd64_window_cap_sinks(gpu_device, window, cap, path):
    w = wl64([(1, 700), (40, 300), (1, 5), (1, 3000), (17, 17)], 16, 4, 16, "hd64-wc",
             sliding_window=window, soft_cap=cap)
    check(w, gpu_device, _sink(16, 2), path=path)


@pytest.mark.parametrize("dt", [E4M3, E5M2])
@pytest.mark.parametrize("sinks", [False, True])
def test_hd64_fp8(gpu_device, dt, sinks):
    w = wl64([(1, 900), (17, 80), (1, 2000), (64, 64)], 32, 8, 32, "hd64-fp8", kv_dtype=dt,
             k_scale=0.7, v_scale=1.3)
    check(w, gpu_device, _sink(32, 3) if sinks else None)


@pytest.mark.parametrize("hkv,dt", [(3, BF16), (1, E4M3), (3, E4M3), (5, BF16)])
def test_hd64_heads_not_multiple_of_packing(gpu_device, hkv, dt):
    """Padding heads of every written record are zero (bit exact)."""
    w = wl64([(1, 300), (9, 40), (1, 33)], 2 * hkv, hkv, 16, "hd64-pad", kv_dtype=dt)
    check(w, gpu_device, _sink(2 * hkv, 4))


def test_hd64_f32(gpu_device):
    w = wl64([(1, 70), (5, 20), (1, 300)], 8, 2, 16, "hd64-f32", q_dtype=torch.float32,
             kv_dtype=torch.float32)
    check(w, gpu_device, _sink(8, 5))


@pytest.mark.parametrize("kv_len,q_len", [(48, 16), (33, 1)])
def test_hd64_skip_kv_update(gpu_device, kv_len, q_len):
    """test_rpa_skip_kv_update.py:98-182: garbage K/V with skip_kv_update leave
    the cache untouched and read the cached keys."""
    w = wl64([(q_len, kv_len)], 4, 2, 16, "hd64-skip")
    garbage = torch.randn(w.k.shape).to(w.k.dtype)
    w.k.copy_(garbage)
    w.v.copy_(garbage)
    check(w, gpu_device, _sink(4, 6), skip_kv_update=True)
    check(w, gpu_device, None, skip_kv_update=True)


def test_hd64_sink_extremes(gpu_device):
    """A -inf sink is no sink; a sink far above every logit sends rows to 0."""
    w = wl64([(1, 500), (30, 60)], 8, 2, 16, "hd64-sink-ext")
    plain, _ = _run(w, gpu_device, None)
    none, _ = _run(w, gpu_device, torch.full((8,), float("-inf")))
    assert torch.equal(plain, none)
    big, _ = _run(w, gpu_device, torch.full((8,), 1e4))
    assert big.float().abs().max().item() == 0.0


def test_hd64_lse_with_sink_unsupported(gpu_device):
    w = wl64([(1, 40)], 4, 2, 16, "hd64-lse").to(gpu_device)
    out = torch.empty(w.q.shape, dtype=w.q.dtype, device=gpu_device)
    lse = torch.empty(w.q.shape[:2], dtype=torch.float32, device=gpu_device)
    p, ps, hp, pack, _ = w.kv_cache.shape
    with pytest.raises(RuntimeError):
        R.rpa._rpa_forward_impl(w.q, w.k, w.v, w.kv_cache.view(p, ps, 2 * hp, pack, 64),
                                w.kv_lens, w.page_indices, w.cu_q_lens, w.distribution, out,
                                use_causal_mask=True, skip_kv_update=False, sm_scale=0.125,
                                sliding_window=None, soft_cap=None, q_scale=None,
                                k_scale=None, v_scale=None, lse=lse,
                                attention_sink=torch.zeros(4, device=gpu_device))


def test_hd64_backend_with_sinks(gpu_device):
    """The backend routes head_size 64 to the hd64 kernel with the layer's
    sinks (attention_interface.py:418-436), on the hd64 cache it allocates."""
    hq, hkv = 16, 4
    w = wl64([(1, 700), (37, 300), (1, 33), (64, 64)], hq, hkv, 16, "hd64-backend",
             sliding_window=256)
    shape = B.RpaAttentionBackend.get_kv_cache_shape(w.kv_cache.shape[0], 16, hkv, 64, BF16)
    assert tuple(shape) == tuple(w.kv_cache.shape)
    sink = _sink(hq, 7)
    exp_out, exp_cache = O.ref_ragged_paged_attention_hd64(*w.args(), sink, mode="fp32",
                                                           **w.kwargs)
    impl = B.RpaAttentionBackendImpl(num_heads=hq, head_size=64, scale=w.kwargs["sm_scale"],
                                     num_kv_heads=hkv, alibi_slopes=None, sliding_window=256,
                                     kv_cache_dtype="auto", sinks=sink.to(BF16).to(gpu_device))
    impl.process_weights_after_loading(BF16)
    g = w.to(gpu_device)
    T = w.q.shape[0]
    meta = B.AttentionMetadata(input_positions=None, block_tables=g.page_indices,
                               seq_lens=g.kv_lens, query_start_loc=g.cu_q_lens,
                               request_distribution=g.distribution)
    out = impl.forward(SimpleNamespace(), g.q.reshape(T, hq * 64), g.k.reshape(T, -1),
                       g.v.reshape(T, -1), g.kv_cache, meta)
    torch.cuda.synchronize()
    n = w.num_tokens
    # The sinks went through bf16 on the way in, as a checkpoint's would.
    exp_out, _ = O.ref_ragged_paged_attention_hd64(*w.args(), sink.to(BF16).float(),
                                                   mode="fp32", **w.kwargs)
    assert_close(out[:n].reshape(n, hq, 64).cpu(), exp_out, 2e-2, 2e-2, "backend hd64")
    assert bytes_equal(g.kv_cache.cpu(), exp_cache)


@pytest.mark.parametrize("dt", [BF16, E4M3])
@pytest.mark.parametrize("window", [3, 64])
def test_hd64_noncausal_window(gpu_device, window, dt):
    """kernel_hd64.py:155-158, :443-446: without the causal mask the window
    still drops keys j <= pos - W of every row (this runs on the generic kernels)."""
    scales = dict(k_scale=0.75, v_scale=1.25) if dt == E4M3 else {}
    w = wl64([(1, 700), (40, 300), (1, 5), (17, 17), (3, 90)], 16, 4, 16, "hd64-nc-window",
             sliding_window=window, kv_dtype=dt, **scales)
    check(w, gpu_device, _sink(16, 3), use_causal_mask=False)


def test_hd64_custom_op_matches_eager(gpu_device):
    """Eager hd64 calls run the op body directly; the registered op (the path
    torch.compile keeps opaque) must give the same bytes."""
    w = wl64([(1, 700), (40, 300), (1, 5)], 16, 4, 16, "hd64-op", sliding_window=64)
    g = w.to(gpu_device)
    sink = _sink(16, 4).to(gpu_device)
    out_e, _ = R.ragged_paged_attention_hd64(*g.args(), sink, **w.kwargs)
    out_o = torch.ops.rpa_amd.ragged_paged_attention_hd64(
        *g.args(), sink, True, False, float(w.kwargs["sm_scale"]), 64, 0.0, False, 1.0, 1.0, 1.0)
    torch.cuda.synchronize()
    n = w.num_tokens
    assert torch.equal(out_e[:n].view(torch.int16), out_o[:n].view(torch.int16))
