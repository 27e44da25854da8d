"""GPU parity tests: the HIP library (through its C ABI, via the Python API)
against the CPU oracle on identical seeded inputs.

Bars: the cache write is bit exact; outputs are within atol = rtol = 2e-2
(bf16 KV) or 5e-2 (fp8 KV) of the oracle's fp32-accumulation mode.  Case lists
follow the reference's tests (tests/kernels/experimental/batched_rpa/
correctness_test.py:472-986, tests/kernels/test_rpa_skip_kv_update.py:98-182,
tests/kernels/test_rpa_bundled.py:58-227).
"""

import sys

import pytest
import torch

from oracle import rpa_oracle as O
from rpa_testlib import assert_close, bytes_diff, bytes_equal

import vllm_torchtpu_amd as R
import vllm_torchtpu_amd.workloads as W
from vllm_torchtpu_amd import _native as N

pytestmark = pytest.mark.gpu

BF16, E4M3, E5M2 = torch.bfloat16, torch.float8_e4m3fn, torch.float8_e5m2
TOL = {BF16: 2e-2, E4M3: 5e-2, E5M2: 5e-2, torch.float32: 2e-2, torch.float16: 2e-2}


def _log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def run_gpu(w, dev, path=N.RPA_PATH_AUTO, **extra):
    g = w.to(dev)
    kw = dict(w.kwargs)
    kw.update(extra)
    if path == N.RPA_PATH_AUTO:
        out, cache = R.ragged_paged_attention(*g.args(), **kw)
    else:
        out = torch.empty(g.q.shape, dtype=g.q.dtype, device=dev)
        q = g.q
        R.rpa._rpa_forward_impl(q, g.k, g.v, g.kv_cache, g.kv_lens, g.page_indices,
                                g.cu_q_lens, g.distribution, out,
                                use_causal_mask=kw.get("use_causal_mask", True),
                                skip_kv_update=kw.get("skip_kv_update", False),
                                sm_scale=kw["sm_scale"],
                                sliding_window=kw.get("sliding_window"),
                                soft_cap=kw.get("soft_cap"), q_scale=kw.get("q_scale"),
                                k_scale=kw.get("k_scale"), v_scale=kw.get("v_scale"),
                                path=path)
        cache = g.kv_cache
    torch.cuda.synchronize()
    return out[:w.num_tokens].cpu(), cache.cpu()


def check(w, dev, path=N.RPA_PATH_AUTO, **extra):
    _log(f"[rpa-gpu] case {w.name} seqs={w.seq_lens[:6]}{'...' if len(w.seq_lens) > 6 else ''}"
         f" q={tuple(w.q.shape)} cache={tuple(w.kv_cache.shape)} {w.kv_cache.dtype} path={path}"
         f" kw={ {k: v for k, v in {**w.kwargs, **extra}.items() if k != 'sm_scale'} }")
    kw = dict(w.kwargs)
    kw.update(extra)
    exp_out, exp_cache = O.ref_ragged_paged_attention(*w.args(), mode="fp32", **kw)
    out, cache = run_gpu(w, dev, path, **extra)
    tol = TOL[w.kv_cache.dtype]
    assert_close(out, exp_out, tol, tol, f"{w.name} output")
    assert bytes_equal(cache, exp_cache), f"{w.name}: cache differs from the oracle"
    return out


# ---------------------------------------------------------------------------
# cache write
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("dt", [BF16, E4M3, torch.float32])
@pytest.mark.parametrize("d", [128, 80])
def test_kv_cache_update_bit_exact(gpu_device, dt, d):
    w = W.make_workload([(5, 18), (1, 33), (16, 48), (3, 3), (1, 1)], 8, 2, d, 16,
                        kv_dtype=dt, seed=21, max_num_seqs=7, max_num_tokens=40,
                        k_scale=0.5 if dt == E4M3 else None, v_scale=0.5 if dt == E4M3 else None)
    _log(f"[rpa-gpu] kv update {dt} d={d}")
    expect = O.update_kv_cache_np(w.k, w.v, w.kv_cache, w.kv_lens, w.page_indices,
                                  w.cu_q_lens, w.distribution)
    g = w.to(gpu_device)
    R.rpa_kv_cache_update(g.k, g.v, g.kv_cache, g.kv_lens, g.page_indices, g.cu_q_lens,
                          g.distribution)
    torch.cuda.synchronize()
    assert bytes_equal(g.kv_cache.cpu(), expect)


def test_kv_cache_update_nan_payloads(gpu_device):
    """NaN and -0.0 in new K/V are copied as bits."""
    w = W.make_workload([(4, 20)], 4, 2, 128, 16, seed=22)
    w.k[0, 0, :4] = torch.tensor([float("nan"), -0.0, float("inf"), -float("inf")])
    expect = O.update_kv_cache_np(w.k, w.v, w.kv_cache, w.kv_lens, w.page_indices,
                                  w.cu_q_lens, w.distribution)
    g = w.to(gpu_device)
    R.rpa_kv_cache_update(g.k, g.v, g.kv_cache, g.kv_lens, g.page_indices, g.cu_q_lens,
                          g.distribution)
    torch.cuda.synchronize()
    assert bytes_equal(g.kv_cache.cpu(), expect)


# ---------------------------------------------------------------------------
# attention: reference case lists
# ---------------------------------------------------------------------------
BASIC = [(192, 328), (128, 180), (64, 255)]
DECODE16 = [(1, k) for k in (18, 129, 597, 122, 64, 322, 463, 181, 1107, 123, 31, 18, 1229,
                             229, 87, 1328)]
PREFILL16 = [(5, 18), (15, 129), (120, 597), (100, 122), (21, 64), (32, 322), (251, 463),
             (40, 181), (64, 1107), (99, 123), (10, 31), (5, 18), (3, 1229), (120, 229),
             (9, 87), (2, 1328)]
MIXED16 = [(5, 18), (1, 129), (120, 597), (1, 122), (1, 64), (32, 322), (251, 463), (1, 181),
           (1, 1107), (99, 123), (1, 31), (5, 18), (3, 1229), (117, 229), (1, 87), (1, 1328)]

PATHS = [N.RPA_PATH_AUTO, N.RPA_PATH_GENERIC]


@pytest.mark.parametrize("path", PATHS)
@pytest.mark.parametrize("ps", [16, 32])
def test_basic(gpu_device, path, ps):
    check(W.make_workload(BASIC, 32, 8, 128, ps, seed=1234, name="basic"), gpu_device, path)


@pytest.mark.parametrize("dt", [BF16, E4M3])
@pytest.mark.parametrize("q_len", [1, 5])
@pytest.mark.parametrize("ps", [128, 256, 512])
def test_large_page_sizes(gpu_device, ps, q_len, dt):
    """correctness_test.py:470-520: page sizes 128-512 with kv_lens that are not
    multiples of 128; q_len 1 takes the decode kernel, 5 the prefill kernel."""
    seqs = [(q_len, n) for n in (18, 129, 597, 1107, 31, 1328)]
    check(W.make_workload(seqs, 32, 8, 128, ps, kv_dtype=dt, seed=44,
                          name=f"ps{ps}-q{q_len}"), gpu_device)


@pytest.mark.parametrize("path", PATHS)
@pytest.mark.parametrize("name,seqs", [("decode", DECODE16), ("prefill", PREFILL16),
                                       ("mixed", MIXED16)])
def test_segments(gpu_device, path, name, seqs):
    n = len(seqs)
    dist = [n, n, n] if name == "decode" else [0, 0, n]
    check(W.make_workload(seqs, 32, 8, 128, 16, seed=1234, distribution=dist, name=name),
          gpu_device, path)


@pytest.mark.parametrize("num_seqs", [1, 17])
@pytest.mark.parametrize("heads", [(32, 8), (12, 2), (5, 1), (3, 3)])
@pytest.mark.parametrize("d", [80, 240])
def test_complex_shapes(gpu_device, num_seqs, heads, d):
    g = torch.Generator().manual_seed(1234)
    ql = torch.randint(1, 100, (num_seqs,), generator=g)
    kl = ql + torch.randint(0, 50, (num_seqs,), generator=g)
    seqs = list(zip(ql.tolist(), kl.tolist()))
    check(W.make_workload(seqs, heads[0], heads[1], d, 16, seed=5, name="complex"), gpu_device)


@pytest.mark.parametrize("d", [128, 256])
def test_prefill_kernel_writes_without_decode_kernel(gpu_device, d):
    """qpk > 16 has no decode kernel, so the prefill launch plans the cache
    writes itself, in 512-thread (d 128) or 256-thread (d 256) workgroups; the
    first sequences' rows must all be written (their kv_len entries share LDS
    with the plan's reduction slots)."""
    seqs = [(17, 80), (1, 300), (64, 64), (5, 18), (1, 33), (40, 41)]
    for rep in range(3):
        check(W.make_workload(seqs, 24, 1, d, 16, seed=90 + rep, name=f"no-decode-{rep}"),
              gpu_device)


@pytest.mark.parametrize("window", [None, 5, 128])
def test_sliding_window(gpu_device, window):
    g = torch.Generator().manual_seed(1234)
    ql = torch.randint(1, 100, (5,), generator=g)
    kl = ql + torch.randint(0, 50, (5,), generator=g)
    check(W.make_workload(list(zip(ql.tolist(), kl.tolist())), 4, 4, 128, 16, seed=6,
                          sliding_window=window, name="window"), gpu_device)


@pytest.mark.parametrize("cap", [None, 50.0, 2.0])
def test_soft_cap(gpu_device, cap):
    g = torch.Generator().manual_seed(1234)
    ql = torch.randint(1, 100, (2,), generator=g)
    kl = ql + torch.randint(0, 50, (2,), generator=g)
    w = W.make_workload(list(zip(ql.tolist(), kl.tolist())), 16, 2, 128, 16, seed=7,
                        soft_cap=cap, name="softcap")
    w.q.mul_(4.0)  # push logits into the capped range
    check(w, gpu_device)


@pytest.mark.parametrize("cap,qmul", [(50.0, 8.0), (50.0, 0.05), (60.0, 30.0), (80.0, 8.0)])
def test_soft_cap_d256_logit_range(gpu_device, cap, qmul):
    """head_dim 256 prefill rows whose capped logits spread over (-cap, cap):
    the kernel fixes each row's reference max at its first tile when the cap
    bounds the logits (cap <= 60) and rescales otherwise (cap 80).  Rows see
    up to ~2000 keys whose magnitude grows with position, so their maxima move
    far from the first tile's; tiny q (qmul 0.05) keeps every logit near 0."""
    g = torch.Generator().manual_seed(4321)
    seqs = [(96, 2000), (33, 700), (128, 128), (1, 1500)]
    w = W.make_workload(seqs, 8, 4, 256, 16, seed=int(torch.randint(0, 1000, (1,), generator=g)),
                        soft_cap=cap, distribution=[0, 0, len(seqs)], name="cap256")
    w.q.mul_(qmul)
    # Keys of later pages are larger (x1 .. x4), so a row's max keeps growing
    # past its first tile's.  K is the even combined head: [..., head, 0, :].
    pps = w.page_indices.shape[0] // w.kv_lens.shape[0]
    for s in range(len(seqs)):
        npg = (int(w.kv_lens[s]) + 15) // 16
        for j in range(npg):
            pg = int(w.page_indices[s * pps + j])
            w.kv_cache[pg, :, :, 0, :] *= 1.0 + 3.0 * j / max(npg - 1, 1)
    check(w, gpu_device)


@pytest.mark.parametrize("dt", [E4M3, E5M2])
@pytest.mark.parametrize("scales", [(0.5, 0.5), (None, None), (1.7, 0.6)])
def test_fp8_kv(gpu_device, dt, scales):
    check(W.make_workload(BASIC, 32, 8, 128, 16, kv_dtype=dt, seed=1234, k_scale=scales[0],
                          v_scale=scales[1], name="fp8"), gpu_device)


@pytest.mark.parametrize("dt", [E4M3, E5M2])
def test_q_scale(gpu_device, dt):
    check(W.make_workload(BASIC, 32, 8, 128, 16, kv_dtype=dt, seed=1234, k_scale=0.5,
                          v_scale=0.5, q_scale=0.5, name="q_scale"), gpu_device)


def test_f32(gpu_device):
    check(W.make_workload(MIXED16, 32, 8, 128, 16, q_dtype=torch.float32,
                          kv_dtype=torch.float32, seed=3, name="f32"), gpu_device)


@pytest.mark.parametrize("seqs", [MIXED16, DECODE16])
def test_f16(gpu_device, seqs):
    """f16 queries and KV (kernel.py:1447-1453 accepts any float KV dtype): the
    shape-generic kernels, f16 output."""
    n = len(seqs)
    check(W.make_workload(seqs, 32, 8, 128, 16, q_dtype=torch.float16, kv_dtype=torch.float16,
                          seed=4, distribution=[0, 0, n], name="f16"), gpu_device)


def test_non_causal(gpu_device):
    check(W.make_workload([(5, 40), (16, 16), (1, 70)], 8, 2, 128, 16, seed=8, name="nc"),
          gpu_device, use_causal_mask=False)


@pytest.mark.parametrize("kv_len,q_len", [(48, 16), (33, 1)])
def test_skip_kv_update(gpu_device, kv_len, q_len):
    w = W.make_workload([(q_len, kv_len)], 4, 2, 128, 16, seed=9, name="skip")
    exp_out, _ = O.ref_ragged_paged_attention(*w.args(), mode="fp32", skip_kv_update=True,
                                              **w.kwargs)
    out, cache = run_gpu(w, gpu_device, skip_kv_update=True)
    assert_close(out, exp_out, 2e-2, 2e-2, "skip_kv_update output")
    assert bytes_equal(cache, w.kv_cache)


def test_nan_poison_isolation(gpu_device):
    w = W.make_workload([(1, k) for k in (129, 2048, 8, 7, 257, 259, 8, 511)], 8, 2, 128, 16,
                        seed=10, nan_fill=True, max_num_seqs=10, max_num_tokens=12,
                        name="nan-decode")
    out = check(w, gpu_device)
    assert torch.isfinite(out).all()
    w = W.make_workload([(q, q + 40) for q in (5, 33, 1, 64)], 8, 2, 128, 16, seed=11,
                        nan_fill=True, name="nan-prefill")
    out = check(w, gpu_device)
    assert torch.isfinite(out).all()


@pytest.mark.parametrize("qh,kvh,seqs,kv_dtype", [
    (8, 2, [(1, 129), (1, 2048), (1, 8), (1, 77)], BF16),             # decode kernel only
    (8, 2, [(1, 300), (17, 80), (1, 33), (40, 41), (1, 1000)], BF16),  # decode + prefill
    (24, 1, [(17, 80), (1, 300), (5, 18)], BF16),                     # qpk > 16: no decode kernel
    (32, 8, [(1, 513), (3, 70), (1, 64)], E4M3),
])
def test_unused_sequence_slots_are_ignored(gpu_device, qh, kvh, seqs, kv_dtype):
    """Every kernel's plan loads kv_lens and cu_q_lens of all max_num_seqs
    slots before it knows num_seqs (distribution[2]); slots past num_seqs must
    change nothing, whatever they hold (the reference reads only s < num_seqs,
    kernel.py:1345-1349)."""
    n = len(seqs)
    w = W.make_workload(seqs, qh, kvh, 128, 16, kv_dtype=kv_dtype, seed=40 + n,
                        max_num_seqs=n + 6, name="unused-slots",
                        **({"k_scale": 0.5, "v_scale": 0.5} if kv_dtype == E4M3 else {}))
    w.kv_lens[n:] = torch.tensor([1 << 30, -5, 7, 1 << 20, 0, 3], dtype=torch.int32)
    last = int(w.cu_q_lens[n])
    w.cu_q_lens[n + 1:] = torch.tensor([last - 3, last + 4096, -1, last + 1, 1 << 29, last],
                                       dtype=torch.int32)
    check(w, gpu_device)


def test_nan_sequence_stays_in_its_rows(gpu_device):
    w = W.make_workload([(3, 40), (1, 100), (5, 77)], 8, 2, 128, 16, seed=12, name="nanseq")
    S = w.kv_lens.shape[0]
    pps = w.page_indices.shape[0] // S
    pages = w.page_indices[pps:pps + O.cdiv(100, 16)].long()
    w.kv_cache[pages] = float("nan")
    out, _ = run_gpu(w, gpu_device)
    assert torch.isnan(out[3:4].float()).all()
    assert torch.isfinite(out[:3].float()).all() and torch.isfinite(out[4:].float()).all()


def _check_dq(w, dev, q_len, what):
    """Oracle against the GPU path with decode groups of q_len tokens
    (decode_query_size is a scheduling choice: the oracle takes none)."""
    exp_out, exp_cache = O.ref_ragged_paged_attention(*w.args(), mode="fp32", **w.kwargs)
    out, cache = run_gpu(w, dev, decode_query_size=q_len)
    tol = TOL[w.kv_cache.dtype]
    assert_close(out, exp_out, tol, tol, f"{what} output")
    assert bytes_equal(cache, exp_cache), f"{what}: cache differs from the oracle"
    return out


@pytest.mark.parametrize("q_len", [1, 4])
def test_nan_cached_kv_stays_in_its_sequence(gpu_device, q_len):
    """correctness_test.py:703-727: every cached K/V page of sequence 1 holds NaN;
    only that sequence's rows may be NaN, and every other row equals the oracle
    (decode groups of q_len tokens, all sequences on the decode path)."""
    seqs = [(q_len, k) for k in (129, 597, 256, 512, 768, 256, 1024, 512)]
    n = len(seqs)
    w = W.make_workload(seqs, 32, 8, 128, 16, seed=48, distribution=[n, n, n],
                        name=f"nan-kv-q{q_len}")
    S = w.kv_lens.shape[0]
    pps = w.page_indices.shape[0] // S
    w.kv_cache[w.page_indices[pps:pps + O.cdiv(597, 16)].long()] = float("nan")
    _log(f"[rpa-gpu] case {w.name}")
    out = _check_dq(w, gpu_device, q_len, w.name)
    assert torch.isnan(out[q_len:2 * q_len].float()).all()
    assert torch.isfinite(out[:q_len].float()).all()
    assert torch.isfinite(out[2 * q_len:].float()).all()


@pytest.mark.parametrize("dt", [BF16, E4M3])
@pytest.mark.parametrize("q_len", [1, 4])
def test_nan_cached_kv_does_not_poison_partial_tiles(gpu_device, q_len, dt):
    """correctness_test.py:731-757: page size 256 and short sequences, so most
    tiles are partly past a sequence's keys; every cache slot and page no
    sequence uses holds NaN, and so does every cached K/V page of sequence 1.
    Only sequence 1's rows may be NaN; the others equal the oracle."""
    lens = (129, 2048, 8, 7, 257, 259, 8, 511)
    seqs = [(q_len, k) for k in lens]
    n = len(seqs)
    w = W.make_workload(seqs, 8, 2, 128, 256, kv_dtype=dt, seed=50, nan_fill=True,
                        distribution=[n, n, n], name=f"nan-partial-q{q_len}")
    S = w.kv_lens.shape[0]
    pps = w.page_indices.shape[0] // S
    w.kv_cache[w.page_indices[pps:pps + O.cdiv(lens[1], 256)].long()] = float("nan")
    _log(f"[rpa-gpu] case {w.name} {dt}")
    out = _check_dq(w, gpu_device, q_len, w.name)
    assert torch.isnan(out[q_len:2 * q_len].float()).all()
    assert torch.isfinite(out[:q_len].float()).all()
    assert torch.isfinite(out[2 * q_len:].float()).all()


@pytest.mark.parametrize("dt", [BF16, E4M3])
@pytest.mark.parametrize("q_len", [1, 4])
@pytest.mark.parametrize("d", [128, 256])
def test_nan_new_kv_stays_in_its_sequence(gpu_device, d, q_len, dt):
    """correctness_test.py:759-790: NaN new keys and values of one short decode
    (sequence 128 / q_len of a batch of them, page size 256) reach only that
    sequence's rows and its own cache slots."""
    bad = 128 // q_len
    seqs = [(q_len, 4 + q_len)] * (bad + 3)
    n = len(seqs)
    w = W.make_workload(seqs, 8, 2, d, 256, kv_dtype=dt, seed=49, distribution=[n, n, n],
                        name=f"nan-new-d{d}-q{q_len}")
    t0 = int(w.cu_q_lens[bad])
    w.k[t0:t0 + q_len] = float("nan")
    w.v[t0:t0 + q_len] = float("nan")
    _log(f"[rpa-gpu] case {w.name} {dt}")
    out = _check_dq(w, gpu_device, q_len, w.name)
    assert torch.isnan(out[t0:t0 + q_len].float()).all()
    assert torch.isfinite(out[:t0].float()).all()
    assert torch.isfinite(out[t0 + q_len:].float()).all()


def test_bundled_matches_flat(gpu_device):
    """test_rpa_bundled.py:173-227: bundled block-major == per-layer flat, bitwise;
    and both equal the oracle on that layer (kernel.py:2011-2061: logical page p
    of layer l is flat page p * num_layers + l, updated in place)."""
    layers, P = 3, 96
    w = W.make_workload([(1, 128)] * 4 + [(32, 192)] * 4, 16, 4, 128, 16, seed=13,
                        num_pages=P, distribution=[4, 8, 8], name="bundled")
    g = torch.Generator().manual_seed(0)
    init = torch.randn(layers, *w.kv_cache.shape, generator=g).to(BF16)
    dev = gpu_device
    n = w.num_tokens
    for layer in range(layers):
        # The oracle on this layer's flat cache: the bundle's pages p * layers +
        # layer are exactly init[layer][p].
        args = list(w.args())
        args[3] = init[layer].clone()
        exp_out, exp_cache = O.ref_ragged_paged_attention(*args, mode="fp32", **w.kwargs)
        flat = w.to(dev)
        flat_cache = init[layer].clone().to(dev)
        out_ref, _ = R.ragged_paged_attention(flat.q, flat.k, flat.v, flat_cache, flat.kv_lens,
                                              flat.page_indices, flat.cu_q_lens,
                                              flat.distribution, **w.kwargs)
        bundle = init.clone().transpose(0, 1).contiguous().to(dev)
        out_b, bundle = R.ragged_paged_attention_bundled(
            flat.q, flat.k, flat.v, bundle, layer, flat.kv_lens, flat.page_indices,
            flat.cu_q_lens, flat.distribution, **w.kwargs)
        torch.cuda.synchronize()
        assert bytes_equal(out_ref[:n].cpu(), out_b[:n].cpu())
        assert bytes_equal(flat_cache.cpu(), bundle[:, layer].cpu())
        assert_close(out_b[:n], exp_out[:n], 2e-2, 2e-2, f"bundled layer {layer} vs oracle")
        assert bytes_equal(bundle[:, layer].cpu(), exp_cache), \
            bytes_diff(bundle[:, layer].cpu(), exp_cache)
        others = [x for x in range(layers) if x != layer]
        assert bytes_equal(bundle[:, others].cpu(), init.transpose(0, 1)[:, others].contiguous())


# ---------------------------------------------------------------------------
# BASELINE configurations at full size
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("idx", [1, 2, 3, 4, 5])
def test_baseline_config(gpu_device, idx):
    check(W.baseline_config(idx), gpu_device)


# ---------------------------------------------------------------------------
# decode path edge cases (single-token rows, split-K)
# ---------------------------------------------------------------------------
DECODE_EDGE = [(1, k) for k in (1, 2, 31, 32, 33, 100, 511, 512, 513, 1000, 4097, 10000)]


@pytest.mark.parametrize("heads", [(32, 8), (16, 1), (8, 8), (12, 4)])
@pytest.mark.parametrize("dt", [BF16, E4M3, E5M2])
def test_decode_edges(gpu_device, heads, dt):
    scales = dict(k_scale=0.8, v_scale=1.3) if dt != BF16 else {}
    check(W.make_workload(DECODE_EDGE, heads[0], heads[1], 128, 16, kv_dtype=dt, seed=31,
                          distribution=[12, 12, 12], name="decode-edge", **scales), gpu_device)


@pytest.mark.parametrize("window,cap", [(5, None), (128, None), (1, None), (None, 30.0),
                                        (4096, 50.0)])
def test_decode_window_cap(gpu_device, window, cap):
    check(W.make_workload(DECODE_EDGE, 16, 4, 128, 32, seed=32, sliding_window=window,
                          soft_cap=cap, name="decode-wc"), gpu_device)


@pytest.mark.parametrize("d", [256, 192, 64])
def test_decode_head_dims(gpu_device, d):
    check(W.make_workload(DECODE_EDGE, 16, 8, d, 16, seed=33, name=f"decode-d{d}"), gpu_device)


@pytest.mark.parametrize("n,kv_max,dt", [(300, 3000, BF16), (600, 600, BF16), (600, 600, E4M3)])
def test_decode_many_seqs(gpu_device, n, kv_max, dt):
    """600 sequences x 8 kv heads = 4800 pairs: more than the merge wavefronts of
    the second launch (at most 512 workgroups x 8), so some merge more than one
    pair -- bf16 in the LDS-DMA kernel, fp8 in the register-staged one."""
    g = torch.Generator().manual_seed(34)
    kvl = torch.randint(1, kv_max, (n,), generator=g).tolist()
    check(W.make_workload([(1, k) for k in kvl], 32, 8, 128, 16, kv_dtype=dt, seed=34,
                          name=f"decode-{n}"), gpu_device)


def test_decode_f32_out(gpu_device):
    """bf16 q with an f32 cache is not the decode path's; f32 q/out is generic."""
    check(W.make_workload(DECODE_EDGE, 8, 2, 128, 16, q_dtype=torch.float32,
                          kv_dtype=torch.float32, seed=35, name="decode-f32"), gpu_device)


def test_decode_repeated_calls(gpu_device):
    """The decode partials live in a persistent per-device workspace; back-to-back
    calls (and a different batch afterwards) must not see each other's partials."""
    w = W.make_workload([(1, k) for k in (4000, 33, 2048, 700, 1)], 32, 8, 128, 16, seed=36,
                        name="decode-repeat")
    exp_out, exp_cache = O.ref_ragged_paged_attention(*w.args(), mode="fp32", **w.kwargs)
    g = w.to(gpu_device)
    for rep in range(3):
        out, cache = R.ragged_paged_attention(*g.args(), **w.kwargs)
        torch.cuda.synchronize()
        assert_close(out[:w.num_tokens].cpu(), exp_out, 2e-2, 2e-2, f"repeat {rep}")
        assert bytes_equal(cache.cpu(), exp_cache)
    # A different batch on the same workspace afterwards.
    check(W.make_workload(DECODE_EDGE, 32, 8, 128, 16, seed=37, name="decode-after"), gpu_device)


def test_back_to_back_calls_without_sync(gpu_device):
    """Calls queued on one stream with no synchronization between them share the
    device's workspace (decode partials and plan): call i's merges must read call
    i's partials, not those of call i + 1 that the next decode kernel writes.
    Two decode batches and a mixed batch take turns nine times, then every
    output is checked."""
    a = W.make_workload([(1, k) for k in (4000, 33, 2048, 700, 1)], 32, 8, 128, 16, seed=38,
                        name="b2b-a")
    b = W.make_workload([(1, k) for k in (1500, 3000, 64, 900, 2500)], 32, 8, 128, 16,
                        seed=39, name="b2b-b")
    c = W.make_workload([(1, 800), (37, 120), (1, 2000), (64, 64)], 32, 8, 128, 16, seed=40,
                        name="b2b-mixed")
    ws = [a, b, c]
    exp = {w.name: O.ref_ragged_paged_attention(*w.args(), mode="fp32", **w.kwargs)[0]
           for w in ws}
    gs = [w.to(gpu_device) for w in ws]
    torch.cuda.synchronize()
    outs = []
    for rep in range(9):
        w, g = ws[rep % 3], gs[rep % 3]
        outs.append((w, R.ragged_paged_attention(*g.args(), **w.kwargs)[0]))
    torch.cuda.synchronize()
    for rep, (w, out) in enumerate(outs):
        assert_close(out[:w.num_tokens].cpu(), exp[w.name], 2e-2, 2e-2, f"{w.name} call {rep}")


def test_custom_op_path_matches_eager_path(gpu_device):
    """Eager calls run the custom op's body directly; the registered ops (the path
    torch.compile keeps opaque) must give the same bytes, with and without out=
    and return_lse."""
    w = W.make_workload([(1, 800), (37, 120), (1, 2000), (64, 64)], 16, 4, 128, 16, seed=41,
                        name="op-path")
    g = w.to(gpu_device)
    kw = w.kwargs
    out_e, _ = R.ragged_paged_attention(*g.args(), **kw)
    out_o = torch.ops.rpa_amd.ragged_paged_attention(
        *g.args(), g.q.dtype, True, False, float(kw["sm_scale"]), 0, 0.0, False, 1.0, 1.0, 1.0,
        N.RPA_PATH_AUTO, 1)
    buf = torch.empty_like(g.q)
    torch.ops.rpa_amd.ragged_paged_attention_out(
        *g.args(), buf, True, False, float(kw["sm_scale"]), 0, 0.0, False, 1.0, 1.0, 1.0,
        N.RPA_PATH_AUTO, 1)
    out_l, _, lse_e = R.ragged_paged_attention(*g.args(), return_lse=True, **kw)
    out_lo, lse_o = torch.ops.rpa_amd.ragged_paged_attention_lse(
        *g.args(), g.q.dtype, True, False, float(kw["sm_scale"]), 0, 0.0, False, 1.0, 1.0, 1.0,
        N.RPA_PATH_AUTO, 1)
    torch.cuda.synchronize()
    n = w.num_tokens
    assert torch.equal(out_e[:n].view(torch.int16), out_o[:n].view(torch.int16))
    assert torch.equal(out_e[:n].view(torch.int16), buf[:n].view(torch.int16))
    assert torch.equal(out_l[:n].view(torch.int16), out_lo[:n].view(torch.int16))
    assert torch.equal(lse_e[:n], lse_o[:n])
    exp = O.ref_ragged_paged_attention(*w.args(), mode="fp32", **kw)[0]
    assert_close(out_e[:n].cpu(), exp, 2e-2, 2e-2, "op-path")


def test_decode_one_pair_many_partials(gpu_device):
    """One long decode pair spread over nearly every decode wavefront (about 900
    partials): the merge combines them 64 units at a time (rpa_merge.h)."""
    check(W.make_workload([(1, 200000)], 8, 1, 128, 256, seed=46, name="one-pair"),
          gpu_device)


def test_1m_context(gpu_device):
    """correctness_test.py:950-985: two decodes of 1M keys, head_dim 256, page size
    256, max_num_seqs 192, distribution [2, 2, 2].  The 4.3 GB cache puts pages
    past 4 GB, and each (sequence, kv head) pair is spread over about 256
    wavefronts."""
    kv = 1 << 20
    w = W.make_workload([(1, kv)] * 2, 8, 2, 256, 256, seed=45, max_num_seqs=192,
                        num_pages=2 * kv // 256 + 8, distribution=[2, 2, 2], name="1m-context")
    check(w, gpu_device)


def test_large_schedule(gpu_device):
    """correctness_test.py:525-551: 1024 decodes, 16 q heads on one kv head (16 rows
    per decode group), head_dim 256, page size 256.  The reference's 8191 keys per
    sequence are cut to 2047 (a 2.1 GB cache) so that building the workload and
    the CPU oracle take seconds, not most of a minute."""
    w = W.make_workload([(1, 2047)] * 1024, 16, 1, 256, 256, seed=47,
                        num_pages=8 * 1024 + 32, name="large-schedule")
    check(w, gpu_device)


def test_stale_plan_entries_past_num_seqs(gpu_device):
    """Merge wavefronts load a pair's plan entries together with the plan's
    sequence count, before they know whether the pair exists
    (rpa_finish_items.h).  After a larger batch on the same workspace, the plan
    slots past a smaller batch's num_seqs hold that batch's split pairs; they
    must be discarded (kernel.py:1345-1349: only s < num_seqs exists).  The
    stale pairs' output rows (token s of the larger batch) are checked rows of
    a prefill sequence in the smaller batches, so a stale merge would show."""
    big = W.make_workload([(1, k) for k in (3000, 2500, 4000, 1800, 3500, 2900, 3300, 2100)],
                          32, 8, 128, 16, seed=41, max_num_seqs=8, name="stale-a")
    check(big, gpu_device)
    for seed, seqs in ((42, [(1, 2200), (1, 3900), (1, 60), (6, 300)]),
                       (43, [(1, 700), (9, 500)])):
        check(W.make_workload(seqs, 32, 8, 128, 16, seed=seed, max_num_seqs=8,
                              name=f"stale-b{len(seqs)}"), gpu_device)


def test_decode_only_measurement_path(gpu_device):
    """RPA_PATH_DECODE_ONLY launches the decode kernel alone: single-unit
    decode rows are final; shapes the decode kernel does not take are rejected."""
    # kv_len <= 32 keys: one 32-key tile, so every sequence is a single unit.
    w = W.make_workload([(1, 20), (1, 7), (1, 32)], 8, 2, 128, 16, seed=38, name="dec-only")
    exp_out, _ = O.ref_ragged_paged_attention(*w.args(), mode="fp32", skip_kv_update=True,
                                              **w.kwargs)
    out, _ = run_gpu(w, gpu_device, path=N.RPA_PATH_DECODE_ONLY, skip_kv_update=True)
    assert_close(out, exp_out, 2e-2, 2e-2, "decode-only path, single-unit rows")
    # Shapes the decode kernel does not take (f32 KV) are rejected.
    p = W.make_workload([(1, 40)], 8, 2, 128, 16, seed=39, q_dtype=torch.float32,
                        kv_dtype=torch.float32, name="f32")
    with pytest.raises(NotImplementedError):
        run_gpu(p, gpu_device, path=N.RPA_PATH_DECODE_ONLY)


@pytest.mark.parametrize("ps,window", [(16, None), (16, 3000), (32, None)])
def test_prefill_long_context(gpu_device, ps, window):
    """Prefill chunks whose key range spans more pages than the kernel keeps in
    LDS (512) read the page table directly; the windowed case starts its range
    mid-sequence."""
    check(W.make_workload([(64, 10000), (1, 9000), (200, 16500)], 16, 4, 128, ps, seed=41,
                          sliding_window=window, distribution=[0, 0, 3], name=f"long-ps{ps}"),
          gpu_device)


@pytest.mark.parametrize("scale", [0.0, -0.05])
def test_non_positive_sm_scale(gpu_device, scale):
    """sm_scale is a plain multiplier: zero gives uniform attention over the
    visible keys, a negative one flips the ranking (decode and prefill rows)."""
    check(W.make_workload([(1, 70), (9, 40), (33, 33)], 8, 2, 128, 16, seed=40,
                          distribution=[1, 1, 3], name=f"scale{scale}", sm_scale=scale),
          gpu_device)


# ---------------------------------------------------------------------------
# return_lse and the LSE merge (batched_rpa/wrapper.py:553, :610-623;
# layers/adapter/cp_attention.py:45-72)
# ---------------------------------------------------------------------------
LSE_CASES = [
    ("decode", dict(seq_lens=DECODE16, hq=32, hkv=8, d=128, ps=16,
                    distribution=[16, 16, 16])),
    ("mixed", dict(seq_lens=MIXED16, hq=32, hkv=8, d=128, ps=16)),
    ("window-cap", dict(seq_lens=[(1, 700), (40, 300), (1, 5)], hq=16, hkv=4, d=128, ps=16,
                        sliding_window=128, soft_cap=30.0)),
    ("d256", dict(seq_lens=[(1, 500), (33, 90)], hq=16, hkv=8, d=256, ps=16)),
    ("fp8", dict(seq_lens=[(1, 900), (17, 80)], hq=32, hkv=8, d=128, ps=32,
                 kv_dtype=E4M3, k_scale=0.7, v_scale=1.3)),
    ("generic-qpk24", dict(seq_lens=[(1, 300), (9, 40)], hq=24, hkv=1, d=128, ps=16)),
    ("f32", dict(seq_lens=[(1, 70), (5, 20)], hq=8, hkv=2, d=64, ps=16,
                 q_dtype=torch.float32, kv_dtype=torch.float32)),
]


@pytest.mark.parametrize("name", [c[0] for c in LSE_CASES])
def test_return_lse(gpu_device, name):
    c = dict(dict(LSE_CASES)[name])
    seq_lens, hq, hkv, d, ps = (c.pop(x) for x in ("seq_lens", "hq", "hkv", "d", "ps"))
    w = W.make_workload(seq_lens, hq, hkv, d, ps, seed=51, name=f"lse-{name}", **c)
    _log(f"[rpa-gpu] return_lse {name}")
    exp_out, exp_cache, exp_lse = O.ref_ragged_paged_attention(*w.args(), mode="fp32",
                                                               return_lse=True, **w.kwargs)
    g = w.to(gpu_device)
    out, cache, lse = R.ragged_paged_attention(*g.args(), return_lse=True, **w.kwargs)
    torch.cuda.synchronize()
    n = w.num_tokens
    tol = TOL[w.kv_cache.dtype]
    assert_close(out[:n].cpu(), exp_out, tol, tol, f"{name} output")
    # The LSE is an fp32 reduction of fp32 logits on both sides.
    assert_close(lse[:n].cpu(), exp_lse, 1e-3, 1e-3, f"{name} lse")
    assert bool(torch.isneginf(lse[n:]).all()), "rows past the batch keep lse -inf"
    assert bytes_equal(cache.cpu(), exp_cache)


@pytest.mark.parametrize("parts,dt", [(2, BF16), (3, torch.float32), (5, BF16), (70, torch.float32)])
def test_merge_attn_states_gpu(gpu_device, parts, dt):
    g = torch.Generator().manual_seed(52)
    T, H, D = 37, 6, 128
    outs = torch.randn(parts, T, H, D, generator=g).to(dt)
    lses = torch.randn(parts, T, H, generator=g) * 3
    lses[0, :5] = float("-inf")          # empty partials
    outs[0, :5] = float("nan")           # ... whose outputs are garbage
    lses[:, 7] = float("-inf")           # a row with no keys anywhere
    lses[parts - 1, 9, 2] = float("nan")  # a NaN lse propagates (torch.maximum)
    exp_out, exp_lse = O.merge_attn_states(outs.double(), lses.double())
    out, lse = R.merge_attn_states(outs.to(gpu_device), lses.to(gpu_device))
    torch.cuda.synchronize()
    assert out.dtype == torch.float32  # the reference's result dtype
    out, lse = out.cpu(), lse.cpu()
    nan_o, nan_l = torch.isnan(exp_out), torch.isnan(exp_lse)
    assert nan_l[9, 2] and nan_o[9, 2].all()
    assert torch.equal(torch.isnan(out), nan_o) and torch.equal(torch.isnan(lse), nan_l)
    assert_close(out[~nan_o], exp_out[~nan_o], 1e-5, 1e-5, "merged output")
    assert_close(lse[~nan_l], exp_lse[~nan_l], 1e-5, 1e-5, "merged lse")
    # bf16 output: the same values rounded.
    ob, lb = R.merge_attn_states(outs.to(gpu_device), lses.to(gpu_device),
                                 out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    assert ob.dtype == BF16
    assert bytes_equal(ob.cpu()[~nan_o], out[~nan_o].to(BF16))
    if parts == 2:
        o2, l2 = R.merge_attn_results(outs[0].to(gpu_device), lses[0].to(gpu_device),
                                      outs[1].to(gpu_device), lses[1].to(gpu_device))
        assert torch.equal(o2.cpu().nan_to_num(), out.nan_to_num())
        assert torch.equal(l2.cpu().nan_to_num(), lse.nan_to_num())
        ref_o, ref_l = O.merge_attn_results(outs[0].double(), lses[0].double(),
                                            outs[1].double(), lses[1].double())
        assert torch.equal(torch.isnan(ref_o), nan_o) and torch.equal(torch.isnan(ref_l), nan_l)


def test_dcp_split_merge_equals_full(gpu_device):
    """Context-parallel decode on one GPU: each sequence's keys are split at a
    page boundary into two shards (two calls over the same cache with their
    own kv_lens and page-table offsets, skip_kv_update), and the LSE merge of
    the shards equals attention over all keys (cp_attention.py:274-348)."""
    ps = 16
    kvl = [4000, 1000, 33, 2500]
    w = W.make_workload([(1, k) for k in kvl], 32, 8, 128, ps, seed=53, name="dcp")
    kw = dict(w.kwargs)
    exp_out, _ = O.ref_ragged_paged_attention(*w.args(), mode="fp32", skip_kv_update=True, **kw)
    g = w.to(gpu_device)
    S = len(kvl)
    pps = w.page_indices.shape[0] // S
    split = [O.cdiv(k, 2 * ps) * ps for k in kvl]          # shard A: keys [0, split)
    lens_a = torch.tensor(split, dtype=torch.int32)
    lens_b = torch.tensor([k - s for k, s in zip(kvl, split)], dtype=torch.int32)
    pt = w.page_indices.view(S, pps)
    pt_b = torch.zeros_like(pt)
    for s in range(S):
        off = split[s] // ps
        pt_b[s, :pps - off] = pt[s, off:]
    outs, lses = [], []
    for lens, table in ((lens_a, pt), (lens_b, pt_b)):
        assert bool((lens > 0).all())
        o, _, l = R.ragged_paged_attention(g.q, g.k, g.v, g.kv_cache, lens.to(gpu_device),
                                           table.reshape(-1).contiguous().to(gpu_device),
                                           g.cu_q_lens, g.distribution, skip_kv_update=True,
                                           return_lse=True, **kw)
        outs.append(o)
        lses.append(l)
    merged, _ = R.merge_attn_results(outs[0], lses[0], outs[1], lses[1])
    torch.cuda.synchronize()
    assert_close(merged[:S].cpu(), exp_out, 2e-2, 2e-2, "merged shards vs full attention")
