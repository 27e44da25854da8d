"""GPU parity for speculative-decoding verify windows: decode sequences with
q_len = K + 1 query tokens, run on the decode kernel when decode_query_size
(batched_rpa/wrapper.py:549, :601-602) covers them.  The oracle computes every
sequence the same way whatever decode_query_size is, so each case is checked
against ref_ragged_paged_attention (fp32 mode) to the usual bars: cache bit
exact, outputs within atol = rtol = 2e-2 (bf16 / f32) or 5e-2 (fp8).

Cases follow the reference's spec-decode test (tests/kernels/experimental/
batched_rpa/correctness_test.py:650-694) and widen it: new tokens that straddle
a tile boundary (32 keys at head_dim 128 bf16, 16 at 256, 64 at fp8 and at the
packed head_dim 64), 16-row groups (qpk 1 x 16 tokens, qpk 2 x 8), windows and
soft caps, fp8, sinks, LSE, skip_kv_update, non-causal rows, long sequences
whose groups are split between wavefronts (the merge path), and batches that
mix groups with q_len above decode_query_size (the prefill kernel's).
"""

import sys

import pytest
import torch

from oracle import rpa_oracle as O
from rpa_testlib import assert_close, bytes_diff, bytes_equal

import vllm_torchtpu_amd as R
import vllm_torchtpu_amd.workloads as W

pytestmark = pytest.mark.gpu

BF16, E4M3, E5M2 = torch.bfloat16, torch.float8_e4m3fn, torch.float8_e5m2
TOL = {BF16: 2e-2, E4M3: 5e-2, E5M2: 5e-2, torch.float32: 2e-2}

# correctness_test.py:655-672.
SPEC16 = [(4, 18), (4, 129), (3, 597), (4, 122), (2, 64), (4, 322), (4, 463), (3, 181),
          (4, 1107), (2, 123), (4, 31), (4, 18), (4, 1229), (3, 229), (4, 87), (4, 1328)]


def _log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def check(w, dev, dq, *, lse=False, **extra):
    kw = dict(w.kwargs)
    kw.update(extra)
    _log(f"[spec-gpu] case {w.name} dq={dq} seqs={w.seq_lens[:6]}"
         f"{'...' if len(w.seq_lens) > 6 else ''} q={tuple(w.q.shape)}"
         f" cache={tuple(w.kv_cache.shape)} {w.kv_cache.dtype} lse={lse} extra={extra}")
    if lse:
        exp_out, exp_cache, exp_lse = O.ref_ragged_paged_attention(
            *w.args(), mode="fp32", return_lse=True, **kw)
    else:
        exp_out, exp_cache = O.ref_ragged_paged_attention(*w.args(), mode="fp32", **kw)
    g = w.to(dev)
    res = R.ragged_paged_attention(*g.args(), decode_query_size=dq, return_lse=lse, **kw)
    torch.cuda.synchronize()
    n = w.num_tokens
    tol = TOL[w.kv_cache.dtype]
    assert_close(res[0][:n].cpu(), exp_out, tol, tol, f"{w.name} output")
    assert bytes_equal(res[1].cpu(), exp_cache), (
        f"{w.name}: cache differs from the oracle: {bytes_diff(res[1].cpu(), exp_cache)}")
    if lse:
        assert_close(res[2][:n].cpu(), exp_lse, 1e-3, 1e-3, f"{w.name} lse")


@pytest.mark.parametrize("dt", [BF16, torch.float32])
def test_reference_spec_decode(gpu_device, dt):
    """correctness_test.py:650-694: (32, 8) heads, head_dim 128, page 16,
    distribution all-decode, decode_query_size 4 (f32 runs the generic path)."""
    w = W.make_workload(SPEC16, 32, 8, 128, 16, q_dtype=dt, kv_dtype=dt, seed=81,
                        num_pages=1000, distribution=[16, 16, 16], name="ref-spec")
    check(w, gpu_device, 4)


@pytest.mark.parametrize("d,dt,kv", [(128, BF16, [33, 34, 35, 64, 65, 31]),
                                     (256, BF16, [17, 18, 19, 32, 33, 16]),
                                     (128, E4M3, [65, 66, 67, 128, 129, 63]),
                                     (64, BF16, [33, 34, 65, 66, 64, 30])])
def test_new_tokens_straddle_tiles(gpu_device, d, dt, kv):
    """q_len 4 groups whose new keys [kv_len - 4, kv_len) cross a tile edge."""
    seqs = [(4, k) for k in kv] + [(3, k + 1) for k in kv]
    scales = dict(k_scale=0.8, v_scale=1.2) if dt == E4M3 else {}
    w = W.make_workload(seqs, 16, 4, d, 16, kv_dtype=dt, seed=82, name=f"straddle-d{d}",
                        **scales)
    check(w, gpu_device, 4)


@pytest.mark.parametrize("heads,ql", [((8, 8), 16), ((8, 4), 8), ((16, 4), 4), ((32, 4), 2)])
def test_sixteen_row_groups(gpu_device, heads, ql):
    seqs = [(ql, k) for k in (ql, 40, 300, 1000, 2500)] + [(1, 77), (ql - 1 or 1, 90)]
    w = W.make_workload(seqs, heads[0], heads[1], 128, 16, seed=83, name="rows16")
    check(w, gpu_device, ql)


@pytest.mark.parametrize("window,cap", [(5, None), (3, 20.0), (128, None), (None, 30.0)])
def test_spec_window_cap(gpu_device, window, cap):
    w = W.make_workload([(4, 700), (4, 6), (3, 300), (4, 4), (2, 129)], 32, 8, 128, 16,
                        seed=84, sliding_window=window, soft_cap=cap, name="spec-wc")
    check(w, gpu_device, 4)


@pytest.mark.parametrize("dt", [E4M3, E5M2])
def test_spec_fp8(gpu_device, dt):
    w = W.make_workload([(4, 900), (2, 80), (4, 2000), (3, 63)], 32, 8, 128, 32, kv_dtype=dt,
                        k_scale=0.7, v_scale=1.3, seed=85, name="spec-fp8")
    check(w, gpu_device, 4)


def test_spec_mixed_with_prefill(gpu_device):
    """Groups above decode_query_size, single tokens and prefill chunks in one
    batch: each row is computed by whichever kernel owns its sequence."""
    seqs = [(1, 500), (4, 600), (5, 700), (3, 40), (64, 64), (2, 2), (100, 300), (4, 4097)]
    w = W.make_workload(seqs, 32, 8, 128, 16, seed=86, name="spec-mixed")
    check(w, gpu_device, 4)
    check(w, gpu_device, 2)


def test_spec_long_split_groups(gpu_device):
    """C2-shaped batch at q_len 4: most groups are cut between wavefronts and
    merged (16-row partial slots)."""
    g = torch.Generator().manual_seed(1002)
    kvl = W._uniform_ints(g, 512, 4096, 64)
    w = W.make_workload([(4, k) for k in kvl], 32, 8, 128, 16, seed=87, num_pages=20000,
                        pages_per_seq=256, distribution=[64, 64, 64], name="spec-c2")
    check(w, gpu_device, 4)
    check(w, gpu_device, 4, lse=True)


def test_spec_lse_skip_noncausal(gpu_device):
    w = W.make_workload([(4, 300), (3, 33), (4, 1500), (2, 2)], 16, 4, 128, 16, seed=88,
                        name="spec-lse")
    check(w, gpu_device, 4, lse=True)
    check(w, gpu_device, 4, skip_kv_update=True)
    check(w, gpu_device, 4, use_causal_mask=False)


def test_spec_sinks_hd64(gpu_device):
    """Sinks with several tokens per group (the sink is per q head, not per
    row): the packed head_dim 64 cache through the C ABI with decode_query_size."""
    hq, hkv = 16, 4
    w = W.make_workload([(4, 700), (3, 33), (4, 66), (2, 1200)], hq, hkv, 64, 16, seed=89,
                        layout="hd64", name="spec-hd64")
    sink = torch.linspace(-1.5, 2.5, hq)
    _log("[spec-gpu] case spec-hd64 sinks dq=4")
    exp_out, exp_cache = O.ref_ragged_paged_attention_hd64(*w.args(), sink, mode="fp32",
                                                           **w.kwargs)
    g = w.to(gpu_device)
    out = torch.empty(g.q.shape, dtype=g.q.dtype, device=gpu_device)
    p, ps, hp, pack, _ = g.kv_cache.shape
    R.rpa._rpa_forward_impl(g.q, g.k, g.v, g.kv_cache.view(p, ps, 2 * hp, pack, 64), g.kv_lens,
                            g.page_indices, g.cu_q_lens, g.distribution, out,
                            use_causal_mask=True, skip_kv_update=False,
                            sm_scale=w.kwargs["sm_scale"], sliding_window=None, soft_cap=None,
                            q_scale=None, k_scale=None, v_scale=None,
                            attention_sink=sink.to(gpu_device), decode_query_size=4)
    torch.cuda.synchronize()
    n = w.num_tokens
    assert_close(out[:n].cpu(), exp_out, 2e-2, 2e-2, "hd64 spec output")
    assert bytes_equal(g.kv_cache.cpu(), exp_cache)


def test_decode_query_size_validation(gpu_device):
    w = W.make_workload([(2, 20)], 8, 2, 128, 16, seed=0).to(gpu_device)
    with pytest.raises(ValueError):
        R.ragged_paged_attention(*w.args(), decode_query_size=0, **w.kwargs)
