"""rpa_forward_noalloc: the entry point that allocates nothing (include/rpa.h).

It runs rpa_forward's kernels on a fixed per-GPU scratch array instead of a
caller workspace.  The GPU test calls both entry points through the C ABI on
copies of the same inputs, twice in a row (the second call smaller, so the
scratch holds the first call's leftovers), and requires identical output and
cache bytes, and the output within the oracle's tolerance.  The host test
checks that a descriptor needing more scratch than the array is refused
before anything is launched.
"""

import ctypes

import pytest
import torch

from oracle import rpa_oracle as O
from rpa_testlib import assert_close, bytes_diff, bytes_equal

import vllm_torchtpu_amd as R
import vllm_torchtpu_amd.workloads as W
from vllm_torchtpu_amd import _native as N


def _desc(g, **over):
    kw = dict(g.kwargs)
    d = R.rpa._make_desc(g.q, g.k, g.kv_cache, g.kv_lens, g.page_indices, g.q.dtype,
                         use_causal_mask=True, skip_kv_update=False, sm_scale=kw["sm_scale"],
                         sliding_window=kw.get("sliding_window"), soft_cap=kw.get("soft_cap"),
                         q_scale=None, k_scale=kw.get("k_scale"), v_scale=kw.get("v_scale"))
    for k, v in over.items():
        setattr(d, k, v)
    return d


def _ptrs(g, out):
    return [g.q.data_ptr(), g.k.data_ptr(), g.v.data_ptr(), g.kv_cache.data_ptr(),
            g.kv_lens.data_ptr(), g.page_indices.data_ptr(), g.cu_q_lens.data_ptr(),
            g.distribution.data_ptr(), out.data_ptr()]


def test_noalloc_refuses_oversize_descriptor():
    """Needs more than RPA_NOALLOC_SCRATCH_BYTES: RPA_ERR_SCRATCH, nothing launched
    (null data pointers are never looked at)."""
    L = N.lib()
    w = W.make_workload([(1, 40)], 64, 8, 128, 16, seed=0, max_num_seqs=2048)
    d = _desc(w)
    assert L.rpa_workspace_size(d) > N.NOALLOC_SCRATCH_BYTES
    code = L.rpa_forward_noalloc(d, *([None] * 9), None)
    assert code == N.RPA_ERR_SCRATCH, code
    assert "rpa_forward_noalloc" in N.status_str(code)


@pytest.mark.gpu
def test_noalloc_matches_workspace_entry_point(gpu_device):
    L = N.lib()
    dev = gpu_device
    stream = torch.cuda.current_stream(dev)
    # Two calls in a row, the second smaller: 40 decode rows plus prefill
    # chunks (decode partials, plan and prefill all in the scratch), then a
    # decode-only batch of fewer sequences and tokens.
    cases = [
        W.make_workload([(1, 700 + 37 * i) for i in range(40)] + [(64, 300), (17, 1000)],
                        32, 8, 128, 16, seed=81, distribution=[40, 40, 42], name="noalloc-1"),
        W.make_workload([(1, 90 + 211 * i) for i in range(9)], 32, 8, 128, 16, seed=82,
                        distribution=[9, 9, 9], name="noalloc-2"),
    ]
    for w in cases:
        print(f"[noalloc] case {w.name} q={tuple(w.q.shape)} seqs={len(w.seq_lens)}", flush=True)
        exp_out, exp_cache = O.ref_ragged_paged_attention(*w.args(), mode="fp32", **w.kwargs)
        ga, gb = w.to(dev), w.to(dev)
        out_a = torch.full(ga.q.shape, float("nan"), dtype=ga.q.dtype, device=dev)
        out_b = torch.full(gb.q.shape, float("nan"), dtype=gb.q.dtype, device=dev)
        d = _desc(ga)
        need = int(L.rpa_workspace_size(d))
        assert 0 < need <= N.NOALLOC_SCRATCH_BYTES
        ws = torch.empty(need, dtype=torch.uint8, device=dev)
        code = L.rpa_forward(d, *_ptrs(ga, out_a), ws.data_ptr(), need, stream.cuda_stream)
        assert code == N.RPA_OK, N.status_str(code)
        code = L.rpa_forward_noalloc(d, *_ptrs(gb, out_b), stream.cuda_stream)
        assert code == N.RPA_OK, N.status_str(code)
        torch.cuda.synchronize()
        n = w.num_tokens
        assert bytes_equal(out_a[:n].cpu(), out_b[:n].cpu()), \
            bytes_diff(out_a[:n].cpu(), out_b[:n].cpu())
        assert bytes_equal(ga.kv_cache.cpu(), gb.kv_cache.cpu())
        assert_close(out_b[:n].cpu(), exp_out[:n], 2e-2, 2e-2, f"{w.name} vs oracle")
        assert bytes_equal(gb.kv_cache.cpu(), exp_cache)
