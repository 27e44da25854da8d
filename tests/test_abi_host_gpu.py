"""The C ABI driven by a non-Python host (tests/abi_host/rpa_abi_host.cpp).

The program allocates its own device buffers and workspace with hipMalloc,
creates its own stream and calls rpa_forward and rpa_forward_lse (the
entry points the reference's ragged_paged_attention,
kernels/ragged_paged_attention/v3/kernel.py:1609-1671, and the batched
wrapper's return_lse, batched_rpa/wrapper.py:553, map to).  Its results are
checked against the golden fixtures: cache bit-exact, output within the
tolerance of the KV dtype, LSE within 1e-3 of the brute force's.
"""

import os
import subprocess
import sys
import tempfile

import numpy as np
import pytest
import torch

from rpa_testlib import assert_close, brute_force_rpa, bytes_diff, bytes_equal

import vllm_torchtpu_amd as R

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import make_golden as G  # noqa: E402

PROGRAM = os.path.join(HERE, "abi_host", "rpa_abi_host")

pytestmark = pytest.mark.gpu

FIXTURES = ["mixed_bf16", "window_cap_bf16", "fp8_e4m3_scales", "d256_decode"]
DESC_FIELDS = ["q_dtype", "kv_dtype", "out_dtype", "max_num_tokens", "num_q_heads",
               "num_kv_heads", "head_dim", "head_dim_padded", "total_num_pages", "page_size",
               "kv_packing", "kv_heads_x2", "max_num_seqs", "pages_per_seq", "use_causal_mask",
               "skip_kv_update", "sliding_window", "has_soft_cap", "soft_cap", "sm_scale",
               "q_scale", "k_scale", "v_scale"]


def _raw(t: torch.Tensor) -> bytes:
    it = {1: torch.uint8, 2: torch.int16, 4: torch.int32}[t.element_size()]
    return t.contiguous().view(it).numpy().tobytes()


def _from_raw(path, like: torch.Tensor) -> torch.Tensor:
    it = {1: torch.uint8, 2: torch.int16, 4: torch.int32}[like.element_size()]
    a = np.fromfile(path, dtype={torch.uint8: np.uint8, torch.int16: np.int16,
                                 torch.int32: np.int32}[it])
    return torch.from_numpy(a).view(like.dtype).reshape(like.shape)


@pytest.mark.parametrize("name", FIXTURES)
def test_c_host_matches_fixture(name):
    assert os.path.exists(PROGRAM), f"{PROGRAM} is not built (make -C tests/abi_host)"
    fx = G.load(os.path.join(HERE, "golden", f"{name}.npz"))
    q, k, v, cache, kvl, pidx, cu, dist = fx["args"]
    kw = dict(fx["kwargs"])
    print(f"[abi-host] fixture {name} q={tuple(q.shape)} cache={tuple(cache.shape)} "
          f"{cache.dtype} kw={kw}", flush=True)
    d = R.rpa._make_desc(q, k, cache, kvl, pidx, q.dtype,
                         use_causal_mask=kw.get("use_causal_mask", True),
                         skip_kv_update=kw.get("skip_kv_update", False),
                         sm_scale=kw["sm_scale"], sliding_window=kw.get("sliding_window"),
                         soft_cap=kw.get("soft_cap"), q_scale=kw.get("q_scale"),
                         k_scale=kw.get("k_scale"), v_scale=kw.get("v_scale"))
    with tempfile.TemporaryDirectory() as tmp:
        with open(os.path.join(tmp, "desc.txt"), "w") as f:
            for fld in DESC_FIELDS:
                f.write(f"{fld} {float(getattr(d, fld))!r}\n")
        for fname, t in (("q", q), ("k", k), ("v", v), ("kv_cache", cache), ("kv_lens", kvl),
                         ("page_indices", pidx), ("cu_q_lens", cu), ("distribution", dist)):
            with open(os.path.join(tmp, f"{fname}.bin"), "wb") as f:
                f.write(_raw(t))
        r = subprocess.run([PROGRAM, tmp], capture_output=True, text=True, timeout=120)
        assert r.returncode == 0, f"rpa_abi_host failed:\n{r.stdout}\n{r.stderr}"
        out = _from_raw(os.path.join(tmp, "out.bin"), q)
        out_lse = _from_raw(os.path.join(tmp, "out_lse.bin"), q)
        lse = _from_raw(os.path.join(tmp, "lse.bin"), torch.empty(q.shape[:2]))
        c1 = _from_raw(os.path.join(tmp, "cache.bin"), cache)
        c2 = _from_raw(os.path.join(tmp, "cache_lse.bin"), cache)
    n = fx["out"].shape[0]
    tol = 5e-2 if cache.element_size() == 1 else 2e-2
    assert bytes_equal(c1, fx["cache"]), bytes_diff(c1, fx["cache"])
    assert bytes_equal(c2, fx["cache"]), bytes_diff(c2, fx["cache"])
    assert_close(out[:n], fx["out"], tol, tol, f"{name}: rpa_forward output")
    assert_close(out_lse[:n], fx["out"], tol, tol, f"{name}: rpa_forward_lse output")
    _, bf_lse = brute_force_rpa(*fx["args"], return_lse=True, **kw)
    assert_close(lse[:n], bf_lse, 1e-3, 1e-3, f"{name}: rpa_forward_lse lse")
