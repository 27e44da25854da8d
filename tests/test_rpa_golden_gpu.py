"""The HIP library against the committed golden fixtures (tests/golden/*.npz):
output within the tolerance of its KV dtype of the fp64 brute force, cache
bit for bit equal to the explicit record copy, through the Python API (which
calls the C ABI)."""

import glob
import os
import sys

import pytest
import torch

from golden import make_golden as G
from rpa_testlib import assert_close, bytes_equal

import vllm_torchtpu_amd as R

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
FIXTURES = sorted(glob.glob(os.path.join(HERE, "golden", "*.npz")))
TOL = {torch.bfloat16: 2e-2, torch.float8_e4m3fn: 5e-2, torch.float8_e5m2: 5e-2,
       torch.float32: 2e-2}


@pytest.mark.parametrize("path", FIXTURES, ids=lambda f: os.path.basename(f)[:-4])
def test_golden_fixture(gpu_device, path):
    fx = G.load(path)
    print(f"[rpa-gpu] golden {fx['name']} seqs={fx['seq_lens']} kw={fx['kwargs']}", flush=True)
    sys.stdout.flush()
    args = [a.to(gpu_device) for a in fx["args"]]
    out, cache = R.ragged_paged_attention(*args, **fx["kwargs"])
    torch.cuda.synchronize()
    n = fx["out"].shape[0]
    tol = TOL[fx["cache"].dtype]
    assert_close(out[:n].cpu(), fx["out"], tol, tol, f"{fx['name']} output")
    assert bytes_equal(cache.cpu(), fx["cache"]), f"{fx['name']}: cache differs from the fixture"
