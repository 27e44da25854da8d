"""Writes the golden RPA fixtures in this directory (test infrastructure).

The reference (JAX/Pallas, Python 3.12) cannot run here and its own tests
commit no fixtures, so each fixture's expected values come from two
computations that share no code with the oracle or the HIP library:

* expected output: `rpa_testlib.brute_force_rpa`, a per-(row, head, key)
  fp64 loop written from the semantic contract of
  ref_ragged_paged_attention (kernel.py:74-214);
* expected cache: `expected_cache` below, an explicit per-token record copy
  of merge_kv(keys, values) into `page_indices[s * pps + j // ps]`, slot
  `j % ps` (kernel.py:148-166, :1140-1168), on integer views (bit exact).

Inputs are seeded `make_workload` batches shaped after the reference's test
case lists (correctness_test.py:472-986, test_rpa_skip_kv_update.py:98-182).
Tensors are stored as raw integer bits with their dtype names, so bf16 and
fp8 round-trip exactly through numpy; the expected cache is stored as the XOR
of its bits with the input cache's (zero wherever the call must not write).

    python tests/golden/make_golden.py          # rewrite every fixture
"""

from __future__ import annotations

import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
for p in (ROOT, os.path.dirname(HERE)):
    if p not in sys.path:
        sys.path.insert(0, p)

from rpa_testlib import brute_force_rpa  # noqa: E402

import vllm_torchtpu_amd.workloads as W  # noqa: E402

BF16, E4M3, E5M2 = torch.bfloat16, torch.float8_e4m3fn, torch.float8_e5m2

# name -> make_workload arguments.  Decode rows come first in `distribution`,
# as the model runner emits them.
CASES = {
    "mixed_bf16": dict(seq_lens=[(1, 1), (1, 17), (1, 33), (5, 5), (7, 40)], hq=4, hkv=2,
                       d=128, ps=8, seed=101, distribution=[3, 3, 5], max_num_tokens=20,
                       max_num_seqs=6),
    "window_cap_bf16": dict(seq_lens=[(1, 45), (6, 30), (3, 9)], hq=8, hkv=2, d=128, ps=16,
                            seed=102, distribution=[1, 1, 3], sliding_window=8, soft_cap=2.0),
    "fp8_e4m3_scales": dict(seq_lens=[(1, 70), (1, 3), (4, 21)], hq=8, hkv=2, d=128, ps=16,
                            seed=103, kv_dtype=E4M3, k_scale=0.5, v_scale=1.5,
                            distribution=[2, 2, 3]),
    "fp8_e5m2_decode": dict(seq_lens=[(1, 50), (1, 16)], hq=4, hkv=1, d=128, ps=16, seed=104,
                            kv_dtype=E5M2, k_scale=0.75, v_scale=0.5, distribution=[2, 2, 2]),
    "d64_padded": dict(seq_lens=[(1, 26), (4, 12)], hq=6, hkv=3, d=64, ps=8, seed=105,
                       distribution=[1, 1, 2]),
    "d256_decode": dict(seq_lens=[(1, 40), (1, 7), (1, 19)], hq=16, hkv=2, d=256, ps=8,
                        seed=106, distribution=[3, 3, 3]),
    "skip_update_bf16": dict(seq_lens=[(1, 20), (3, 19)], hq=4, hkv=2, d=128, ps=8, seed=107,
                             distribution=[1, 1, 2], skip_kv_update=True),
    "f32_kv_generic": dict(seq_lens=[(2, 9), (1, 5)], hq=2, hkv=1, d=64, ps=4, seed=108,
                           kv_dtype=torch.float32, q_dtype=torch.float32,
                           distribution=[0, 0, 2]),
    "nan_poison_bf16": dict(seq_lens=[(1, 13), (4, 20)], hq=4, hkv=2, d=128, ps=8, seed=109,
                            distribution=[1, 1, 2], nan_fill=True, max_num_seqs=4,
                            max_num_tokens=8),
}

_ITYPE = {1: torch.uint8, 2: torch.int16, 4: torch.int32}
_DTYPES = {str(t): t for t in (BF16, E4M3, E5M2, torch.float32, torch.float16)}


def build(name):
    c = dict(CASES[name])
    seq_lens, hq, hkv, d, ps = (c.pop(x) for x in ("seq_lens", "hq", "hkv", "d", "ps"))
    c.setdefault("pool_factor", 1.0)
    return W.make_workload(seq_lens, hq, hkv, d, ps, name=name, **c)


def bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(_ITYPE[t.element_size()]).numpy().copy()


def from_bits(a: np.ndarray, dtype_name: str) -> torch.Tensor:
    dt = _DTYPES[dtype_name]
    return torch.from_numpy(np.ascontiguousarray(a)).view(dt)


def load(path):
    """Fixture file -> dict of tensors, kwargs and the expected results."""
    z = np.load(path, allow_pickle=False)
    qd, kd = str(z["q_dtype"]), str(z["kv_dtype"])
    cache = from_bits(z["kv_cache"], kd)
    exp_cache = from_bits(z["kv_cache"] ^ z["cache_xor"], kd)
    return dict(
        name=os.path.splitext(os.path.basename(path))[0],
        args=(from_bits(z["q"], qd), from_bits(z["k"], kd), from_bits(z["v"], kd), cache,
              torch.from_numpy(z["kv_lens"]), torch.from_numpy(z["page_indices"]),
              torch.from_numpy(z["cu_q_lens"]), torch.from_numpy(z["distribution"])),
        kwargs=json.loads(str(z["kwargs"])), seq_lens=json.loads(str(z["seq_lens"])),
        out=torch.from_numpy(z["out"]), cache=exp_cache)


def expected_cache(w) -> torch.Tensor:
    """Every new token's record, copied element by element (integer views)."""
    cache = w.kv_cache.clone()
    if w.kwargs.get("skip_kv_update", False):
        return cache
    _, ps, _, _, dp = cache.shape
    S = w.kv_lens.shape[0]
    pps = w.page_indices.shape[0] // S
    hkv, d = w.k.shape[1], w.k.shape[2]
    it = _ITYPE[cache.element_size()]
    ci, ki, vi = cache.view(it), w.k.contiguous().view(it), w.v.contiguous().view(it)
    for s in range(w.num_seqs):
        q0, q1 = int(w.cu_q_lens[s]), int(w.cu_q_lens[s + 1])
        kl = int(w.kv_lens[s])
        for t in range(q0, q1):
            j = kl - (q1 - q0) + (t - q0)
            rec = ci[int(w.page_indices[s * pps + j // ps]), j % ps].reshape(-1, dp)
            for c in range(rec.shape[0]):
                for e in range(dp):
                    h, is_v = c // 2, c % 2
                    if h < hkv and e < d:
                        rec[c, e] = (vi if is_v else ki)[t, h, e]
                    else:
                        rec[c, e] = 0
    return cache


def write(name):
    w = build(name)
    out = brute_force_rpa(*w.args(), **w.kwargs).to(torch.float32)
    cache = expected_cache(w)
    np.savez_compressed(
        os.path.join(HERE, f"{name}.npz"),
        q=bits(w.q), k=bits(w.k), v=bits(w.v), kv_cache=bits(w.kv_cache),
        q_dtype=str(w.q.dtype), kv_dtype=str(w.kv_cache.dtype),
        kv_lens=w.kv_lens.numpy(), page_indices=w.page_indices.numpy(),
        cu_q_lens=w.cu_q_lens.numpy(), distribution=w.distribution.numpy(),
        kwargs=json.dumps(w.kwargs, sort_keys=True), seq_lens=json.dumps(w.seq_lens),
        out=out.numpy(), cache_xor=bits(cache) ^ bits(w.kv_cache))
    return w


def main():
    for name in CASES:
        w = write(name)
        size = os.path.getsize(os.path.join(HERE, f"{name}.npz"))
        print(f"{name}: {w.num_tokens} rows, cache {tuple(w.kv_cache.shape)} "
              f"{w.kv_cache.dtype}, {size // 1024} KiB")


if __name__ == "__main__":
    main()
