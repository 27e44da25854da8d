"""The oracle against the committed golden fixtures (tests/golden/*.npz).

Each fixture's expected output is an fp64 per-element brute force and its
expected cache an explicit per-token record copy (tests/golden/make_golden.py),
neither of which shares code with the oracle.  The oracle's fp32 mode must
agree to fp32 accumulation error, its cache bit for bit; the fixture inputs
must be exactly what the seeded workload generator produces, so the fixtures
and the generated GPU test cases describe the same batches.
"""

import glob
import os

import pytest
import torch

from golden import make_golden as G
from oracle import rpa_oracle as O
from rpa_testlib import assert_close, bytes_equal

HERE = os.path.dirname(os.path.abspath(__file__))
FIXTURES = sorted(glob.glob(os.path.join(HERE, "golden", "*.npz")))
NAMES = [os.path.splitext(os.path.basename(f))[0] for f in FIXTURES]


def test_every_case_has_a_fixture():
    assert sorted(G.CASES) == NAMES


@pytest.mark.parametrize("name", NAMES)
def test_oracle_matches_fixture(name):
    fx = G.load(os.path.join(HERE, "golden", f"{name}.npz"))
    out, cache = O.ref_ragged_paged_attention(*fx["args"], mode="fp32", **fx["kwargs"])
    n = fx["out"].shape[0]
    assert_close(out[:n], fx["out"], 2e-5, 2e-5, f"{name}: oracle fp32 vs fixture")
    out64, _ = O.ref_ragged_paged_attention(*fx["args"], mode="fp64", **fx["kwargs"])
    assert_close(out64[:n], fx["out"], 1e-6, 1e-6, f"{name}: oracle fp64 vs fixture")
    assert bytes_equal(cache, fx["cache"]), f"{name}: oracle cache differs from the fixture"


@pytest.mark.parametrize("name", NAMES)
def test_fixture_inputs_match_generator(name):
    fx = G.load(os.path.join(HERE, "golden", f"{name}.npz"))
    w = G.build(name)
    for got, want in zip(fx["args"], w.args()):
        assert got.dtype == want.dtype and got.shape == want.shape
        assert bytes_equal(got, want), name
    assert fx["kwargs"] == {k: v for k, v in w.kwargs.items()}


def test_fixture_cache_changes_only_new_records():
    """Bytes outside the new tokens' records are unchanged in every fixture."""
    for name in NAMES:
        fx = G.load(os.path.join(HERE, "golden", f"{name}.npz"))
        before, after = fx["args"][3], fx["cache"]
        P, ps = before.shape[:2]
        it = {1: torch.uint8, 2: torch.int16, 4: torch.int32}[before.element_size()]
        diff = (before.view(it).reshape(P * ps, -1) != after.view(it).reshape(P * ps, -1))
        changed = int(diff.any(dim=1).sum())
        new_rows = 0 if fx["kwargs"].get("skip_kv_update") else sum(q for q, _ in fx["seq_lens"])
        assert changed <= new_rows, (name, changed, new_rows)


def _fixture(name):
    return G.load(os.path.join(HERE, "golden", f"{name}.npz"))


def _max_err(fx, args, kwargs):
    out, _ = O.ref_ragged_paged_attention(*args, mode="fp32", **kwargs)
    n = fx["out"].shape[0]
    return (out[:n].double() - fx["out"].double()).abs().max().item()


@pytest.mark.parametrize("mistake", ["window_off_by_one", "no_soft_cap", "no_k_scale",
                                     "no_v_scale", "kv_heads_swapped", "page_table_shifted",
                                     "new_tokens_from_cache"])
def test_fixtures_catch_planted_mistakes(mistake):
    """Plausible slips, planted in the oracle's inputs on the CPU, move the
    result far outside the GPU tolerance (2e-2) on some fixture."""
    name = {"window_off_by_one": "window_cap_bf16", "no_soft_cap": "window_cap_bf16",
            "no_k_scale": "fp8_e4m3_scales", "no_v_scale": "fp8_e4m3_scales",
            "kv_heads_swapped": "mixed_bf16", "page_table_shifted": "mixed_bf16",
            "new_tokens_from_cache": "mixed_bf16"}[mistake]
    fx = _fixture(name)
    args, kw = list(fx["args"]), dict(fx["kwargs"])
    if mistake == "window_off_by_one":
        kw["sliding_window"] += 1
    elif mistake == "no_soft_cap":
        kw.pop("soft_cap")
    elif mistake == "no_k_scale":
        kw.pop("k_scale")
    elif mistake == "no_v_scale":
        kw.pop("v_scale")
    elif mistake == "kv_heads_swapped":
        args[1], args[2] = args[1].flip(1), args[2].flip(1)
        args[3] = args[3].flip(2)
    elif mistake == "page_table_shifted":
        args[5] = args[5].roll(1)
    elif mistake == "new_tokens_from_cache":
        kw["skip_kv_update"] = True
    assert _max_err(fx, args, kw) > 0.1, mistake
