"""Host-side checks that need no GPU: the C ABI library loads and exports every
symbol include/rpa.h declares, descriptor layout agrees with C, host-only
entry points (validation, cache shape, workspace size) behave, and the
Python API refuses to run anywhere but on the GPU."""

import os
import re
import shutil
import subprocess
import tempfile

import pytest
import torch

import vllm_torchtpu_amd as R
from vllm_torchtpu_amd import _native as N
import vllm_torchtpu_amd.workloads  # noqa: F401

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "rpa.h")


def _declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|size_t|const char\*)\s+(rpa_\w+)\s*\(", text,
                                 re.M)))


def test_library_exports_every_declared_symbol():
    L = N.lib()
    declared = _declared_functions()
    assert declared, "no declarations parsed from include/rpa.h"
    assert sorted(N.EXPORTED_SYMBOLS) == declared
    for name in declared:
        assert hasattr(L, name), name
    assert L.rpa_abi_version() == N.ABI_VERSION


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not available")
def test_desc_layout_matches_c():
    src = r"""
    #include <stdio.h>
    #include <stddef.h>
    #include "rpa.h"
    int main(void) {
      printf("%zu %zu %zu %zu %zu %zu %zu\n", sizeof(rpa_desc), offsetof(rpa_desc, soft_cap),
             offsetof(rpa_desc, sm_scale), offsetof(rpa_desc, path),
             offsetof(rpa_desc, decode_query_size), offsetof(rpa_desc, window_all_rows),
             offsetof(rpa_desc, reserved));
      return 0;
    }
    """
    with tempfile.TemporaryDirectory() as d:
        c = os.path.join(d, "t.c")
        open(c, "w").write(src)
        exe = os.path.join(d, "t")
        subprocess.check_call(["gcc", "-I", os.path.join(ROOT, "include"), c, "-o", exe])
        vals = [int(x) for x in subprocess.check_output([exe]).split()]
    D = N.RpaDesc
    assert vals == [__import__("ctypes").sizeof(D), D.soft_cap.offset, D.sm_scale.offset,
                    D.path.offset, D.decode_query_size.offset, D.window_all_rows.offset,
                    D.reserved.offset]


def _desc(**over):
    w = R.workloads.make_workload([(3, 20), (1, 9)], 8, 2, 128, 16, seed=0)
    d = R.rpa._make_desc(w.q, w.k, w.kv_cache, w.kv_lens, w.page_indices, torch.bfloat16,
                         use_causal_mask=True, skip_kv_update=False, sm_scale=0.1,
                         sliding_window=None, soft_cap=None, q_scale=None, k_scale=None,
                         v_scale=None)
    for k, v in over.items():
        setattr(d, k, v)
    return d


def test_validate_desc_codes():
    L = N.lib()
    assert L.rpa_validate_desc(_desc()) == N.RPA_OK
    assert L.rpa_validate_desc(_desc(abi_version=99)) == N.RPA_ERR_ABI
    assert L.rpa_validate_desc(_desc(num_q_heads=7)) == N.RPA_ERR_INVALID_ARG
    assert L.rpa_validate_desc(_desc(head_dim_padded=256)) == N.RPA_ERR_INVALID_ARG
    assert L.rpa_validate_desc(_desc(kv_heads_x2=6)) == N.RPA_ERR_INVALID_ARG
    assert L.rpa_validate_desc(_desc(has_soft_cap=1, soft_cap=0.0)) == N.RPA_ERR_INVALID_ARG
    # f16 q and KV (any float KV dtype, kernel.py:1447-1453) run on the generic kernels.
    assert L.rpa_validate_desc(_desc(kv_dtype=N.RPA_DTYPE_F16, q_dtype=N.RPA_DTYPE_F16,
                                     out_dtype=N.RPA_DTYPE_F16)) == N.RPA_OK
    assert L.rpa_validate_desc(_desc(out_dtype=99)) in (N.RPA_ERR_INVALID_ARG,
                                                        N.RPA_ERR_UNSUPPORTED)
    assert L.rpa_validate_desc(_desc(decode_query_size=-1)) == N.RPA_ERR_INVALID_ARG
    assert L.rpa_workspace_size(_desc()) > 0
    assert L.rpa_workspace_size(_desc(abi_version=99)) == 0
    with pytest.raises(ValueError):
        N.check(N.RPA_ERR_INVALID_ARG, "x")
    with pytest.raises(NotImplementedError):
        N.check(N.RPA_ERR_UNSUPPORTED, "x")
    with pytest.raises(RuntimeError):
        N.check(N.RPA_ERR_LAUNCH, "x")


@pytest.mark.parametrize("hkv,d,dt", [(2, 128, torch.bfloat16), (1, 80, torch.float8_e4m3fn),
                                      (3, 240, torch.float32)])
def test_native_cache_shape_matches_python(hkv, d, dt):
    import ctypes
    out = (ctypes.c_int64 * 5)()
    assert N.lib().rpa_get_kv_cache_shape(11, 32, hkv, d, N.rpa_dtype(dt), out) == 0
    assert tuple(out) == R.get_kv_cache_shape(11, 32, hkv, d, dt)


def test_no_cpu_path():
    w = R.workloads.make_workload([(3, 20), (1, 9)], 8, 2, 128, 16, seed=0)
    with pytest.raises(RuntimeError, match="no CPU path"):
        R.ragged_paged_attention(*w.args(), **w.kwargs)


def test_mask_value_policy():
    w = R.workloads.make_workload([(3, 20)], 8, 2, 128, 16, seed=0)
    with pytest.raises(NotImplementedError):
        R.ragged_paged_attention(*w.args(), mask_value=-1.0, **w.kwargs)


def test_static_validation_memo_keeps_errors():
    """A signature that passed validation is remembered; a failing one is not, and
    any argument the rules read (a dtype, a window) makes a new signature."""
    w = R.workloads.make_workload([(3, 20), (1, 9)], 8, 2, 128, 16, seed=0)
    for _ in range(2):
        with pytest.raises(RuntimeError, match="no CPU path"):
            R.ragged_paged_attention(*w.args(), **w.kwargs)
    for _ in range(2):
        with pytest.raises(ValueError):
            R.ragged_paged_attention(*w.args(), sliding_window=0, **w.kwargs)
    args = list(w.args())
    args[4] = args[4].to(torch.int64)
    for _ in range(2):
        with pytest.raises(ValueError, match="int32"):
            R.ragged_paged_attention(*args, **w.kwargs)
    with pytest.raises(ValueError):
        R.ragged_paged_attention(*w.args(), use_causal_mask=True, skip_kv_mask=True,
                                 **w.kwargs)


def test_custom_op_fake_shape():
    from torch._subclasses.fake_tensor import FakeTensorMode
    w = R.workloads.make_workload([(3, 20), (1, 9)], 8, 2, 128, 16, seed=0)
    W64 = R.workloads.make_workload([(3, 20), (1, 9)], 8, 2, 64, 16, seed=0, layout="hd64")
    with FakeTensorMode() as mode:
        args = [mode.from_tensor(t) for t in w.args()]
        out = torch.ops.rpa_amd.ragged_paged_attention(
            *args, torch.bfloat16, True, False, 0.1, 0, 0.0, False, 1.0, 1.0, 1.0, 0, 4)
        s = torch.ops.rpa_amd.ragged_paged_attention_hd64(
            *[mode.from_tensor(t) for t in W64.args()], None, True, False, 0.1, 0, 0.0, False,
            1.0, 1.0, 1.0)
    assert tuple(out.shape) == tuple(w.q.shape) and out.dtype == torch.bfloat16
    assert tuple(s.shape) == tuple(W64.q.shape)


def test_rpa_case_ranges():
    dist = torch.tensor([3, 5, 9], dtype=torch.int32)
    assert [tuple(int(x) for x in c.get_range(dist)) for c in R.RpaCase] == [
        (0, 3), (3, 5), (5, 9)]
    assert [c.symbol for c in R.RpaCase] == ["d", "p", "m"]
