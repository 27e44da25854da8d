"""ctypes binding of librpa_hip.so (C ABI declared in include/rpa.h).

The library is built in-tree by `make -C vllm-torchtpu_amd/csrc` (or
`__graft_entry__.build()`).  torch is imported first so that torch's HIP
runtime (same SONAME, libamdhip64.so.7) is the one the library binds to:
one runtime per process.  There is no fallback: if the library is missing,
every entry point raises.
"""

from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (must be loaded before the HIP library)

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "librpa_hip.so")

ABI_VERSION = 1

RPA_DTYPE_F32 = 0
RPA_DTYPE_BF16 = 1
RPA_DTYPE_F16 = 2
RPA_DTYPE_FP8_E4M3FN = 3
RPA_DTYPE_FP8_E5M2 = 4

RPA_OK = 0
RPA_ERR_INVALID_ARG = -1
RPA_ERR_UNSUPPORTED = -2
RPA_ERR_WORKSPACE = -3
RPA_ERR_LAUNCH = -4
RPA_ERR_NULL_PTR = -5
RPA_ERR_ABI = -6
RPA_ERR_SCRATCH = -7

# Fixed per-GPU scratch of rpa_forward_noalloc (RPA_NOALLOC_SCRATCH_BYTES).
NOALLOC_SCRATCH_BYTES = 32 << 20

RPA_PATH_AUTO = 0
RPA_PATH_GENERIC = 1
RPA_PATH_DECODE_ONLY = 2  # measurement: the decode kernel alone

_TORCH_TO_RPA = {
    torch.float32: RPA_DTYPE_F32,
    torch.bfloat16: RPA_DTYPE_BF16,
    torch.float16: RPA_DTYPE_F16,
    torch.float8_e4m3fn: RPA_DTYPE_FP8_E4M3FN,
    torch.float8_e5m2: RPA_DTYPE_FP8_E5M2,
}

# Every symbol include/rpa.h declares.
EXPORTED_SYMBOLS = (
    "rpa_abi_version",
    "rpa_status_str",
    "rpa_validate_desc",
    "rpa_get_kv_cache_shape",
    "rpa_workspace_size",
    "rpa_kv_cache_update",
    "rpa_forward",
    "rpa_forward_lse",
    "rpa_forward_ex",
    "rpa_merge_attn_states",
    "rpa_forward_noalloc",
)


class RpaDesc(ctypes.Structure):
    """Mirror of `struct rpa_desc` (include/rpa.h)."""

    _fields_ = [
        ("abi_version", ctypes.c_int32),
        ("q_dtype", ctypes.c_int32),
        ("kv_dtype", ctypes.c_int32),
        ("out_dtype", ctypes.c_int32),
        ("max_num_tokens", ctypes.c_int32),
        ("num_q_heads", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("head_dim_padded", ctypes.c_int32),
        ("total_num_pages", ctypes.c_int32),
        ("page_size", ctypes.c_int32),
        ("kv_packing", ctypes.c_int32),
        ("kv_heads_x2", ctypes.c_int32),
        ("max_num_seqs", ctypes.c_int32),
        ("pages_per_seq", ctypes.c_int32),
        ("use_causal_mask", ctypes.c_int32),
        ("skip_kv_update", ctypes.c_int32),
        ("sliding_window", ctypes.c_int32),
        ("has_soft_cap", ctypes.c_int32),
        ("soft_cap", ctypes.c_float),
        ("sm_scale", ctypes.c_float),
        ("q_scale", ctypes.c_float),
        ("k_scale", ctypes.c_float),
        ("v_scale", ctypes.c_float),
        ("path", ctypes.c_int32),
        ("decode_query_size", ctypes.c_int32),
        ("window_all_rows", ctypes.c_int32),
        ("reserved", ctypes.c_int32 * 5),
    ]


_LIB = None


class NativeLibraryMissing(RuntimeError):
    pass


def lib() -> ctypes.CDLL:
    """Load librpa_hip.so once; raise if it has not been built."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(LIB_PATH):
        raise NativeLibraryMissing(
            f"{LIB_PATH} is not built: run `make -C vllm-torchtpu_amd/csrc` "
            "(or __graft_entry__.build()); there is no non-HIP fallback.")
    L = ctypes.CDLL(LIB_PATH)
    P = ctypes.c_void_p
    desc_p = ctypes.POINTER(RpaDesc)
    L.rpa_abi_version.restype = ctypes.c_int
    L.rpa_abi_version.argtypes = []
    L.rpa_status_str.restype = ctypes.c_char_p
    L.rpa_status_str.argtypes = [ctypes.c_int]
    L.rpa_validate_desc.restype = ctypes.c_int
    L.rpa_validate_desc.argtypes = [desc_p]
    L.rpa_get_kv_cache_shape.restype = ctypes.c_int
    L.rpa_get_kv_cache_shape.argtypes = [ctypes.c_int32] * 5 + [ctypes.POINTER(ctypes.c_int64)]
    L.rpa_workspace_size.restype = ctypes.c_size_t
    L.rpa_workspace_size.argtypes = [desc_p]
    L.rpa_kv_cache_update.restype = ctypes.c_int
    L.rpa_kv_cache_update.argtypes = [desc_p] + [P] * 8
    L.rpa_forward.restype = ctypes.c_int
    L.rpa_forward.argtypes = [desc_p] + [P] * 10 + [ctypes.c_size_t, P]
    L.rpa_forward_lse.restype = ctypes.c_int
    L.rpa_forward_lse.argtypes = [desc_p] + [P] * 11 + [ctypes.c_size_t, P]
    L.rpa_forward_ex.restype = ctypes.c_int
    L.rpa_forward_ex.argtypes = [desc_p] + [P] * 12 + [ctypes.c_size_t, P]
    L.rpa_forward_noalloc.restype = ctypes.c_int
    L.rpa_forward_noalloc.argtypes = [desc_p] + [P] * 10
    L.rpa_merge_attn_states.restype = ctypes.c_int
    L.rpa_merge_attn_states.argtypes = [ctypes.c_int32, ctypes.c_int64, ctypes.c_int32,
                                        ctypes.c_int32, ctypes.c_int32, P, P, P, P, P]
    if L.rpa_abi_version() != ABI_VERSION:
        raise NativeLibraryMissing(
            f"librpa_hip.so ABI {L.rpa_abi_version()} != expected {ABI_VERSION}; rebuild it")
    _LIB = L
    return L


def rpa_dtype(dt: torch.dtype) -> int:
    try:
        return _TORCH_TO_RPA[dt]
    except KeyError:
        raise ValueError(f"dtype {dt} is not supported by the RPA library") from None


def status_str(code: int) -> str:
    return lib().rpa_status_str(code).decode()


def check(code: int, what: str) -> None:
    """Map a status code to the exception the reference raises for it."""
    if code == RPA_OK:
        return
    msg = f"{what}: {status_str(code)} (status {code})"
    if code == RPA_ERR_INVALID_ARG:
        raise ValueError(msg)
    if code == RPA_ERR_UNSUPPORTED:
        raise NotImplementedError(msg)
    raise RuntimeError(msg)
