"""Seeded synthetic RPA workloads (the benchmark configurations and test cases).

Inputs follow the reference's own test conventions
(tests/kernels/experimental/batched_rpa/correctness_test.py:199-330 and
tests/kernels/test_rpa_bundled.py:58-114 of vllm-torchtpu): i.i.d. N(0,1)
Q/K/V, pages drawn from a seeded shuffled pool, sequences given as
(q_len, kv_len) pairs.  Tensors are built on the CPU with a torch.Generator
and moved by the caller.
"""

from __future__ import annotations

import dataclasses

import torch

from .quantization import quantize_kv
from .util import cdiv, get_dtype_packing
from .rpa import get_kv_cache_shape
from .rpa_hd64 import get_kv_cache_shape_hd64


@dataclasses.dataclass
class Workload:
    name: str
    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    kv_cache: torch.Tensor
    kv_lens: torch.Tensor
    page_indices: torch.Tensor
    cu_q_lens: torch.Tensor
    distribution: torch.Tensor
    kwargs: dict
    seq_lens: list  # [(q_len, kv_len)]

    @property
    def num_seqs(self) -> int:
        return int(self.distribution[2])

    @property
    def num_tokens(self) -> int:
        return int(self.cu_q_lens[self.num_seqs])

    def to(self, device) -> "Workload":
        f = lambda t: t.to(device)  # noqa: E731
        return dataclasses.replace(self, q=f(self.q), k=f(self.k), v=f(self.v),
                                   kv_cache=f(self.kv_cache), kv_lens=f(self.kv_lens),
                                   page_indices=f(self.page_indices),
                                   cu_q_lens=f(self.cu_q_lens),
                                   distribution=f(self.distribution))

    def args(self):
        return (self.q, self.k, self.v, self.kv_cache, self.kv_lens, self.page_indices,
                self.cu_q_lens, self.distribution)


def make_workload(seq_lens, num_q_heads, num_kv_heads, head_dim, page_size, *,
                  q_dtype=torch.bfloat16, kv_dtype=torch.bfloat16, seed=0,
                  num_pages=None, pool_factor=1.25, max_num_seqs=None,
                  max_num_tokens=None, pages_per_seq=None, distribution=None,
                  k_scale=None, v_scale=None, nan_fill=False, name="custom",
                  layout="v3", **kwargs) -> Workload:
    """Build one ragged batch.

    seq_lens: list of (q_len, kv_len).  Each sequence takes cdiv(kv_len, ps)
    distinct pages from a seeded permutation of the pool.  The cache holds
    N(0,1) values (quantised with k_scale/v_scale for fp8) everywhere; with
    nan_fill, every cache row, page and page-table slot no sequence uses is
    NaN (or -1 for the table), as the reference's poison tests do
    (correctness_test.py:280-323).  layout "hd64" builds the head_dim 64
    packed cache of ragged_paged_attention_hd64 (K|V of a head in one row).
    """
    g = torch.Generator().manual_seed(seed)
    n = len(seq_lens)
    q_lens = [a for a, _ in seq_lens]
    kv_lens = [b for _, b in seq_lens]
    for ql, kl in seq_lens:
        assert 0 < ql <= kl, (ql, kl)
    max_num_seqs = max(max_num_seqs or n, n, 1)
    total_q = sum(q_lens)
    T = max(max_num_tokens or total_q, total_q, 1)
    pps = max(pages_per_seq or 0, max(cdiv(k, page_size) for k in kv_lens) if n else 1)
    used_pages = sum(cdiv(k, page_size) for k in kv_lens)
    if num_pages is None:
        num_pages = max(int(used_pages * pool_factor) + 1, used_pages + 1)
    assert num_pages >= used_pages

    def randn(*shape):
        return torch.randn(*shape, generator=g, dtype=torch.float32)

    q = randn(T, num_q_heads, head_dim).to(q_dtype)
    kv_is_fp8 = get_dtype_packing(kv_dtype) == 4
    kf, vf = randn(T, num_kv_heads, head_dim), randn(T, num_kv_heads, head_dim)
    if kv_is_fp8:
        k, v = quantize_kv(kv_dtype, kf, vf, k_scale or 1.0, v_scale or 1.0)
    else:
        k, v = kf.to(kv_dtype), vf.to(kv_dtype)

    hd64 = layout == "hd64"
    assert layout in ("v3", "hd64") and (not hd64 or head_dim == 64)
    if hd64:
        shape = get_kv_cache_shape_hd64(num_pages, page_size, num_kv_heads, head_dim, kv_dtype)
    else:
        shape = get_kv_cache_shape(num_pages, page_size, num_kv_heads, head_dim, kv_dtype)
    cache_f = randn(*shape)
    if kv_is_fp8 and hd64:
        # K halves of each row with k_scale, V halves with v_scale.
        half = torch.arange(128).view(1, 1, 1, 1, 128) >= 64
        scale = torch.where(half, torch.tensor(v_scale or 1.0), torch.tensor(k_scale or 1.0))
        info = torch.finfo(kv_dtype)
        kv_cache = torch.clamp(cache_f / scale, info.min, info.max).to(kv_dtype)
    elif kv_is_fp8:
        # K rows (even combined heads) with k_scale, V rows with v_scale.
        pack = shape[3]
        c = torch.arange(shape[2] * pack).view(shape[2], pack)
        scale = torch.where(c % 2 == 0, torch.tensor(k_scale or 1.0),
                            torch.tensor(v_scale or 1.0)).view(1, 1, shape[2], pack, 1)
        info = torch.finfo(kv_dtype)
        kv_cache = torch.clamp(cache_f / scale, info.min, info.max).to(kv_dtype)
    else:
        kv_cache = cache_f.to(kv_dtype)

    perm = torch.randperm(num_pages, generator=g).to(torch.int32)
    page_indices = torch.zeros(max_num_seqs * pps, dtype=torch.int32)
    off = 0
    for s, kl in enumerate(kv_lens):
        cnt = cdiv(kl, page_size)
        page_indices[s * pps:s * pps + cnt] = perm[off:off + cnt]
        off += cnt
    if nan_fill:
        used = torch.zeros(num_pages, dtype=torch.bool)
        if kv_cache.element_size() == 1:
            # fp8 tensors take no masked writes: write the NaN byte (0x7F in both
            # e4m3fn and e5m2) through a byte view.
            flat = kv_cache.view(torch.uint8).view(num_pages, page_size, -1)
            nan = 0x7F
        else:
            flat = kv_cache.view(num_pages, page_size, -1)
            nan = float("nan")
        for s, kl in enumerate(kv_lens):
            cnt = cdiv(kl, page_size)
            pages = page_indices[s * pps:s * pps + cnt].long()
            used[pages] = True
            tail = cnt * page_size - kl  # unused rows of the last page
            if tail:
                flat[pages[-1], page_size - tail:] = nan
            page_indices[s * pps + cnt:(s + 1) * pps] = -1
        flat[~used] = nan
        page_indices[n * pps:] = -1
    cu = torch.zeros(max_num_seqs + 1, dtype=torch.int32)
    cu[1:n + 1] = torch.cumsum(torch.tensor(q_lens, dtype=torch.int64), 0).to(torch.int32)
    cu[n + 1:] = cu[n]
    kvl = torch.zeros(max_num_seqs, dtype=torch.int32)
    kvl[:n] = torch.tensor(kv_lens, dtype=torch.int32)
    if distribution is None:
        distribution = [0, 0, n]
    dist = torch.tensor(distribution, dtype=torch.int32)
    kw = dict(sm_scale=head_dim ** -0.5)
    if k_scale is not None:
        kw["k_scale"] = float(k_scale)
    if v_scale is not None:
        kw["v_scale"] = float(v_scale)
    kw.update(kwargs)
    return Workload(name, q, k, v, kv_cache, kvl, page_indices, cu, dist, kw,
                    list(seq_lens))


def prefill_part(w: Workload) -> Workload:
    """The sequences of `w` with more than one query token, alone: the same
    cache, the same page-table rows, distribution [0, 0, n] (the prefill
    kernel's share of a mixed batch, timed by itself)."""
    S = w.kv_lens.shape[0]
    pps = w.page_indices.shape[0] // S
    n = w.num_seqs
    keep = [s for s in range(n) if int(w.cu_q_lens[s + 1]) - int(w.cu_q_lens[s]) > 1]
    m = len(keep)
    cu = torch.zeros(m + 1, dtype=torch.int32)
    kvl = torch.zeros(m, dtype=torch.int32)
    pages = torch.empty(m * pps, dtype=torch.int32)
    rows = []
    for i, s in enumerate(keep):
        c0, c1 = int(w.cu_q_lens[s]), int(w.cu_q_lens[s + 1])
        cu[i + 1] = cu[i] + (c1 - c0)
        kvl[i] = w.kv_lens[s]
        pages[i * pps:(i + 1) * pps] = w.page_indices[s * pps:(s + 1) * pps]
        rows.append(torch.arange(c0, c1))
    idx = torch.cat(rows) if rows else torch.zeros(0, dtype=torch.int64)
    return Workload(w.name + "-prefill", w.q[idx].contiguous(), w.k[idx].contiguous(),
                    w.v[idx].contiguous(), w.kv_cache, kvl, pages, cu,
                    torch.tensor([0, 0, m], dtype=torch.int32), dict(w.kwargs),
                    [w.seq_lens[s] for s in keep])


def _uniform_ints(g, lo, hi, n):
    return torch.randint(lo, hi + 1, (n,), generator=g).tolist()


def baseline_config(idx: int, seed: int | None = None) -> Workload:
    """The five configurations of BASELINE.json `configs`, 1-based."""
    seed = 1000 + idx if seed is None else seed
    g = torch.Generator().manual_seed(seed)
    if idx == 1:
        kvl = _uniform_ints(g, 64, 512, 4)
        return make_workload([(1, k) for k in kvl], 8, 2, 128, 16, seed=seed, num_pages=128,
                             pages_per_seq=32, distribution=[4, 4, 4], name="C1")
    if idx == 2:
        kvl = _uniform_ints(g, 512, 4096, 64)
        return make_workload([(1, k) for k in kvl], 32, 8, 128, 16, seed=seed,
                             num_pages=20000, pages_per_seq=256, distribution=[64, 64, 64],
                             name="C2")
    if idx == 3:
        dec = _uniform_ints(g, 1024, 8192, 120)
        ctx = _uniform_ints(g, 0, 4096, 8)
        seqs = [(1, k) for k in dec] + [(512, c + 512) for c in ctx]
        return make_workload(seqs, 64, 8, 128, 32, seed=seed, pages_per_seq=256,
                             distribution=[120, 120, 128], name="C3")
    if idx == 4:
        kvl = _uniform_ints(g, 16384, 32768, 16)
        ks = 0.5 + 1.5 * torch.rand((), generator=g).item()
        vs = 0.5 + 1.5 * torch.rand((), generator=g).item()
        return make_workload([(1, k) for k in kvl], 32, 8, 128, 64, seed=seed,
                             kv_dtype=torch.float8_e4m3fn, k_scale=ks, v_scale=vs,
                             pages_per_seq=512, distribution=[16, 16, 16], name="C4")
    if idx == 5:
        kvl = _uniform_ints(g, 2048, 16384, 32)
        seqs = [(1, k) for k in kvl[:16]] + [(256, k) for k in kvl[16:]]
        return make_workload(seqs, 16, 8, 256, 16, seed=seed, pages_per_seq=1024,
                             distribution=[16, 16, 32], sliding_window=4096, soft_cap=50.0,
                             name="C5")
    raise ValueError(idx)


# ---------------------------------------------------------------------------
# Algorithmic work of a call (what the benchmark's roofline divides by time).
# ---------------------------------------------------------------------------
def _attended_keys(kv_len, q_len, sliding_window):
    """Keys a sequence's rows read from HBM at least once: R_s."""
    if sliding_window is None:
        return kv_len
    return min(kv_len, q_len + sliding_window - 1)


def algorithmic_bytes(kv_lens, cu_q_lens, num_seqs, hq, hkv, d, dp, page_size,
                      q_bytes, kv_bytes, out_bytes, sliding_window=None, kv_write=True):
    """Algorithmic HBM bytes of one RPA call: KV read of R_s tokens per
    sequence (the new tokens, read from the k/v inputs, included once), the
    new-KV write into pages (unless kv_write is False, i.e. skip_kv_update),
    Q read, O write, page-table and metadata reads."""
    total = 0
    rec = 2 * hkv * dp * kv_bytes
    for s in range(num_seqs):
        q_len = int(cu_q_lens[s + 1]) - int(cu_q_lens[s])
        kv_len = int(kv_lens[s])
        total += _attended_keys(kv_len, q_len, sliding_window) * rec
        if kv_write:
            total += q_len * rec
        total += q_len * hq * d * (q_bytes + out_bytes)
        total += cdiv(kv_len, page_size) * 4
    total += (3 * num_seqs + 4) * 4
    return total


def decode_kernel_bytes(kv_lens, cu_q_lens, num_seqs, hq, hkv, d, dp, page_size, q_bytes,
                        kv_bytes, sliding_window=None):
    """Algorithmic HBM bytes of the decode kernel alone, attention only
    (skip_kv_update): the KV records of every decode sequence's key range,
    its q row and its page-table entries, plus the metadata.  Output rows are
    not counted (multi-unit sequences write theirs in the finish kernel)."""
    total = 0
    rec = 2 * hkv * dp * kv_bytes
    for s in range(num_seqs):
        q_len = int(cu_q_lens[s + 1]) - int(cu_q_lens[s])
        kv_len = int(kv_lens[s])
        if q_len != 1 or kv_len < 1:
            continue
        total += _attended_keys(kv_len, 1, sliding_window) * rec
        total += hq * d * q_bytes
        total += cdiv(kv_len, page_size) * 4
    total += (3 * num_seqs + 4) * 4
    return total


def algorithmic_flops(kv_lens, cu_q_lens, num_seqs, hq, d, sliding_window=None):
    """4 * D * Hq * (sum over q rows of attended keys): QK^T and PV."""
    tot = 0
    for s in range(num_seqs):
        q_len = int(cu_q_lens[s + 1]) - int(cu_q_lens[s])
        kv_len = int(kv_lens[s])
        for i in range(q_len):
            a = kv_len - q_len + i + 1
            if sliding_window is not None:
                a = min(a, sliding_window)
            tot += a
    return 4 * d * hq * tot


def prefill_flops(kv_lens, cu_q_lens, num_seqs, hq, d, sliding_window=None):
    """algorithmic_flops over the rows of sequences with q_len > 1."""
    tot = 0
    for s in range(num_seqs):
        q_len = int(cu_q_lens[s + 1]) - int(cu_q_lens[s])
        if q_len > 1:
            tot += algorithmic_flops([kv_lens[s]], [0, q_len], 1, hq, d, sliding_window)
    return tot
