"""Attention backend (vllm-torchtpu_amd/backend.py) end to end on the GPU:
RpaAttentionBackendImpl.forward against the CPU oracle, bf16 and with fp8
quantize-on-write (attention.py:1560-1569), in vLLM's 2-D layout, and for a
KV-shared layer (no key/value: the cache is read as it is)."""

from types import SimpleNamespace

import pytest
import torch

from oracle import rpa_oracle as O
from rpa_testlib import assert_close, bytes_equal

import vllm_torchtpu_amd.workloads as W
from vllm_torchtpu_amd import backend as B
from vllm_torchtpu_amd.quantization import quantize_kv

pytestmark = pytest.mark.gpu

SEQS = [(1, 700), (37, 300), (1, 33), (64, 64)]


def _metadata(g):
    return B.AttentionMetadata(input_positions=None, block_tables=g.page_indices,
                               seq_lens=g.kv_lens, query_start_loc=g.cu_q_lens,
                               request_distribution=g.distribution)


@pytest.mark.parametrize("kv_dtype", ["auto", "fp8"])
def test_backend_forward(gpu_device, kv_dtype):
    hq, hkv, d = 32, 8, 128
    fp8 = kv_dtype == "fp8"
    ks, vs = (0.8, 1.6) if fp8 else (1.0, 1.0)
    w = W.make_workload(SEQS, hq, hkv, d, 16, seed=61, name="backend",
                        kv_dtype=torch.float8_e4m3fn if fp8 else torch.bfloat16,
                        k_scale=ks if fp8 else None, v_scale=vs if fp8 else None,
                        sliding_window=256, soft_cap=40.0)
    # The layer's bf16 K/V; the backend quantizes them on write.
    g_ = torch.Generator().manual_seed(62)
    k_bf = torch.randn(w.k.shape, generator=g_).to(torch.bfloat16)
    v_bf = torch.randn(w.v.shape, generator=g_).to(torch.bfloat16)
    k_in, v_in = (quantize_kv(torch.float8_e4m3fn, k_bf, v_bf, ks, vs) if fp8 else (k_bf, v_bf))
    kw = dict(w.kwargs)
    exp_out, exp_cache = O.ref_ragged_paged_attention(
        w.q, k_in, v_in, w.kv_cache, w.kv_lens, w.page_indices, w.cu_q_lens, w.distribution,
        mode="fp32", **kw)
    impl = B.RpaAttentionBackendImpl(num_heads=hq, head_size=d, scale=kw["sm_scale"],
                                     num_kv_heads=hkv, alibi_slopes=None, sliding_window=256,
                                     kv_cache_dtype=kv_dtype, logits_soft_cap=40.0)
    g = w.to(gpu_device)
    T = w.q.shape[0]
    out_buf = torch.zeros(T, hq * d, dtype=torch.bfloat16, device=gpu_device)
    layer = SimpleNamespace(_k_scale_float=ks, _v_scale_float=vs)
    out = impl.forward(layer, g.q.reshape(T, hq * d), k_bf.reshape(T, -1).to(gpu_device),
                       v_bf.reshape(T, -1).to(gpu_device), g.kv_cache, _metadata(g),
                       output=out_buf)
    torch.cuda.synchronize()
    n = w.num_tokens
    tol = 5e-2 if fp8 else 2e-2
    assert out.shape == (T, hq * d) and torch.equal(out, out_buf)
    assert_close(out[:n].reshape(n, hq, d).cpu(), exp_out, tol, tol, "backend output")
    assert bytes_equal(g.kv_cache.cpu(), exp_cache), "cache write differs"


def test_backend_kv_shared_layer(gpu_device):
    hq, hkv, d = 16, 4, 128
    w = W.make_workload(SEQS, hq, hkv, d, 16, seed=63, name="shared")
    kw = dict(w.kwargs)
    exp_out, _ = O.ref_ragged_paged_attention(*w.args(), mode="fp32", skip_kv_update=True, **kw)
    impl = B.RpaAttentionBackendImpl(num_heads=hq, head_size=d, scale=kw["sm_scale"],
                                     num_kv_heads=hkv, alibi_slopes=None, sliding_window=None,
                                     kv_cache_dtype="auto", kv_sharing_target_layer_name="l0")
    g = w.to(gpu_device)
    before = g.kv_cache.clone()
    out = impl.forward(None, g.q, None, None, g.kv_cache, _metadata(g))
    torch.cuda.synchronize()
    n = w.num_tokens
    assert_close(out[:n].cpu(), exp_out, 2e-2, 2e-2, "shared-layer output")
    assert torch.equal(g.kv_cache, before), "a KV-shared layer must not write the cache"
