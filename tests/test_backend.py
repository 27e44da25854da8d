"""Attention-backend glue (vllm-torchtpu_amd/backend.py) on the CPU, in the
style of the reference's glue tests (tests/layers/adapter/
test_attention_head_padding.py:109-176: the kernel replaced by a fake that
records what it receives).  The GPU end-to-end checks are in
test_backend_gpu.py."""

import math
from types import SimpleNamespace

import pytest
import torch

from vllm_torchtpu_amd import backend as B

BF16, E4M3, E5M2 = torch.bfloat16, torch.float8_e4m3fn, torch.float8_e5m2


def test_kv_cache_shape_and_page_bytes():
    BE = B.RpaAttentionBackend
    # "auto" is vLLM's offloading probe: num_blocks at dim 0, packing 1.
    assert BE.get_kv_cache_shape(10, 16, 8, 128) == (10, 16, 16, 1, 128)
    assert BE.get_kv_cache_shape(10, 16, 8, 128, "bfloat16") == (10, 16, 8, 2, 128)
    assert BE.get_kv_cache_shape(10, 16, 8, 128, "fp8") == (10, 16, 4, 4, 128)
    assert BE.get_kv_cache_shape(10, 16, 8, 128, E5M2) == (10, 16, 4, 4, 128)
    assert BE.get_kv_cache_shape(3, 32, 3, 80, BF16) == (3, 32, 3, 2, 128)
    assert BE.get_kv_cache_shape(3, 32, 1, 256, "fp8_e4m3") == (3, 32, 1, 4, 256)
    # head_size 64: K|V packed along one 128-wide row (Kx2 = num_kv_heads).
    assert BE.get_kv_cache_shape(10, 16, 8, 64) == (10, 16, 8, 1, 128)
    assert BE.get_kv_cache_shape(10, 16, 8, 64, BF16) == (10, 16, 4, 2, 128)
    assert BE.get_kv_cache_shape(10, 16, 3, 64, "fp8") == (10, 16, 1, 4, 128)
    assert BE.get_kv_cache_page_size_bytes(16, 8, 64, BF16) == 16 * 8 * 128 * 2
    # one page = block_size records of Kx2 * Dp elements
    assert BE.get_kv_cache_page_size_bytes(16, 8, 128, BF16) == 16 * 16 * 128 * 2
    assert BE.get_kv_cache_page_size_bytes(16, 8, 128, "fp8") == 16 * 16 * 128
    with pytest.raises(ValueError):
        BE.get_kv_cache_page_size_bytes(16, 8, 128, "auto")
    with pytest.raises(ValueError):
        B.resolve_kv_cache_dtype("int4")
    assert BE.get_kv_cache_stride_order() == (0, 1, 2, 3, 4)
    assert BE.get_kv_cache_stride_order(True) == (1, 0, 2, 3, 4, 5)
    assert BE.get_name() == "FLASH_ATTN" and BE.get_impl_cls() is B.RpaAttentionBackendImpl


@pytest.mark.parametrize("max_model_len,expect", [(1024, 64), (2048, 128), (8192, 256),
                                                  (8193, 128), (200, 16), (32768, 128),
                                                  (4000, 256), (3000, 256), (1000, 64)])
def test_page_size_policy(max_model_len, expect):
    # attention.py:733-758 in closed form: >8192 -> 128, else
    # clamp(next_pow2(len) / 16, 16, 256).
    assert B.RpaAttentionBackend.get_page_size(max_model_len) == expect


def test_head_padding_rule():
    assert B.kv_page_head_padding((4, 2, 128), (4, 2, 128), 128, 64) == 0
    assert B.kv_page_head_padding((4, 2, 256), (4, 2, 128), 256, 128) == 128
    assert B.kv_page_head_padding((2, 2, 128), (4, 2, 128), 128, 128) == 0


def test_impl_validation():
    mk = dict(num_heads=4, head_size=128, scale=1.0, num_kv_heads=2, sliding_window=None,
              kv_cache_dtype="auto")
    with pytest.raises(NotImplementedError):
        B.RpaAttentionBackendImpl(alibi_slopes=[1.0], **mk)
    with pytest.raises(NotImplementedError):
        B.RpaAttentionBackendImpl(alibi_slopes=None, attn_type="encoder", **mk)
    impl = B.RpaAttentionBackendImpl(alibi_slopes=None, **dict(mk, kv_cache_dtype="fp8_e5m2"))
    assert impl.kv_cache_quantized_dtype == E5M2


def _run(head_size, pool_heads, pool_head_size, *, kv_cache_dtype="bf16", two_d=True,
         shared=False, scales=(1.0, 1.0), out_buf=False):
    num_heads, num_kv_heads, q_len = 4, 4, 3
    impl = B.RpaAttentionBackendImpl(
        num_heads=num_heads, head_size=head_size, scale=0.5, num_kv_heads=num_kv_heads,
        alibi_slopes=None, sliding_window=7, kv_cache_dtype=kv_cache_dtype,
        logits_soft_cap=20.0, kv_sharing_target_layer_name="l0" if shared else None)
    cache_dt = impl.kv_cache_quantized_dtype or BF16
    kv_cache = torch.zeros(B.RpaAttentionBackend.get_kv_cache_shape(
        2, 16, pool_heads, pool_head_size, cache_dt), dtype=cache_dt)
    shape_q = (q_len, num_heads * head_size) if two_d else (q_len, num_heads, head_size)
    query = torch.randn(shape_q).to(BF16)
    key = torch.randn(q_len, num_kv_heads * head_size).to(BF16)
    seen = {}

    def fake_kernel(kv, q, k, v, seq_lens, block_tables, qsl, dist, sink, out=None):
        seen.update(q=q, k=k, v=v, sink=sink, direct=out is not None)
        if out is not None:  # the kernel writes the caller's buffer
            assert out.shape == q.shape and out.dtype == q.dtype
            out.fill_(2)
            return out
        return torch.ones_like(q) * 2
    built = {}

    def fake_build(q_scale, k_scale, v_scale, skip_kv_update=False):
        built.update(q_scale=q_scale, k_scale=k_scale, v_scale=v_scale, skip=skip_kv_update)
        return fake_kernel
    impl._build_rpa_kernel = fake_build
    md = B.AttentionMetadata(
        input_positions=torch.arange(q_len, dtype=torch.int32),
        block_tables=torch.zeros(1, dtype=torch.int32),
        seq_lens=torch.tensor([q_len], dtype=torch.int32),
        query_start_loc=torch.tensor([0, q_len], dtype=torch.int32),
        request_distribution=torch.tensor([0, 0, 1], dtype=torch.int32))
    layer = SimpleNamespace(_k_scale_float=scales[0], _v_scale_float=scales[1])
    output = torch.zeros(shape_q, dtype=BF16) if out_buf else None
    out = impl.forward(layer, query, None if shared else key, None if shared else key.clone(),
                       kv_cache, md, output=output)
    return out, output, seen, built, query


def test_forward_query_width_and_layout():
    # A layer on its own page gets no padding.
    for hs, ph, phs in ((128, 4, 128), (64, 4, 64)):
        out, _, seen, _, q = _run(hs, ph, phs)
        assert seen["q"].shape[-1] == hs and out.shape == q.shape
    # A head_dim 64 layer on a head_dim 128 pool page (a wider spec's) is
    # padded to 128 and goes to the v3 layout (attention.py:215-247).
    out, _, seen, _, q = _run(64, 4, 128)
    assert seen["q"].shape[-1] == 128 and out.shape == q.shape
    # A 128-wide layer on a 256-wide pool is padded to 256, then sliced back.
    out, _, seen, _, q = _run(128, 4, 256)
    assert seen["q"].shape == (3, 4, 256) and out.shape == q.shape
    assert torch.equal(seen["q"][..., 128:], torch.zeros_like(seen["q"][..., 128:]))
    # 3-D in, 3-D out; the output buffer is written in place, by the kernel
    # itself (no temporary and copy) when no head padding is involved.
    out, buf, seen, _, q = _run(128, 4, 128, two_d=False, out_buf=True)
    assert out.shape == q.shape and torch.equal(buf, out) and seen["direct"]
    assert out.data_ptr() == buf.data_ptr()
    out, buf, seen, _, q = _run(128, 4, 128, two_d=True, out_buf=True)
    assert out.data_ptr() == buf.data_ptr() and seen["direct"] and torch.equal(buf, out)
    # A padded pool page: the kernel writes a temporary, then the slice is copied.
    out, buf, seen, _, q = _run(128, 4, 256, two_d=True, out_buf=True)
    assert not seen["direct"] and torch.equal(buf, out)


def test_forward_quantize_on_write():
    out, _, seen, built, _ = _run(128, 4, 128, kv_cache_dtype="fp8", scales=(0.5, 2.0))
    assert seen["k"].dtype == E4M3 and seen["v"].dtype == E4M3
    assert built == dict(q_scale=None, k_scale=0.5, v_scale=2.0, skip=False)
    with pytest.raises(ValueError):
        _run(128, 4, 128, kv_cache_dtype="fp8", scales=(0.0, 1.0))


def test_forward_kv_shared_layer():
    _, _, seen, built, _ = _run(128, 4, 128, shared=True)
    assert built["skip"] is True
    assert bool((seen["k"] == 0).all())


def test_forward_profiling_call():
    impl = B.RpaAttentionBackendImpl(num_heads=2, head_size=128, scale=1.0, num_kv_heads=1,
                                     alibi_slopes=None, sliding_window=None,
                                     kv_cache_dtype="auto")
    q = torch.randn(5, 256)
    out = impl.forward(None, q, q[:, :128], q[:, :128], torch.empty(0), None)
    assert torch.equal(out, torch.ones_like(q))


def test_kernel_registry_caches_per_config():
    impl = B.RpaAttentionBackendImpl(num_heads=2, head_size=128, scale=1.0, num_kv_heads=1,
                                     alibi_slopes=None, sliding_window=None,
                                     kv_cache_dtype="auto")
    a = impl._build_rpa_kernel(None, None, None)
    assert impl._build_rpa_kernel(None, None, None) is a
    assert impl._build_rpa_kernel(None, 0.5, 2.0) is not a
    assert impl._build_rpa_kernel(None, None, None, skip_kv_update=True) is not a


def test_sinks_routing():
    """Sinks are kept (as f32 after loading) and only the head_dim 64 kernel
    takes them (attention_interface.py:418-436)."""
    sinks = torch.randn(4).to(BF16)
    impl = B.RpaAttentionBackendImpl(num_heads=4, head_size=128, scale=1.0, num_kv_heads=2,
                                     alibi_slopes=None, sliding_window=None,
                                     kv_cache_dtype="auto", sinks=sinks)
    impl.process_weights_after_loading(BF16)
    assert impl.sinks.dtype == torch.float32 and torch.equal(impl.sinks, sinks.float())
    with pytest.raises(AssertionError):
        B.RpaAttentionBackendImpl(num_heads=4, head_size=128, scale=1.0, num_kv_heads=2,
                                  alibi_slopes=None, sliding_window=None,
                                  kv_cache_dtype="auto", sinks=torch.zeros(3))
    kernel = impl._build_rpa_kernel(None, None, None)
    q = torch.zeros(2, 4, 128, dtype=BF16)
    with pytest.raises(NotImplementedError, match="head_dim==64"):
        kernel(None, q, q[:, :2], q[:, :2], None, torch.zeros(1, dtype=torch.int32), None,
               None, impl.sinks)


def test_workspace_is_never_freed_and_not_grown_in_capture(monkeypatch):
    """A captured graph keeps the workspace pointer of its calls: a larger
    workspace replaces the old one for later calls but the old one stays
    alive, and growing during a capture raises (rpa.py _workspace)."""
    from vllm_torchtpu_amd import rpa

    dev = torch.device("cpu")
    monkeypatch.setattr(rpa, "_WORKSPACES", {})
    monkeypatch.setattr(rpa, "_RETIRED", [])
    a = rpa._workspace(dev, 100)
    assert rpa._workspace(dev, 50) is a
    b = rpa._workspace(dev, 1000)
    assert b is not a and b.numel() >= 1000 and any(x is a for x in rpa._RETIRED)
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: True)
    cuda_dev = torch.device("cuda", 0)
    monkeypatch.setitem(rpa._WORKSPACES, rpa._ws_key(cuda_dev), b)
    assert rpa._workspace(cuda_dev, 1000) is b        # no growth: fine under capture
    with pytest.raises(RuntimeError, match="graph capture"):
        rpa._workspace(cuda_dev, 10 ** 6)

