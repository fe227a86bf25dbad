"""fdllm_kv_attn_fwd_noalloc: the allocation-free variant of fdllm_kv_attn_fwd.

Called through the C ABI (ctypes) on the same descriptors as fdllm_kv_attn_fwd with
a caller workspace; the two share their kernels, so the outputs must be identical.
Two calls in a row, the second on a smaller input, so the second call runs on the
scratch the first one left behind (its counters must have been reset).
"""
import ctypes

import pytest
import torch

from fast_v2_amd import _ffi, ops, workloads
from oracle import attention as oa

pytestmark = pytest.mark.gpu


def _desc(q, kp, vp, sl, scale, pt, page_size, out):
    d = ops._attn_desc(q, kp, vp, sl, out, scale, _ffi.MASK_SEQLEN, 32, None, pt, page_size, 0)
    return d


def _with_workspace(gpu, q, kp, vp, sl, scale, pt, page_size):
    out = torch.empty_like(q)
    d = _desc(q, kp, vp, sl, scale, pt, page_size, out)
    need = ctypes.c_size_t(0)
    _ffi.check(_ffi.lib().fdllm_kv_attn_workspace_size(ctypes.byref(d), ctypes.byref(need)),
               "fdllm_kv_attn_workspace_size")
    ws = torch.zeros(max(int(need.value), 1), dtype=torch.uint8, device=gpu)
    _ffi.check(_ffi.lib().fdllm_kv_attn_fwd(ctypes.byref(d), ws.data_ptr(), int(need.value),
                                            _ffi.stream_ptr(gpu)), "fdllm_kv_attn_fwd")
    torch.cuda.synchronize(gpu)
    return out, int(need.value)


def _no_alloc(gpu, q, kp, vp, sl, scale, pt, page_size):
    out = torch.empty_like(q)
    d = _desc(q, kp, vp, sl, scale, pt, page_size, out)
    rc = _ffi.lib().fdllm_kv_attn_fwd_noalloc(ctypes.byref(d), _ffi.stream_ptr(gpu))
    _ffi.check(rc, "fdllm_kv_attn_fwd_noalloc")
    torch.cuda.synchronize(gpu)
    return out


@pytest.mark.parametrize("active", [8, 32])
def test_noalloc_matches_workspace_entry_point(gpu, active):
    """Sub-block (8 active queries: split decode kernel, merge in the last workgroup)
    and full-block (32: split prefill kernel + merge kernel) calls at 7B geometry,
    batch 16, then a smaller batch on the same scratch."""
    cases = [workloads.kv_decode_paged(seed=20, batch=16, active=active),
             workloads.kv_decode_paged(seed=21, batch=5, active=active, min_prefix=300, max_prefix=2500)]
    for i, wl in enumerate(cases):
        print(f"case noalloc active={active} call {i} B={wl.q.shape[0]}", flush=True)
        args = (wl.q.to(gpu), wl.k_pool.to(gpu), wl.v_pool.to(gpu), wl.seqlens.to(gpu), wl.scale,
                wl.page_table.to(gpu), wl.page_size)
        ref, need = _with_workspace(gpu, *args)
        assert 0 < need <= _ffi.KV_ATTN_SCRATCH_BYTES
        got = _no_alloc(gpu, *args)
        assert torch.equal(got, ref), f"call {i}: noalloc output differs from fdllm_kv_attn_fwd"
        exp = oa.attention_np(wl.q.float(), wl.k_pool.float(), wl.v_pool.float(), wl.seqlens, wl.scale,
                              page_table=wl.page_table, page_size=wl.page_size)
        torch.testing.assert_close(got.float().cpu(), torch.from_numpy(exp).float(), atol=1e-2, rtol=1e-2)


def test_noalloc_fp32_key_splits(gpu):
    """fp32 calls: the fp32 kernel with its keys split over workgroups, each row block
    merged by its last split to arrive through the arrival counters at the head of the
    scratch (the 12 / 2-head block of 32 queries over 544 keys, five splits), then 300 keys
    on the same scratch; bit-exact against the workspace entry point, within 1e-5 of the
    float64 oracle."""
    wl = workloads.kv_decode_fp32_small(seed=0)
    g = torch.Generator().manual_seed(22)
    small = (torch.randn(1, 32, 12, 128, generator=g), torch.randn(1, 300, 2, 128, generator=g),
             torch.randn(1, 300, 2, 128, generator=g), torch.tensor([300], dtype=torch.int32))
    for i, (q, k, v, sl) in enumerate([(wl.q, wl.k_cache, wl.v_cache, wl.seqlens), small]):
        print(f"case noalloc fp32 call {i} keys={int(sl[0])}", flush=True)
        args = (q.to(gpu), k.to(gpu), v.to(gpu), sl.to(gpu), 128 ** -0.5, None, 0)
        ref, need = _with_workspace(gpu, *args)
        assert 0 < need <= _ffi.KV_ATTN_SCRATCH_BYTES
        got = _no_alloc(gpu, *args)
        assert torch.equal(got, ref), f"call {i}: noalloc output differs from fdllm_kv_attn_fwd"
        exp = oa.attention_np(q.float(), k.float(), v.float(), sl, 128 ** -0.5)
        torch.testing.assert_close(got.cpu(), torch.from_numpy(exp).float(), atol=1e-5, rtol=1e-5)


def test_noalloc_rejects_calls_beyond_the_scratch(gpu):
    """A call that needs more workspace than the scratch holds is refused before any
    launch, with FDLLM_ERR_WORKSPACE and a message naming the limit."""
    B, Hq, Hkv, D = 64, 32, 8, 128
    q = torch.zeros(B, 32, Hq, D, dtype=torch.bfloat16, device=gpu)  # 128 rows per KV head
    kc = torch.zeros(B, 16, Hkv, D, dtype=torch.bfloat16, device=gpu)
    sl = torch.full((B,), 16, dtype=torch.int32, device=gpu)
    out = torch.empty_like(q)
    d = ops._attn_desc(q, kc, kc, sl, out, D ** -0.5, _ffi.MASK_SEQLEN, 32, None, None, 0, 0)
    d.max_seqlen = 160 * 64 * 8  # sizes the split plan for long sequences: many slots
    need = ctypes.c_size_t(0)
    _ffi.check(_ffi.lib().fdllm_kv_attn_workspace_size(ctypes.byref(d), ctypes.byref(need)), "size")
    assert need.value > _ffi.KV_ATTN_SCRATCH_BYTES
    rc = _ffi.lib().fdllm_kv_attn_fwd_noalloc(ctypes.byref(d), _ffi.stream_ptr(gpu))
    assert rc == _ffi.FDLLM_ERR_WORKSPACE
    assert b"maximum" in _ffi.lib().fdllm_last_error()
