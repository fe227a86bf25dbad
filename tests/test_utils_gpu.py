"""GPU parity of the drop-in cache objects and the hip attention backend.

Cache writes are compared bit for bit with the reference semantics restated on
the CPU with torch indexing (static_kv_cache.py:132-160, :218-247;
block_sparse_cache.py:112-132; dynamic_block_kv.py:39-43, whose CPU test
tests/test_dkv.py:56-71 checks that unselected rows stay untouched). Attention
goes through AttentionBackend('hip') and is checked against the float64 oracle
at atol = rtol = 1e-2.
"""
import numpy as np
import pytest
import torch

from fast_v2_amd.utils import attention_backends as ab
from fast_v2_amd.utils import BlockSparseCache, DynamicBlockKV, StaticBlockCache, StaticKVCache
from oracle import attention as oa

pytestmark = pytest.mark.gpu

ATOL = RTOL = 1e-2


@pytest.fixture(scope="module")
def hip_backend(gpu):
    ab.get_attention_backend.cache_clear()
    be = ab.get_attention_backend("auto")
    assert be.name == "hip", "auto must select the HIP backend on gfx950"
    return be


def test_static_kv_cache_update_advances_after_last_layer(gpu):
    L, B, S, H, D = 3, 2, 96, 4, 128
    c = StaticKVCache(B, S, L, H, D, torch.bfloat16, gpu)
    g = torch.Generator().manual_seed(0)
    exp_k = torch.zeros(L, B, S, H, D, dtype=torch.bfloat16)
    exp_v = torch.zeros_like(exp_k)
    pos = 0
    for n in (40, 32, 8):
        for layer in range(L):
            k = torch.randn(B, n, H, D, generator=g).to(torch.bfloat16)
            v = torch.randn(B, n, H, D, generator=g).to(torch.bfloat16)
            ret_k, _ = c.update(k.to(gpu), v.to(gpu), layer)
            assert ret_k.shape == (B, pos + n, H, D)
            exp_k[layer, :, pos:pos + n] = k
            exp_v[layer, :, pos:pos + n] = v
            # the pointer moves only after the last layer
            assert c.get_seq_length() == (pos + n if layer == L - 1 else pos)
        pos += n
        assert c.cache_seqlens.tolist() == [pos] * B
    for layer in range(L):
        assert torch.equal(c.key_cache[layer].cpu(), exp_k[layer])
        assert torch.equal(c.value_cache[layer].cpu(), exp_v[layer])


def test_static_kv_cache_scratch_and_sparse_writes(gpu):
    L, B, S, H, D = 2, 3, 128, 4, 128
    c = StaticKVCache(B, S, L, H, D, torch.bfloat16, gpu)
    g = torch.Generator().manual_seed(1)
    before = [k.clone().cpu() for k in c.key_cache]
    c.set_kv_write_start(64)
    c.prepare_write_idx(32)
    k = torch.randn(B, 32, H, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, 32, H, D, generator=g).to(torch.bfloat16)
    c.write_scratch_compiled(k.to(gpu), v.to(gpu), 1)
    exp = before[1].clone()
    exp[:, 64:96] = k
    assert torch.equal(c.key_cache[1].cpu(), exp)
    assert torch.equal(c.key_cache[0].cpu(), before[0])  # other layers untouched
    assert c.get_seq_length() == 0  # scratch writes never advance the pointer
    # sparse: per-token positions
    posn = torch.stack([torch.randperm(S, generator=g)[:5] for _ in range(B)])
    k2 = torch.randn(B, 5, H, D, generator=g).to(torch.bfloat16)
    c.write_sparse(k2.to(gpu), k2.to(gpu), 1, posn.to(gpu))
    for b in range(B):
        exp[b, posn[b]] = k2[b]
    assert torch.equal(c.key_cache[1].cpu(), exp)
    assert torch.equal(c.value_cache[1].cpu()[:, posn[0]][0], k2[0])


def test_static_block_cache(gpu):
    bc = StaticBlockCache(2, 32, 2, 4, 128, torch.bfloat16, gpu)
    g = torch.Generator().manual_seed(2)
    full = torch.randn(2, 32, 4, 128, generator=g).to(torch.bfloat16)
    k, v = bc.update(full.to(gpu), full.to(gpu), 1)
    assert len(bc) == 2 and torch.equal(k.cpu(), full)
    sub = torch.randn(2, 8, 4, 128, generator=g).to(torch.bfloat16)
    bc.write(sub.to(gpu), sub.to(gpu), 1, 16)
    exp = full.clone()
    exp[:, 16:24] = sub
    assert torch.equal(bc[1][0].cpu(), exp) and torch.equal(bc[1][1].cpu(), exp)


def test_block_sparse_cache_scatter(gpu):
    L, B, blk, Hd = 2, 3, 32, 3584
    sc = BlockSparseCache(L, B, blk, Hd, torch.bfloat16, gpu)
    g = torch.Generator().manual_seed(3)
    base = torch.randn(B, blk, Hd, generator=g).to(torch.bfloat16)
    sc.cache_attn_output(1, base.to(gpu))
    sc.cache_mlp_output(0, base.to(gpu))
    idx = torch.stack([torch.randperm(blk, generator=g)[:7] for _ in range(B)])
    vals = torch.randn(B, 7, Hd, generator=g).to(torch.bfloat16)
    sc.scatter_attn_output(1, idx.to(gpu), vals.to(gpu))
    sc.scatter_mlp_output(0, idx.to(gpu), vals.to(gpu))
    exp = base.clone()
    exp.scatter_(1, idx.unsqueeze(-1).expand(-1, -1, Hd), vals)
    assert torch.equal(sc.get_attn_output(1).cpu(), exp)
    assert torch.equal(sc.get_mlp_output(0).cpu(), exp)
    assert not sc.get_attn_output(0).any()


def test_dynamic_block_kv_scatter_leaves_other_rows(gpu):
    dk = DynamicBlockKV(1, 3, 2, 4, 32, 128, torch.bfloat16, gpu)
    g = torch.Generator().manual_seed(4)
    full = torch.randn(2, 4, 32, 128, generator=g).to(torch.bfloat16)
    dk.write_full(2, full.to(gpu), full.to(gpu))
    idx = torch.tensor([[1, 5, 30], [0, 2, 31]])
    new = torch.randn(2, 4, 3, 128, generator=g).to(torch.bfloat16)
    dk.write(2, new.to(gpu), (-new).to(gpu), idx.to(gpu))
    exp = full.clone()
    exp.scatter_(2, idx[:, None, :, None].expand(-1, 4, -1, 128), new)
    k, v = dk.get(2)
    assert torch.equal(k.cpu(), exp)
    exp_v = full.clone()
    exp_v.scatter_(2, idx[:, None, :, None].expand(-1, 4, -1, 128), -new)
    assert torch.equal(v.cpu(), exp_v)


def test_hip_backend_flash_kvcache(gpu, hip_backend):
    g = torch.Generator().manual_seed(5)
    B, Sq, Hq, Hkv, D, S = 4, 8, 28, 4, 128, 700
    q = torch.randn(B, Sq, Hq, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, S, Hkv, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, S, Hkv, D, generator=g).to(torch.bfloat16)
    sl = torch.tensor([700, 33, 512, 64], dtype=torch.int32)
    out = hip_backend.flash_kvcache_attention(q.to(gpu), k.to(gpu), v.to(gpu), sl.to(gpu))
    assert out.shape == q.shape and out.dtype == q.dtype
    exp = oa.attention_np(q.float(), k.float(), v.float(), sl)
    np.testing.assert_allclose(out.float().cpu().numpy(), exp, atol=ATOL, rtol=RTOL)
    # the SDPA shim (the reference's own CPU statement) agrees too
    shim = oa.sdpa_kvcache(q.float(), k.float(), v.float(), sl)
    np.testing.assert_allclose(out.float().cpu().numpy(), shim.numpy(), atol=ATOL, rtol=RTOL)
    # causal=True: flash_attn_with_kvcache's bottom-right alignment
    outc = hip_backend.flash_kvcache_attention(q.to(gpu), k.to(gpu), v.to(gpu), sl.to(gpu), is_causal=True)
    expc = oa.attention_np(q.float(), k.float(), v.float(), sl, mask_mode=oa.MASK_CAUSAL)
    np.testing.assert_allclose(outc.float().cpu().numpy(), expc, atol=ATOL, rtol=RTOL)


@pytest.mark.parametrize("causal", [False, True])
def test_hip_backend_bhsd_attention(gpu, hip_backend, causal):
    g = torch.Generator().manual_seed(6)
    B, Hq, Hkv, S, D = 2, 12, 2, 200, 128
    q = torch.randn(B, Hq, S, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, Hkv, S, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, Hkv, S, D, generator=g).to(torch.bfloat16)
    out = hip_backend.attention(q.to(gpu), k.to(gpu), v.to(gpu), is_causal=causal)
    assert out.shape == (B, Hq, S, D)
    exp = oa.attention_np(q.transpose(1, 2).float(), k.transpose(1, 2).float(), v.transpose(1, 2).float(),
                          [S, S], mask_mode=oa.MASK_CAUSAL if causal else oa.MASK_SEQLEN)
    np.testing.assert_allclose(out.transpose(1, 2).float().cpu().numpy(), exp, atol=ATOL, rtol=RTOL)
    with pytest.raises(RuntimeError, match="attn_mask"):
        hip_backend.attention(q.to(gpu), k.to(gpu), v.to(gpu), attn_mask=torch.zeros(S, S, device=gpu))
