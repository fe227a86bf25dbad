"""GPU parity of the fused RoPE + KV cache write (fdllm_rope_kv_write).

Bar: bit-exact. The kernel rounds to the 16-bit type after each product and after
the sum, which is what the eager expression q * cos + rotate_half(q) * sin of the
reference (utils/attention_backends.py:777-788) does, and cache writes are copies.
The oracle here is that torch expression itself, run on the same inputs.
"""
import pytest
import torch

from fast_v2_amd import ops
from fast_v2_amd.e2e import model as em
from fast_v2_amd.e2e import sampler as es
from fast_v2_amd.utils import attention_backends as ab

pytestmark = pytest.mark.gpu


def _rope_torch(x, cos, sin):
    cos, sin = cos.unsqueeze(2), sin.unsqueeze(2)
    h = x.shape[-1] // 2
    return x * cos + torch.cat((-x[..., h:], x[..., :h]), dim=-1) * sin


def _tables(S, D, start, dtype, gpu, theta=1e6):
    inv = 1.0 / (theta ** (torch.arange(0, D, 2, dtype=torch.float32, device=gpu) / D))
    pos = torch.arange(start, start + S, device=gpu).float()
    emb = torch.cat([pos[:, None] * inv[None]] * 2, dim=-1)
    return emb.cos().to(dtype)[None], emb.sin().to(dtype)[None]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("S,Hq,Hkv,D", [(32, 28, 4, 128), (8, 28, 4, 128), (5, 12, 2, 64), (16, 8, 8, 128)])
def test_rope_kv_write_bit_exact(gpu, dtype, S, Hq, Hkv, D):
    g = torch.Generator(device="cpu").manual_seed(S * 100 + Hq + D)
    B, L, LB = 3, 300, 32
    q = (torch.randn(B, S, Hq, D, generator=g) * 3).to(dtype).to(gpu)
    k = (torch.randn(B, S, Hkv, D, generator=g) * 3).to(dtype).to(gpu)
    v = torch.randn(B, S, Hkv, D, generator=g).to(dtype).to(gpu)
    cos, sin = _tables(S, D, 1234, dtype, gpu)
    ws = torch.tensor([0, 100, L - 3], dtype=torch.int32, device=gpu)  # the last one runs off the end
    off, boff = 2, 8 if S <= 8 else 0
    kc = torch.full((B, L, Hkv, D), 7.0, dtype=dtype, device=gpu)
    vc = kc.clone()
    kb = torch.full((B, LB, Hkv, D), -5.0, dtype=dtype, device=gpu)
    vb = kb.clone()
    print(f"case rope {dtype} S={S} {Hq}/{Hkv} D={D}", flush=True)
    q_rot, (k_rot, v_copy) = ops.rope_kv_write(q, k, v, cos, sin, kc, vc, write_start=ws, write_offset=off,
                                               k_block=kb, v_block=vb, block_offset=boff, kv_out=True)
    q_ref, k_ref = _rope_torch(q, cos, sin), _rope_torch(k, cos, sin)
    assert torch.equal(q_rot, q_ref)
    assert torch.equal(k_rot, k_ref) and torch.equal(v_copy, v)
    kc_ref = torch.full_like(kc, 7.0)
    vc_ref = kc_ref.clone()
    for b in range(B):
        p0 = int(ws[b]) + off
        n = max(0, min(S, L - p0))
        kc_ref[b, p0:p0 + n] = k_ref[b, :n]
        vc_ref[b, p0:p0 + n] = v[b, :n]
    assert torch.equal(kc, kc_ref) and torch.equal(vc, vc_ref)
    kb_ref = torch.full_like(kb, -5.0)
    vb_ref = kb_ref.clone()
    nb = min(S, LB - boff)
    kb_ref[:, boff:boff + nb] = k_ref[:, :nb]
    vb_ref[:, boff:boff + nb] = v[:, :nb]
    assert torch.equal(kb, kb_ref) and torch.equal(vb, vb_ref)


def test_rope_in_place_and_broadcast_tables(gpu):
    """q_out aliasing q, per-sequence cos/sin tables, no cache destinations."""
    g = torch.Generator(device="cpu").manual_seed(5)
    B, S, Hq, Hkv, D = 2, 8, 28, 4, 128
    q = torch.randn(B, S, Hq, D, generator=g).to(torch.bfloat16).to(gpu)
    k = torch.randn(B, S, Hkv, D, generator=g).to(torch.bfloat16).to(gpu)
    v = torch.randn(B, S, Hkv, D, generator=g).to(torch.bfloat16).to(gpu)
    c0, s0 = _tables(S, D, 10, torch.bfloat16, gpu)
    c1, s1 = _tables(S, D, 900, torch.bfloat16, gpu)
    cos, sin = torch.cat([c0, c1]), torch.cat([s0, s1])
    ref = _rope_torch(q, cos, sin)
    out = ops.rope_kv_write(q, k, v, cos, sin, q_out=q)
    assert out.data_ptr() == q.data_ptr() and torch.equal(q, ref)


@pytest.mark.parametrize("use_block_cache", [True, False])
def test_fused_forward_equals_unfused(gpu, use_block_cache):
    """The patched attention forward with the fused kernel and with torch RoPE + separate
    cache writes (the reference's statement) give identical generations and caches."""
    cfg = em.BlockDiffusionConfig(num_hidden_layers=2)
    model = em.build_model(cfg, gpu)
    x = torch.randint(0, cfg.vocab_size - 1, (4, 64), generator=torch.Generator().manual_seed(4)).to(gpu)
    outs = []
    for fused in (True, False):
        ab.FUSED_ROPE_CACHE_WRITE = fused
        try:
            out, st = es.generate(model, x, max_new_tokens=96, use_block_cache=use_block_cache,
                                  impl=es.HipStaticAttention(graphs=False))
        finally:
            ab.FUSED_ROPE_CACHE_WRITE = True
        outs.append(out)
    assert torch.equal(outs[0], outs[1])
