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
    saved = ab.FUSED_QKV_PROJECTION
    ab.FUSED_QKV_PROJECTION = False  # projections by nn.Linear on both sides: RoPE + writes compared alone
    try:
        for fused in (True, False):
            ab.FUSED_ROPE_CACHE_WRITE = fused
            try:
                out, st = es.generate(model, x, max_new_tokens=96, use_block_cache=use_block_cache,
                                      impl=es.HipStaticAttention(graphs=False))
            finally:
                ab.FUSED_ROPE_CACHE_WRITE = True
            outs.append(out)
    finally:
        ab.FUSED_QKV_PROJECTION = saved
    assert torch.equal(outs[0], outs[1])


# ---------------------------------------------------------------------------
# q / k / v projections fused with RoPE + cache write (fdllm_qkv_rope_kv_write)

def _qkv_case(B, S, H, Hq, Hkv, dtype, gpu, exact, seed, x_pad=0):
    """x [B, S, H] (a view with row stride H + x_pad), weights [heads * 128, H], biases.
    exact: small multiples of 1/16 whose products and sums are exact in fp32, so every
    summation order gives the same projection and the result is fixed bit for bit."""
    g = torch.Generator().manual_seed(seed)
    D = 128
    if exact:
        def mk(*shape):
            return (torch.randint(-4, 5, shape, generator=g).float() / 16).to(dtype)
        xf = torch.randint(-3, 4, (B, S, H + x_pad), generator=g).float().to(dtype)
        wq, wk, wv = mk(Hq * D, H), mk(Hkv * D, H), mk(Hkv * D, H)
        bq, bk, bv = mk(Hq * D), mk(Hkv * D), mk(Hkv * D)
    else:
        xf = torch.randn(B, S, H + x_pad, generator=g).to(dtype)
        wq, wk, wv = ((torch.randn(n * D, H, generator=g) * 0.02).to(dtype) for n in (Hq, Hkv, Hkv))
        bq, bk, bv = ((torch.randn(n * D, generator=g) * 0.1).to(dtype) for n in (Hq, Hkv, Hkv))
    t = [u.to(gpu) for u in (xf, wq, bq, wk, bk, wv, bv)]
    x = t[0][..., :H]
    return x, t[1:]


def _ulps(a, b):
    ai = a.contiguous().view(torch.int16).to(torch.int32)
    bi = b.contiguous().view(torch.int16).to(torch.int32)
    ai = torch.where(ai < 0, -(ai & 0x7FFF), ai)
    bi = torch.where(bi < 0, -(bi & 0x7FFF), bi)
    return (ai - bi).abs()


@pytest.mark.parametrize("B,S,H,Hq,Hkv,dtype,x_pad", [
    (16, 32, 3584, 28, 4, torch.bfloat16, 0),   # the 7B full-block forward: 512 token rows
    (16, 8, 3584, 28, 4, torch.bfloat16, 0),    # the 7B sub-block forward: 128 rows
    (3, 37, 256, 4, 2, torch.bfloat16, 64),     # 111 rows: one ragged tile; padded x rows
    (5, 64, 512, 2, 1, torch.float16, 0),       # 320 rows: three tiles, the last ragged
])
def test_qkv_rope_exact_inputs_bit_exact(gpu, B, S, H, Hq, Hkv, dtype, x_pad):
    """With inputs whose products and sums are exact in fp32, the fused kernel equals
    the projections (float64, rounded once to the 16-bit type, as a linear layer with
    bias rounds) + the eager RoPE + the cache writes bit for bit: a transposed operand,
    a wrong row, column or head, a dropped bias or K step would all show."""
    D = 128
    x, (wq, bq, wk, bk, wv, bv) = _qkv_case(B, S, H, Hq, Hkv, dtype, gpu, True, B * S + H, x_pad)
    cos, sin = _tables(S, D, 517, dtype, gpu)
    L, LB = S + 40, max(S, 32)
    ws = torch.arange(B, dtype=torch.int32, device=gpu) * 3
    kc = torch.full((B, L, Hkv, D), 7.0, dtype=dtype, device=gpu)
    vc = kc.clone()
    kb = torch.full((B, LB, Hkv, D), -5.0, dtype=dtype, device=gpu)
    vb = kb.clone()
    print(f"case qkv exact B={B} S={S} H={H} {Hq}/{Hkv} {dtype}", flush=True)
    q_rot, (k_rot, v_out) = ops.qkv_rope_kv_write(x, wq, bq, wk, bk, wv, bv, cos, sin, kc, vc, write_start=ws,
                                                  write_offset=1, k_block=kb, v_block=vb, block_offset=0,
                                                  kv_out=True)
    x64 = x.double().cpu()  # exact: float64 holds every sum, so this is the projection

    def proj(w, b_, n):
        return (x64 @ w.double().cpu().T + b_.double().cpu()).to(dtype).view(B, S, n, D).to(gpu)
    q, k, v = proj(wq, bq, Hq), proj(wk, bk, Hkv), proj(wv, bv, Hkv)
    q_ref, k_ref = _rope_torch(q, cos, sin), _rope_torch(k, cos, sin)
    assert torch.equal(v_out, v)
    assert torch.equal(q_rot, q_ref)
    assert torch.equal(k_rot, k_ref)
    kc_ref, vc_ref = torch.full_like(kc, 7.0), torch.full_like(vc, 7.0)
    for b in range(B):
        p0 = int(ws[b]) + 1
        n = max(0, min(S, L - p0))  # rows past the cache's length are skipped
        kc_ref[b, p0:p0 + n], vc_ref[b, p0:p0 + n] = k_ref[b, :n], v[b, :n]
    assert torch.equal(kc, kc_ref) and torch.equal(vc, vc_ref)
    kb_ref, vb_ref = torch.full_like(kb, -5.0), torch.full_like(vb, -5.0)
    kb_ref[:, :S], vb_ref[:, :S] = k_ref, v
    assert torch.equal(kb, kb_ref) and torch.equal(vb, vb_ref)


@pytest.mark.parametrize("S", [32, 8])
def test_qkv_rope_random_weights_within_rounding(gpu, S):
    """7B shapes with N(0, 0.02) weights: the projections agree with a float64
    restatement rounded to bf16 to within one ulp or the fp32 sum's rounding error near
    zero (fp32 MFMA sums in another order can round the other way), 99 % of them
    exactly, and the rotated rows with the eager RoPE of those projections to within
    what one flipped input can move them."""
    B, H, Hq, Hkv, D = 16, 3584, 28, 4, 128
    x, (wq, bq, wk, bk, wv, bv) = _qkv_case(B, S, H, Hq, Hkv, torch.bfloat16, gpu, False, S)
    cos, sin = _tables(S, D, 700, torch.bfloat16, gpu)
    print(f"case qkv random S={S}", flush=True)
    q_rot, (k_rot, v_out) = ops.qkv_rope_kv_write(x, wq, bq, wk, bk, wv, bv, cos, sin, kv_out=True)
    x64 = x.double().cpu()

    def proj(w, b_, n):
        return (x64 @ w.double().cpu().T + b_.double().cpu()).to(torch.bfloat16).view(B, S, n, D)
    v_ref = proj(wv, bv, Hkv)
    got = v_out.cpu()
    du = _ulps(got, v_ref)
    # one ulp of the result, or the fp32 sum's own error near zero (|y| ~ 1e-3 has ulps
    # of 1e-5, below the rounding error of 3584 fp32 additions of terms ~0.02)
    ulp = v_ref.float().abs() * 2.0 ** -7
    assert bool(((got.float() - v_ref.float()).abs() <= ulp + 1e-4).all())
    assert float((du == 0).float().mean()) > 0.99
    q_ref = _rope_torch(proj(wq, bq, Hq).to(gpu), cos, sin).cpu()
    k_ref = _rope_torch(proj(wk, bk, Hkv).to(gpu), cos, sin).cpu()
    for got, ref in ((q_rot.cpu(), q_ref), (k_rot.cpu(), k_ref)):
        torch.testing.assert_close(got.float(), ref.float(), atol=2e-2, rtol=2e-2)
        assert float((_ulps(got, ref) == 0).float().mean()) > 0.98


def test_qkv_fused_forward_matches_unfused(gpu):
    """The patched forward with the fused projections against nn.Linear projections +
    the fused RoPE: the logits of a prefill and of a diffusion step agree to within the
    projections' last-bit rounding."""
    cfg = em.BlockDiffusionConfig(num_hidden_layers=2)
    model = em.build_model(cfg, gpu)
    x = torch.randint(0, cfg.vocab_size - 1, (4, 96), generator=torch.Generator().manual_seed(6)).to(gpu)
    logits = []
    saved = ab.FUSED_QKV_PROJECTION
    for fused in (True, False):
        ab.FUSED_QKV_PROJECTION = fused
        try:
            cache, _ = es.HipStaticAttention(graphs=False).make_caches(4, 256, cfg, torch.bfloat16, gpu, False)
            orig = ab.patch_attention_layers(model, ab.get_attention_backend("hip"))
            try:
                pre = model(x[:, :64], cache, update_past_key_values=True).float()
                cache.set_kv_write_start(64)
                cache.set_scratch_seqlens(96)
                step = model(x[:, 64:96], cache, cache_position=torch.arange(64, 96, device=gpu)).float()
            finally:
                ab.unpatch_attention_layers(model, orig)
        finally:
            ab.FUSED_QKV_PROJECTION = saved
        logits.append((pre, step))
    for a, b in zip(logits[0], logits[1]):
        rel = float((a - b).norm() / b.norm())
        assert rel < 2e-2, rel
        assert float((a.argmax(-1) == b.argmax(-1)).float().mean()) > 0.9

