"""Pins the attention oracle (CPU only, no GPU, no HIP library).

Each check is chosen so that a plausible mistake in the oracle fails it:
  * committed golden vectors (torch CPU SDPA after the GQA expand of
    tests/test_focus.py:216-219, and a float64 numpy product) — a wrong scale,
    GQA map or mask changes the output far beyond the tolerance;
  * an independent pure-Python brute force on tiny shapes;
  * closed forms: one visible key gives that key's value row, identical keys
    give the mean of the visible values;
  * invariants: keys past cache_seqlens have no influence, permuting visible
    keys changes nothing, G = 1 equals per-head attention;
  * the block-causal mask, enumerated by hand (modeling.py:145-150);
  * planted mistakes (a wrong GQA head map, an off-by-one length, a flipped
    block comparison) must fail the checks above.
"""
import math
from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attention as oa

GOLDEN = Path(__file__).resolve().parent / "golden"


def _golden():
    z = np.load(GOLDEN / "kv_decode_small.npz")
    return {k: z[k] for k in z.files}


def test_golden_sdpa_shim_fp32():
    z = _golden()
    q, k, v = (torch.from_numpy(z[n]) for n in ("q", "k", "v"))
    out = oa.sdpa_kvcache(q, k, v, torch.from_numpy(z["seqlens"]), scaling=float(z["scale"]))
    np.testing.assert_allclose(out.numpy(), z["out"], atol=2e-5, rtol=2e-5)
    np.testing.assert_allclose(z["out"], z["out_f64"], atol=1e-4, rtol=1e-4)


def test_golden_brute_force_f64():
    z = _golden()
    out = oa.attention_np(z["q"], z["k"], z["v"], z["seqlens"], float(z["scale"]))
    np.testing.assert_allclose(out, z["out_f64"], atol=1e-10, rtol=1e-10)


def test_golden_default_scale_is_inverse_sqrt_head_dim():
    z = _golden()
    assert math.isclose(float(z["scale"]), 128 ** -0.5)
    out = oa.attention_np(z["q"], z["k"], z["v"], z["seqlens"])  # scale=None
    np.testing.assert_allclose(out, z["out_f64"], atol=1e-10, rtol=1e-10)


def test_planted_wrong_gqa_map_fails_golden():
    """h -> h % Hkv instead of h // G: the oracle must disagree with the golden."""
    z = _golden()
    H, Hkv = z["q"].shape[2], z["k"].shape[2]
    G = H // Hkv
    # emulate the wrong map by permuting query heads so that head h meets KV head h % Hkv
    wrong = np.empty_like(z["q"])
    for h in range(H):
        # under the right map, head j uses KV head j // G; pick j with j // G == h % Hkv
        j = (h % Hkv) * G + (h // Hkv) % G
        wrong[:, :, j] = z["q"][:, :, h]
    out = oa.attention_np(wrong, z["k"], z["v"], z["seqlens"], float(z["scale"]))
    assert not np.allclose(out, z["out_f64"], atol=1e-2, rtol=1e-2)


def test_planted_off_by_one_length_fails_golden():
    z = _golden()
    out = oa.attention_np(z["q"], z["k"], z["v"], z["seqlens"] - 1, float(z["scale"]))
    assert not np.allclose(out, z["out_f64"], atol=1e-3, rtol=1e-3)


def _loops(q, k, v, seqlens, scale, mask_mode=oa.MASK_SEQLEN, block=32, q_start=None):
    """Pure-Python brute force: one query row, one head at a time."""
    B, Sq, H, D = q.shape
    Hkv = k.shape[2]
    G = H // Hkv
    out = np.zeros((B, Sq, H, D))
    for b in range(B):
        L = int(seqlens[b])
        qs = L - Sq if q_start is None else int(q_start[b])
        for t in range(Sq):
            qpos = qs + t
            for h in range(H):
                kh = h // G
                keys = []
                for j in range(L):
                    if mask_mode == oa.MASK_CAUSAL and j > qpos:
                        continue
                    if mask_mode == oa.MASK_BLOCK_CAUSAL and (qpos < 0 or j // block > qpos // block):
                        continue
                    keys.append(j)
                if not keys:
                    continue
                s = [sum(float(q[b, t, h, d]) * float(k[b, j, kh, d]) for d in range(D)) * scale for j in keys]
                m = max(s)
                w = [math.exp(x - m) for x in s]
                tot = sum(w)
                for d in range(D):
                    out[b, t, h, d] = sum(wi * float(v[b, j, kh, d]) for wi, j in zip(w, keys)) / tot
    return out


@pytest.mark.parametrize("mask_mode", [oa.MASK_SEQLEN, oa.MASK_CAUSAL, oa.MASK_BLOCK_CAUSAL])
def test_brute_force_loops_tiny(mask_mode):
    rng = np.random.default_rng(mask_mode)
    B, Sq, H, Hkv, D, S = 3, 5, 6, 2, 8, 13
    q = rng.standard_normal((B, Sq, H, D))
    k = rng.standard_normal((B, S, Hkv, D))
    v = rng.standard_normal((B, S, Hkv, D))
    seqlens = np.array([13, 7, 0])
    got = oa.attention_np(q, k, v, seqlens, 0.3, mask_mode=mask_mode, mask_block=4)
    exp = _loops(q, k, v, seqlens, 0.3, mask_mode, 4)
    np.testing.assert_allclose(got, exp, atol=1e-12, rtol=1e-12)
    if mask_mode == oa.MASK_SEQLEN:
        # the SDPA shim on the sequences with at least one key (it gives NaN for none)
        sd = oa.sdpa_kvcache(*(torch.from_numpy(x[:2]) for x in (q, k, v)), torch.tensor([13, 7]),
                             scaling=0.3)
        np.testing.assert_allclose(sd.numpy(), exp[:2], atol=1e-10)


def test_closed_forms_single_key_and_equal_keys():
    rng = np.random.default_rng(1)
    B, Sq, H, Hkv, D, S = 2, 4, 8, 2, 16, 20
    q = rng.standard_normal((B, Sq, H, D))
    k = rng.standard_normal((B, S, Hkv, D))
    v = rng.standard_normal((B, S, Hkv, D))
    # one visible key -> that value row, for every head of the group
    out = oa.attention_np(q, k, v, [1, 1])
    for h in range(H):
        np.testing.assert_allclose(out[:, :, h], np.broadcast_to(v[:, None, 0, h // 4], (B, Sq, D)), atol=1e-12)
    # identical keys -> the mean of the visible values
    k2 = np.broadcast_to(k[:, :1], k.shape).copy()
    out = oa.attention_np(q, k2, v, [20, 9])
    for b, L in enumerate((20, 9)):
        for h in range(H):
            np.testing.assert_allclose(out[b, :, h], np.broadcast_to(v[b, :L, h // 4].mean(0), (Sq, D)), atol=1e-12)
    # torch shim: same closed form
    sd = oa.sdpa_kvcache(torch.from_numpy(q), torch.from_numpy(k2), torch.from_numpy(v), torch.tensor([20, 9]))
    np.testing.assert_allclose(sd.numpy(), out, atol=1e-10)


def test_masked_keys_have_no_influence_and_permutation_invariance():
    rng = np.random.default_rng(2)
    B, Sq, H, Hkv, D, S = 2, 8, 28, 4, 32, 64
    q = rng.standard_normal((B, Sq, H, D))
    k = rng.standard_normal((B, S, Hkv, D))
    v = rng.standard_normal((B, S, Hkv, D))
    seqlens = np.array([40, 17])
    base = oa.attention_np(q, k, v, seqlens)
    kp, vp = k.copy(), v.copy()
    for b, L in enumerate(seqlens):
        kp[b, L:] = 1e4
        vp[b, L:] = -1e4
    np.testing.assert_allclose(oa.attention_np(q, kp, vp, seqlens), base, atol=1e-12)
    sd = oa.sdpa_kvcache(*(torch.from_numpy(x) for x in (q, kp, vp)), torch.from_numpy(seqlens))
    np.testing.assert_allclose(sd.numpy(), base, atol=1e-9)
    # permuting the visible keys (with their values) changes nothing
    kq, vq = k.copy(), v.copy()
    for b, L in enumerate(seqlens):
        perm = rng.permutation(L)
        kq[b, :L] = k[b, perm]
        vq[b, :L] = v[b, perm]
    np.testing.assert_allclose(oa.attention_np(q, kq, vq, seqlens), base, atol=1e-12)


def test_mha_reduces_to_per_head_sdpa():
    torch.manual_seed(0)
    B, Sq, H, D, S = 2, 6, 3, 16, 10
    q, k, v = torch.randn(B, Sq, H, D), torch.randn(B, S, H, D), torch.randn(B, S, H, D)
    got = oa.sdpa_kvcache(q, k, v, torch.tensor([S, S]))
    for h in range(H):
        exp = F.scaled_dot_product_attention(q[:, :, h].unsqueeze(1), k[:, :, h].unsqueeze(1),
                                             v[:, :, h].unsqueeze(1)).squeeze(1)
        torch.testing.assert_close(got[:, :, h], exp, atol=1e-6, rtol=1e-6)


def test_paged_layout_equals_contiguous():
    rng = np.random.default_rng(3)
    B, Sq, H, Hkv, D, ps = 3, 4, 4, 2, 8, 4
    seqlens = np.array([9, 16, 3])
    npages = [(L + ps - 1) // ps for L in seqlens]
    pool_k = rng.standard_normal((sum(npages) + 2, ps, Hkv, D))
    pool_v = rng.standard_normal(pool_k.shape)
    perm = rng.permutation(pool_k.shape[0])
    table = np.zeros((B, max(npages)), dtype=np.int64)
    off = 0
    for b, n in enumerate(npages):
        table[b, :n] = perm[off:off + n]
        off += n
    q = rng.standard_normal((B, Sq, H, D))
    kc = np.zeros((B, 16, Hkv, D))
    vc = np.zeros_like(kc)
    for b in range(B):
        for j in range(seqlens[b]):
            kc[b, j] = pool_k[table[b, j // ps], j % ps]
            vc[b, j] = pool_v[table[b, j // ps], j % ps]
    a = oa.attention_np(q, pool_k, pool_v, seqlens, page_table=table, page_size=ps)
    c = oa.attention_np(q, kc, vc, seqlens)
    np.testing.assert_allclose(a, c, atol=1e-14)


def test_block_causal_mask_by_hand():
    m = oa.block_causal_mask(4, 4, 2)
    exp = torch.tensor([[1, 1, 0, 0], [1, 1, 0, 0], [1, 1, 1, 1], [1, 1, 1, 1]], dtype=torch.bool)
    assert torch.equal(m, exp)
    # queries of the second 32-block of a 64-token prefill with a 32-token past
    m = oa.block_causal_mask(32, 96, 32, past_len=64)
    assert m[:, :96].all()
    m = oa.block_causal_mask(64, 64, 32)
    assert m[:32, :32].all() and not m[:32, 32:].any() and m[32:].all()
    # planted mistake: a strict comparison would hide the own block
    q_idx, kv_idx = torch.arange(4), torch.arange(4)
    strict = (q_idx[:, None] // 2) > (kv_idx[None, :] // 2)
    assert not torch.equal(strict, oa.block_causal_mask(4, 4, 2))


def test_block_causal_last_block_equals_kvcache_attention():
    """The last block's queries of a block-causal prefill see every key, so they
    equal kv-cache attention with L = S."""
    torch.manual_seed(4)
    B, S, H, Hkv, D, blk = 2, 96, 6, 2, 16, 32
    q, k, v = torch.randn(B, S, H, D), torch.randn(B, S, Hkv, D), torch.randn(B, S, Hkv, D)
    full = oa.sdpa_block_causal(q, k, v, blk)
    last = oa.sdpa_kvcache(q[:, -blk:], k, v, torch.tensor([S, S]))
    torch.testing.assert_close(full[:, -blk:], last, atol=1e-5, rtol=1e-5)
    # and the brute force agrees on every block
    np_out = oa.attention_np(q.numpy(), k.numpy(), v.numpy(), [S, S], mask_mode=oa.MASK_BLOCK_CAUSAL,
                             mask_block=blk, q_start=[0, 0])
    np.testing.assert_allclose(full.numpy(), np_out, atol=1e-5, rtol=1e-5)
    # first block sees only itself
    first = oa.sdpa_kvcache(q[:, :blk], k[:, :blk], v[:, :blk], torch.tensor([blk, blk]))
    torch.testing.assert_close(full[:, :blk], first, atol=1e-5, rtol=1e-5)


def test_repeat_kv_map():
    x = torch.arange(2 * 3 * 1 * 1, dtype=torch.float32).reshape(2, 3, 1, 1)
    r = oa.repeat_kv(x, 4)
    assert r.shape == (2, 12, 1, 1)
    for h in range(12):
        assert torch.equal(r[:, h], x[:, h // 4])


def test_e2e_oracle_attention_variants():
    """The eager e2e oracle's float32 attention equals the SDPA shim; its bf16-P variant
    differs only by the rounding of the probabilities (bounded by bf16 resolution)."""
    from oracle.e2e_eager import kvcache_attention_f32
    g = torch.Generator().manual_seed(9)
    q, k, v = torch.randn(3, 5, 8, 32, generator=g), torch.randn(3, 40, 2, 32, generator=g), \
        torch.randn(3, 40, 2, 32, generator=g)
    sl = torch.tensor([40, 9, 1])
    ref = oa.sdpa_kvcache(q, k, v, sl, scaling=0.2)
    torch.testing.assert_close(kvcache_attention_f32(q, k, v, sl, 0.2, False), ref, atol=1e-5, rtol=1e-5)
    lo = kvcache_attention_f32(q, k, v, sl, 0.2, True)
    assert 0 < (lo - ref).abs().max() < 2e-2
    # one visible key: p = 1 exactly in bf16, so both variants return that value row
    torch.testing.assert_close(lo[2], v[2, 0].repeat_interleave(4, 0)[None].expand(5, 8, 32), atol=0, rtol=0)


def test_cache_write_matches_slice_assignment_and_paging():
    """cache_write_np against torch slice assignment (the StaticKVCache.update
    statement, static_kv_cache.py:132-160, one start per sequence), the paged layout
    against the contiguous one, and the capacity rule; a planted off-by-one start
    fails."""
    g = torch.Generator().manual_seed(3)
    B, S, Hkv, D, T = 3, 96, 2, 8, 20
    cache = torch.randn(B, S, Hkv, D, generator=g)
    new = torch.randn(B, T, Hkv, D, generator=g)
    starts = [0, 37, 86]  # the last one runs past the capacity: rows 96.. are dropped
    exp = cache.clone()
    for b, s0 in enumerate(starts):
        n = min(T, S - s0)
        exp[b, s0:s0 + n] = new[b, :n]
    got = oa.cache_write_np(cache.numpy(), new.numpy(), starts)
    assert np.array_equal(got, exp.numpy())
    assert np.array_equal(got[2, 86:], new[2, :10].numpy())
    planted = oa.cache_write_np(cache.numpy(), new.numpy(), [s + 1 for s in starts])
    assert not np.array_equal(planted, exp.numpy())
    # paged: shuffled 32-key pages hold the same rows after the same write
    ps, per = 32, S // 32
    perm = torch.randperm(B * per, generator=g)
    pt = perm.view(B, per).numpy()
    pool = np.zeros((B * per, ps, Hkv, D), dtype=np.float32)
    for b in range(B):
        for i in range(per):
            pool[pt[b, i]] = cache[b, i * ps:(i + 1) * ps].numpy()
    pool2 = oa.cache_write_np(pool, new.numpy(), starts, page_table=pt, page_size=ps)
    for b in range(B):
        back = np.concatenate([pool2[pt[b, i]] for i in range(per)], axis=0)
        assert np.array_equal(back, exp[b].numpy())


def test_e2e_oracle_caches_follow_the_static_cache_rules():
    """The eager e2e oracle's caches: update() stores at the committed length and moves
    it only after the last layer (static_kv_cache.py:132-160); write_scratch_compiled()
    stores at kv_write_start without moving it (:218-229); the block cache's write()
    stores at the block offset. Each equals cache_write_np's per-sequence store; a
    planted pointer move after the first layer would fail the second layer's rows."""
    from oracle.e2e_eager import TorchBlockCache, TorchKVCache
    g = torch.Generator().manual_seed(11)
    B, L, H, D, layers = 2, 24, 2, 8, 3
    c = TorchKVCache(B, L, layers, H, D, torch.float32, "cpu")
    k1, v1 = torch.randn(B, 5, H, D, generator=g), torch.randn(B, 5, H, D, generator=g)
    for layer in range(layers):
        before = c.key_cache[layer].clone()
        c.update(k1 + layer, v1 - layer, layer)
        exp = oa.cache_write_np(before.numpy(), (k1 + layer).numpy(), [0, 0])
        np.testing.assert_array_equal(c.key_cache[layer].numpy(), exp)
        assert c.get_seq_length() == (5 if layer == layers - 1 else 0)
    k2 = torch.randn(B, 3, H, D, generator=g)
    for layer in range(layers):
        before = c.key_cache[layer].clone()
        c.update(k2, k2, layer)
        np.testing.assert_array_equal(c.key_cache[layer].numpy(), oa.cache_write_np(before.numpy(), k2.numpy(), [5, 5]))
    assert c.get_seq_length() == 8
    c.set_kv_write_start(8)
    k3 = torch.randn(B, 4, H, D, generator=g)
    before = c.value_cache[1].clone()
    c.write_scratch_compiled(k3, k3, 1)
    np.testing.assert_array_equal(c.value_cache[1].numpy(), oa.cache_write_np(before.numpy(), k3.numpy(), [8, 8]))
    assert c.get_seq_length() == 8
    bc = TorchBlockCache(B, 32, layers, H, D, torch.float32, "cpu")
    kb = torch.randn(B, 8, H, D, generator=g)
    before = bc.key_cache[2].clone()
    bc.write(kb, kb, 2, 16)
    np.testing.assert_array_equal(bc.key_cache[2].numpy(), oa.cache_write_np(before.numpy(), kb.numpy(), [16, 16]))


def test_e2e_oracle_rope_is_the_pairwise_rotation():
    """The eager oracle's RoPE, q * cos + rotate_half(q) * sin (modeling.py:168-200), is the
    rotation of each pair (x_i, x_{i + D/2}) by the angle of its frequency:
    (x cos t - y sin t, y cos t + x sin t), written out element by element here. Position 0
    is the identity, norms are kept, and a dot product of a rotated query and key depends
    only on the distance of their positions. A planted sign error in rotate_half fails the
    explicit rotation."""
    from oracle.e2e_eager import _rotate_half
    g = torch.Generator().manual_seed(11)
    D, P = 16, 9
    x = torch.randn(P, D, generator=g, dtype=torch.float64)
    inv_freq = 1.0 / (10000.0 ** (torch.arange(0, D, 2, dtype=torch.float64) / D))
    ang = torch.arange(P, dtype=torch.float64)[:, None] * inv_freq[None, :]  # [P, D/2]
    emb = torch.cat((ang, ang), dim=-1)
    cos, sin = emb.cos(), emb.sin()
    got = x * cos + _rotate_half(x) * sin
    h = D // 2
    exp = torch.empty_like(x)
    for p in range(P):
        for i in range(h):
            c, s = math.cos(ang[p, i].item()), math.sin(ang[p, i].item())
            exp[p, i] = x[p, i] * c - x[p, i + h] * s
            exp[p, i + h] = x[p, i + h] * c + x[p, i] * s
    torch.testing.assert_close(got, exp, atol=1e-12, rtol=0)
    torch.testing.assert_close(got[0], x[0], atol=0, rtol=0)
    torch.testing.assert_close(got.norm(dim=-1), x.norm(dim=-1), atol=1e-12, rtol=0)
    q, k = torch.randn(D, generator=g, dtype=torch.float64), torch.randn(D, generator=g, dtype=torch.float64)

    def rot(v, p):
        return v * cos[p] + _rotate_half(v) * sin[p]
    assert abs(rot(q, 5) @ rot(k, 2) - rot(q, 7) @ rot(k, 4)) < 1e-12
    planted = x * cos + torch.cat((x[..., h:], -x[..., :h]), dim=-1) * sin
    assert not torch.allclose(planted, exp)
