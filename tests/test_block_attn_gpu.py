"""GPU parity of the block attention kernel against the oracle.

Bar: atol = rtol = 1e-2 against the float64 brute force (bf16 inputs, fp32
softmax/accumulation in the kernel), on the same seeded inputs.

Covers: the fp32 golden block-decode case (12/2 heads, 512 + 32 keys) run in
bf16; the 7B-geometry bs16 paged sub-block decode at full size; the contiguous
static-cache layout vs the paged layout (identical outputs); full 32-token
blocks (224 rows per KV head); split-KV on/off; causal and block-causal masks;
block-causal prefill with its KV-cache write; ragged lengths, empty sequences,
a single visible key; fp16; head_dim 64; NaN in every row no query may see (past
the lengths, unreferenced pages) leaving every kernel family's output unchanged; query
rows read through non-contiguous strides.
"""
from pathlib import Path

import numpy as np
import pytest
import torch

from fast_v2_amd import _ffi, ops, workloads
from oracle import attention as oa

pytestmark = pytest.mark.gpu

ATOL = RTOL = 1e-2
GOLDEN = Path(__file__).resolve().parent / "golden"


def _check(got: torch.Tensor, exp: np.ndarray, atol=ATOL, rtol=RTOL):
    got = got.float().cpu().numpy()
    assert np.isfinite(got).all()
    np.testing.assert_allclose(got, exp, atol=atol, rtol=rtol)


def test_golden_small_decode_bf16(gpu):
    """fp32 golden (torch CPU SDPA, 1 x 32 queries x 12/2 heads, 544 keys) vs the bf16 kernel."""
    z = np.load(GOLDEN / "kv_decode_small.npz")
    q = torch.from_numpy(z["q"]).to(torch.bfloat16)
    k = torch.from_numpy(z["k"]).to(torch.bfloat16)
    v = torch.from_numpy(z["v"]).to(torch.bfloat16)
    seq = torch.from_numpy(z["seqlens"])
    out = ops.block_attn(q.to(gpu), k.to(gpu), v.to(gpu), seq.to(gpu), float(z["scale"]))
    # inputs were rounded to bf16: compare with both the bf16-input brute force (tight)
    # and the fp32 golden output (loose, input rounding included)
    _check(out, oa.attention_np(q.float(), k.float(), v.float(), seq, float(z["scale"])))
    _check(out, z["out"], atol=3e-2, rtol=3e-2)


def test_golden_small_decode_fp32(gpu):
    """The small fp32 decode (batch 1, 12 / 2 heads, 512 + 32 keys) at its own precision: the fp32 golden (torch CPU SDPA, 1 x 32 queries x
    12/2 heads over 512 + 32 keys) against the fp32 kernel on the same fp32 inputs, within
    1e-5 (both accumulate in fp32; only the summation order differs)."""
    z = np.load(GOLDEN / "kv_decode_small.npz")
    q, k, v = (torch.from_numpy(z[n]) for n in ("q", "k", "v"))
    assert q.dtype == k.dtype == v.dtype == torch.float32
    seq = torch.from_numpy(z["seqlens"])
    out = ops.block_attn(q.to(gpu), k.to(gpu), v.to(gpu), seq.to(gpu), float(z["scale"]))
    assert out.dtype == torch.float32
    np.testing.assert_allclose(out.cpu().numpy(), z["out"], atol=1e-5, rtol=1e-5)
    # and the float64 brute force of the oracle
    np.testing.assert_allclose(out.cpu().numpy(), oa.attention_np(q, k, v, seq, float(z["scale"])),
                               atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("kv_split", [64, 192, 320, 0, 4096])
def test_fp32_key_splits(gpu, kv_split):
    """fp32 kernel with its keys split over workgroups and the partials folded by the
    combine kernel: 64-key splits (one chunk each), uneven splits (192, 320 keys of 544),
    the automatic choice and one split; the fp32 golden within 1e-5, and a paged
    block-causal call with q_start whose row blocks see different key counts (some of a
    block's splits hold keys past some of its rows' limits) against the float64 brute
    force."""
    print(f"case fp32 kv_split={kv_split}", flush=True)
    z = np.load(GOLDEN / "kv_decode_small.npz")
    q, k, v = (torch.from_numpy(z[n]) for n in ("q", "k", "v"))
    seq = torch.from_numpy(z["seqlens"])
    out = ops.block_attn(q.to(gpu), k.to(gpu), v.to(gpu), seq.to(gpu), float(z["scale"]), kv_split=kv_split)
    np.testing.assert_allclose(out.cpu().numpy(), z["out"], atol=1e-5, rtol=1e-5)
    g = torch.Generator().manual_seed(kv_split + 7)
    B, S, Hq, Hkv, D, Sq, ps = 3, 640, 8, 2, 128, 40, 32
    seqlens = torch.tensor([600, 0, 233], dtype=torch.int32)
    q_start = torch.tensor([560, 0, 150], dtype=torch.int32)
    q2 = torch.randn(B, Sq, Hq, D, generator=g)
    k2 = torch.randn(B, S, Hkv, D, generator=g)
    v2 = torch.randn(B, S, Hkv, D, generator=g)
    n_pages = S // ps
    pt = torch.randperm(B * n_pages, generator=g).view(B, n_pages).to(torch.int32)
    kp = torch.empty(B * n_pages, ps, Hkv, D)
    vp = torch.empty_like(kp)
    for b in range(B):
        for j in range(n_pages):
            kp[pt[b, j]] = k2[b, j * ps:(j + 1) * ps]
            vp[pt[b, j]] = v2[b, j * ps:(j + 1) * ps]
    out2 = ops.block_attn(q2.to(gpu), kp.to(gpu), vp.to(gpu), seqlens.to(gpu), None,
                          mask_mode=_ffi.MASK_BLOCK_CAUSAL, mask_block=32, q_start=q_start.to(gpu),
                          page_table=pt.to(gpu), page_size=ps, kv_split=kv_split).cpu().numpy()
    exp = oa.attention_np(q2, k2, v2, seqlens, None, mask_mode=_ffi.MASK_BLOCK_CAUSAL, mask_block=32,
                          q_start=q_start)
    np.testing.assert_allclose(out2, exp, atol=1e-5, rtol=1e-5)
    assert np.count_nonzero(out2[1]) == 0


@pytest.mark.parametrize("mask_mode", [_ffi.MASK_SEQLEN, _ffi.MASK_CAUSAL, _ffi.MASK_BLOCK_CAUSAL])
@pytest.mark.parametrize("paged", [False, True])
def test_fp32_masks_paged_and_gqa(gpu, mask_mode, paged):
    """fp32 kernel: every mask mode, contiguous and paged caches, GQA 1 / 4 / 8, head_dim
    64 and 128, ragged and empty lengths, q_start given or not; within 1e-5 of the float64
    brute force."""
    g = torch.Generator().manual_seed(100 + 10 * mask_mode + paged)
    for Hq, Hkv, D, Sq in ((12, 2, 128, 32), (8, 8, 64, 5), (16, 4, 128, 1)):
        B, S, ps = 3, 160, 16
        seqlens = torch.tensor([150, 0, 77], dtype=torch.int32)
        q = torch.randn(B, Sq, Hq, D, generator=g)
        k = torch.randn(B, S, Hkv, D, generator=g)
        v = torch.randn(B, S, Hkv, D, generator=g)
        q_start = torch.tensor([150 - Sq, 0, 40], dtype=torch.int32) if Sq > 1 else None
        print(f"case fp32 mask={mask_mode} paged={paged} Hq={Hq} Hkv={Hkv} D={D} Sq={Sq}", flush=True)
        exp = oa.attention_np(q, k, v, seqlens, None, mask_mode=mask_mode, mask_block=32, q_start=q_start)
        if paged:
            n_pages = S // ps
            perm = torch.randperm(B * n_pages, generator=g)
            pt = perm.view(B, n_pages).to(torch.int32)
            kp = torch.empty(B * n_pages, ps, Hkv, D)
            vp = torch.empty_like(kp)
            for b in range(B):
                for j in range(n_pages):
                    kp[pt[b, j]] = k[b, j * ps:(j + 1) * ps]
                    vp[pt[b, j]] = v[b, j * ps:(j + 1) * ps]
            out = ops.block_attn(q.to(gpu), kp.to(gpu), vp.to(gpu), seqlens.to(gpu), None, mask_mode=mask_mode,
                                 mask_block=32, q_start=None if q_start is None else q_start.to(gpu),
                                 page_table=pt.to(gpu), page_size=ps)
        else:
            out = ops.block_attn(q.to(gpu), k.to(gpu), v.to(gpu), seqlens.to(gpu), None, mask_mode=mask_mode,
                                 mask_block=32, q_start=None if q_start is None else q_start.to(gpu))
        got = out.cpu().numpy()
        np.testing.assert_allclose(got, exp, atol=1e-5, rtol=1e-5)
        assert np.count_nonzero(got[1]) == 0  # the empty sequence


@pytest.mark.parametrize("kv_split", [0, 64, 256, 1 << 20])
def test_paged_subblock_decode_7b_bs16(gpu, kv_split):
    wl = workloads.kv_decode_paged(seed=0)
    print(f"case paged decode bs16 kv_split={kv_split} lens={wl.seqlens.tolist()}", flush=True)
    out = ops.block_attn(wl.q.to(gpu), wl.k_pool.to(gpu), wl.v_pool.to(gpu), wl.seqlens.to(gpu), wl.scale,
                         page_table=wl.page_table.to(gpu), page_size=wl.page_size,
                         kv_split=min(kv_split, 1 << 16) if kv_split else 0)
    exp = oa.attention_np(wl.q.float(), wl.k_pool.float(), wl.v_pool.float(), wl.seqlens, wl.scale,
                          page_table=wl.page_table, page_size=wl.page_size)
    _check(out, exp)


def _paged_to_contig(wl, max_s):
    B = wl.q.shape[0]
    Hkv, D = wl.k_pool.shape[2], wl.k_pool.shape[3]
    k = torch.zeros(B, max_s, Hkv, D, dtype=wl.k_pool.dtype)
    v = torch.zeros_like(k)
    for b in range(B):
        L = int(wl.seqlens[b])
        pos = torch.arange(L)
        pages = wl.page_table[b, pos // wl.page_size].long()
        k[b, :L] = wl.k_pool[pages, pos % wl.page_size]
        v[b, :L] = wl.v_pool[pages, pos % wl.page_size]
    return k, v


def test_contiguous_equals_paged(gpu):
    """The static BSHD cache [B, max_S, Hkv, D] (identity pages) gives bit-identical output."""
    wl = workloads.kv_decode_paged(seed=1, batch=6, min_prefix=64, max_prefix=1024)
    k, v = _paged_to_contig(wl, 1100)
    a = ops.block_attn(wl.q.to(gpu), wl.k_pool.to(gpu), wl.v_pool.to(gpu), wl.seqlens.to(gpu), wl.scale,
                       page_table=wl.page_table.to(gpu), page_size=wl.page_size)
    b = ops.block_attn(wl.q.to(gpu), k.to(gpu), v.to(gpu), wl.seqlens.to(gpu), wl.scale)
    assert torch.equal(a.cpu(), b.cpu())
    # and the SDPA shim (the reference's CPU statement) agrees within tolerance
    exp = oa.sdpa_kvcache(wl.q.float(), k.float(), v.float(), wl.seqlens, scaling=wl.scale)
    _check(b, exp.numpy())


@pytest.mark.parametrize("q_len", [1, 8, 32, 37])
@pytest.mark.parametrize("mask_mode", [_ffi.MASK_SEQLEN, _ffi.MASK_CAUSAL, _ffi.MASK_BLOCK_CAUSAL])
def test_masks_and_row_counts(gpu, q_len, mask_mode):
    g = torch.Generator().manual_seed(q_len * 10 + mask_mode)
    B, Hq, Hkv, D, max_s = 3, 28, 4, 128, 700
    seqlens = torch.tensor([600, 37, 700], dtype=torch.int32)
    q = torch.randn(B, q_len, Hq, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, max_s, Hkv, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, max_s, Hkv, D, generator=g).to(torch.bfloat16)
    print(f"case masks q_len={q_len} mode={mask_mode}", flush=True)
    out = ops.block_attn(q.to(gpu), k.to(gpu), v.to(gpu), seqlens.to(gpu), None, mask_mode=mask_mode,
                         mask_block=32, kv_split=128)
    exp = oa.attention_np(q.float(), k.float(), v.float(), seqlens, None, mask_mode=mask_mode, mask_block=32)
    _check(out, exp)


def test_edge_lengths(gpu):
    """Empty sequence -> zeros; one visible key -> that value row; keys past the length ignored."""
    g = torch.Generator().manual_seed(7)
    B, Sq, Hq, Hkv, D, S = 4, 8, 28, 4, 128, 300
    q = torch.randn(B, Sq, Hq, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, S, Hkv, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, S, Hkv, D, generator=g).to(torch.bfloat16)
    seqlens = torch.tensor([0, 1, 65, 300], dtype=torch.int32)
    # poison everything past each length with huge (finite) values
    kp, vp = k.clone(), v.clone()
    for b in range(B):
        kp[b, int(seqlens[b]):] = 3e4
        vp[b, int(seqlens[b]):] = -3e4
    out = ops.block_attn(q.to(gpu), kp.to(gpu), vp.to(gpu), seqlens.to(gpu), kv_split=64).cpu()
    assert torch.count_nonzero(out[0]) == 0
    one_key = v[1, 0].float().repeat_interleave(Hq // Hkv, 0)[None].expand(Sq, Hq, D)
    torch.testing.assert_close(out[1].float(), one_key, atol=0, rtol=0)
    exp = oa.attention_np(q.float(), k.float(), v.float(), seqlens)
    _check(out, exp)


def test_fp16_and_head_dim_64(gpu):
    g = torch.Generator().manual_seed(11)
    for dtype, D, Hq, Hkv in ((torch.float16, 128, 28, 4), (torch.bfloat16, 64, 12, 2), (torch.float16, 64, 8, 8)):
        B, Sq, S = 2, 32, 333
        q = torch.randn(B, Sq, Hq, D, generator=g).to(dtype)
        k = torch.randn(B, S, Hkv, D, generator=g).to(dtype)
        v = torch.randn(B, S, Hkv, D, generator=g).to(dtype)
        seqlens = torch.tensor([333, 200], dtype=torch.int32)
        print(f"case {dtype} D={D} {Hq}/{Hkv}", flush=True)
        out = ops.block_attn(q.to(gpu), k.to(gpu), v.to(gpu), seqlens.to(gpu), kv_split=128)
        _check(out, oa.attention_np(q.float(), k.float(), v.float(), seqlens))


def test_block_causal_prefill_with_cache_write(gpu):
    """Block-causal prefill: write K/V into the static cache, attend with the block mask."""
    wl = workloads.block_prefill(seed=0, batch=2, seq_len=512)
    B, S, Hkv, D = wl.k.shape
    kc = torch.zeros(B, 1024, Hkv, D, dtype=torch.bfloat16, device=gpu)
    vc = torch.zeros_like(kc)
    ops.kv_cache_write(wl.k.to(gpu), wl.v.to(gpu), kc, vc, write_offset=0)
    assert torch.equal(kc[:, :S].cpu(), wl.k) and torch.count_nonzero(kc[:, S:]) == 0
    seqlens = torch.full((B,), S, dtype=torch.int32, device=gpu)
    out = ops.block_attn(wl.q.to(gpu), kc, vc, seqlens, wl.scale, mask_mode=_ffi.MASK_BLOCK_CAUSAL,
                         mask_block=wl.block)
    exp = oa.sdpa_block_causal(wl.q.float(), wl.k.float(), wl.v.float(), wl.block)
    _check(out, exp.numpy())


def test_block_causal_prefill_full_size_sampled(gpu):
    """4 x 4096 block-causal prefill with the K/V cache write fused into the call (the
    benchmarked config): the cache holds the new rows bit for bit, the output equals the
    separate write + attention bit for bit, and sampled query blocks match the brute force."""
    wl = workloads.block_prefill(seed=0)
    B, S, Hkv, D = wl.k.shape
    kc = torch.full((B, S, Hkv, D), 7.0, dtype=torch.bfloat16, device=gpu)
    vc = torch.full_like(kc, -7.0)
    seqlens = torch.full((B,), S, dtype=torch.int32, device=gpu)
    k, v = wl.k.to(gpu), wl.v.to(gpu)
    out = ops.block_attn(wl.q.to(gpu), kc, vc, seqlens, wl.scale, mask_mode=_ffi.MASK_BLOCK_CAUSAL,
                         mask_block=wl.block, k_new=k, v_new=v)
    assert torch.equal(kc, k) and torch.equal(vc, v)
    ku, vu = torch.empty_like(kc), torch.empty_like(vc)
    ops.kv_cache_write(k, v, ku, vu)
    ref = ops.block_attn(wl.q.to(gpu), ku, vu, seqlens, wl.scale, mask_mode=_ffi.MASK_BLOCK_CAUSAL,
                         mask_block=wl.block)
    assert torch.equal(out, ref)
    # the cache write by the copy kernel (FDLLM_ATTN_CACHE_WRITE_KERNEL): same cache, same output
    kf, vf = torch.full_like(kc, 7.0), torch.full_like(vc, -7.0)
    out_f = ops.block_attn(wl.q.to(gpu), kf, vf, seqlens, wl.scale, mask_mode=_ffi.MASK_BLOCK_CAUSAL,
                           mask_block=wl.block, k_new=k, v_new=v, cache_write_kernel=True)
    assert torch.equal(kf, k) and torch.equal(vf, v)
    assert torch.equal(out_f, ref)
    out = out.cpu()
    for blk in (0, 1, 63, 64, 127):
        t0 = blk * wl.block
        qs = torch.full((B,), t0, dtype=torch.int32)
        exp = oa.attention_np(wl.q[:, t0:t0 + wl.block].float(), wl.k.float(), wl.v.float(),
                              torch.full((B,), S), wl.scale, mask_mode=oa.MASK_BLOCK_CAUSAL,
                              mask_block=wl.block, q_start=qs)
        _check(out[:, t0:t0 + wl.block], exp)


def test_flash_kvcache_op_and_meta(gpu):
    wl = workloads.kv_decode_paged(seed=2, batch=2, min_prefix=64, max_prefix=256)
    k, v = _paged_to_contig(wl, 320)
    out = torch.ops.fdllm.flash_kvcache(wl.q.to(gpu), k.to(gpu), v.to(gpu), wl.seqlens.to(gpu), wl.scale, False)
    _check(out, oa.attention_np(wl.q.float(), k.float(), v.float(), wl.seqlens, wl.scale))
    meta = torch.ops.fdllm.flash_kvcache(wl.q.to("meta"), k.to("meta"), v.to("meta"),
                                         wl.seqlens.to("meta"), wl.scale, False)
    assert meta.shape == wl.q.shape and meta.device.type == "meta"


def test_repeated_split_calls_rearm(gpu):
    """Split-KV calls in a row on one workspace give bit-identical results."""
    wl = workloads.kv_decode_paged(seed=3, batch=4, min_prefix=512, max_prefix=2048)
    q, kp, vp = wl.q.to(gpu), wl.k_pool.to(gpu), wl.v_pool.to(gpu)
    pt, sl = wl.page_table.to(gpu), wl.seqlens.to(gpu)
    first = ops.block_attn(q, kp, vp, sl, wl.scale, page_table=pt, page_size=wl.page_size, kv_split=128)
    for _ in range(20):
        again = ops.block_attn(q, kp, vp, sl, wl.scale, page_table=pt, page_size=wl.page_size, kv_split=128)
    assert torch.equal(first, again)


@pytest.mark.parametrize("balanced", [False, True])
@pytest.mark.parametrize("case", ["batch80_fixed_chunks", "one_long_capped", "batch64_all_lanes", "hkv1_256_slots"])
def test_split_decode_partitions(gpu, case, balanced):
    """The split decode kernels' key partitions at their edges: more than 64 sequences
    (fixed 5120-key chunks), one sequence long enough to need the 16-split cap next to
    empty and one-tile sequences, exactly 64 sequences (every lane of the search), and one
    KV head (256 slots per head); balanced selects the runs across sequence boundaries
    instead of the per-sequence splits."""
    g = torch.Generator().manual_seed(len(case))
    hq, hkv = 28, 4
    if case == "batch80_fixed_chunks":
        lens = torch.randint(1, 400, (80,), generator=g)
        lens[3], lens[50] = 5200, 5121
    elif case == "one_long_capped":
        lens = torch.tensor([0, 20000, 31, 32, 33])
    elif case == "batch64_all_lanes":
        lens = torch.randint(0, 700, (64,), generator=g)
    else:
        hq, hkv = 4, 1
        lens = torch.randint(100, 3000, (20,), generator=g)
    B, D, Sq = len(lens), 128, 8
    max_s = int(lens.max())
    q = torch.randn(B, Sq, hq, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, max_s, hkv, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, max_s, hkv, D, generator=g).to(torch.bfloat16)
    sl = lens.to(torch.int32)
    print(f"case partition {case} balanced={balanced} B={B} max_len={max_s}", flush=True)
    if case == "batch80_fixed_chunks":
        # a split call with few sequences first fills the workspace right after the
        # counter region; the 320 counters of this call must not read those partials
        small = workloads.kv_decode_paged(seed=9, batch=4, min_prefix=2048, max_prefix=4096)
        ops.block_attn(small.q.to(gpu), small.k_pool.to(gpu), small.v_pool.to(gpu), small.seqlens.to(gpu),
                       small.scale, page_table=small.page_table.to(gpu), page_size=small.page_size)
    out = ops.block_attn(q.to(gpu), k.to(gpu), v.to(gpu), sl.to(gpu), balanced_splits=balanced)
    _check(out, oa.attention_np(q.float(), k.float(), v.float(), sl))


@pytest.mark.parametrize("case", ["many_short", "fewer_pairs_than_slots", "empty_runs", "all_empty",
                                  "block_causal_qstart", "head_major_pages", "fp16_contig_bhsd", "gqa1_q64"])
def test_balanced_decode_runs(gpu, case):
    """The balanced split decode kernel (opt-in): runs of quads that cross sequence boundaries.
    many_short: 64 sequences of 0-200 keys, so one workgroup's run spans many sequences
    (more pieces than query blocks staged at the start); fewer_pairs_than_slots: 3
    sequences of 1-2 pairs (only P of the slots work); empty_runs: empty sequences
    between long ones; all_empty: every sequence empty (zero rows); block_causal_qstart:
    the block-causal mask with explicit query starts; head_major_pages: a page pool stored
    head-major; fp16_contig_bhsd: fp16 over a head-major contiguous cache; gqa1_q64: 64
    query rows of one head per KV head. Each against the float64 oracle, and against the
    default per-sequence splits (checked against the oracle too) within the same bound."""
    g = torch.Generator().manual_seed(sum(map(ord, case)))
    hq, hkv, Sq, D, dtype = 28, 4, 8, 128, torch.bfloat16
    mode, qst, pt, page = _ffi.MASK_SEQLEN, None, None, 0
    if case == "many_short":
        lens = torch.randint(0, 201, (64,), generator=g)
    elif case == "fewer_pairs_than_slots":
        lens = torch.tensor([10, 64, 100])
    elif case == "empty_runs":
        lens = torch.tensor([3000, 0, 0, 2048, 0, 1, 4100, 0])
    elif case == "all_empty":
        lens = torch.zeros(5, dtype=torch.int64)
    elif case == "block_causal_qstart":
        lens = torch.randint(500, 3000, (12,), generator=g)
        mode = _ffi.MASK_BLOCK_CAUSAL
        qst = (lens - Sq - torch.randint(0, 40, (12,), generator=g)).clamp(min=0).to(torch.int32)
    elif case == "head_major_pages":
        lens = None
    elif case == "fp16_contig_bhsd":
        lens, dtype = torch.randint(1, 2500, (16,), generator=g), torch.float16
    else:
        hq, hkv, Sq = 4, 4, 64
        lens = torch.randint(1, 1500, (10,), generator=g)
    if case == "head_major_pages":
        wl = workloads.kv_decode_paged(seed=3, batch=16, head_major=True)
        q, k, v, sl, pt, page = wl.q, wl.k_pool, wl.v_pool, wl.seqlens, wl.page_table, wl.page_size
        assert k.stride(1) == D and k.stride(2) == page * D  # one KV head's page is one contiguous run
        exp = oa.attention_np(q.float(), k.float(), v.float(), sl, wl.scale, page_table=pt, page_size=page)
    else:
        B = len(lens)
        max_s = max(1, int(lens.max()))
        q = torch.randn(B, Sq, hq, D, generator=g).to(dtype)
        k = torch.randn(B, max_s, hkv, D, generator=g).to(dtype)
        v = torch.randn(B, max_s, hkv, D, generator=g).to(dtype)
        if case == "fp16_contig_bhsd":
            k = k.permute(0, 2, 1, 3).contiguous().permute(0, 2, 1, 3)
            v = v.permute(0, 2, 1, 3).contiguous().permute(0, 2, 1, 3)
        sl = lens.to(torch.int32)
        exp = oa.attention_np(q.float(), k.float(), v.float(), sl, mask_mode=mode, mask_block=32, q_start=qst)
    print(f"case balanced decode {case} B={q.shape[0]} lens={sl.tolist()}", flush=True)
    args = dict(mask_mode=mode, mask_block=32, q_start=None if qst is None else qst.to(gpu),
                page_table=None if pt is None else pt.to(gpu), page_size=page)
    kd, vd = k.to(gpu), v.to(gpu)
    assert kd.stride() == k.stride() and vd.stride() == v.stride()  # the copy keeps the storage order
    out = ops.block_attn(q.to(gpu), kd, vd, sl.to(gpu), balanced_splits=True, **args)
    _check(out, exp)
    ref = ops.block_attn(q.to(gpu), kd, vd, sl.to(gpu), **args)
    _check(out, ref.float().cpu().numpy())
    _check(ref, exp)
    if case == "all_empty":
        assert torch.count_nonzero(out) == 0 and torch.count_nonzero(ref) == 0
    # a second call re-arms the arrival counters: identical output
    again = ops.block_attn(q.to(gpu), kd, vd, sl.to(gpu), balanced_splits=True, **args)
    assert torch.equal(out, again)


@pytest.mark.parametrize("batch,page_size", [(16, 32), (40, 16)])
def test_split_decode_page_table_staging(gpu, batch, page_size):
    """Paged split decode with a page table small enough to be read whole at the start
    (16 x 130 ids) and one too large for that (40 x 250 ids), which stages only the
    workgroup's own page ids."""
    wl = workloads.kv_decode_paged(seed=11, batch=batch, min_prefix=1024, max_prefix=3968, page_size=page_size)
    print(f"case page table {tuple(wl.page_table.shape)}", flush=True)
    out = ops.block_attn(wl.q.to(gpu), wl.k_pool.to(gpu), wl.v_pool.to(gpu), wl.seqlens.to(gpu), wl.scale,
                         page_table=wl.page_table.to(gpu), page_size=page_size)
    _check(out, oa.attention_np(wl.q.float(), wl.k_pool.float(), wl.v_pool.float(), wl.seqlens, wl.scale,
                                page_table=wl.page_table, page_size=page_size))


def test_fp32_split_counters_rearm_under_graph_replay(gpu):
    """The fp32 kernel's key splits are merged by each row block's last split to arrive,
    which resets the row block's arrival counter: after the call every counter reads zero,
    and a captured call replayed several times (eager fp32 calls of another shape in
    between, on the same workspace) matches the eager result on every replay."""
    wl = workloads.kv_decode_fp32_small(seed=0)
    q, k, v, sl = wl.q.to(gpu), wl.k_cache.to(gpu), wl.v_cache.to(gpu), wl.seqlens.to(gpu)
    g = torch.Generator().manual_seed(23)
    oq = torch.randn(2, 16, 8, 64, generator=g).to(gpu)
    ok = torch.randn(2, 400, 2, 64, generator=g).to(gpu)
    ov = torch.randn(2, 400, 2, 64, generator=g).to(gpu)
    osl = torch.tensor([400, 250], dtype=torch.int32).to(gpu)

    def call():
        return ops.block_attn(q, k, v, sl, wl.scale)

    def other_call():
        return ops.block_attn(oq, ok, ov, osl, None, mask_mode=_ffi.MASK_CAUSAL)

    eager = call()
    _check(eager, oa.attention_np(wl.q.float(), wl.k_cache.float(), wl.v_cache.float(), wl.seqlens, wl.scale),
           atol=1e-5, rtol=1e-5)
    other_eager = other_call()
    _check(other_eager, oa.attention_np(oq.cpu(), ok.cpu(), ov.cpu(), osl.cpu(), mask_mode=_ffi.MASK_CAUSAL),
           atol=1e-5, rtol=1e-5)
    torch.cuda.synchronize(gpu)
    ws = ops._WORKSPACE.get(0, gpu)
    assert int(ws[:64 * 1024].view(torch.int32).abs().sum()) == 0, "arrival counters not reset"
    s = torch.cuda.Stream(gpu)
    s.wait_stream(torch.cuda.current_stream(gpu))
    with torch.cuda.stream(s):
        call()  # workspace for this stream exists before capture
        torch.cuda.synchronize(gpu)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            out = call()
    torch.cuda.current_stream(gpu).wait_stream(s)
    for _ in range(4):
        graph.replay()
        torch.cuda.synchronize(gpu)
        assert torch.equal(out, eager)
        assert torch.equal(other_call(), other_eager)
        torch.cuda.synchronize(gpu)


def test_split_decode_counters_rearm_under_graph_replay(gpu):
    """The split decode kernel's last workgroup per KV head merges the partials and
    resets that head's arrival counter: after every call the counters read zero, and a
    captured call replayed several times (eager calls of another size in between)
    matches the eager result on every replay."""
    wl = workloads.kv_decode_paged(seed=6, batch=16, min_prefix=2048, max_prefix=4096)
    q, kp, vp = wl.q.to(gpu), wl.k_pool.to(gpu), wl.v_pool.to(gpu)
    pt, sl = wl.page_table.to(gpu), wl.seqlens.to(gpu)
    other = workloads.kv_decode_paged(seed=7, batch=3, min_prefix=700, max_prefix=3000)
    oq, okp, ovp = other.q.to(gpu), other.k_pool.to(gpu), other.v_pool.to(gpu)
    opt, osl = other.page_table.to(gpu), other.seqlens.to(gpu)

    def call():
        return ops.block_attn(q, kp, vp, sl, wl.scale, page_table=pt, page_size=wl.page_size)

    def other_call():
        return ops.block_attn(oq, okp, ovp, osl, other.scale, page_table=opt, page_size=other.page_size)

    eager = call()
    _check(eager, oa.attention_np(wl.q.float(), wl.k_pool.float(), wl.v_pool.float(), wl.seqlens, wl.scale,
                                  page_table=wl.page_table, page_size=wl.page_size))
    other_eager = other_call()
    torch.cuda.synchronize(gpu)
    units = q.shape[0] * kp.shape[2]
    ws = ops._WORKSPACE.get(0, gpu)
    assert int(ws[:4 * units].view(torch.int32).abs().sum()) == 0, "arrival counters not reset"
    s = torch.cuda.Stream(gpu)
    s.wait_stream(torch.cuda.current_stream(gpu))
    with torch.cuda.stream(s):
        call()  # workspace for this stream exists before capture
        torch.cuda.synchronize(gpu)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            out = call()
    torch.cuda.current_stream(gpu).wait_stream(s)
    for _ in range(4):
        graph.replay()
        torch.cuda.synchronize(gpu)
        assert torch.equal(out, eager)
        assert torch.equal(other_call(), other_eager)
        torch.cuda.synchronize(gpu)


def test_workspace_growth_keeps_captured_graph_valid(gpu):
    """A graph captured with a sub-block decode call keeps the stream's workspace
    address; a later, larger full-block call on the same stream grows the workspace.
    The old buffer must stay allocated (never handed back to the allocator), so every
    replay after the growth is still bit-identical to the eager result."""
    small = workloads.kv_decode_paged(seed=10, batch=4, min_prefix=1024, max_prefix=2048)
    big = workloads.kv_decode_paged(seed=11, batch=16, active=32)
    sq, skp, svp = small.q.to(gpu), small.k_pool.to(gpu), small.v_pool.to(gpu)
    spt, ssl = small.page_table.to(gpu), small.seqlens.to(gpu)
    bq, bkp, bvp = big.q.to(gpu), big.k_pool.to(gpu), big.v_pool.to(gpu)
    bpt, bsl = big.page_table.to(gpu), big.seqlens.to(gpu)
    print("case workspace growth: graph B=4 sub-block, eager B=16 full block", flush=True)

    def small_call():
        return ops.block_attn(sq, skp, svp, ssl, small.scale, page_table=spt, page_size=small.page_size)

    def big_call():
        return ops.block_attn(bq, bkp, bvp, bsl, big.scale, page_table=bpt, page_size=big.page_size)

    s = torch.cuda.Stream(gpu)
    s.wait_stream(torch.cuda.current_stream(gpu))
    with torch.cuda.stream(s):
        eager = small_call()  # creates this stream's (small) workspace
        torch.cuda.synchronize(gpu)
        ws_small = ops._WORKSPACE.get(0, gpu).data_ptr()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            out = small_call()
        big_eager = big_call()  # grows the workspace of the same stream
        torch.cuda.synchronize(gpu)
        assert ops._WORKSPACE.get(0, gpu).data_ptr() != ws_small, "the full-block call did not grow the workspace"
        # churn the caching allocator: a freed workspace would be handed out here
        junk = [torch.full((1 << 20,), 7, dtype=torch.uint8, device=gpu) for _ in range(8)]
        for _ in range(4):
            graph.replay()
            assert torch.equal(big_call(), big_eager)
            torch.cuda.synchronize(gpu)
            assert torch.equal(out, eager)
        del junk
    torch.cuda.current_stream(gpu).wait_stream(s)
    _check(eager, oa.attention_np(small.q.float(), small.k_pool.float(), small.v_pool.float(), small.seqlens,
                                  small.scale, page_table=small.page_table, page_size=small.page_size))


def test_workspace_reuse_across_shapes(gpu):
    """One workspace serves consecutive split calls of different sizes: a large call
    after a small one must not merge partials the small call left behind."""
    small = workloads.kv_decode_paged(seed=4, batch=2, min_prefix=512, max_prefix=1024)
    ops.block_attn(small.q.to(gpu), small.k_pool.to(gpu), small.v_pool.to(gpu), small.seqlens.to(gpu),
                   small.scale, page_table=small.page_table.to(gpu), page_size=small.page_size, kv_split=64)
    wl = workloads.block_prefill(seed=0, batch=2, seq_len=512)
    B, S, Hkv, D = wl.k.shape
    kc = torch.zeros(B, 1024, Hkv, D, dtype=torch.bfloat16, device=gpu)
    vc = torch.zeros_like(kc)
    kc[:, :S] = wl.k.to(gpu)
    vc[:, :S] = wl.v.to(gpu)
    sl = torch.full((B,), S, dtype=torch.int32, device=gpu)
    exp = oa.sdpa_block_causal(wl.q.float(), wl.k.float(), wl.v.float(), wl.block).numpy()
    for split in (64, 256, 0):
        out = ops.block_attn(wl.q.to(gpu), kc, vc, sl, wl.scale, mask_mode=_ffi.MASK_BLOCK_CAUSAL,
                             mask_block=wl.block, kv_split=split)
        _check(out, exp)


@pytest.mark.parametrize("page_size", [16, 64, 256])
def test_page_sizes(gpu, page_size):
    wl = workloads.kv_decode_paged(seed=5, batch=5, min_prefix=96, max_prefix=1500, page_size=page_size)
    print(f"case page_size={page_size} lens={wl.seqlens.tolist()}", flush=True)
    for split in (0, 128):
        out = ops.block_attn(wl.q.to(gpu), wl.k_pool.to(gpu), wl.v_pool.to(gpu), wl.seqlens.to(gpu), wl.scale,
                             page_table=wl.page_table.to(gpu), page_size=page_size, kv_split=split)
        exp = oa.attention_np(wl.q.float(), wl.k_pool.float(), wl.v_pool.float(), wl.seqlens, wl.scale,
                              page_table=wl.page_table, page_size=page_size)
        _check(out, exp)


def test_bad_page_size_rejected(gpu):
    wl = workloads.kv_decode_paged(seed=5, batch=2, min_prefix=96, max_prefix=200, page_size=48)
    with pytest.raises(RuntimeError, match="page_size"):
        ops.block_attn(wl.q.to(gpu), wl.k_pool.to(gpu), wl.v_pool.to(gpu), wl.seqlens.to(gpu), wl.scale,
                       page_table=wl.page_table.to(gpu), page_size=48)


@pytest.mark.parametrize("hq,hkv,q_len", [(28, 4, 8), (28, 4, 1), (8, 8, 8), (16, 2, 32), (4, 1, 64), (32, 8, 4)])
@pytest.mark.parametrize("paged", [False, True])
def test_decode_kernel_vs_general(gpu, hq, hkv, q_len, paged):
    """Split-KV decode kernel, all-heads decode kernel and the general kernel agree with the
    oracle (and each other) across KV-head counts, rows per head up to 64, ragged lengths
    and split sizes."""
    g = torch.Generator().manual_seed(hq * 100 + hkv * 10 + q_len + paged)
    B, D = 5, 128
    if paged:
        wl = workloads.kv_decode_paged(seed=hq + hkv, batch=B, num_q_heads=hq, num_kv_heads=hkv,
                                       min_prefix=32, max_prefix=1600, active=q_len, page_size=64)
        q, kc, vc, sl, pt, ps = wl.q, wl.k_pool, wl.v_pool, wl.seqlens, wl.page_table, 64
        exp = oa.attention_np(q.float(), kc.float(), vc.float(), sl, page_table=pt, page_size=ps)
    else:
        max_s = 1700
        q = torch.randn(B, q_len, hq, D, generator=g).to(torch.bfloat16)
        kc = torch.randn(B, max_s, hkv, D, generator=g).to(torch.bfloat16)
        vc = torch.randn(B, max_s, hkv, D, generator=g).to(torch.bfloat16)
        sl = torch.tensor([1700, 33, 1, 640, 1299], dtype=torch.int32)
        pt, ps = None, 0
        exp = oa.attention_np(q.float(), kc.float(), vc.float(), sl)
    print(f"case decode-vs-general {hq}/{hkv} q_len={q_len} paged={paged}", flush=True)
    args = dict(page_table=pt.to(gpu) if pt is not None else None, page_size=ps)
    outs = []
    for split in (0, 64, 1 << 16):
        for dec, allh in ((True, False), (True, True), (False, False)):
            o = ops.block_attn(q.to(gpu), kc.to(gpu), vc.to(gpu), sl.to(gpu), kv_split=split, decode_kernel=dec,
                               all_heads_decode=allh, **args)
            _check(o, exp)
            outs.append(o.float().cpu())
    for o in outs[1:]:
        torch.testing.assert_close(o, outs[0], atol=2e-2, rtol=2e-2)


def _paginate(k, v, page_size, g):
    """Contiguous [B, S, Hkv, D] caches -> a shuffled page pool and its page table."""
    B, S, Hkv, D = k.shape
    per = (S + page_size - 1) // page_size
    perm = torch.randperm(B * per, generator=g)
    kp = torch.zeros(B * per, page_size, Hkv, D, dtype=k.dtype)
    vp = torch.zeros_like(kp)
    pt = torch.zeros(B, per, dtype=torch.int32)
    for b in range(B):
        for i in range(per):
            pg = int(perm[b * per + i])
            pt[b, i] = pg
            n = min(page_size, S - i * page_size)
            kp[pg, :n] = k[b, i * page_size:i * page_size + n]
            vp[pg, :n] = v[b, i * page_size:i * page_size + n]
    return kp, vp, pt


@pytest.mark.parametrize("layout", ["fused_qkv_slice", "heads_outer"])
@pytest.mark.parametrize("case", ["sub_block", "full_block", "prefill"])
def test_strided_query_rows(gpu, case, layout):
    """Query rows read through their strides: a slice of a fused q / k / v projection
    ([B, S, Hq + 8, D] cut to its first Hq heads) or a [B, H, S, D] tensor seen as
    [B, S, H, D]. The split decode kernel loads them per lane; the split prefill
    (full-block) and prefill kernels without a cache write load them straight into LDS
    through a descriptor over the sequence's rows. Against the oracle on the same values,
    and the general kernel on the same call."""
    g = torch.Generator().manual_seed(sum(map(ord, case + layout)))
    if case in ("sub_block", "full_block"):
        wl = workloads.kv_decode_paged(seed=7, batch=4, active=8 if case == "sub_block" else 32)
        q0, kc, vc, sl, scale = wl.q, wl.k_pool, wl.v_pool, wl.seqlens, wl.scale
        args = dict(page_table=wl.page_table.to(gpu), page_size=wl.page_size)
        exp = oa.attention_np(q0.float(), kc.float(), vc.float(), sl, scale, page_table=wl.page_table,
                              page_size=wl.page_size)
    else:  # 300 queries x GQA 7 = 2100 rows per KV head: the prefill kernel, block-causal
        B, Sq, hq, hkv, lens = 1, 300, 28, 4, [700]
        q0 = torch.randn(B, Sq, hq, 128, generator=g).to(torch.bfloat16)
        kc = torch.randn(B, max(lens), hkv, 128, generator=g).to(torch.bfloat16)
        vc = torch.randn(B, max(lens), hkv, 128, generator=g).to(torch.bfloat16)
        sl = torch.tensor(lens, dtype=torch.int32)
        scale = None
        args = dict(mask_mode=_ffi.MASK_BLOCK_CAUSAL, mask_block=32)
        exp = oa.attention_np(q0.float(), kc.float(), vc.float(), sl, mask_mode=_ffi.MASK_BLOCK_CAUSAL,
                              mask_block=32)
    B, Sq, Hq, D = q0.shape
    if layout == "fused_qkv_slice":
        big = torch.randn(B, Sq, Hq + 8, D, generator=g).to(q0.dtype)
        big[:, :, :Hq] = q0
        q = big.to(gpu)[:, :, :Hq]
        assert q.stride(1) == (Hq + 8) * D and q.stride(2) == D
    else:
        q = q0.transpose(1, 2).contiguous().to(gpu).transpose(1, 2)
        assert q.stride(1) == D and q.stride(2) == Sq * D
    print(f"case strided query {case} {layout}", flush=True)
    for dk in (True, False):
        out = ops.block_attn(q, kc.to(gpu), vc.to(gpu), sl.to(gpu), scale, decode_kernel=dk, **args)
        _check(out, exp)


@pytest.mark.parametrize("case", [
    "gqa7_block_causal_prefix",   # 28/4 heads, cached prefix + new rows, block-causal
    "gqa7_fp16_paged64",          # the same in fp16 over 64-key pages
    "gqa7_paged32",               # 32-key pages: two pages per 64-key tile
    "gqa7_paged16",               # 16-key pages: the general kernel takes the call
    "mha_causal_paged256",        # 8/8 heads (G = 1), causal, 256-key pages
    "gqa8_full_ragged",           # 16/2 heads, every key visible, ragged lengths
    "gqa4_block64_one_head",      # 4/1 heads, 64-key blocks
])
def test_prefill_kernel(gpu, case):
    """The prefill kernel (>= 2048 query rows per KV head) against the float64 oracle
    across head groupings, masks, dtypes, paging, cached prefixes and row counts that
    are not multiples of its 256-row blocks."""
    g = torch.Generator().manual_seed(sum(map(ord, case)))
    dtype, page, mode, blk = torch.bfloat16, 0, _ffi.MASK_BLOCK_CAUSAL, 32
    if case == "gqa7_block_causal_prefix":
        B, Sq, hq, hkv, lens = 2, 300, 28, 4, [812, 300]
    elif case == "gqa7_fp16_paged64":
        B, Sq, hq, hkv, lens, dtype, page = 2, 300, 28, 4, [812, 333], torch.float16, 64
    elif case == "gqa7_paged32":
        B, Sq, hq, hkv, lens, page = 2, 300, 28, 4, [700, 333], 32
    elif case == "gqa7_paged16":
        B, Sq, hq, hkv, lens, page = 2, 300, 28, 4, [700, 333], 16
    elif case == "mha_causal_paged256":
        B, Sq, hq, hkv, lens, mode, page = 1, 2100, 8, 8, [2400], _ffi.MASK_CAUSAL, 256
    elif case == "gqa8_full_ragged":
        B, Sq, hq, hkv, lens, mode = 2, 600, 16, 2, [900, 650], _ffi.MASK_SEQLEN
    else:
        B, Sq, hq, hkv, lens, blk = 1, 1000, 4, 1, [1000], 64
    D, max_s = 128, max(lens)
    q = torch.randn(B, Sq, hq, D, generator=g).to(dtype)
    k = torch.randn(B, max_s, hkv, D, generator=g).to(dtype)
    v = torch.randn(B, max_s, hkv, D, generator=g).to(dtype)
    sl = torch.tensor(lens, dtype=torch.int32)
    print(f"case prefill {case}", flush=True)
    if page:
        kc, vc, pt = _paginate(k, v, page, g)
        args = dict(page_table=pt.to(gpu), page_size=page)
    else:
        kc, vc, args = k, v, {}
    exp = oa.attention_np(q.float(), k.float(), v.float(), sl, mask_mode=mode, mask_block=blk)
    for prefill in (True, False):  # False: the general kernel on the same call
        out = ops.block_attn(q.to(gpu), kc.to(gpu), vc.to(gpu), sl.to(gpu), mask_mode=mode, mask_block=blk,
                             decode_kernel=prefill, **args)
        _check(out, exp)


def test_split_prefill_merge_under_graph_replay(gpu):
    """Full-block calls (32 active queries): the split kernel writes each (sequence, KV
    head)'s slots and split count on every call for the merge kernel. Eager calls of
    two batch sizes in turn on one workspace (a different table at a different offset
    each time) keep their results, and a captured call replayed several times, with
    those eager calls in between, matches the eager result on every replay."""
    wl = workloads.kv_decode_paged(seed=8, batch=16, active=32)
    q, kp, vp = wl.q.to(gpu), wl.k_pool.to(gpu), wl.v_pool.to(gpu)
    pt, sl = wl.page_table.to(gpu), wl.seqlens.to(gpu)
    other = workloads.kv_decode_paged(seed=9, batch=5, active=32, min_prefix=200, max_prefix=3500)
    oq, okp, ovp = other.q.to(gpu), other.k_pool.to(gpu), other.v_pool.to(gpu)
    opt, osl = other.page_table.to(gpu), other.seqlens.to(gpu)
    print("case full-block graph replay B=16 / eager B=5", flush=True)

    def call():
        return ops.block_attn(q, kp, vp, sl, wl.scale, page_table=pt, page_size=wl.page_size)

    def other_call():
        return ops.block_attn(oq, okp, ovp, osl, other.scale, page_table=opt, page_size=other.page_size)

    eager = call()
    _check(eager, oa.attention_np(wl.q.float(), wl.k_pool.float(), wl.v_pool.float(), wl.seqlens, wl.scale,
                                  page_table=wl.page_table, page_size=wl.page_size))
    other_eager = other_call()
    _check(other_eager, oa.attention_np(other.q.float(), other.k_pool.float(), other.v_pool.float(), other.seqlens,
                                        other.scale, page_table=other.page_table, page_size=other.page_size))
    assert torch.equal(call(), eager)
    s = torch.cuda.Stream(gpu)
    s.wait_stream(torch.cuda.current_stream(gpu))
    with torch.cuda.stream(s):
        call()  # workspace for this stream exists before capture
        torch.cuda.synchronize(gpu)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            out = call()
    torch.cuda.current_stream(gpu).wait_stream(s)
    for _ in range(4):
        graph.replay()
        torch.cuda.synchronize(gpu)
        assert torch.equal(out, eager)
        assert torch.equal(other_call(), other_eager)
        torch.cuda.synchronize(gpu)


@pytest.mark.parametrize("case", ["bs16_paged32", "ragged_contig", "fp16_paged64", "fixed_chunks", "gqa8_256_rows",
                                  "rows91_contig"])
def test_block_decode_split_prefill_kernel(gpu, case):
    """A whole 32-token block per step (64 < rows per KV head <= 256): the prefill
    kernel's math with split keys and the merge kernel that follows it, against the
    oracle and against the general kernel on the same call."""
    split, dtype, decode_args = 0, torch.bfloat16, {}
    if case == "bs16_paged32":
        wl = workloads.kv_decode_paged(seed=0, active=32)
    elif case == "fp16_paged64":
        wl = workloads.kv_decode_paged(seed=3, batch=6, active=32, page_size=64, dtype=torch.float16)
    elif case == "fixed_chunks":
        wl = workloads.kv_decode_paged(seed=4, batch=5, active=32)
        split = 128
    elif case == "gqa8_256_rows":
        wl = workloads.kv_decode_paged(seed=5, batch=3, num_q_heads=16, num_kv_heads=2, active=32)
    else:
        wl = None
    if wl is not None:
        q, kc, vc, sl = wl.q, wl.k_pool, wl.v_pool, wl.seqlens
        args = dict(page_table=wl.page_table.to(gpu), page_size=wl.page_size)
        exp = oa.attention_np(q.float(), kc.float(), vc.float(), sl, wl.scale, page_table=wl.page_table,
                              page_size=wl.page_size)
        scale = wl.scale
    else:
        g = torch.Generator().manual_seed(12)
        B, Sq, Hq, Hkv, D, S = 5, 32, 28, 4, 128, 3000
        if case == "rows91_contig":  # 13 queries x GQA 7: the merge's last 32-row chunk holds 27 rows
            Sq = 13
        q = torch.randn(B, Sq, Hq, D, generator=g).to(dtype)
        kc = torch.randn(B, S, Hkv, D, generator=g).to(dtype)
        vc = torch.randn(B, S, Hkv, D, generator=g).to(dtype)
        sl = torch.tensor([3000, 0, 1, 97, 2048], dtype=torch.int32)
        args, scale = {}, None
        exp = oa.attention_np(q.float(), kc.float(), vc.float(), sl)
    print(f"case block decode {case}", flush=True)
    for dk in (True, False):
        out = ops.block_attn(q.to(gpu), kc.to(gpu), vc.to(gpu), sl.to(gpu), scale, kv_split=split,
                             decode_kernel=dk, **args)
        _check(out, exp)


@pytest.mark.parametrize("case", [
    "prefill_q0_contig",        # 4 KV heads x 4200 rows: prefill kernel, every key new
    "prefix_paged32_mixed",     # cached prefix ending inside a 32-key half (per-lane sources)
    "prefix_paged64_fp16",      # fp16, 64-key pages, prefix on a page boundary
    "commit_split_paged32",     # a whole 32-token block per sequence: split prefill kernel
    "commit_split_misaligned",  # the same with prefixes that are not multiples of 32
    "short_visible_qstart",     # explicit q_start, new rows past the visible length
    "past_capacity",            # new rows past the cache's end are dropped
    "qstart_cache_past_new",    # explicit q_start, visible cache rows past the last new row
    "qstart_block_causal",      # explicit unaligned q_start, block-causal, cache rows past the new ones
    "subblock_fallback",        # 8 queries: split decode kernel, cache write kernel first
    "head64_fallback",          # head_dim 64: the general kernel, cache write kernel first
])
@pytest.mark.parametrize("in_kernel", [False, True])
def test_fused_cache_write(gpu, case, in_kernel):
    """k_new / v_new: the call stores the query tokens' K / V rows into the cache at
    q_start + t and attends over the updated cache, from inside the prefill kernels
    (in_kernel, where the shape has them and q_start is implicit) or by its copy kernel
    (FDLLM_ATTN_CACHE_WRITE_KERNEL, and every call with an explicit q_start). The cache must equal
    the oracle's write bit for bit, the output must equal the same call made as a
    separate cache write followed by the attention (bit for bit) and match the float64
    oracle over the written cache."""
    g = torch.Generator().manual_seed(sum(map(ord, case)))
    dtype, page, mode, blk, D, hq, hkv, explicit_qs = torch.bfloat16, 0, _ffi.MASK_BLOCK_CAUSAL, 32, 128, 28, 4, False
    if case == "prefill_q0_contig":
        B, Sq, qs, cap, lens = 2, 600, [0, 0], 700, None
    elif case == "prefix_paged32_mixed":
        B, Sq, qs, cap, lens, page = 2, 400, [45, 130], 640, None, 32
    elif case == "prefix_paged64_fp16":
        B, Sq, qs, cap, lens, page, dtype = 2, 400, [64, 192], 640, None, 64, torch.float16
    elif case == "commit_split_paged32":
        B, Sq, qs, cap, lens, page = 5, 32, [1024, 64, 0, 2016, 320], 2112, None, 32
    elif case == "commit_split_misaligned":
        B, Sq, qs, cap, lens = 5, 32, [1000, 77, 5, 0, 2049], 2112, None
    elif case == "short_visible_qstart":
        B, Sq, qs, cap, lens, mode, explicit_qs = 2, 400, [96, 10], 600, [446, 330], _ffi.MASK_SEQLEN, True
    elif case == "past_capacity":
        B, Sq, qs, cap, lens, explicit_qs = 1, 600, [100], 650, [650], True
    elif case == "qstart_cache_past_new":
        # keys [q_start + Sq, seqlens) are cache rows this call does not write: they
        # must be read from the cache, not from the new rows of the next sequence
        B, Sq, qs, cap, lens, mode, explicit_qs = 3, 300, [40, 0, 257], 900, [440, 400, 657], _ffi.MASK_SEQLEN, True
    elif case == "qstart_block_causal":
        B, Sq, qs, cap, lens, page, explicit_qs = 2, 270, [45, 301], 960, [415, 700], 32, True
    elif case == "subblock_fallback":
        B, Sq, qs, cap, lens, page = 4, 8, [1000, 500, 64, 2047], 2112, None, 32
    else:
        B, Sq, qs, cap, lens, D, hq, hkv = 3, 300, [0, 33, 128], 512, None, 64, 8, 2
    if lens is None:
        lens = [q0 + Sq for q0 in qs]
    print(f"case fused cache write {case} in_kernel={in_kernel}", flush=True)
    q = torch.randn(B, Sq, hq, D, generator=g).to(dtype)
    kc0 = torch.randn(B, cap, hkv, D, generator=g).to(dtype)
    vc0 = torch.randn(B, cap, hkv, D, generator=g).to(dtype)
    kn = torch.randn(B, Sq, hkv, D, generator=g).to(dtype)
    vn = torch.randn(B, Sq, hkv, D, generator=g).to(dtype)
    sl = torch.tensor(lens, dtype=torch.int32)
    qst = torch.tensor(qs, dtype=torch.int32)
    if page:
        kp0, vp0, pt = _paginate(kc0, vc0, page, g)
        args = dict(page_table=pt.to(gpu), page_size=page)
    else:
        kp0, vp0, pt, args = kc0, vc0, None, {}
    exp_k = oa.cache_write_np(kp0.numpy() if dtype == torch.float16 else kp0.view(torch.int16).numpy(),
                              kn.numpy() if dtype == torch.float16 else kn.view(torch.int16).numpy(), qs,
                              page_table=pt, page_size=page or None, capacity=cap)
    exp_v = oa.cache_write_np(vp0.numpy() if dtype == torch.float16 else vp0.view(torch.int16).numpy(),
                              vn.numpy() if dtype == torch.float16 else vn.view(torch.int16).numpy(), qs,
                              page_table=pt, page_size=page or None, capacity=cap)
    qarg = dict(q_start=qst.to(gpu)) if explicit_qs else {}
    kf, vf = kp0.to(gpu), vp0.to(gpu)
    out = ops.block_attn(q.to(gpu), kf, vf, sl.to(gpu), mask_mode=mode, mask_block=blk, k_new=kn.to(gpu),
                         v_new=vn.to(gpu), cache_write_kernel=not in_kernel, **qarg, **args)
    as_np = (lambda t: t.cpu().numpy()) if dtype == torch.float16 else (lambda t: t.cpu().view(torch.int16).numpy())
    assert np.array_equal(as_np(kf), exp_k), "K cache differs from the oracle's write"
    assert np.array_equal(as_np(vf), exp_v), "V cache differs from the oracle's write"
    # the unfused statement: the cache write kernel, then the attention
    ku, vu = kp0.to(gpu), vp0.to(gpu)
    ops.kv_cache_write(kn.to(gpu), vn.to(gpu), ku, vu, write_start=qst.to(gpu), **args)
    ref = ops.block_attn(q.to(gpu), ku, vu, sl.to(gpu), mask_mode=mode, mask_block=blk, **qarg, **args)
    assert torch.equal(ku, kf) and torch.equal(vu, vf)
    assert torch.equal(out, ref), "fused call differs from write + attention"
    kx = torch.from_numpy(exp_k).view(dtype) if dtype != torch.float16 else torch.from_numpy(exp_k)
    vx = torch.from_numpy(exp_v).view(dtype) if dtype != torch.float16 else torch.from_numpy(exp_v)
    _check(out, oa.attention_np(q.float(), kx.float(), vx.float(), torch.clamp(sl, max=cap), mask_mode=mode,
                                mask_block=blk, q_start=qst, page_table=pt, page_size=page or None))


@pytest.mark.parametrize("B", [16000, 20000])
@pytest.mark.parametrize("paged", [False, True])
def test_large_batch_grid(gpu, B, paged):
    """Thousands of sequences of one KV head (q_len 1, 0-96 visible keys). 16000: more
    sequences than the per-sequence partition takes, so the split decode kernel runs with
    fixed chunks on a grid whose third dimension is the batch; 20000: more (sequence, KV
    head) pairs than the split kernel's arrival counters, so the all-heads decode kernel
    takes the call on a grid whose second dimension is the batch. Within the bars of the
    float64 oracle on a sample of 400 sequences; an empty sequence gives zero rows."""
    print(f"case large batch B={B} paged={paged}", flush=True)
    g = torch.Generator().manual_seed(23 + B)
    Sq, Hq, Hkv, D, S = 1, 2, 1, 128, 96
    q = torch.randn(B, Sq, Hq, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, S, Hkv, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, S, Hkv, D, generator=g).to(torch.bfloat16)
    seqlens = torch.randint(0, S + 1, (B,), generator=g, dtype=torch.int32)
    seqlens[:3] = torch.tensor([0, 1, S], dtype=torch.int32)
    if paged:
        kp, vp, pt = _paginate(k, v, 32, g)
        out = ops.block_attn(q.to(gpu), kp.to(gpu), vp.to(gpu), seqlens.to(gpu), page_table=pt.to(gpu),
                             page_size=32).cpu()
    else:
        out = ops.block_attn(q.to(gpu), k.to(gpu), v.to(gpu), seqlens.to(gpu)).cpu()
    assert torch.count_nonzero(out[0]) == 0
    # the oracle on a sample of the sequences (the kernel's grid covers all of them)
    sel = torch.cat([torch.arange(3), torch.randperm(B - 3, generator=g)[:397] + 3])
    exp = oa.attention_np(q[sel].float(), k[sel].float(), v[sel].float(), seqlens[sel])
    _check(out[sel], exp)


def _poison_paged(pool: torch.Tensor, page_table: torch.Tensor, seqlens: torch.Tensor, page_size: int,
                  extra_pages: int, fill: float) -> torch.Tensor:
    """The pool with `extra_pages` unreferenced pages appended and every (page, slot) that
    no sequence sees (past its length, or on a page no table entry names) set to `fill`."""
    P = pool.shape[0]
    out = torch.cat([pool, torch.zeros((extra_pages,) + tuple(pool.shape[1:]), dtype=pool.dtype)])
    seen = torch.zeros(P + extra_pages, page_size, dtype=torch.bool)
    for b in range(page_table.shape[0]):
        n = int(seqlens[b])
        for j in range(0, n, page_size):
            seen[int(page_table[b, j // page_size]), : min(page_size, n - j)] = True
    out[~seen] = fill
    return out


@pytest.mark.parametrize("case", ["paged_subblock", "paged_full_block", "static_split", "static_general",
                                  "block_causal_prefill", "fp32"])
def test_unread_rows_poisoned_with_nan(gpu, case):
    """Keys past each sequence's visible length have no influence (the invariant the reference's
    SDPA shim states with its -inf mask, tests/test_focus.py:220-224): every K/V row that no
    query may see (slots past the length, unreferenced pages, static-cache rows past the
    length) is set to NaN, and the output must be bit for bit the output with zeros there,
    on every kernel family the dispatcher picks (split decode, full-block ring split, static
    cache split and general kernels, block-causal prefill ring, fp32)."""
    print(f"case poisoned rows {case}", flush=True)
    nan = float("nan")
    if case.startswith("paged"):
        wl = workloads.kv_decode_paged(seed=41, batch=16, active=8 if case == "paged_subblock" else 32)
        sl = wl.seqlens.clone()
        sl[::3] -= 7  # partial last pages
        outs = []
        for fill in (0.0, nan):
            kp = _poison_paged(wl.k_pool, wl.page_table, sl, wl.page_size, 3, fill)
            vp = _poison_paged(wl.v_pool, wl.page_table, sl, wl.page_size, 3, fill)
            outs.append(ops.block_attn(wl.q.to(gpu), kp.to(gpu), vp.to(gpu), sl.to(gpu), wl.scale,
                                       page_table=wl.page_table.to(gpu), page_size=wl.page_size).cpu())
        exp = oa.attention_np(wl.q.float(), wl.k_pool.float(), wl.v_pool.float(), sl, wl.scale,
                              page_table=wl.page_table, page_size=wl.page_size)
    else:
        g = torch.Generator().manual_seed(43)
        dt = torch.float32 if case == "fp32" else torch.bfloat16
        if case == "block_causal_prefill":
            B, Sq, Hq, Hkv, S = 2, 512, 28, 4, 640
            sl = torch.tensor([512, 576], dtype=torch.int32)  # queries at positions sl - 512 ..
        elif case == "fp32":
            B, Sq, Hq, Hkv, S = 1, 32, 12, 2, 600
            sl = torch.tensor([544], dtype=torch.int32)
        else:
            B, Sq, Hq, Hkv, S = 6, 8, 28, 4, 1500
            sl = torch.tensor([1, 31, 33, 700, 1029, 1400], dtype=torch.int32)
        q = torch.randn(B, Sq, Hq, 128, generator=g).to(dt)
        k = torch.randn(B, S, Hkv, 128, generator=g).to(dt)
        v = torch.randn(B, S, Hkv, 128, generator=g).to(dt)
        kw = {}
        if case == "block_causal_prefill":
            kw = dict(mask_mode=_ffi.MASK_BLOCK_CAUSAL, mask_block=32)
        elif case == "static_general":
            kw = dict(decode_kernel=False, kv_split=64)
        outs = []
        for fill in (0.0, nan):
            kc, vc = k.clone(), v.clone()
            for b in range(B):
                kc[b, int(sl[b]):] = fill
                vc[b, int(sl[b]):] = fill
            outs.append(ops.block_attn(q.to(gpu), kc.to(gpu), vc.to(gpu), sl.to(gpu), **kw).cpu())
        if case == "block_causal_prefill":
            exp = None  # the block-causal kernel's values are checked elsewhere; here only the invariant
        else:
            exp = oa.attention_np(q.float(), k.float(), v.float(), sl)
    torch.cuda.synchronize()
    assert torch.isfinite(outs[1]).all(), "NaN from an unread row reached the output"
    assert torch.equal(outs[0], outs[1]), "rows past the visible lengths changed the output"
    if exp is not None:
        _check(outs[0], exp)
