"""GPU parity of the gather + RMSNorm kernels against the oracle.

Cases: the reference's own case table (cuda_bench/test_correctness.py:129-144,
indices drawn with replacement, unit weight), the gather+RMSNorm workload at
full size (bf16 [4096 x 3584], 1024 distinct rows, weight ~ N(1, 0.02)), every
norm mode, fp16, odd hidden sizes (generic path), strided hidden, out-of-range
indices, empty inputs.

Bars: gathered rows bit-exact; normalised rows within atol = rtol = 1e-2, and
within one bf16 ulp of the oracle (two in the weight-after-cast order, whose
intermediate bf16 rounding can land on the neighbouring value when the sum of
squares is accumulated in a different order).
"""
import numpy as np
import pytest
import torch

from fast_v2_amd import ops, workloads
from fast_v2_amd import _ffi
from fast_v2_amd.cuda_bench import fused_sparse_extension as fse
from oracle import gather_rmsnorm as og

pytestmark = pytest.mark.gpu

ATOL = RTOL = 1e-2


def _ulp_diff_bf16(a: torch.Tensor, b: torch.Tensor) -> int:
    ai = a.contiguous().view(torch.int16).to(torch.int32).cpu()
    bi = b.contiguous().view(torch.int16).to(torch.int32).cpu()
    # map sign-magnitude to a monotone integer line
    ai = torch.where(ai < 0, -(ai & 0x7FFF), ai)
    bi = torch.where(bi < 0, -(bi & 0x7FFF), bi)
    return int((ai - bi).abs().max()) if ai.numel() else 0


class _Norm(torch.nn.Module):
    def __init__(self, w, eps):
        super().__init__()
        self.weight = torch.nn.Parameter(w)
        self.variance_epsilon = eps


REF_CASES = [
    # (B, S, H, T, eps, dtype)  cuda_bench/test_correctness.py:129-144
    (1, 64, 128, 7, 1e-6, torch.bfloat16),
    (2, 128, 256, 16, 1e-5, torch.bfloat16),
    (1, 512, 3584, 32, 1e-6, torch.bfloat16),
    (2, 256, 512, 24, 1e-6, torch.bfloat16),
    (1, 32, 64, 5, 1e-6, torch.float32),
    (3, 48, 96, 11, 1e-6, torch.float32),
    (1, 128, 512, 40, 1e-6, torch.float32),
]


@pytest.mark.parametrize("B,S,H,T,eps,dtype", REF_CASES)
def test_model_path_pair_reference_cases(gpu, B, S, H, T, eps, dtype):
    print(f"case B={B} S={S} H={H} T={T} {dtype}", flush=True)
    g = torch.Generator().manual_seed(0)
    hidden = torch.randn(B, S, H, generator=g).to(dtype)
    idx = torch.randint(0, S, (B, T), generator=g)
    w = torch.ones(H, dtype=dtype)
    ref_g, ref_n = og.ref_gather_input_rmsnorm(hidden, idx, w, eps)
    pair = fse.fused_gather_input_rmsnorm_pair(hidden.to(gpu), idx.to(gpu), _Norm(w.to(gpu), eps))
    assert pair is not None
    got_g, got_n = (t.cpu() for t in pair)
    assert got_g.dtype == dtype and got_n.dtype == dtype
    assert torch.equal(got_g, ref_g)
    torch.testing.assert_close(got_n.float(), ref_n.float(), atol=ATOL, rtol=RTOL)
    if dtype == torch.bfloat16:
        assert _ulp_diff_bf16(got_n, ref_n) <= 1


def test_full_size_rows_all_modes(gpu):
    wl = workloads.gather_rmsnorm_rows(seed=0)
    print("case gather_rmsnorm_rows 1x4096x3584 T=1024", flush=True)
    hid, idx, w = wl.hidden.to(gpu), wl.indices.to(gpu), wl.weight.to(gpu)
    h64 = wl.hidden.float().numpy()
    for mode in (og.NORM_PLAIN, og.NORM_WEIGHT_FP32, og.NORM_WEIGHT_AFTER_CAST):
        normed, gathered = ops.gather_rmsnorm(hid, idx, w, wl.eps, mode, with_gathered=True)
        exp_g, exp_n = og.gather_rmsnorm_np(h64, wl.indices.numpy(), wl.weight.float().numpy(), wl.eps,
                                            mode, "bf16")
        assert torch.equal(gathered.cpu(), wl.hidden[0, wl.indices[0]].unsqueeze(0))
        got = normed.float().cpu().numpy()
        np.testing.assert_allclose(got, exp_n, atol=ATOL, rtol=RTOL)
        # fp32 x*rsqrt in the kernel vs float64 in the oracle may round to neighbouring
        # bf16 values; in the weight-after-cast order that intermediate is rounded once
        # more after the product, so one step can become two.
        bound = 2 if mode == og.NORM_WEIGHT_AFTER_CAST else 1
        assert _ulp_diff_bf16(normed.cpu(), torch.from_numpy(exp_n).to(torch.bfloat16)) <= bound, mode
    # the torch restatement of the model path agrees too
    ref_g, ref_n = og.ref_gather_input_rmsnorm(wl.hidden, wl.indices, wl.weight, wl.eps)
    normed, gathered = ops.gather_rmsnorm(hid, idx, w, wl.eps, og.NORM_WEIGHT_AFTER_CAST, True)
    assert torch.equal(gathered.cpu(), ref_g)
    assert _ulp_diff_bf16(normed.cpu(), ref_n) <= 2


def test_reference_fp32_entry_points(gpu):
    """get_fused_ops() surface: gather_rmsnorm_cuda / fused_select_norm (weight in fp32)
    and fused_gather_input_rmsnorm_pair (no weight), fp32 as in the reference kernels."""
    g = torch.Generator().manual_seed(1)
    hidden = torch.randn(2, 100, 384, generator=g)
    idx = torch.randint(0, 100, (2, 17), generator=g)
    w = torch.randn(384, generator=g)
    ext = fse.get_fused_ops()
    assert ext is not None
    exp = og.ref_gather_rmsnorm_fp32w(hidden, idx, w, 1e-5)
    for fn in (ext.gather_rmsnorm_cuda, ext.fused_select_norm):
        got = fn(hidden.to(gpu), idx.to(gpu), w.to(gpu), 1e-5).cpu()
        torch.testing.assert_close(got, exp, atol=1e-5, rtol=1e-5)
    g_ref, n_ref = og.ref_gather_pair_plain(hidden, idx, 1e-6)
    g_got, n_got = ext.fused_gather_input_rmsnorm_pair(hidden.to(gpu), idx.to(gpu), 1e-6)
    assert torch.equal(g_got.cpu(), g_ref)
    torch.testing.assert_close(n_got.cpu(), n_ref, atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("H", [3584, 4096, 100, 1000, 8200, 2056, 8192, 2048])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_hidden_sizes_and_fp16(gpu, H, dtype):
    print(f"case H={H} {dtype}", flush=True)
    g = torch.Generator().manual_seed(H)
    hidden = (3 * torch.randn(2, 33, H, generator=g)).to(dtype)
    idx = torch.randint(0, 33, (2, 9), generator=g)
    w = (1 + 0.1 * torch.randn(H, generator=g)).to(dtype)
    normed, gathered = ops.gather_rmsnorm(hidden.to(gpu), idx.to(gpu), w.to(gpu), 1e-6,
                                          og.NORM_WEIGHT_AFTER_CAST, True)
    tag = "bf16" if dtype == torch.bfloat16 else "f16"
    exp_g, exp_n = og.gather_rmsnorm_np(hidden.float().numpy(), idx.numpy(), w.float().numpy(), 1e-6,
                                        og.NORM_WEIGHT_AFTER_CAST, tag)
    assert torch.equal(gathered.cpu(), torch.stack([hidden[b, idx[b]] for b in range(2)]))
    np.testing.assert_allclose(normed.float().cpu().numpy(), exp_n, atol=ATOL, rtol=RTOL)


@pytest.mark.parametrize("H,dtype,tag", [
    (2056, torch.bfloat16, "bf16"),   # 257 16-byte vectors: the last one held by a single lane
    (6152, torch.bfloat16, "bf16"),   # 769 vectors: 13 per lane, the generic path
    (8192, torch.float16, "f16"),     # 1024 vectors: the widest row held in registers
    (3588, torch.float32, "f32"),     # fp32 rows, 897 vectors: the generic path
])
@pytest.mark.parametrize("mode", [og.NORM_WEIGHT_AFTER_CAST, og.NORM_PLAIN])
def test_long_rows_with_bad_indices(gpu, H, dtype, tag, mode):
    """Rows of 2 K - 8 K elements on the register and generic paths, with out-of-range
    indices mixed in (zero rows, no read)."""
    print(f"case long rows H={H} {tag} mode={mode}", flush=True)
    g = torch.Generator().manual_seed(H + mode)
    B, S, T = 3, 21, 11
    hidden = (2 * torch.randn(B, S, H, generator=g)).to(dtype)
    idx = torch.randint(0, S, (B, T), generator=g)
    idx[0, 0] = -1
    idx[1, T - 1] = S
    idx[2, 5] = -(1 << 40)
    w = (1 + 0.1 * torch.randn(H, generator=g)).to(dtype)
    normed, gathered = ops.gather_rmsnorm(hidden.to(gpu), idx.to(gpu), w.to(gpu), 1e-6, mode, True)
    normed, gathered = normed.float().cpu(), gathered.cpu()
    ok = (idx >= 0) & (idx < S)
    assert torch.count_nonzero(normed[~ok]) == 0 and torch.count_nonzero(gathered[~ok]) == 0
    safe = idx.clamp(0, S - 1)
    exp_g, exp_n = og.gather_rmsnorm_np(hidden.float().numpy(), safe.numpy(), w.float().numpy(), 1e-6, mode, tag)
    okn = ok.numpy()
    assert np.array_equal(gathered.float().numpy()[okn], exp_g[okn])
    np.testing.assert_allclose(normed.numpy()[okn], exp_n[okn], atol=ATOL, rtol=RTOL)


def test_strided_hidden_and_bad_indices(gpu):
    g = torch.Generator().manual_seed(3)
    base = torch.randn(2, 50, 2 * 512, generator=g).to(torch.bfloat16)
    hidden = base[:, :, :512]  # row stride 1024, last dim contiguous
    idx = torch.randint(0, 50, (2, 12), generator=g)
    idx[0, 3] = -1
    idx[1, 5] = 50  # out of range -> zero rows, no out-of-bounds read
    w = torch.ones(512, dtype=torch.bfloat16)
    normed, gathered = ops.gather_rmsnorm(hidden.to(gpu), idx.to(gpu), w.to(gpu), 1e-6,
                                          og.NORM_WEIGHT_AFTER_CAST, True)
    normed, gathered = normed.cpu(), gathered.cpu()
    assert torch.count_nonzero(normed[0, 3]) == 0 and torch.count_nonzero(gathered[1, 5]) == 0
    ok = torch.ones(2, 12, dtype=torch.bool)
    ok[0, 3] = ok[1, 5] = False
    safe = idx.clamp(0, 49)
    ref_g, ref_n = og.ref_gather_input_rmsnorm(hidden.contiguous(), safe, w, 1e-6)
    assert torch.equal(gathered[ok], ref_g[ok])
    assert _ulp_diff_bf16(normed[ok], ref_n[ok]) <= 1


def test_closed_forms(gpu):
    H = 256
    hidden = torch.zeros(1, 4, H)
    hidden[0, 1] = 0.5          # constant row c -> c / sqrt(c^2 + eps)
    hidden[0, 2] = torch.linspace(-3, 3, H)
    hidden = hidden.to(torch.bfloat16)
    idx = torch.tensor([[0, 1, 2, 1]])
    w = torch.ones(H, dtype=torch.bfloat16)
    normed, _ = ops.gather_rmsnorm(hidden.to(gpu), idx.to(gpu), w.to(gpu), 1e-6, og.NORM_WEIGHT_AFTER_CAST, False)
    normed = normed.float().cpu()
    assert torch.count_nonzero(normed[0, 0]) == 0
    c = 0.5
    assert torch.allclose(normed[0, 1], torch.full((H,), c / (c * c + 1e-6) ** 0.5), atol=4e-3)
    rms = normed[0, 2].pow(2).mean().sqrt()
    assert abs(float(rms) - 1.0) < 1e-2


def test_empty_and_errors(gpu):
    hidden = torch.randn(1, 8, 64, device=gpu, dtype=torch.bfloat16)
    idx = torch.zeros(1, 0, dtype=torch.int64, device=gpu)
    n, gth = ops.gather_rmsnorm(hidden, idx, None, 1e-6, og.NORM_PLAIN, True)
    assert n.shape == (1, 0, 64) and gth.shape == (1, 0, 64)
    with pytest.raises(RuntimeError):
        ops.gather_rmsnorm(hidden.cpu(), idx.cpu(), None, 1e-6, og.NORM_PLAIN, True)


def _np_bits(t: torch.Tensor) -> np.ndarray:
    """The tensor's bit patterns as integers (bit-exact comparison of any 2- or 4-byte dtype)."""
    t = t.detach().cpu().contiguous()
    return t.view(torch.int16 if t.element_size() == 2 else torch.int32).numpy()


@pytest.mark.parametrize("B,S,T,H,dtype,two,row_pad,bad", [
    (2, 40, 7, 384, torch.bfloat16, True, 0, False),       # 48 vectors per row
    (1, 4096, 1024, 3584, torch.bfloat16, True, 0, False),  # the 1024 x 3584 workload, two destinations
    (2, 64, 9, 4096, torch.float16, True, 0, False),       # 512 vectors: the largest register-staged row
    (1, 64, 5, 8192, torch.bfloat16, True, 0, False),      # 1024 vectors: the looped row path
    (2, 30, 6, 37, torch.bfloat16, True, 0, False),        # 74-byte rows: element loop
    (2, 30, 6, 100, torch.float32, True, 0, False),        # fp32, 25 vectors
    (3, 50, 11, 256, torch.bfloat16, False, 0, False),     # one destination
    (2, 48, 8, 512, torch.bfloat16, True, 64, True),       # padded rows, out-of-range indices skipped
])
def test_scatter_rows(gpu, B, S, T, H, dtype, two, row_pad, bad):
    """fdllm_scatter_rows bit-exact against the oracle (scatter_and_return_cuda,
    fused_gather_norm.cu:79-119) and torch's scatter_; rows no index names keep their
    contents."""
    g = torch.Generator().manual_seed(5 + H)
    vals = torch.randn(B, T, H, generator=g).to(dtype)
    idx = torch.stack([torch.randperm(S, generator=g)[:T] for _ in range(B)])
    if bad:
        idx[0, 1], idx[1, 3] = -1, S
    base_c = torch.randn(B, S, H + row_pad, generator=g).to(dtype)
    base_u = torch.randn(B, S, H + row_pad, generator=g).to(dtype)
    exp_c, exp_u = og.scatter_rows_np(_np_bits(vals), idx.numpy(), _np_bits(base_c[..., :H]),
                                      _np_bits(base_u[..., :H]) if two else None)
    if not bad:
        ii = idx.unsqueeze(-1).expand(-1, -1, H)
        assert np.array_equal(_np_bits(base_c[..., :H].clone().scatter_(1, ii, vals)), exp_c)
    c_full, u_full = base_c.to(gpu), base_u.to(gpu)
    c_gpu, u_gpu = c_full[..., :H], u_full[..., :H]
    ret = ops.scatter_rows(vals.to(gpu), idx.to(gpu), c_gpu, u_gpu if two else None)
    torch.cuda.synchronize()
    assert np.array_equal(_np_bits(c_gpu), exp_c)
    if two:
        assert ret.data_ptr() == u_gpu.data_ptr()
        assert np.array_equal(_np_bits(u_gpu), exp_u)
    else:
        assert ret is None
        assert torch.equal(u_full.cpu(), base_u)
    if row_pad:  # the padding columns are never written
        assert torch.equal(c_full[..., H:].cpu(), base_c[..., H:])


@pytest.mark.parametrize("rows,H,dtype", [
    (128, 3584, torch.bfloat16),   # the 7B sub-block step: 16 sequences x 8 tokens
    (2048, 3584, torch.bfloat16),  # a 4 x 512-token prompt
    (37, 2056, torch.bfloat16),    # 257 vectors: the last one per lane ragged
    (5, 4096, torch.float16),
    (3, 8, torch.bfloat16),
])
def test_add_rmsnorm(gpu, rows, H, dtype):
    """The decoder layer's residual add + norm: the sum bit-exact against the 16-bit torch
    add, the norm bit-exact against the gather kernel on that sum (the norm the model used
    before the add was fused) and within the gather bars of the oracle."""
    print(f"case add_rmsnorm rows={rows} H={H} {dtype}", flush=True)
    g = torch.Generator().manual_seed(rows + H)
    x = (2 * torch.randn(rows, H, generator=g)).to(dtype)
    r = (2 * torch.randn(rows, H, generator=g)).to(dtype)
    w = (1 + 0.05 * torch.randn(H, generator=g)).to(dtype)
    s_exp = x + r
    for wt in (w, w.float()):
        s, n = ops.add_rmsnorm(x.to(gpu), r.to(gpu), wt.to(gpu), 1e-6)
        assert torch.equal(s.cpu(), s_exp)
        idx = torch.arange(rows, dtype=torch.int64, device=gpu)[None]
        n_gather, _ = ops.gather_rmsnorm(s[None], idx, wt.to(gpu), 1e-6, og.NORM_WEIGHT_AFTER_CAST, False)
        assert torch.equal(n.cpu(), n_gather[0].cpu())
        tag = "bf16" if dtype == torch.bfloat16 else "f16"
        _, exp_n = og.gather_rmsnorm_np(s_exp.float().numpy()[None], np.arange(rows)[None], wt.float().numpy(), 1e-6,
                                        og.NORM_WEIGHT_AFTER_CAST, tag)
        np.testing.assert_allclose(n.float().cpu().numpy(), exp_n[0], atol=ATOL, rtol=RTOL)
        if dtype == torch.bfloat16:
            assert _ulp_diff_bf16(n.cpu(), torch.from_numpy(exp_n[0]).to(torch.bfloat16)) <= 2
    # plain mode (no weight) and the torch statement of the model norm
    s, n = ops.add_rmsnorm(x.to(gpu), r.to(gpu), None, 1e-6, og.NORM_PLAIN)
    _, exp_n = og.gather_rmsnorm_np(s_exp.float().numpy()[None], np.arange(rows)[None], None, 1e-6, og.NORM_PLAIN,
                                    "bf16" if dtype == torch.bfloat16 else "f16")
    np.testing.assert_allclose(n.float().cpu().numpy(), exp_n[0], atol=ATOL, rtol=RTOL)


def test_add_rmsnorm_errors(gpu):
    x = torch.randn(4, 100, device=gpu, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="hidden_size|H="):
        ops.add_rmsnorm(x, x.clone(), torch.ones(100, device=gpu), 1e-6)  # H not a multiple of 8
    y = torch.randn(4, 64, device=gpu, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError):
        ops.add_rmsnorm(y, y.half(), torch.ones(64, device=gpu), 1e-6)
    s, n = ops.add_rmsnorm(y[:0], y[:0], torch.ones(64, device=gpu), 1e-6)
    assert s.shape == (0, 64) and n.shape == (0, 64)


@pytest.mark.parametrize("shape,dtype", [
    ((128, 18944), torch.bfloat16),   # the 7B MLP at the sub-block step
    ((3, 77, 24), torch.bfloat16),
    ((1024, 512), torch.float16),
])
def test_silu_mul(gpu, shape, dtype):
    """silu(gate) * up: bit-exact against the torch statement on the GPU (SiLU in fp32,
    rounded, then the 16-bit product), within one ulp of a float64 restatement."""
    print(f"case silu_mul {shape} {dtype}", flush=True)
    g = torch.Generator().manual_seed(sum(shape))
    gate = (4 * torch.randn(*shape, generator=g)).to(dtype)
    up = torch.randn(*shape, generator=g).to(dtype)
    gate[..., :4] = torch.tensor([0.0, -0.0, 30.0, -30.0])   # zeros and saturated ends
    got = ops.silu_mul(gate.to(gpu), up.to(gpu))
    exp = torch.nn.functional.silu(gate.to(gpu)) * up.to(gpu)
    assert torch.equal(got.cpu(), exp.cpu())
    g64 = gate.double()
    sg = (g64 / (1 + torch.exp(-g64))).to(dtype).double()
    ref = (sg * up.double()).to(dtype)
    if dtype == torch.bfloat16:
        assert _ulp_diff_bf16(got.cpu(), ref) <= 1
    else:
        torch.testing.assert_close(got.cpu(), ref, atol=1e-3, rtol=1e-3)


def test_silu_mul_errors(gpu):
    a = torch.randn(7, device=gpu, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="multiple of 8"):
        ops.silu_mul(a, a.clone())
    with pytest.raises(RuntimeError):
        ops.silu_mul(torch.randn(8, device=gpu), torch.randn(8, device=gpu))


def test_scatter_colliding_indices(gpu):
    """Indices that repeat within a sequence (a collision). The reference kernel's writers
    race element by element (fused_gather_norm.cu:79-99: each thread stores its element to
    both destinations), so which writer an element ends with is unspecified, and the two
    destinations may end with different writers. What holds: every element of a
    destination row aimed at holds that element of one of the value rows aimed at it, in
    each destination, and every other row keeps its contents."""
    g = torch.Generator().manual_seed(41)
    B, S, T, H = 2, 16, 12, 256
    vals = torch.randn(B, T, H, generator=g).to(torch.bfloat16)
    idx = torch.randint(0, 5, (B, T), generator=g)  # rows 0-4 only: many collisions
    cache = torch.randn(B, S, H, generator=g).to(torch.bfloat16)
    cur = torch.randn(B, S, H, generator=g).to(torch.bfloat16)
    c_gpu, u_gpu = cache.to(gpu), cur.to(gpu)
    ops.scatter_rows(vals.to(gpu), idx.to(gpu), c_gpu, u_gpu)
    c_out, u_out = c_gpu.cpu(), u_gpu.cpu()
    for b in range(B):
        for r in range(S):
            src = [t for t in range(T) if int(idx[b, t]) == r]
            if not src:
                assert torch.equal(c_out[b, r], cache[b, r]) and torch.equal(u_out[b, r], cur[b, r])
                continue
            cand = vals[b, src]  # [writers, H]
            for name, got in (("cache", c_out[b, r]), ("current", u_out[b, r])):
                assert bool((got[None] == cand).any(0).all()), \
                    f"{name} row {b},{r}: an element matches none of its {len(src)} writers"


@pytest.mark.parametrize("H", [8, 64])
def test_gather_and_scatter_large_batch(gpu, H):
    """70000 sequences (more than a 65535-high grid dimension): the gather takes its generic
    kernel and the scatter one row per workgroup; bit-exact rows, the norm within the bars."""
    print(f"case large batch gather/scatter H={H}", flush=True)
    g = torch.Generator().manual_seed(43 + H)
    B, S, T = 70000, 3, 2
    hidden = torch.randn(B, S, H, generator=g).to(torch.bfloat16)
    idx = torch.randint(0, S, (B, T), generator=g)
    w = (1 + 0.05 * torch.randn(H, generator=g)).to(torch.bfloat16)
    normed, gathered = ops.gather_rmsnorm(hidden.to(gpu), idx.to(gpu), w.to(gpu), 1e-6,
                                          og.NORM_WEIGHT_AFTER_CAST, True)
    exp_g = torch.gather(hidden, 1, idx.unsqueeze(-1).expand(-1, -1, H))
    assert torch.equal(gathered.cpu(), exp_g)
    _, ref_n = og.ref_gather_input_rmsnorm(hidden, idx, w, 1e-6)
    torch.testing.assert_close(normed.float().cpu(), ref_n.float(), atol=ATOL, rtol=RTOL)
    vals = torch.randn(B, T, H, generator=g).to(torch.bfloat16)
    sidx = torch.stack([torch.randperm(S, generator=g)[:T] for _ in range(64)]).repeat(B // 64 + 1, 1)[:B]
    cache = hidden.clone()
    c_gpu = cache.to(gpu)
    ops.scatter_rows(vals.to(gpu), sidx.to(gpu), c_gpu)
    exp_c = cache.clone().scatter_(1, sidx.unsqueeze(-1).expand(-1, -1, H), vals)
    assert torch.equal(c_gpu.cpu(), exp_c)


@pytest.mark.parametrize("H,dtype", [(3584, torch.bfloat16), (128, torch.bfloat16), (4096, torch.float16),
                                     (2056, torch.bfloat16), (512, torch.float32)])
def test_unselected_rows_poisoned_with_nan(gpu, H, dtype):
    """Only the selected rows are read: NaN in every row no index names leaves the normed
    rows and the gathered copy bit for bit as with zeros there, on every width class (the
    register-vector kernels and the element loop) and for fp32 hidden states."""
    print(f"case poisoned gather H={H} {dtype}", flush=True)
    g = torch.Generator().manual_seed(H)
    B, S, T = 2, 300, 77
    hidden = torch.randn(B, S, H, generator=g).to(dtype)
    idx = torch.stack([torch.randperm(S, generator=g)[:T] for _ in range(B)])
    w = (1 + 0.02 * torch.randn(H, generator=g)).to(dtype)
    outs = []
    for fill in (0.0, float("nan")):
        h = hidden.clone()
        keep = torch.zeros(B, S, dtype=torch.bool)
        keep[torch.arange(B)[:, None], idx] = True
        h[~keep] = fill
        normed, gathered = ops.gather_rmsnorm(h.to(gpu), idx.to(gpu), w.to(gpu), 1e-6)
        outs.append((normed.cpu(), gathered.cpu()))
    torch.cuda.synchronize()
    assert torch.isfinite(outs[1][0]).all() and torch.isfinite(outs[1][1]).all()
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
    assert torch.equal(outs[1][1], hidden[torch.arange(B)[:, None], idx])
