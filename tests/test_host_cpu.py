"""Host-side logic that needs no GPU: backend selection and its failure modes,
the cache objects' bookkeeping (lengths, write position, masks, compaction),
the torch ops' Meta implementations, RoPE, and the rule that every compute
entry point refuses CPU tensors instead of computing on the CPU.
"""
import math

import pytest
import torch

from fast_v2_amd import _ffi, ops
from fast_v2_amd.cuda_bench import fused_sparse_extension as fse
from fast_v2_amd.utils import attention_backends as ab
from fast_v2_amd.utils import BlockSparseCache, DynamicBlockKV, StaticBlockCache, StaticKVCache
from oracle import attention as oa

pytestmark = pytest.mark.skipif(torch.cuda.is_available(), reason="CPU-only behaviour")


def test_backend_selection_without_gpu():
    ab.get_attention_backend.cache_clear()
    be = ab.get_attention_backend()
    assert be.name == "sdpa"
    assert ab.get_attention_backend() is be  # lru-cached singleton
    ab.get_attention_backend.cache_clear()
    with pytest.raises(RuntimeError, match="gfx950"):
        ab.get_attention_backend("hip")
    ab.get_attention_backend.cache_clear()
    assert ab.get_attention_backend("flash2").name == "sdpa"
    ab.get_attention_backend.cache_clear()


def test_sdpa_backend_kvcache_raises_like_the_reference():
    be = ab.AttentionBackend(ab.AttentionBackend.SDPA)
    q = torch.randn(1, 8, 4, 16)
    k = torch.randn(1, 32, 2, 16)
    with pytest.raises(RuntimeError, match="hip backend"):
        be.flash_kvcache_attention(q, k, k, torch.tensor([20], dtype=torch.int32))
    with pytest.raises(ValueError):
        ab.AttentionBackend("nonsense").attention(q, k, k)


def test_sdpa_backend_attention_matches_oracle():
    torch.manual_seed(0)
    q, k, v = torch.randn(2, 6, 5, 16), torch.randn(2, 2, 9, 16), torch.randn(2, 2, 9, 16)
    out = ab.AttentionBackend("sdpa").attention(q, k, v)
    exp = oa.attention_np(q.transpose(1, 2).numpy(), k.transpose(1, 2).numpy(), v.transpose(1, 2).numpy(), [9, 9])
    torch.testing.assert_close(out.transpose(1, 2), torch.from_numpy(exp).float(), atol=1e-5, rtol=1e-5)


def test_hip_backend_refuses_cpu_tensors():
    be = ab.AttentionBackend(ab.AttentionBackend.HIP)
    q = torch.randn(1, 8, 4, 16, dtype=torch.bfloat16)
    k = torch.randn(1, 32, 2, 16, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError):
        be.flash_kvcache_attention(q, k, k, torch.tensor([20], dtype=torch.int32))
    with pytest.raises(RuntimeError):
        be.attention(q.transpose(1, 2), k.transpose(1, 2), k.transpose(1, 2))


def test_ops_refuse_cpu_tensors():
    h = torch.randn(1, 8, 64, dtype=torch.bfloat16)
    idx = torch.zeros(1, 2, dtype=torch.int64)
    with pytest.raises(RuntimeError, match="GPU"):
        ops.gather_rmsnorm(h, idx, None, 1e-6, _ffi.NORM_PLAIN)
    with pytest.raises(RuntimeError, match="GPU"):
        ops.scatter_rows(h[:, :2], idx, h)
    k = torch.zeros(1, 4, 2, 64, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="GPU"):
        ops.kv_cache_write(k, k, torch.zeros(1, 16, 2, 64, dtype=torch.bfloat16),
                           torch.zeros(1, 16, 2, 64, dtype=torch.bfloat16))
    with pytest.raises(RuntimeError, match="GPU"):
        ops.block_attn(torch.zeros(1, 4, 4, 64, dtype=torch.bfloat16), k, k, torch.tensor([4]))


def test_fused_sparse_extension_returns_none_for_cpu_hidden():
    class Norm(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.weight = torch.nn.Parameter(torch.ones(64))
            self.variance_epsilon = 1e-6
    h = torch.randn(1, 8, 64)
    assert fse.fused_gather_input_rmsnorm_pair(h, torch.zeros(1, 2, dtype=torch.long), Norm()) is None


_LATCH_PROBE = r"""
import logging, sys
import torch
from fast_v2_amd.cuda_bench import fused_sparse_extension as fse

records = []
class H(logging.Handler):
    def emit(self, r):
        records.append(r)
logging.getLogger(fse.__name__).addHandler(H())

class FakeCudaHidden:          # only .is_cuda is read before the library check
    is_cuda = True
class Norm(torch.nn.Module):
    def __init__(self):
        super().__init__()
        self.weight = torch.nn.Parameter(torch.ones(64))
        self.variance_epsilon = 1e-6

first = fse.get_fused_ops()
second = fse.get_fused_ops()
pair = fse.fused_gather_input_rmsnorm_pair(FakeCudaHidden(), torch.zeros(1, 2, dtype=torch.long), Norm())
errors = [r for r in records if r.levelno >= logging.ERROR]
print(first is None, second is None, pair is None, len(errors), fse._OPS_FAILED)
"""


def test_get_fused_ops_latches_a_load_failure(tmp_path):
    """A library that cannot load: get_fused_ops() returns None, logs once and latches
    (reference cuda_bench/fused_sparse_extension.py:25-48), and the model-path wrapper
    returns None so the caller takes its PyTorch path (:70-78)."""
    import os
    import subprocess
    import sys
    from pathlib import Path

    env = dict(os.environ, FDLLM_HIP_LIB=str(tmp_path / "missing" / "libfdllm_hip.so"))
    root = Path(__file__).resolve().parents[1]
    proc = subprocess.run([sys.executable, "-c", _LATCH_PROBE], cwd=root, env=env, capture_output=True,
                          text=True, timeout=300)
    assert proc.returncode == 0, proc.stderr
    assert proc.stdout.split() == ["True", "True", "True", "1", "True"], proc.stdout


def test_get_fused_ops_loads_the_built_library():
    if not _ffi.LIB_PATH.exists():
        pytest.skip("libfdllm_hip.so not built")
    ext = fse.get_fused_ops()
    assert ext is not None and fse.get_fused_ops() is ext
    for name in ("gather_rmsnorm_cuda", "scatter_and_return_cuda", "fused_select_norm",
                 "fused_gather_input_rmsnorm_pair"):
        assert callable(getattr(ext, name))


def test_meta_implementations():
    q = torch.empty(2, 8, 28, 128, dtype=torch.bfloat16, device="meta")
    k = torch.empty(2, 512, 4, 128, dtype=torch.bfloat16, device="meta")
    sl = torch.empty(2, dtype=torch.int32, device="meta")
    out = torch.ops.fdllm.flash_kvcache(q, k, k, sl, 0.1, False)
    assert out.shape == q.shape and out.device.type == "meta"
    out = torch.ops.fdllm.block_attn(q, k, k, sl, 0.1, 2, 32, None, None, 0)
    assert out.shape == q.shape
    h = torch.empty(1, 4096, 3584, dtype=torch.bfloat16, device="meta")
    idx = torch.empty(1, 1024, dtype=torch.int64, device="meta")
    n, g = torch.ops.fdllm.gather_rmsnorm(h, idx, None, 1e-6, 0, True)
    assert n.shape == (1, 1024, 3584) and g.shape == (1, 1024, 3584)
    n, g = torch.ops.fdllm.gather_rmsnorm(h, idx, None, 1e-6, 0, False)
    assert g.numel() == 0


def test_static_kv_cache_bookkeeping():
    c = StaticKVCache(batch_size=3, max_seq_len=64, num_layers=4, num_kv_heads=2, head_dim=8,
                      dtype=torch.bfloat16, device="cpu")
    assert len(c.key_cache) == 4 and c.key_cache[1].shape == (3, 64, 2, 8)
    # the per-layer buffers are views of one allocation, one layer apart
    step = c.key_cache[1].data_ptr() - c.key_cache[0].data_ptr()
    assert step == 3 * 64 * 2 * 8 * 2
    assert c.get_seq_length() == 0 and len(c) == 0
    c.set_scratch_seqlens(40)
    assert c.scratch_seqlens.tolist() == [40, 40, 40] and c.scratch_seqlens.dtype == torch.int32
    c.set_kv_write_start(32)
    assert int(c.kv_write_start) == 32 and c._write_start.tolist() == [32, 32, 32]
    c.kv_write_start.fill_(48)  # direct writers are picked up by prepare_write_idx
    c.prepare_write_idx(8)
    assert c._write_start.tolist() == [48, 48, 48]
    m = c.get_seqused_mask(10)
    assert m.shape == (3, 1, 1, 64)
    assert (m[..., :10] == 0).all() and torch.isinf(m[..., 10:]).all()
    mb = c.get_seqused_mask_batched(torch.tensor([1, 5, 64]))
    assert torch.isinf(mb[0, ..., 1:]).all() and (mb[2] == 0).all()
    k = torch.randn(3, 4, 2, 8).to(torch.bfloat16)
    with pytest.raises(RuntimeError):  # the write kernels need the GPU
        c.update(k, k, 0)
    with pytest.raises(RuntimeError, match="do not match"):
        c.update(torch.zeros(2, 4, 2, 8, dtype=torch.bfloat16), torch.zeros(2, 4, 2, 8, dtype=torch.bfloat16), 0)
    # compaction keeps the selected rows, in order
    c.key_cache[2][1, 5, 1, 3] = 7.0
    c.cache_seqlens.copy_(torch.tensor([10, 20, 30], dtype=torch.int32))
    c.compact_batch(torch.tensor([1, 2]))
    assert c.batch_size == 2 and c.key_cache[2].shape == (2, 64, 2, 8)
    assert float(c.key_cache[2][0, 5, 1, 3]) == 7.0
    assert c.cache_seqlens.tolist() == [20, 30] and c._write_start.shape == (2,)
    c.restore_full_batch()
    assert c.batch_size == 3 and c.key_cache[0].shape == (3, 64, 2, 8)
    c.zero_and_reset()
    assert c.get_seq_length() == 0 and int(c.kv_write_start) == 0


def test_block_caches_bookkeeping():
    bc = StaticBlockCache(2, 32, 3, 4, 16, torch.bfloat16, "cpu")
    assert len(bc) == 0 and bc.get_seq_length() == 0
    assert bc[1][0].shape == (2, 32, 4, 16)
    bc._num_initialized = 2
    assert len(bc) == 2 and bc.get_seq_length() == 32
    bc.reset()
    assert len(bc) == 0
    bc.compact_batch(torch.tensor([1]))
    assert bc.key_cache[0].shape == (1, 32, 4, 16)

    sc = BlockSparseCache(3, 2, 32, 64, torch.bfloat16, "cpu")
    x = torch.randn(2, 32, 64).to(torch.bfloat16)
    sc.cache_attn_output(1, x)
    assert torch.equal(sc.get_attn_output(1), x) and not sc.get_attn_output(0).any()
    sc.compact_batch(torch.tensor([1]))
    assert torch.equal(sc.get_attn_output(1)[0], x[1])

    dk = DynamicBlockKV(2, 4, 2, 4, 32, 16, torch.bfloat16, "cpu")
    assert sorted(dk.k) == [2, 3] and dk.get(3)[0].shape == (2, 4, 32, 16)
    kk = torch.randn(2, 4, 32, 16).to(torch.bfloat16)
    dk.write_full(2, kk, kk)
    assert torch.equal(dk.get(2)[1], kk)
    with pytest.raises(RuntimeError):
        dk.write(2, kk[:, :, :3], kk[:, :, :3], torch.zeros(2, 3, dtype=torch.long))


def test_rope_is_a_rotation_of_half_pairs():
    """RoPE pairs element i with i + D/2 and rotates the pair by the position angle."""
    torch.manual_seed(0)
    B, S, H, D = 2, 5, 3, 8
    q, k = torch.randn(B, S, H, D), torch.randn(B, S, 1, D)
    theta = torch.rand(B, S, D // 2) * 6.0
    cos = torch.cat([theta.cos(), theta.cos()], -1)
    sin = torch.cat([theta.sin(), theta.sin()], -1)
    qe, ke = ab._apply_rotary_pos_emb(q, k, cos, sin)
    zq = torch.complex(q[..., :D // 2], q[..., D // 2:]) * torch.polar(torch.ones_like(theta), theta)[:, :, None]
    torch.testing.assert_close(qe, torch.cat([zq.real, zq.imag], -1), atol=1e-6, rtol=1e-6)
    # norms are preserved
    torch.testing.assert_close(ke.norm(dim=-1), k.norm(dim=-1), atol=1e-5, rtol=1e-5)
    assert math.isclose(float(qe.norm()), float(q.norm()), rel_tol=1e-5)


def test_timeline_phase_statistics():
    """fast_v2_amd.timeline.analyse on hand-made stamps (100 MHz ticks): idle slots,
    single-split units and merging workgroups are told apart, and the phase ends and
    durations come out in µs from the first start."""
    import numpy as np
    from fast_v2_amd import timeline as tlm
    st = np.zeros((6, tlm.STAMPS), dtype=np.int64)
    t0 = 1_000_000
    #                 start  part  first  loop   arrive  merge   info (b, split, n_act, ntiles)
    st[0, :7] = [t0, t0 + 100, t0 + 400, t0 + 1500, t0 + 1700, t0 + 1950, (0 << 48) | (0 << 32) | (2 << 16) | 20]
    st[1, :7] = [t0 + 50, t0 + 150, t0 + 450, t0 + 1600, t0 + 1800, 0, (0 << 48) | (1 << 32) | (2 << 16) | 21]
    st[2, :7] = [t0 + 20, t0 + 130, t0 + 420, t0 + 1200, t0 + 1300, 0, (1 << 48) | (0 << 32) | (1 << 16) | 10]
    st[3, :2] = [t0 + 30, t0 + 140]  # an idle slot: start and partition only
    res = tlm.analyse(st)
    assert res["workgroups"] == 4 and res["active"] == 3 and res["merging"] == 1
    assert res["tiles_per_workgroup"] == (10.0, 20.0, 21.0)
    assert res["start"] == (0.0, 0.25, 0.5)
    assert res["merge written"] == (19.5, 19.5, 19.5)
    assert math.isclose(res["span"], 19.5)
    assert np.allclose(res["d_loop"], (7.8, 11.0, 11.5))
    assert np.allclose(res["d_merge"], (2.5, 2.5, 2.5))


def test_bench_refuses_more_than_one_gpu():
    """bench.py --gpus N with N > 1 prints one JSON line saying the build targets one GPU
    and exits with status 2, before touching torch or a device."""
    import json
    import subprocess
    import sys
    from pathlib import Path
    root = Path(__file__).resolve().parents[1]
    out = subprocess.run([sys.executable, str(root / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                         timeout=120, cwd=root)
    assert out.returncode == 2
    line = json.loads(out.stdout.strip().splitlines()[-1])
    assert line["n_gpus"] == 2 and "one GPU" in line["error"]
