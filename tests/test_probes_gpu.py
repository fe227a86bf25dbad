"""The measurement probes bench.py times beside the calls they bound
(include/fdllm_probes.h, lib/libfdllm_probes.so): the gathered copy reproduces
hidden[idx] bit for bit (rows of 16 B to 16 KB, every width class of the kernel), the
plain read of a paged or contiguous cache runs to completion without writing its sink
(the fold of the rows never hits the sentinel on random data), and a call the probe
cannot run returns -1 before any launch."""
import ctypes
from pathlib import Path

import pytest
import torch

from fast_v2_amd import workloads

pytestmark = pytest.mark.gpu

LIB = Path(__file__).resolve().parent.parent / "fast_v2_amd" / "lib" / "libfdllm_probes.so"


def _lib():
    lib = ctypes.CDLL(str(LIB))
    vp, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32
    lib.fdllm_probe_read_kv.argtypes = [vp, vp, i64, i64, i64, i64, i64, i64, vp, i32, i32, vp,
                                        ctypes.c_int, ctypes.c_int, ctypes.c_int, vp, vp]
    lib.fdllm_probe_read_kv.restype = ctypes.c_int
    lib.fdllm_probe_copy_rows.argtypes = [vp, i64, ctypes.c_int, vp, vp, ctypes.c_int, ctypes.c_int, vp]
    lib.fdllm_probe_copy_rows.restype = ctypes.c_int
    lib.fdllm_probe_mfma.argtypes = [ctypes.c_int, ctypes.c_int, vp, vp]
    lib.fdllm_probe_mfma.restype = ctypes.c_int
    return lib


def _stream():
    return torch.cuda.current_stream().cuda_stream


@pytest.mark.parametrize("rows,cols,src_rows", [(1024, 3584, 4096), (7, 8, 20), (33, 4096, 64), (5, 8192, 9)])
def test_probe_copy_rows_matches_indexing(gpu, rows, cols, src_rows):
    print(f"case probe copy rows={rows} cols={cols}", flush=True)
    g = torch.Generator().manual_seed(rows + cols)
    src = torch.randn(src_rows, cols, generator=g).to(torch.bfloat16).to(gpu)
    idx = torch.randint(0, src_rows, (rows,), generator=g).to(gpu)
    dst = torch.empty(rows, cols, dtype=torch.bfloat16, device=gpu)
    rc = _lib().fdllm_probe_copy_rows(src.data_ptr(), cols * 2, src_rows, idx.data_ptr(), dst.data_ptr(), rows,
                                      cols * 2, _stream())
    assert rc == 0
    torch.cuda.synchronize()
    assert torch.equal(dst, src[idx])


@pytest.mark.parametrize("paged", [True, False])
def test_probe_read_kv_runs(gpu, paged):
    print(f"case probe read paged={paged}", flush=True)
    wl = workloads.kv_decode_paged(seed=3, batch=16)
    kp, vp_ = wl.k_pool.to(gpu), wl.v_pool.to(gpu)
    sl = wl.seqlens.to(gpu)
    sink = torch.zeros(4, dtype=torch.int32, device=gpu)
    lib = _lib()
    if paged:
        pt = wl.page_table.to(gpu)
        k, v = kp, vp_
        args = (pt.data_ptr(), pt.shape[1], wl.page_size)
    else:
        B, maxs = wl.seqlens.shape[0], int(wl.seqlens.max())
        k = torch.randn(B, maxs, kp.shape[-2], kp.shape[-1], device=gpu).to(torch.bfloat16)
        v = torch.randn_like(k)
        args = (None, 0, 0)
    ks, vs = k.stride(), v.stride()
    rc = lib.fdllm_probe_read_kv(k.data_ptr(), v.data_ptr(), ks[0], ks[1], ks[2], vs[0], vs[1], vs[2], *args,
                                 sl.data_ptr(), wl.seqlens.shape[0], k.shape[-2], 64, sink.data_ptr(), _stream())
    assert rc == 0
    torch.cuda.synchronize()
    assert int(sink.abs().sum()) == 0


def test_probe_rejects_bad_calls(gpu):
    lib = _lib()
    sink = torch.zeros(4, dtype=torch.int32, device=gpu)
    sl = torch.ones(2, dtype=torch.int32, device=gpu)
    k = torch.zeros(2, 64, 4, 128, dtype=torch.bfloat16, device=gpu)
    ks = k.stride()
    # slots not a multiple of 8
    assert lib.fdllm_probe_read_kv(k.data_ptr(), k.data_ptr(), ks[0], ks[1], ks[2], ks[0], ks[1], ks[2], None, 0, 0,
                                   sl.data_ptr(), 2, 4, 12, sink.data_ptr(), _stream()) == -1
    # rows wider than the copy kernel takes
    src = torch.zeros(4, 16384, dtype=torch.bfloat16, device=gpu)
    idx = torch.zeros(2, dtype=torch.int64, device=gpu)
    dst = torch.zeros(2, 16384, dtype=torch.bfloat16, device=gpu)
    assert lib.fdllm_probe_copy_rows(src.data_ptr(), 16384 * 2, 4, idx.data_ptr(), dst.data_ptr(), 2, 16384 * 2,
                                     _stream()) == -1
    # MFMA rate probe: no workgroups, no rounds, no sink
    out = torch.zeros(256, dtype=torch.float32, device=gpu)
    assert lib.fdllm_probe_mfma(0, 8, out.data_ptr(), _stream()) == -1
    assert lib.fdllm_probe_mfma(1, 0, out.data_ptr(), _stream()) == -1
    assert lib.fdllm_probe_mfma(1, 8, None, _stream()) == -1


def test_probe_mfma_runs(gpu):
    """The MFMA rate probe runs to completion on a full grid (one workgroup per compute
    unit) and leaves its sink untouched (the sums never hit the sink's constant)."""
    print("case probe mfma", flush=True)
    wgs = torch.cuda.get_device_properties(gpu).multi_processor_count
    sink = torch.zeros(wgs * 256, dtype=torch.float32, device=gpu)
    assert _lib().fdllm_probe_mfma(wgs, 64, sink.data_ptr(), _stream()) == 0
    torch.cuda.synchronize()
    assert int(torch.count_nonzero(sink)) == 0
