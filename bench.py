#!/usr/bin/env python3
"""Benchmark of the block-diffusion hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline] [--only NAME]

Headline (one JSON line on stdout): the block-decode attention step at 7B
geometry — 16 sequences, 28 query / 4 KV heads, head_dim 128, prefixes uniform
in {1024..4096} step 32 plus the current 32-token block, 8 active queries (one
sub-block), 32-token KV pages, bf16. One step = one attention call of one layer;
the K timed steps walk through 28 separate layer pools (2.4 GB of KV), so every
call streams its KV from HBM rather than from the 256 MB last-level cache.

The K steps are captured in one HIP graph and replayed once inside the timed
region, bracketed by torch.cuda.synchronize(); HIP events recorded on the same
stream give the per-step time, i.e. the average kernel duration plus the
inter-kernel gap.

Also reported (same run, under "extra"): the same step with all 32 block queries
active (the full-block forward), gather + RMSNorm (bf16 [4096 x 3584], 1024 rows), the
row scatter of those 1024 rows back into two [4096 x 3584] destinations, and
block-causal prefill with its KV-cache write (4 x 4096 tokens), each with its own
roofline.

cpu_baseline: the reference's CPU path for the same workload, the SDPA shim of
tests/test_focus.py:205-228 (oracle.attention.sdpa_kvcache), on the host cores.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import tempfile
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA, TFLOP/s
METRIC = "block-attn step µs + % HBM/MFMA peak; gen tokens/s (7B geom, bs16)"
LAYERS = 28
TRAFFIC_FILE = ROOT / "profiles" / "traffic.json"


def _log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def _time_graph(torch, step_fn, steps: int, warmup: int) -> float:
    """Run `warmup` eager steps, capture `steps` steps in one graph, replay it once
    untimed, then time one replay. Returns microseconds per step.

    Warm-up runs on the capture stream so that any per-stream scratch the ops keep
    (the split-KV workspace) exists before capture starts."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for i in range(warmup):
            step_fn(i)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for i in range(steps):
            step_fn(i)
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    g.replay()
    end.record()
    torch.cuda.synchronize()
    us = start.elapsed_time(end) * 1e3 / steps
    del g
    return us


def _time_graphs_rotating(torch, step_fns: dict, steps: int, warmup: int, rounds: int = 3) -> dict:
    """Capture `steps` steps of each function in a graph of its own (after `warmup` eager
    steps on the capture stream), then time one replay of each in turn, `rounds` times
    over; returns the median µs per step of each. Interleaving keeps clock and cache
    state from favouring whichever form would otherwise be timed last."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graphs = {}
    for name, fn in step_fns.items():
        with torch.cuda.stream(s):
            for i in range(warmup):
                fn(i)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            for i in range(steps):
                fn(i)
        torch.cuda.synchronize()
        graphs[name] = g
    for g in graphs.values():
        g.replay()
    torch.cuda.synchronize()
    times = {name: [] for name in graphs}
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    for _ in range(rounds):
        for name, g in graphs.items():
            start.record()
            g.replay()
            end.record()
            torch.cuda.synchronize()
            times[name].append(start.elapsed_time(end) * 1e3 / steps)
    del graphs
    return {name: sorted(t)[len(t) // 2] for name, t in times.items()}


_PROBES = None


def _probes():
    """ctypes handle of lib/libfdllm_probes.so (the measurement probes: include/fdllm_probes.h)."""
    global _PROBES
    if _PROBES is None:
        import ctypes
        path = ROOT / "fast_v2_amd" / "lib" / "libfdllm_probes.so"
        if not path.exists():
            raise RuntimeError(f"{path} is not built; run `python -m fast_v2_amd.build`")
        lib = ctypes.CDLL(str(path))
        vp, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32
        lib.fdllm_probe_read_kv.argtypes = [vp, vp, i64, i64, i64, i64, i64, i64, vp, i32, i32, vp,
                                            ctypes.c_int, ctypes.c_int, ctypes.c_int, vp, vp]
        lib.fdllm_probe_read_kv.restype = ctypes.c_int
        lib.fdllm_probe_copy_rows.argtypes = [vp, i64, ctypes.c_int, vp, vp, ctypes.c_int, ctypes.c_int, vp]
        lib.fdllm_probe_copy_rows.restype = ctypes.c_int
        lib.fdllm_probe_mfma.argtypes = [ctypes.c_int, ctypes.c_int, vp, vp]
        lib.fdllm_probe_mfma.restype = ctypes.c_int
        _PROBES = lib
    return _PROBES


def _stream_ptr(torch):
    return torch.cuda.current_stream().cuda_stream


def _traffic(name: str):
    try:
        data = json.loads(TRAFFIC_FILE.read_text())
        return data.get(name)
    except (OSError, ValueError):
        return None


def _roofline(bound: str, achieved: float, peak: float, unit: str, traffic):
    return {"bound": bound, "achieved": round(achieved, 2), "peak": peak, "unit": unit,
            "frac": round(achieved / peak, 4), "traffic": traffic}


# ---------------------------------------------------------------------------
def bench_decode(torch, args):
    from fast_v2_amd import ops, workloads

    dev = torch.device("cuda", 0)
    wl = workloads.kv_decode_paged(seed=0)
    layers = args.layers
    # layer 0 holds the seeded pool (shared with the CPU baseline); further layers are
    # N(0,1) pools drawn on the device, same page table
    gen = torch.Generator(device=dev).manual_seed(1)
    kp = torch.empty((layers,) + tuple(wl.k_pool.shape), dtype=wl.k_pool.dtype, device=dev)
    vp = torch.empty_like(kp)
    kp[0].copy_(wl.k_pool)
    vp[0].copy_(wl.v_pool)
    for layer in range(1, layers):
        kp[layer].normal_(generator=gen)
        vp[layer].normal_(generator=gen)
    q = wl.q.to(dev)
    pt = wl.page_table.to(dev)
    sl = wl.seqlens.to(dev)
    page_size = wl.page_size
    if args.layout == "paged_hm":
        # head-major pages: each page stored [Hkv, page_size, D], so one KV head's page is one
        # contiguous run (page_size x D x 2 B); viewed as [num_pages, page_size, Hkv, D]
        kp = kp.permute(0, 1, 3, 2, 4).contiguous().permute(0, 1, 3, 2, 4)
        vp = vp.permute(0, 1, 3, 2, 4).contiguous().permute(0, 1, 3, 2, 4)
        torch.cuda.empty_cache()
    if args.layout in ("contig", "bhsd"):
        # the reference's static cache layout [B, max_S, Hkv, D] per layer (identity pages)
        B = q.shape[0]
        max_s = int(wl.seqlens.max())
        pos = torch.arange(max_s, device=dev)
        idx = pt[:, (pos // page_size).clamp(max=pt.shape[1] - 1)].long()  # [B, max_S]
        kc = kp[:, idx, pos % page_size]  # [layers, B, max_S, Hkv, D]
        vc = vp[:, idx, pos % page_size]
        if args.layout == "bhsd":
            # head-major storage [layers, B, Hkv, max_S, D] viewed as [layers, B, max_S, Hkv, D]
            kc = kc.permute(0, 1, 3, 2, 4).contiguous().permute(0, 1, 3, 2, 4)
            vc = vc.permute(0, 1, 3, 2, 4).contiguous().permute(0, 1, 3, 2, 4)
        kp, vp, pt, page_size = kc, vc, None, 0
        torch.cuda.empty_cache()
    _log(f"decode: lens={wl.seqlens.tolist()} layout={args.layout} "
         f"kv={2 * kp.numel() * 2 / 2**30:.2f} GiB over {layers} layers")
    out = torch.empty_like(q)
    B, Sq, Hq, D = q.shape
    Hkv = kp.shape[-2]

    def step(i):
        layer = i % layers
        ops.block_attn(q, kp[layer], vp[layer], sl, wl.scale, page_table=pt, page_size=page_size,
                       out=out, kv_split=args.kv_split, balanced_splits=args.balanced_splits)

    # graph replay must reproduce the eager result bit for bit: the last captured step
    # reads layer (steps - 1) % layers, the eager reference the same layer
    step(args.steps - 1)
    eager = out.clone()
    us = _time_graph(torch, step, args.steps, args.warmup)
    if not torch.equal(out, eager):
        raise RuntimeError("decode: graph replay output differs from the eager call")
    extra_layouts = {}
    if args.layout == "paged_hm":
        # the same values in token-major pages ([page_size, Hkv, D] per page, the paged layout
        # of flash_attn_with_kvcache's block table), timed the same way
        kt = kp.contiguous()
        vt = vp.contiguous()

        def step_tm(i):
            ops.block_attn(q, kt[i % layers], vt[i % layers], sl, wl.scale, page_table=pt, page_size=page_size,
                           out=out, kv_split=args.kv_split, balanced_splits=args.balanced_splits)

        step_tm(args.steps - 1)
        eager_tm = out.clone()
        extra_layouts["us_per_step_token_major_pages"] = _time_graph(torch, step_tm, args.steps, args.warmup)
        if not torch.equal(out, eager_tm):
            raise RuntimeError("decode (token-major pages): graph replay output differs from the eager call")
        # the same values in the other page layout: the same arithmetic, so the same bits
        extra_layouts["token_major_output_bit_identical"] = bool(torch.equal(eager_tm, eager))
        del kt, vt
        torch.cuda.empty_cache()
    # the practical floor of the call: a plain read of the same K/V bytes in the same tile
    # pattern and launch shape (one KV head per workgroup, 32-key tiles, 64 slots per head),
    # no math, timed through the same graph path
    probes = _probes()
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    kst, vst = kp[0].stride(), vp[0].stride()

    def read_step(i):
        layer = i % layers
        rc = probes.fdllm_probe_read_kv(kp[layer].data_ptr(), vp[layer].data_ptr(), kst[0], kst[1], kst[2],
                                        vst[0], vst[1], vst[2], pt.data_ptr() if pt is not None else None,
                                        pt.shape[1] if pt is not None else 0, page_size, sl.data_ptr(), B, Hkv,
                                        max(8, (256 // Hkv + 7) // 8 * 8), sink.data_ptr(), _stream_ptr(torch))
        if rc != 0:
            raise RuntimeError(f"fdllm_probe_read_kv failed ({rc})")

    us_read = _time_graph(torch, read_step, args.steps, args.warmup)
    nbytes = workloads.decode_bytes(wl.seqlens, Hq, Hkv, D, Sq)
    flops = workloads.decode_flops(wl.seqlens, Hq, D, Sq)
    gbs = nbytes / (us * 1e-6) / 1e9
    res = {
        "us_per_step": us,
        "bytes_per_step": nbytes,
        "flops_per_step": flops,
        "achieved_gbs": gbs,
        "tflops": flops / (us * 1e-6) / 1e12,
        "roofline": _roofline("hbm", gbs, HBM_PEAK_GBS, "GB/s", _traffic("kv_attn_decode_bs16")),
        "us_per_model_step_28_layers": us * LAYERS,
        "seqlens": wl.seqlens.tolist(),
        "layout": args.layout,
        **extra_layouts,
        "ceiling": {
            "read_us_per_step": us_read,
            "read_bytes": nbytes - workloads.decode_bytes(wl.seqlens * 0, Hq, Hkv, D, Sq),
            "step_vs_read": us / us_read,
            "note": ("plain read of every visible K/V row of the step (fdllm_probe_read_kv: one KV head per "
                     "workgroup, 32-key tiles, two tiles in flight per team, keys dealt evenly over 64 slots "
                     "per head, no math), same pages and layer pools, same graph path"),
        },
    }
    del q, kp, vp, pt, sl, out
    torch.cuda.empty_cache()
    return res, wl


def bench_decode_full(torch, args):
    """The same 16 sequences with all 32 block queries active (the full-block forward of a
    diffusion step): 224 query rows per KV head, run on the prefill kernel's 32x32 MFMA
    tiles with key splits, then the merge kernel (two kernels per step). Same KV pools and
    page table layout as the headline step, N(0, 1) on the device."""
    from fast_v2_amd import ops, workloads

    dev = torch.device("cuda", 0)
    wl = workloads.kv_decode_paged(seed=0, active=32)
    layers = args.layers
    gen = torch.Generator(device=dev).manual_seed(1)
    kp = torch.empty((layers,) + tuple(wl.k_pool.shape), dtype=wl.k_pool.dtype, device=dev)
    if args.layout == "paged_hm":  # the headline's page layout: [Hkv, page_size, D] per page
        kp = kp.transpose(-3, -2).contiguous().transpose(-3, -2)
    vp = torch.empty_like(kp)
    kp.normal_(generator=gen)
    vp.normal_(generator=gen)
    q = wl.q.to(dev)
    pt = wl.page_table.to(dev)
    sl = wl.seqlens.to(dev)
    out = torch.empty_like(q)
    B, Sq, Hq, D = q.shape
    Hkv = kp.shape[-2]

    def step(i):
        ops.block_attn(q, kp[i % layers], vp[i % layers], sl, wl.scale, page_table=pt,
                       page_size=wl.page_size, out=out)

    # graph replay must reproduce the eager result bit for bit (both kernels of the step)
    step(args.steps - 1)
    eager = out.clone()
    us = _time_graph(torch, step, args.steps, args.warmup)
    if not torch.equal(out, eager):
        raise RuntimeError("full-block decode: graph replay output differs from the eager call")
    nbytes = workloads.decode_bytes(wl.seqlens, Hq, Hkv, D, Sq)
    flops = workloads.decode_flops(wl.seqlens, Hq, D, Sq)
    gbs = nbytes / (us * 1e-6) / 1e9
    res = {
        "us_per_step": us,
        "bytes_per_step": nbytes,
        "flops_per_step": flops,
        "achieved_gbs": gbs,
        "tflops": flops / (us * 1e-6) / 1e12,
        "roofline": _roofline("hbm", gbs, HBM_PEAK_GBS, "GB/s", _traffic("kv_attn_decode_full_bs16")),
    }
    del q, kp, vp, pt, sl, out
    torch.cuda.empty_cache()
    return res


def cpu_baseline_decode(torch, wl, warmup: int = 10, measured: int = 50, what: str = "the full bs16 batch"):
    """Reference CPU path (SDPA shim) on the same bs16 inputs, bf16, contiguous static cache."""
    from oracle import attention as oa

    B, Sq, Hq, D = wl.q.shape
    Hkv = wl.k_pool.shape[-2]
    max_s = int(wl.seqlens.max())
    layer_k, layer_v = wl.k_pool, wl.v_pool
    k = torch.zeros(B, max_s, Hkv, D, dtype=wl.q.dtype)
    v = torch.zeros_like(k)
    for b in range(B):
        L = int(wl.seqlens[b])
        pos = torch.arange(L)
        pages = wl.page_table[b, pos // wl.page_size].long()
        k[b, :L] = layer_k[pages, pos % wl.page_size]
        v[b, :L] = layer_v[pages, pos % wl.page_size]
    st = _cpu_protocol(torch, lambda: oa.sdpa_kvcache(wl.q, k, v, wl.seqlens, scaling=wl.scale), warmup, measured)
    return _cpu_result(st, "us/step", f"SDPA shim (tests/test_focus.py:205-228 restated in oracle/attention.py), "
                       f"bf16, {what} of one layer, contiguous [16, {max_s}, 4, 128] cache")


# ---------------------------------------------------------------------------
def bench_gather(torch, args):
    from fast_v2_amd import _ffi, ops, workloads

    dev = torch.device("cuda", 0)
    wl = workloads.gather_rmsnorm_rows(seed=0)
    # 48 copies of the 29 MB hidden states: the rows one cycle touches (48 x 7.3 MB) exceed
    # the 256 MB last-level cache, so every call reads its rows from HBM
    copies = 48
    hs = [wl.hidden.to(dev)]
    for _ in range(copies - 1):
        hs.append(hs[0].clone())
    idx = wl.indices.to(dev)
    w = wl.weight.to(dev)
    res = {}
    for name, with_g in (("normed", False), ("pair", True)):
        def step(i, with_g=with_g):
            ops.gather_rmsnorm(hs[i % copies], idx, w, wl.eps, _ffi.NORM_WEIGHT_AFTER_CAST, with_g)
        steps = args.gather_steps
        us = _time_graph(torch, step, steps, min(args.warmup, 32))
        T, H = idx.shape[1], wl.hidden.shape[2]
        nbytes = workloads.gather_bytes(T, H, 2, with_gathered=with_g)
        gbs = nbytes / (us * 1e-6) / 1e9
        res[name] = {"us_per_call": us, "bytes_per_call": nbytes, "achieved_gbs": gbs,
                     "roofline": _roofline("hbm", gbs, HBM_PEAK_GBS, "GB/s",
                                           _traffic(f"gather_rmsnorm_{name}"))}
    # The practical ceiling of a call this size, timed the same way (graph of the same
    # number of nodes, inputs rotated through the same 48 HBM-resident slabs): a plain
    # gathered copy of the same rows (fdllm_probe_copy_rows: dst[t] = hidden[idx[t]], one
    # wave per row, all loads before the stores; the normed call's bytes less the 15 KB of
    # weight and indices), and an empty kernel node (torch.cuda._sleep(0)).
    T, H, S = idx.shape[1], wl.hidden.shape[2], wl.hidden.shape[1]
    dst = torch.empty((T, H), dtype=wl.hidden.dtype, device=dev)
    probes = _probes()

    def copy_step(i):
        rc = probes.fdllm_probe_copy_rows(hs[i % copies].data_ptr(), H * 2, S, idx.data_ptr(), dst.data_ptr(), T,
                                          H * 2, _stream_ptr(torch))
        if rc != 0:
            raise RuntimeError(f"fdllm_probe_copy_rows failed ({rc})")

    copy_step(0)
    torch.cuda.synchronize()
    if not torch.equal(dst, wl.hidden[0, wl.indices[0]].to(dev)):
        raise RuntimeError("the probe copy does not reproduce the gathered rows")
    us_copy = _time_graph(torch, copy_step, args.gather_steps, min(args.warmup, 32))
    us_empty = _time_graph(torch, lambda i: torch.cuda._sleep(0), args.gather_steps, min(args.warmup, 32))
    copy_bytes = 2 * T * H * 2
    res["ceiling"] = {
        "copy_us_per_call": us_copy, "copy_bytes": copy_bytes,
        "copy_gbs": copy_bytes / (us_copy * 1e-6) / 1e9,
        "empty_kernel_us_per_node": us_empty,
        "normed_vs_copy": res["normed"]["us_per_call"] / us_copy,
        "note": ("gathered copy of the 1024 x 3584 bf16 rows by a hand-written gfx950 kernel "
                 "(fdllm_probe_copy_rows: one wave per row, every load issued before the stores; read + "
                 "write, the normed call's bytes less the 15 KB of weight and indices) and an empty kernel "
                 "node, each as a graph of the same length as the gather's"),
    }
    del hs, dst
    torch.cuda.empty_cache()
    return res


def bench_scatter(torch, args):
    """The row scatter at the gather's size (scatter_and_return_cuda,
    fused_gather_norm.cu:79-119): 1024 rows of 3584 bf16 written back to two
    [1, 4096, 3584] destinations (the block cache and the current hidden states). The
    values and destination pairs rotate through 24 sets (24 x 66 MB), so every call reads
    and writes HBM rather than the last-level cache."""
    from fast_v2_amd import ops, workloads

    dev = torch.device("cuda", 0)
    wl = workloads.gather_rmsnorm_rows(seed=0)
    B, S, H = wl.hidden.shape
    T = wl.indices.shape[1]
    sets = 24
    g = torch.Generator().manual_seed(1)
    vals0 = torch.randn(B, T, H, generator=g).to(wl.hidden.dtype)
    vals = [vals0.to(dev)] + [torch.empty_like(vals0, device=dev) for _ in range(sets - 1)]
    for v in vals[1:]:
        v.copy_(vals[0])
    caches = [wl.hidden.to(dev) for _ in range(sets)]
    curs = [c.clone() for c in caches]
    idx = wl.indices.to(dev)

    def step(i):
        j = i % sets
        ops.scatter_rows(vals[j], idx, caches[j], curs[j])

    # bit-exact against torch's scatter_ on the first set
    step(0)
    torch.cuda.synchronize()
    exp = wl.hidden.clone().scatter_(1, wl.indices.unsqueeze(-1).expand(-1, -1, H), vals0).to(dev)
    if not (torch.equal(caches[0], exp) and torch.equal(curs[0], exp)):
        raise RuntimeError("scatter: the destinations differ from torch's scatter_")
    us = _time_graph(torch, step, args.gather_steps, min(args.warmup, 32))
    nbytes = workloads.scatter_bytes(T, H, 2, destinations=2)
    gbs = nbytes / (us * 1e-6) / 1e9
    res = {"us_per_call": us, "bytes_per_call": nbytes, "achieved_gbs": gbs,
           "roofline": _roofline("hbm", gbs, HBM_PEAK_GBS, "GB/s", _traffic("scatter_rows")),
           "shape": {"rows": T, "hidden": H, "seq_len": S, "destinations": 2, "dtype": "bf16"}}
    del vals, caches, curs, exp
    torch.cuda.empty_cache()
    return res


def bench_prefill(torch, args):
    from fast_v2_amd import _ffi, ops, workloads

    dev = torch.device("cuda", 0)
    wl = workloads.block_prefill(seed=0)
    q, k, v = wl.q.to(dev), wl.k.to(dev), wl.v.to(dev)
    B, S, Hq, D = q.shape
    Hkv = k.shape[2]
    kc = torch.zeros(B, S, Hkv, D, dtype=q.dtype, device=dev)
    vc = torch.zeros_like(kc)
    sl = torch.full((B,), S, dtype=torch.int32, device=dev)
    out = torch.empty_like(q)

    def whole_call(i):
        # the whole 4 x 4096-token prefill call: the K/V rows stored into the cache and the attention, in
        # one fdllm_kv_attn_fwd (the prefill kernel stores the rows itself)
        ops.block_attn(q, kc, vc, sl, wl.scale, mask_mode=_ffi.MASK_BLOCK_CAUSAL, mask_block=wl.block, out=out,
                       k_new=k, v_new=v)

    def copy_kernel_write(i):
        # the same call with the rows stored by a copy kernel ahead of the prefill kernel
        ops.block_attn(q, kc, vc, sl, wl.scale, mask_mode=_ffi.MASK_BLOCK_CAUSAL, mask_block=wl.block, out=out,
                       k_new=k, v_new=v, cache_write_kernel=True)

    def attn_only(i):
        ops.block_attn(q, kc, vc, sl, wl.scale, mask_mode=_ffi.MASK_BLOCK_CAUSAL, mask_block=wl.block, out=out)

    steps = args.prefill_steps
    whole_call(0)
    if not torch.equal(kc, k) or not torch.equal(vc, v):
        raise RuntimeError("prefill: the call left a cache that differs from the new K/V rows")
    kc.zero_()
    vc.zero_()
    copy_kernel_write(0)
    if not torch.equal(kc, k) or not torch.equal(vc, v):
        raise RuntimeError("prefill: the copy-kernel cache write left a cache that differs from the new K/V rows")
    # the three forms timed in rotation (a form timed first, right after other work, ran
    # 10-15 us slower than in a later slot): three rounds, the median per form
    us = _time_graphs_rotating(torch, {"call": whole_call, "attn": attn_only, "copy": copy_kernel_write},
                               steps, 2, rounds=3)
    us_full, us_attn, us_copy = us["call"], us["attn"], us["copy"]
    flops = workloads.prefill_flops(B, S, Hq, D, wl.block)
    nbytes = workloads.prefill_bytes(B, S, Hq, Hkv, D)
    tf = flops / (us_full * 1e-6) / 1e12
    res = {"us_per_call": us_full, "us_attention_only": us_attn, "us_copy_kernel_then_attention": us_copy,
           "flops": flops, "bytes_with_cache_write": nbytes,
           "roofline": _roofline("mfma", tf, MFMA_BF16_PEAK_TFLOPS, "TFLOP/s", _traffic("kv_attn_prefill_fused")),
           "tflops_attention_only": flops / (us_attn * 1e-6) / 1e12}
    del q, k, v, kc, vc, out
    torch.cuda.empty_cache()
    return res


def bench_mfma_ceiling(torch):
    """Sustained bf16 MFMA rate of this GPU, the ceiling the MFMA-bound calls (prefill,
    full-block step) are compared with beside the nominal peak: fdllm_probe_mfma, one
    workgroup per compute unit, one wave per SIMD, four independent
    v_mfma_f32_32x32x16_bf16 chains per wave on register operands (the prefill kernel's
    instruction), no memory traffic. HIP events on the stream the probe runs on; the
    median of five launches after one untimed."""
    import statistics

    dev = torch.device("cuda", 0)
    wgs = torch.cuda.get_device_properties(dev).multi_processor_count
    rounds = 8192
    sink = torch.zeros(wgs * 256, dtype=torch.float32, device=dev)
    probes = _probes()

    def launch():
        rc = probes.fdllm_probe_mfma(wgs, rounds, sink.data_ptr(), _stream_ptr(torch))
        if rc != 0:
            raise RuntimeError(f"fdllm_probe_mfma failed ({rc})")

    launch()
    torch.cuda.synchronize()
    times = []
    for _ in range(5):
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        launch()
        end.record()
        end.synchronize()
        times.append(start.elapsed_time(end) * 1e3)
    us = statistics.median(times)
    flops = wgs * 4 * rounds * 4 * 32768
    return {"tflops": flops / (us * 1e-6) / 1e12, "us": us, "workgroups": wgs, "rounds_per_wave": rounds,
            "note": ("fdllm_probe_mfma: the rate v_mfma_f32_32x32x16_bf16 sustains on every SIMD at once "
                     "(the clock runs below its nominal 2.4 GHz under sustained MFMA load); roofline.peak "
                     "stays the published 2500 TFLOP/s")}


def bench_small_fp32(torch, args):
    """The small fp32 decode on the GPU: the fp32 attention kernel on the fp32 workload (batch 1, 32
    queries x 12 / 2 heads over 512 + 32 keys, head_dim 128), the call as the caller
    makes it (one graph node per call)."""
    from fast_v2_amd import ops, workloads

    dev = torch.device("cuda", 0)
    wl = workloads.kv_decode_fp32_small(seed=0)
    q, k, v, sl = wl.q.to(dev), wl.k_cache.to(dev), wl.v_cache.to(dev), wl.seqlens.to(dev)
    out = torch.empty_like(q)

    def step(i):
        ops.block_attn(q, k, v, sl, wl.scale, out=out)
    step(0)
    eager = out.clone()
    us = _time_graph(torch, step, 200, 4)
    if not torch.equal(out, eager):
        raise RuntimeError("fp32 attention: graph replay output differs from the eager call")
    flops = 4 * 32 * 12 * 128 * 544
    return {"us_per_call": us, "gflops": flops / (us * 1e-6) / 1e9,
            "workload": "fp32, q [1, 32, 12, 128] over 544 keys of 2 KV heads (kv_attn_f32_kernel)"}


def bench_qkv(torch, args):
    """The q / k / v projections of one 7B-layout layer with RoPE and the static-cache
    write: the fused kernel (ops.qkv_rope_kv_write) against three nn.Linear GEMMs +
    ops.rope_kv_write, for the full-block (16 x 32), sub-block (16 x 8) and a 4 x 512
    prefill forward; 28 layers' weights cycled so each call reads its weights from HBM,
    both forms timed in rotation. Not part of the default run (``--only qkv``)."""
    from fast_v2_amd import ops

    dev = torch.device("cuda", 0)
    H, Hq, Hkv, D, layers = 3584, 28, 4, 128, 28
    g = torch.Generator(device=dev).manual_seed(0)
    W = [[(torch.randn(n * D, H, device=dev, generator=g) * 0.02).to(torch.bfloat16) for n in (Hq, Hkv, Hkv)]
         for _ in range(layers)]
    Bs = [[(torch.randn(n * D, device=dev, generator=g) * 0.1).to(torch.bfloat16) for n in (Hq, Hkv, Hkv)]
          for _ in range(layers)]
    res = {}
    for B, S in ((16, 32), (16, 8), (4, 512)):
        x = torch.randn(B, S, H, device=dev, generator=g).to(torch.bfloat16)
        inv = 1.0 / (1e6 ** (torch.arange(0, D, 2, device=dev).float() / D))
        emb = torch.cat([torch.arange(S, device=dev).float()[:, None] * inv[None]] * 2, -1)
        cos, sin = emb.cos().to(torch.bfloat16)[None], emb.sin().to(torch.bfloat16)[None]
        kc = torch.zeros(B, S + 64, Hkv, D, dtype=torch.bfloat16, device=dev)
        vc = torch.zeros_like(kc)
        ws = torch.zeros(B, dtype=torch.int32, device=dev)

        def fused(i):
            w, b = W[i % layers], Bs[i % layers]
            ops.qkv_rope_kv_write(x, w[0], b[0], w[1], b[1], w[2], b[2], cos, sin, kc, vc, write_start=ws)

        def unfused(i):
            w, b = W[i % layers], Bs[i % layers]
            q = torch.nn.functional.linear(x, w[0], b[0]).view(B, S, Hq, D)
            k = torch.nn.functional.linear(x, w[1], b[1]).view(B, S, Hkv, D)
            v = torch.nn.functional.linear(x, w[2], b[2]).view(B, S, Hkv, D)
            ops.rope_kv_write(q, k, v, cos, sin, kc, vc, write_start=ws)
        us = _time_graphs_rotating(torch, {"fused": fused, "unfused": unfused}, 2 * layers, 2, rounds=3)
        flops = 2.0 * B * S * H * (Hq + 2 * Hkv) * D
        res[f"{B}x{S}"] = {"us_fused": us["fused"], "us_linear_then_rope": us["unfused"],
                           "tflops_fused": flops / (us["fused"] * 1e-6) / 1e12}
    del W, Bs
    torch.cuda.empty_cache()
    return res


def bench_e2e(torch, args):
    """End-to-end block-diffusion generation with the random-init 7B-layout model on the
    HIP path: batch 16, 512-token prompts, ``--e2e-tokens`` new tokens, 32-token blocks,
    8-token sub-blocks, threshold 0.9, block cache on. tokens/s = generated tokens /
    generation wall time (eval.py:425-429); one short untimed run first."""
    from fast_v2_amd.e2e import model as em
    from fast_v2_amd.e2e import sampler as es

    dev = torch.device("cuda", 0)
    t0 = time.perf_counter()
    if args.e2e_weights:
        from fast_v2_amd.e2e import weights as ew
        model = ew.load_model(args.e2e_weights, dev)
        cfg = model.config
    else:
        cfg = em.BlockDiffusionConfig()
        model = em.build_model(cfg, dev)
    torch.cuda.synchronize()
    build_s = time.perf_counter() - t0
    g = torch.Generator().manual_seed(0)
    x = torch.randint(0, cfg.vocab_size - 1, (16, 512), generator=g).to(dev)
    # GEMM solutions: torch TunableOp benchmarks the hipBLASLt / rocBLAS candidates of
    # every GEMM shape the warm-up meets (prefill, full block, sub-block, commit) and
    # keeps the fastest; tuning is off again before the timed run
    tun = torch.cuda.tunable
    tun.enable(True)
    tun.tuning_enable(True)
    tun.set_filename(os.path.join(tempfile.gettempdir(), f"fdllm_tunableop_{os.getpid()}_%d.csv"))
    _log(f"e2e: model built in {build_s:.1f} s; warm-up with GEMM tuning")
    last = [time.perf_counter()]

    def progress(stats, phase):
        # one line at most every 20 s, written when a forward has been issued
        now = time.perf_counter()
        if now - last[0] >= 20.0:
            last[0] = now
            _log(f"e2e {phase}: {stats.forwards} forwards, {stats.commits} commits")
    es.generate(model, x, max_new_tokens=64, use_block_cache=True,
                progress=lambda st_: progress(st_, "warm-up"))  # warm-up (and GEMM tuning)
    tun.tuning_enable(False)
    _log("e2e: timed generation")
    out, st = es.generate(model, x, max_new_tokens=args.e2e_tokens, use_block_cache=True,
                          progress=lambda st_: progress(st_, "timed run"))
    # the same generation with the q / k / v projections in the RoPE + cache-write kernel
    # (off by default: its projections differ from the library GEMM's in the last bit)
    _log("e2e: timed generation with the fused q / k / v projections")
    out_f, st_f = es.generate(model, x, max_new_tokens=args.e2e_tokens, use_block_cache=True,
                              impl=es.HipStaticAttention(fused_qkv=True),
                              progress=lambda st_: progress(st_, "timed run, fused projections"))
    tun.enable(False)
    res = {"tokens_per_s": round(st.tokens_per_second, 1),
           "tokens_per_s_fused_qkv_projection": round(st_f.tokens_per_second, 1),
           "generated_tokens": st.generated_tokens,
           "seconds": round(st.seconds, 3), "forwards": st.forwards, "commits": st.commits,
           "ms_per_forward": round(st.seconds * 1e3 / max(st.forwards, 1), 3),
           "tokens_per_step": round(sum(st.step_tokens) / max(len(st.step_tokens), 1), 3),
           "params": em.param_count(cfg), "model_build_s": round(build_s, 2),
           "gemm_tuning": "torch TunableOp over hipBLASLt / rocBLAS solutions, tuned in the warm-up",
           "forwards_graphed": "diffusion steps and commits replayed from HIP graphs; the prompt prefill runs eagerly (once per generation)",
           "weights": args.e2e_weights or ("random init (N(0, 0.02), zero biases, unit norms) except the mask "
                                           "token's lm_head row, which is zero: a random model may otherwise "
                                           "predict the mask token, which the unmask rule writes back, and the "
                                           "block never completes"),
           "config": "28 layers, hidden 3584, 28/4 heads, vocab 152064, bf16; batch 16, prompt 512, "
                     f"{args.e2e_tokens} new tokens, block 32, sub-block 8, threshold 0.9 (p > 0.9), block cache on"}
    del model, out, out_f, x
    torch.cuda.empty_cache()
    return res


def calibrate_copies(torch):
    """Plain torch device copies (read N + write N bytes) timed the same way as the
    kernels: the practical bandwidth of a kernel of that size, launch gap included."""
    res = {}
    for mb in (7, 48, 256, 1024):
        n = mb << 20
        bufs = [torch.empty(n, dtype=torch.uint8, device="cuda") for _ in range(4 if mb < 256 else 2)]
        dsts = [torch.empty(n, dtype=torch.uint8, device="cuda") for _ in bufs]

        def step(i):
            dsts[i % len(bufs)].copy_(bufs[i % len(bufs)])
        steps = 200 if mb < 256 else 20
        us = _time_graph(torch, step, steps, 4)
        res[f"copy_{mb}MiB"] = {"us": round(us, 2), "GBs_read_plus_write": round(2 * n / (us * 1e-6) / 1e9, 1)}
        del bufs, dsts
    torch.cuda.empty_cache()
    # the decode step's read pattern at a size where its fixed phases no longer count:
    # fdllm_probe_read_kv over a contiguous [64, 4096, 4, 128] bf16 cache (537 MB of K and
    # V), stored head-major (one KV head's keys one contiguous run, as the head-major pages
    # of the headline step) or token-major (a head's key rows 256 B at a 1 KB stride), the
    # keys dealt over 64 / 128 / 256 slots per KV head (1 / 2 / 4 workgroups of 512
    # threads per compute unit)
    probes = _probes()
    B, S, H, D = 64, 4096, 4, 128
    sl = torch.full((B,), S, dtype=torch.int32, device="cuda")
    sink = torch.zeros(4, dtype=torch.int32, device="cuda")
    n = B * S * H * D * 2 * 2
    for layout in ("head_major", "token_major"):
        if layout == "head_major":
            k = torch.randn(B, H, S, D, device="cuda").to(torch.bfloat16).transpose(1, 2)
        else:
            k = torch.randn(B, S, H, D, device="cuda").to(torch.bfloat16)
        v = torch.randn_like(k)  # the same strides as k
        ks, vs = k.stride(), v.stride()
        for slots in (64, 128, 256):
            def step(i, slots=slots, k=k, v=v, ks=ks, vs=vs):
                rc = probes.fdllm_probe_read_kv(k.data_ptr(), v.data_ptr(), ks[0], ks[1], ks[2], vs[0], vs[1],
                                                vs[2], None, 0, 0, sl.data_ptr(), B, H, slots, sink.data_ptr(),
                                                _stream_ptr(torch))
                if rc != 0:
                    raise RuntimeError(f"fdllm_probe_read_kv failed ({rc})")
            us = _time_graph(torch, step, 20, 4)
            res[f"read_kv_537MB_{layout}_{slots}_slots"] = {"us": round(us, 2),
                                                            "GBs_read": round(n / (us * 1e-6) / 1e9, 1)}
        del k, v
    # the headline's sub-block decode step at four times the length, where its fixed phases
    # (partition, first tiles, split merge) count less, beside the plain read of the same
    # rows: batch 16, prefixes U{8192..16352} step 32 + the 32-token block, 64-token pages
    # (16 x 256 page-table entries, the staging both the kernel and the probe take), 28 / 4
    # heads, 8 active queries, head-major pages, 2 layer pools (> 600 MB) cycled
    from fast_v2_amd import ops as _ops, workloads as _wls
    wl = _wls.kv_decode_paged(seed=0, batch=16, min_prefix=8192, max_prefix=16352, page_size=64)
    L = 2
    kpool = torch.empty((L,) + tuple(wl.k_pool.shape), dtype=torch.bfloat16, device="cuda")
    kpool = kpool.permute(0, 1, 3, 2, 4).contiguous().permute(0, 1, 3, 2, 4)  # head-major pages
    vpool = torch.empty_like(kpool)
    gen = torch.Generator(device="cuda").manual_seed(5)
    kpool.normal_(generator=gen)
    vpool.normal_(generator=gen)
    q64, pt64, sl64 = wl.q.to("cuda"), wl.page_table.to("cuda"), wl.seqlens.to("cuda")
    out64 = torch.empty_like(q64)

    def dstep(i):
        _ops.block_attn(q64, kpool[i % L], vpool[i % L], sl64, wl.scale, page_table=pt64, page_size=wl.page_size,
                        out=out64)

    def rstep(i):
        k_, v_ = kpool[i % L], vpool[i % L]
        ks_, vs_ = k_.stride(), v_.stride()
        rc = probes.fdllm_probe_read_kv(k_.data_ptr(), v_.data_ptr(), ks_[0], ks_[1], ks_[2], vs_[0], vs_[1], vs_[2],
                                        pt64.data_ptr(), pt64.shape[1], wl.page_size, sl64.data_ptr(), 16,
                                        k_.shape[-2], 64, sink.data_ptr(), _stream_ptr(torch))
        if rc != 0:
            raise RuntimeError(f"fdllm_probe_read_kv failed ({rc})")
    nb64 = _wls.decode_bytes(wl.seqlens, q64.shape[2], kpool.shape[-2], q64.shape[3], q64.shape[1])
    ud = _time_graph(torch, dstep, 40, 4)
    ur = _time_graph(torch, rstep, 40, 4)
    rb64 = int(wl.seqlens.sum()) * kpool.shape[-2] * 128 * 2 * 2
    res["decode_bs16_long"] = {"us": round(ud, 2), "bytes": nb64, "GBs": round(nb64 / (ud * 1e-6) / 1e9, 1),
                          "read_us": round(ur, 2), "read_GBs": round(rb64 / (ur * 1e-6) / 1e9, 1),
                          "step_vs_read": round(ud / ur, 3)}
    del kpool, vpool
    torch.cuda.empty_cache()
    # the gather + RMSNorm call and the gathered copy of the same rows at more rows, where
    # the call's fixed cost (launch, index load, one row round trip) counts less: rows of
    # 3584 bf16 drawn from [1, 2 x rows, 3584] hidden states, enough slabs cycled (>= 600
    # MB) that every call reads its rows from HBM, not from the 256 MB last-level cache
    from fast_v2_amd import _ffi, ops, workloads
    for rows in (1024, 4096, 16384):
        wl = workloads.gather_rmsnorm_rows(seed=0, seq_len=2 * rows, rows=rows)
        n_slabs = max(4, -(-600_000_000 // wl.hidden.numel() // 2))
        slabs = [wl.hidden.to("cuda")]
        slabs += [slabs[0].clone() for _ in range(n_slabs - 1)]
        idx, w = wl.indices.to("cuda"), wl.weight.to("cuda")
        H = wl.hidden.shape[2]
        dst = torch.empty(rows, H, dtype=torch.bfloat16, device="cuda")

        def gstep(i, slabs=slabs, idx=idx, w=w, wl=wl):
            ops.gather_rmsnorm(slabs[i % len(slabs)], idx, w, wl.eps, _ffi.NORM_WEIGHT_AFTER_CAST, False)

        def cstep(i, slabs=slabs, idx=idx, dst=dst, rows=rows, H=H):
            rc = probes.fdllm_probe_copy_rows(slabs[i % len(slabs)].data_ptr(), H * 2, 2 * rows, idx.data_ptr(),
                                              dst.data_ptr(), rows, H * 2, _stream_ptr(torch))
            if rc != 0:
                raise RuntimeError(f"fdllm_probe_copy_rows failed ({rc})")
        nb = workloads.gather_bytes(rows, H, 2)
        steps = 200 if rows < 16384 else 50
        ug = _time_graph(torch, gstep, steps, 4)
        uc = _time_graph(torch, cstep, steps, 4)
        res[f"gather_rmsnorm_{rows}_rows"] = {"us": round(ug, 2), "GBs": round(nb / (ug * 1e-6) / 1e9, 1),
                                              "copy_us": round(uc, 2),
                                              "copy_GBs": round((nb - H * 2 - rows * 8) / (uc * 1e-6) / 1e9, 1),
                                              "slabs": n_slabs}
        del slabs, dst
    torch.cuda.empty_cache()
    return res


def _cpu_protocol(torch, fn, warmup: int = 10, measured: int = 50):
    """The reference's timing protocol (tests/bench_compile.py:179-214): `warmup`
    untimed calls, then `measured` timed ones; median and the mean after dropping the
    fastest and slowest 10 %. Threads: every core this process may run on."""
    torch.set_num_threads(len(os.sched_getaffinity(0)))
    for _ in range(warmup):
        fn()
    lat = []
    for _ in range(measured):
        t0 = time.perf_counter()
        fn()
        lat.append(time.perf_counter() - t0)
    lat.sort()
    trim = max(1, len(lat) // 10)
    kept = lat[trim:-trim]
    return {"median_us": round(lat[len(lat) // 2] * 1e6, 1),
            "trimmed_mean_us": round(sum(kept) / len(kept) * 1e6, 1),
            "warmup": warmup, "measured": measured, "cores": torch.get_num_threads()}


def _cpu_result(st, unit: str, sample: str, scale: float = 1.0):
    """cpu_baseline object: value = median x scale (the sample's share of the workload)."""
    return {"value": round(st["median_us"] * scale, 1), "unit": unit, "cores": st["cores"], "kind": "port",
            "median_us_sample": st["median_us"], "trimmed_mean_us_sample": st["trimmed_mean_us"],
            "protocol": f"{st['warmup']} warm-up + {st['measured']} timed calls; median, 10 %-trimmed mean",
            "sample": sample}


def cpu_baseline_gather(torch):
    """Reference CPU path for gather + RMSNorm: ref_gather_input_rmsnorm
    (cuda_bench/test_correctness.py:33-50) on the full bf16 [4096 x 3584] / 1024-row call."""
    from fast_v2_amd import workloads
    from oracle import gather_rmsnorm as og

    wl = workloads.gather_rmsnorm_rows(seed=0)
    st = _cpu_protocol(torch, lambda: og.ref_gather_input_rmsnorm(wl.hidden, wl.indices, wl.weight, wl.eps))
    return _cpu_result(st, "us/call", "ref_gather_input_rmsnorm (cuda_bench/test_correctness.py:33-50 restated in "
                       "oracle/gather_rmsnorm.py), the whole call (gathered + normed outputs)")


def cpu_baseline_scatter(torch):
    """Reference CPU path for the row scatter: torch's scatter_ (the reference's PyTorch
    statement of this step, cuda_bench/bench_sparse_cuda.py:88-96) into both destinations
    of scatter_and_return_cuda, bf16 [1, 4096, 3584], 1024 rows; the whole call."""
    from fast_v2_amd import workloads

    wl = workloads.gather_rmsnorm_rows(seed=0)
    H = wl.hidden.shape[2]
    vals = torch.randn(1, wl.indices.shape[1], H, generator=torch.Generator().manual_seed(1)).to(wl.hidden.dtype)
    cache, cur = wl.hidden.clone(), wl.hidden.clone()
    ii = wl.indices.unsqueeze(-1).expand(-1, -1, H)

    def call():
        cache.scatter_(1, ii, vals)
        cur.scatter_(1, ii, vals)
    st = _cpu_protocol(torch, call)
    return _cpu_result(st, "us/call", "torch CPU scatter_ of the 1024 bf16 rows into both [1, 4096, 3584] "
                       "destinations (cuda_bench/bench_sparse_cuda.py:88-96, applied to the cache and the "
                       "current hidden states as scatter_and_return_cuda writes them), the whole call")


def cpu_baseline_prefill(torch):
    """Reference CPU path for block-causal prefill: SDPA with the block-causal bool mask
    (modeling.py:145-150, :398-411) on sequence 0 of the 4; value = 4 x that time."""
    from fast_v2_amd import workloads
    from oracle import attention as oa

    wl = workloads.block_prefill(seed=0)
    q, k, v = wl.q[:1], wl.k[:1], wl.v[:1]
    st = _cpu_protocol(torch, lambda: oa.sdpa_block_causal(q, k, v, wl.block, scaling=wl.scale))
    return _cpu_result(st, "us/call", "SDPA with the block-causal mask (oracle/attention.py sdpa_block_causal), "
                       "bf16, sequence 0 of the 4 ([1, 4096, 28, 128] against 4 KV heads); value = 4 x the "
                       "sample's median (the sequences are the same size)", scale=4.0)


def cpu_baseline_small_fp32(torch):
    """The small fp32 decode on the CPU: the SDPA shim in fp32, batch 1, 12 / 2 heads, 512 prefix + 32
    block keys, 32 queries (the reference's only CPU statement of the kv-cache attention)."""
    from fast_v2_amd import workloads
    from oracle import attention as oa

    wl = workloads.kv_decode_fp32_small(seed=0)
    st = _cpu_protocol(torch, lambda: oa.sdpa_kvcache(wl.q, wl.k_cache, wl.v_cache, wl.seqlens, scaling=wl.scale))
    flops = 4 * 32 * 12 * 128 * 544
    res = _cpu_result(st, "us/call", "SDPA shim (tests/test_focus.py:205-228 restated in oracle/attention.py), "
                      "fp32, q [1, 32, 12, 128] over 544 keys of 2 KV heads, the whole call")
    res["gflops"] = round(flops / (st["median_us"] * 1e-6) / 1e9, 2)
    return res


def cpu_baseline_e2e_step(torch):
    """The end-to-end generation step on the CPU (the whole 7B model at batch 16 does not fit a bounded sample):
    one decoder layer of the random-init 7B-layout model running a sub-block diffusion
    step (16 sequences x 8 tokens at positions 512..519, attention over the 512-token
    prompt plus the 32-token block through the SDPA shim, the reference's eager path
    restated in oracle/e2e_eager.py), and the lm_head over the same 128 rows; value =
    28 x layer + lm_head, an extrapolation from the two timed pieces."""
    from fast_v2_amd.e2e import model as em
    from oracle.e2e_eager import TorchKVCache, eager_attention_forward

    cfg = em.BlockDiffusionConfig()
    B, S, P = 16, 8, 512
    g = torch.Generator().manual_seed(0)
    dt = torch.bfloat16
    with torch.no_grad():
        layer = em.DecoderLayer(cfg, 0).to(dt)
        for mod in layer.modules():
            if isinstance(mod, torch.nn.Linear):
                mod.weight.normal_(0.0, cfg.initializer_range, generator=g)
                if mod.bias is not None:
                    mod.bias.zero_()
        lm_head = torch.nn.Linear(cfg.hidden_size, cfg.vocab_size, bias=False).to(dt)
        lm_head.weight.normal_(0.0, cfg.initializer_range, generator=g)
    layer.self_attn.forward = eager_attention_forward(layer.self_attn, False)
    cache = TorchKVCache(B, P + 64, 1, cfg.num_key_value_heads, cfg.head_dim, dt, "cpu")
    cache.key_cache[0].normal_(generator=g)
    cache.value_cache[0].normal_(generator=g)
    cache.set_kv_write_start(P)
    cache.set_scratch_seqlens(P + cfg.bd_size)
    h = torch.randn(B, S, cfg.hidden_size, generator=g).to(dt)
    d = cfg.head_dim
    inv_freq = 1.0 / (cfg.rope_theta ** (torch.arange(0, d, 2, dtype=torch.float32) / d))
    freqs = torch.arange(P, P + S).float()[:, None] * inv_freq[None, :]
    emb = torch.cat((freqs, freqs), dim=-1)
    pe = (emb.cos().to(dt)[None], emb.sin().to(dt)[None])

    def run_layer():
        with torch.no_grad():
            hh, m = layer(h, pe, cache, False, None, None)
            hh + m

    def run_head():
        with torch.no_grad():
            lm_head(h)
    st_l = _cpu_protocol(torch, run_layer)
    st_h = _cpu_protocol(torch, run_head)
    per_step = cfg.num_hidden_layers * st_l["median_us"] + st_h["median_us"]
    tokens_per_s = B / (per_step * 1e-6)  # at least one token per sequence per step
    return {"value": round(per_step, 1), "unit": "us/diffusion step (extrapolated)", "cores": st_l["cores"],
            "kind": "port", "layer": st_l, "lm_head": st_h,
            "tokens_per_s_at_one_token_per_row_per_step": round(tokens_per_s, 2),
            "sample": ("one decoder layer (eager torch + SDPA shim, bf16) on a 16 x 8-token sub-block step "
                       "over 544 visible keys, and the lm_head on the same 128 rows; value = 28 x layer median "
                       "+ lm_head median (extrapolated to the 28-layer model; embedding and final norm left out)")}


# ---------------------------------------------------------------------------
def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1120, help="timed attention steps (multiple of 28 keeps layers balanced)")
    ap.add_argument("--warmup", type=int, default=56)
    ap.add_argument("--gather-steps", type=int, default=2000)
    ap.add_argument("--prefill-steps", type=int, default=20)
    ap.add_argument("--kv-split", type=int, default=0, help="keys per split-KV work item (0 = automatic)")
    ap.add_argument("--layers", type=int, default=LAYERS, help="layer pools cycled by the decode steps")
    ap.add_argument("--layout", choices=["paged", "paged_hm", "contig", "bhsd"], default="paged_hm",
                    help="KV layout: 32-token pages (token-major), 32-token pages stored head-major, the "
                         "contiguous [B, max_S, Hkv, D] static cache, or the same cache stored head-major")
    ap.add_argument("--balanced-splits", action="store_true",
                    help="decode: deal all sequences' keys evenly over the workgroups (runs across sequences)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--only", choices=["decode", "decode_full", "gather", "scatter", "prefill", "e2e", "qkv"],
                    default=None)
    ap.add_argument("--e2e-tokens", type=int, default=1024, help="tokens generated in the end-to-end leg")
    ap.add_argument("--no-e2e", action="store_true", help="skip the end-to-end generation leg")
    ap.add_argument("--e2e-weights", default=None,
                    help="local checkpoint directory (config.json + *.safetensors) instead of random weights")
    ap.add_argument("--calibrate", action="store_true",
                    help="also time plain device copies of the workloads' sizes (practical bandwidth floor)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="first run a plain 512 MiB device copy (for HBM counter calibration)")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this build targets one GPU: the block-decode attention and gather+RMSNorm "
                          "kernels run on one GPU's share; multi-GPU runs are not part of it",
                          "n_gpus": args.gpus}), flush=True)
        return 2

    import torch

    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}), flush=True)
        return 1
    from fast_v2_amd import _ffi
    _ffi.lib()  # fail loudly if the HIP library is missing

    if args.copy_calibration:
        src = torch.empty(512 << 20, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    calib = None
    if args.calibrate:
        calib = calibrate_copies(torch)
        _log(f"calibration: {json.dumps(calib)}")

    extra = {}
    decode = wl = None
    if args.only in (None, "decode"):
        decode, wl = bench_decode(torch, args)
        _log(f"decode: {decode['us_per_step']:.2f} us/step, {decode['achieved_gbs']:.0f} GB/s")
    if args.only in (None, "decode_full"):
        extra["block_decode_full"] = bench_decode_full(torch, args)
        _log(f"full-block decode: {extra['block_decode_full']['us_per_step']:.2f} us/step, "
             f"{extra['block_decode_full']['achieved_gbs']:.0f} GB/s, {extra['block_decode_full']['tflops']:.0f} TFLOP/s")
    if args.only in (None, "gather"):
        extra["gather_rmsnorm"] = bench_gather(torch, args)
        g = extra["gather_rmsnorm"]
        _log(f"gather: normed {g['normed']['us_per_call']:.3f} us, pair {g['pair']['us_per_call']:.3f} us; "
             f"plain copy of the rows {g['ceiling']['copy_us_per_call']:.3f} us, empty kernel node "
             f"{g['ceiling']['empty_kernel_us_per_node']:.3f} us")
    if args.only in (None, "scatter"):
        extra["scatter_rows"] = bench_scatter(torch, args)
        _log(f"scatter: {extra['scatter_rows']['us_per_call']:.3f} us, "
             f"{extra['scatter_rows']['achieved_gbs']:.0f} GB/s")
    if args.only is None:
        extra["small_fp32"] = bench_small_fp32(torch, args)
        _log(f"small fp32 decode (batch 1, 12 / 2 heads, 544 keys): {extra['small_fp32']['us_per_call']:.2f} us per call")
    if args.only in (None, "prefill"):
        extra["prefill"] = bench_prefill(torch, args)
        _log(f"prefill: {extra['prefill']['us_per_call']:.1f} us per call with the cache write, "
             f"{extra['prefill']['roofline']['achieved']:.0f} TFLOP/s")

    if "prefill" in extra or "block_decode_full" in extra:
        extra["mfma_ceiling"] = bench_mfma_ceiling(torch)
        mc = extra["mfma_ceiling"]["tflops"]
        if "prefill" in extra:
            extra["prefill"]["frac_of_measured_mfma_rate"] = extra["prefill"]["roofline"]["achieved"] / mc
        if "block_decode_full" in extra:
            extra["block_decode_full"]["frac_of_measured_mfma_rate"] = extra["block_decode_full"]["tflops"] / mc
        _log(f"MFMA ceiling: {mc:.0f} TFLOP/s sustained (bf16 32x32x16 on every SIMD)")
    if args.only == "qkv":
        extra["qkv_projection"] = bench_qkv(torch, args)
        _log("qkv: " + ", ".join(f"{k} fused {v['us_fused']:.1f} us / linear + rope {v['us_linear_then_rope']:.1f} us"
                                  for k, v in extra["qkv_projection"].items()))
    if args.only == "e2e" or (args.only is None and not args.no_e2e):
        extra["e2e"] = bench_e2e(torch, args)
        _log(f"e2e: {extra['e2e']['tokens_per_s']} tokens/s ({extra['e2e']['forwards']} forwards, "
             f"{extra['e2e']['seconds']} s)")

    cpu = None
    if decode is not None and not args.no_cpu_baseline:
        _log("cpu baseline (bs16 sub-block decode step) ...")
        cpu = cpu_baseline_decode(torch, wl)
        _log("cpu baseline (small fp32 decode, SDPA shim) ...")
        extra["small_fp32_cpu"] = cpu_baseline_small_fp32(torch)
    if not args.no_cpu_baseline:
        if "block_decode_full" in extra:
            _log("cpu baseline (bs16 full-block step) ...")
            from fast_v2_amd import workloads as _wls
            extra["block_decode_full"]["cpu_baseline"] = cpu_baseline_decode(
                torch, _wls.kv_decode_paged(seed=0, active=32), warmup=3, measured=15,
                what="the full bs16 batch with all 32 block queries")
        if "gather_rmsnorm" in extra:
            _log("cpu baseline (gather + RMSNorm) ...")
            extra["gather_rmsnorm"]["cpu_baseline"] = cpu_baseline_gather(torch)
        if "scatter_rows" in extra:
            _log("cpu baseline (row scatter) ...")
            extra["scatter_rows"]["cpu_baseline"] = cpu_baseline_scatter(torch)
        if "prefill" in extra:
            _log("cpu baseline (prefill sample) ...")
            extra["prefill"]["cpu_baseline"] = cpu_baseline_prefill(torch)
        if "e2e" in extra:
            _log("cpu baseline (end-to-end diffusion step, one layer + lm_head) ...")
            extra["e2e"]["cpu_baseline"] = cpu_baseline_e2e_step(torch)

    if decode is not None:
        us = decode["us_per_step"]
        line = {
            "metric": METRIC,
            "value": round(us, 3),
            "unit": "us/step",
            "n_gpus": 1,
            "steps": args.steps,
            "warmup": args.warmup,
            "ms_per_step": round(us / 1e3, 6),
            "higher_is_better": False,
            "scaling": "weak",
            "vs_baseline": None,
            "dtype": "bf16",
            "data": "synthetic",
            "config": {
                "workload": ("block-decode attention, 7B geometry: batch 16, 28 query / 4 KV heads, head_dim 128, "
                             "prefix U{1024..4096 step 32} + 32-token block, 8 active queries, 32-token pages "
                             + ("stored head-major ([Hkv, 32, D] per page)" if decode["layout"] == "paged_hm"
                                else f"({decode['layout']} layout)")
                             + ", one layer per step over 28 layer pools"),
                "batch": 16, "q_len": 8, "num_q_heads": 28, "num_kv_heads": 4, "head_dim": 128,
                "kv_layout": decode["layout"],
                "page_size": 32, "layers_cycled": LAYERS, "seqlens": decode["seqlens"],
            },
            "roofline": decode["roofline"],
            "cpu_baseline": cpu,
            "extra": {
                "decode": {k: decode[k] for k in ("bytes_per_step", "flops_per_step", "tflops",
                                                  "us_per_model_step_28_layers", "layout",
                                                  "us_per_step_token_major_pages",
                                                  "token_major_output_bit_identical", "ceiling") if k in decode},
                **extra,
            },
        }
    else:
        line = {"metric": METRIC, "value": None, "extra": extra}
    if calib is not None:
        line.setdefault("extra", {})["copy_calibration"] = calib
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
