"""Per-phase timeline of the split decode kernel on the bs16 sub-block decode step (16
sequences, 8 active queries, 28 query / 4 KV heads, head_dim 128, 32-token pages, the
prefix lengths of workloads.kv_decode_paged(seed=0)).

It loads the instrumented library lib/libfdllm_hip_timeline.so (the production sources
built with FDLLM_TIMELINE by `python -m fast_v2_amd.build --timeline`, beside
lib/libfdllm_hip.so; refused when it is older than a source), in which thread 0 of each
workgroup of kv_split_decode_kernel writes the device's 100 MHz real-time clock at the
end of each phase:

    0 start                      3 key loop done
    1 partition known            4 partial stored and arrival counted
    2 first K/V tiles in LDS        (output written, for a single-split unit)
                                 5 merge written (last workgroup of its unit)

and reports, over the workgroups of one call, when each phase ends relative to the
first workgroup's start, with the median over calls. The calls cycle over 28 layer
pools as the benchmark's decode leg does, so every call reads its K/V from HBM; each
call is preceded by a clear of the stamp buffer and a synchronisation, so the stamps
show the kernel alone (no overlap with the previous call's tail).

    python -m fast_v2_amd.timeline [--calls 56] [--layers 28] [--full-block]

With --full-block all 32 queries of the block are active (the full-block forward): the
call runs kv_prefill_ring_kernel in its split form, whose stamps are 0 start, 1
partition known, 2 first tiles and Q landed, 3 key loop done, 4 partial stores issued,
then the merge kernel (not stamped).
"""
from __future__ import annotations

import argparse
import ctypes
import os
import sys
from pathlib import Path

TIMELINE_LIB = Path(__file__).resolve().parent / "lib" / "libfdllm_hip_timeline.so"
TICK_US = 0.01  # s_memrealtime counts at 100 MHz
STAMPS = 8
MAX_WORKGROUPS = 16384
PHASES = ["start", "partition known", "first tiles in LDS", "key loop done", "partial stored + arrival",
          "merge written"]


def _stats(x):
    import numpy as np
    x = np.asarray(x, dtype=np.float64)
    if x.size == 0:
        return (float("nan"),) * 3
    return float(x.min()), float(np.median(x)), float(x.max())


def analyse(st):
    """Phase-end statistics (µs from the first start) of one call's stamp array [wg, 8]."""
    import numpy as np
    ran = st[:, 0] != 0
    st = st[ran]
    t0 = st[:, 0].min()
    rel = (st - t0).astype(np.float64) * TICK_US
    # a stamp counts only when written after the workgroup's own start in this call: with
    # --back-to-back the buffer is cleared once before the N calls, and a workgroup that
    # merged in an earlier call but not in the last keeps that call's (earlier) stamp
    active = (st[:, 3] != 0) & (st[:, 3] >= st[:, 0])
    merged = (st[:, 5] != 0) & (st[:, 5] >= st[:, 0])
    info = st[:, 6]
    ntiles = (info & 0xFFFF)[active]
    res = {"workgroups": int(ran.sum()), "active": int(active.sum()), "merging": int(merged.sum()),
           "tiles_per_workgroup": _stats(ntiles)}
    for i, name in enumerate(PHASES):
        sel = merged if i == 5 else (active if i >= 2 else np.ones(len(st), dtype=bool))
        res[name] = _stats(rel[sel, i])
    ends = np.where(merged, rel[:, 5], rel[:, 4])[active]
    res["span"] = float(ends.max())
    # durations of each phase per workgroup
    res["d_partition"] = _stats((rel[:, 1] - rel[:, 0])[active])
    res["d_first_tiles"] = _stats((rel[:, 2] - rel[:, 1])[active])
    res["d_loop"] = _stats((rel[:, 3] - rel[:, 2])[active])
    res["d_store_arrive"] = _stats((rel[:, 4] - rel[:, 3])[active])
    res["d_merge"] = _stats((rel[:, 5] - rel[:, 4])[merged])
    return res


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--calls", type=int, default=56)
    ap.add_argument("--layers", type=int, default=28)
    ap.add_argument("--full-block", action="store_true", help="all 32 block queries active")
    ap.add_argument("--token-major", action="store_true",
                    help="pages stored [page_size, Hkv, D] (default: head-major [Hkv, page_size, D])")
    ap.add_argument("--balanced-splits", action="store_true",
                    help="deal all sequences' keys evenly over the workgroups (runs across sequence boundaries)")
    ap.add_argument("--dump", default=None, help="also save every call's raw stamps [calls, workgroups, 8] (.npy)")
    ap.add_argument("--lib", default=None, help="instrumented library to load (default: lib/libfdllm_hip_timeline.so)")
    ap.add_argument("--prefix", type=int, default=None, help="every sequence's cached prefix (default: U{1024..4096})")
    ap.add_argument("--back-to-back", type=int, default=0, metavar="N",
                    help="time each sample as the last of N calls replayed back to back from a HIP graph "
                         "(the benchmark's regime) instead of one call from an idle GPU")
    args = ap.parse_args(argv)
    if "fast_v2_amd._ffi" in sys.modules:
        raise RuntimeError("fast_v2_amd.timeline must load the instrumented library before anything else loads "
                           "the production one: run it as its own process")
    lib_path = Path(args.lib) if args.lib else TIMELINE_LIB
    if args.lib is None:
        from . import build as _build
        if _build._stale(TIMELINE_LIB, _build.DEPS):  # missing, or older than a source
            raise RuntimeError(f"{lib_path} is missing or older than the sources: "
                               "python -m fast_v2_amd.build --timeline")
    if not lib_path.exists():
        raise RuntimeError(f"{lib_path} does not exist")
    os.environ["FDLLM_HIP_LIB"] = str(lib_path)
    import numpy as np
    import torch

    from . import _ffi, ops, workloads

    lib = _ffi.lib()
    attach = lib.fdllm_timeline_attach
    attach.argtypes = [ctypes.c_void_p]
    attach.restype = ctypes.c_int

    dev = torch.device("cuda", 0)
    lens = {} if args.prefix is None else dict(min_prefix=args.prefix, max_prefix=args.prefix)
    wl = workloads.kv_decode_paged(seed=0, active=32 if args.full_block else 8, head_major=not args.token_major, **lens)
    layers = args.layers
    gen = torch.Generator(device=dev).manual_seed(1)
    kp = torch.empty((layers,) + tuple(wl.k_pool.shape), dtype=wl.k_pool.dtype, device=dev)
    if not args.token_major:  # the same storage order as the pool: [layers, pages, Hkv, page_size, D]
        kp = kp.transpose(-3, -2).contiguous().transpose(-3, -2)
    vp = torch.empty_like(kp)
    kp[0].copy_(wl.k_pool)
    vp[0].copy_(wl.v_pool)
    for layer in range(1, layers):
        kp[layer].normal_(generator=gen)
        vp[layer].normal_(generator=gen)
    q, pt, sl = wl.q.to(dev), wl.page_table.to(dev), wl.seqlens.to(dev)
    out = torch.empty_like(q)

    def call(layer):
        ops.block_attn(q, kp[layer], vp[layer], sl, wl.scale, page_table=pt, page_size=wl.page_size, out=out,
                       balanced_splits=args.balanced_splits)

    for i in range(2 * layers):
        call(i % layers)
    torch.cuda.synchronize()
    stamps = torch.zeros(MAX_WORKGROUPS * STAMPS, dtype=torch.int64, device=dev)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    per_call, event_us, dumps = [], [], []
    if attach(ctypes.c_void_p(stamps.data_ptr())) != 0:
        raise RuntimeError("fdllm_timeline_attach failed")
    try:
        graph = None
        if args.back_to_back > 0:
            s = torch.cuda.Stream()
            s.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(s):
                for i in range(2):
                    call(i % layers)
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=s):
                for i in range(args.back_to_back):
                    call(i % layers)
            torch.cuda.synchronize()
        for c in range(args.calls):
            stamps.zero_()
            torch.cuda.synchronize()
            start.record()
            if graph is not None:
                graph.replay()  # every call overwrites the stamps: the last call's remain
            else:
                call(c % layers)
            end.record()
            torch.cuda.synchronize()
            event_us.append(start.elapsed_time(end) * 1e3)
            raw = stamps.view(-1, STAMPS).cpu().numpy()
            per_call.append(analyse(raw))
            if args.dump:
                dumps.append(raw[: 4096].copy())
    finally:
        attach(None)

    if args.dump:
        np.save(args.dump, np.stack(dumps))

    def med(key, j=None):
        vals = [r[key] if j is None else r[key][j] for r in per_call]
        return float(np.median(vals))

    what = ("ring prefill kernel (split form) timeline: bs16 full-block step" if args.full_block else
            "split decode kernel timeline: bs16 sub-block decode step")
    tile = 64 if args.full_block else 32
    print(f"# {what}, {args.calls} calls over {layers} layer pools")
    print()
    print(f"workgroups {med('workgroups'):.0f}, with keys {med('active'):.0f}, merging {med('merging'):.0f}; "
          f"tiles of {tile} keys per workgroup (min / median / max) {med('tiles_per_workgroup', 0):.0f} / "
          f"{med('tiles_per_workgroup', 1):.0f} / {med('tiles_per_workgroup', 2):.0f}")
    print(f"kernel span from the stamps (first start to last end): {med('span'):.2f} us; "
          f"HIP-event time of the same calls (launch from idle included): {float(np.median(event_us)):.2f} us")
    print()
    print("| phase end | first (us) | median (us) | last (us) |")
    print("|---|---|---|---|")
    for name in PHASES:
        print(f"| {name} | {med(name, 0):.2f} | {med(name, 1):.2f} | {med(name, 2):.2f} |")
    print()
    print("| phase duration per workgroup | min (us) | median (us) | max (us) |")
    print("|---|---|---|---|")
    for key, name in (("d_partition", "partition (lengths load + search)"),
                      ("d_first_tiles", "first tiles (page ids, Q, first K/V)"),
                      ("d_loop", "key loop"), ("d_store_arrive", "team merge + partial store + arrival"),
                      ("d_merge", "merge (last workgroup of a unit)")):
        print(f"| {name} | {med(key, 0):.2f} | {med(key, 1):.2f} | {med(key, 2):.2f} |")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
