"""Tensor-level entry points over libfdllm_hip.so, plus their torch.library ops.

Every function here validates its tensors, allocates the outputs with torch
(on the tensors' device, on the current stream) and launches the HIP kernel
through the C ABI. Nothing here computes on the CPU: CPU tensors, unsupported
dtypes or a missing library raise ``RuntimeError``.

torch.library ops (namespace ``fdllm``), each with a Meta implementation so
that graph capture / FakeTensor tracing can infer output shapes without data,
in the manner of ``_wrap_flash_kvcache_as_custom_op``
(utils/attention_backends.py:73-120):

    fdllm::flash_kvcache(Tensor q, Tensor k_cache, Tensor v_cache,
                         Tensor cache_seqlens, float softmax_scale, bool causal) -> Tensor
    fdllm::block_attn(Tensor q, Tensor k_cache, Tensor v_cache, Tensor cache_seqlens,
                      float softmax_scale, int mask_mode, int mask_block,
                      Tensor? q_start, Tensor? page_table, int page_size) -> Tensor
    fdllm::gather_rmsnorm(Tensor hidden, Tensor indices, Tensor? weight, float eps,
                          int norm_mode, bool with_gathered) -> (Tensor, Tensor)
    fdllm::kv_cache_write(Tensor k_new, Tensor v_new, Tensor(a!) k_cache, Tensor(b!) v_cache,
                          Tensor? write_start, int write_offset, Tensor? positions) -> ()
"""
from __future__ import annotations

import ctypes
import math
from typing import Optional, Tuple

import torch

from . import _ffi

# ---------------------------------------------------------------------------
# helpers
# ---------------------------------------------------------------------------

def _require_gpu(*tensors: torch.Tensor) -> torch.device:
    dev = tensors[0].device
    for t in tensors:
        if t.device.type != "cuda":
            raise RuntimeError(
                f"libfdllm_hip kernels need GPU tensors; got a tensor on {t.device}")
        if t.device != dev:
            raise RuntimeError(f"tensors on different devices: {dev} vs {t.device}")
    return dev


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


class _Workspace:
    """Scratch per (device, stream), grown on demand and reused.

    The buffer is zero-filled when allocated: the split-KV decode kernel's
    arrival counters must start at zero, and every call leaves them at zero.
    Partials are written before they are read, so nothing else needs clearing;
    calls on one stream run in order and may share the buffer.

    A buffer that is outgrown is retired, never freed: a HIP graph captured
    earlier on the stream keeps its address and writes counters and partials
    there on every replay, so the memory must not return to the caching
    allocator while the process may still replay such a graph. Each retired
    buffer keeps its counters at zero (every call leaves them so), so a replay
    after any number of larger calls still starts from a clean state.
    """

    def __init__(self) -> None:
        self._bufs: dict = {}
        self._retired: list = []

    def get(self, nbytes: int, device: torch.device) -> torch.Tensor:
        stream = torch.cuda.current_stream(device)
        key = (device.index, stream.cuda_stream)
        buf = self._bufs.get(key)
        if buf is None or buf.numel() < nbytes:
            if buf is not None:
                self._retired.append(buf)
            buf = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
            self._bufs[key] = buf
        return buf


_WORKSPACE = _Workspace()


# ---------------------------------------------------------------------------
# gather + RMSNorm / scatter
# ---------------------------------------------------------------------------

def gather_rmsnorm(
    hidden: torch.Tensor,
    indices: torch.Tensor,
    weight: Optional[torch.Tensor],
    eps: float,
    norm_mode: int = _ffi.NORM_WEIGHT_AFTER_CAST,
    with_gathered: bool = True,
) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """Gather rows ``hidden[b, indices[b, t]]`` and RMS-normalise them in one pass.

    hidden  [B, S, H] (last dim contiguous), bf16 / fp16 / fp32
    indices [B, T] integer (int64 used as is, other integer types converted)
    weight  [H] or None (then norm_mode must be NORM_PLAIN)
    Returns (normed [B, T, H], gathered [B, T, H] or None), both in hidden's dtype.
    """
    if hidden.dim() != 3 or indices.dim() != 2 or indices.shape[0] != hidden.shape[0]:
        raise RuntimeError(
            f"gather_rmsnorm: expected hidden [B,S,H] and indices [B,T]; got "
            f"{tuple(hidden.shape)} and {tuple(indices.shape)}")
    dev = _require_gpu(hidden, indices, *([weight] if weight is not None else []))
    if hidden.stride(-1) != 1:
        hidden = hidden.contiguous()
    if indices.dtype != torch.int64 or indices.stride(-1) != 1:
        indices = indices.to(torch.int64).contiguous()
    if weight is not None:
        weight = weight.contiguous()
        if weight.numel() != hidden.shape[-1]:
            raise RuntimeError("gather_rmsnorm: weight size must equal hidden size")
    elif norm_mode != _ffi.NORM_PLAIN:
        raise RuntimeError("gather_rmsnorm: this norm_mode needs a weight")
    B, S, H = hidden.shape
    T = indices.shape[1]
    normed = torch.empty((B, T, H), dtype=hidden.dtype, device=dev)
    gathered = torch.empty((B, T, H), dtype=hidden.dtype, device=dev) if with_gathered else None
    rc = _ffi.lib().fdllm_gather_rmsnorm(
        hidden.data_ptr(), hidden.stride(0), hidden.stride(1),
        indices.data_ptr(), indices.stride(0),
        _ptr(weight), _ffi.dtype_code(weight.dtype) if weight is not None else 0,
        normed.data_ptr(), _ptr(gathered),
        B, S, T, H, float(eps), _ffi.dtype_code(hidden.dtype), int(norm_mode),
        _ffi.stream_ptr(dev))
    _ffi.check(rc, "fdllm_gather_rmsnorm")
    return normed, gathered


def add_rmsnorm(x: torch.Tensor, residual: torch.Tensor, weight: Optional[torch.Tensor], eps: float,
                norm_mode: int = _ffi.NORM_WEIGHT_AFTER_CAST) -> Tuple[torch.Tensor, torch.Tensor]:
    """``s = x + residual`` (rounded to the rows' dtype) and the RMSNorm of ``s`` in one
    pass over the rows (modeling.py:465-488, 427-432). x, residual [..., H] bf16 / fp16 of
    one shape, H a multiple of 8 (at most 4096). Returns (s, normed), both new tensors."""
    if x.shape != residual.shape or x.dtype != residual.dtype:
        raise RuntimeError("add_rmsnorm: x and residual must share shape and dtype")
    dev = _require_gpu(x, residual, *([weight] if weight is not None else []))
    if x.dtype not in (torch.bfloat16, torch.float16):
        raise RuntimeError("add_rmsnorm: dtype must be bf16 or fp16")
    H = x.shape[-1]
    x, residual = x.contiguous(), residual.contiguous()
    if weight is not None:
        weight = weight.contiguous()
        if weight.numel() != H:
            raise RuntimeError("add_rmsnorm: weight size must equal hidden size")
    elif norm_mode != _ffi.NORM_PLAIN:
        raise RuntimeError("add_rmsnorm: this norm_mode needs a weight")
    out_sum = torch.empty_like(x)
    normed = torch.empty_like(x)
    rc = _ffi.lib().fdllm_add_rmsnorm(
        x.data_ptr(), residual.data_ptr(), _ptr(weight), _ffi.dtype_code(weight.dtype) if weight is not None else 0,
        out_sum.data_ptr(), normed.data_ptr(), x.numel() // H, H, float(eps), _ffi.dtype_code(x.dtype),
        int(norm_mode), _ffi.stream_ptr(dev))
    _ffi.check(rc, "fdllm_add_rmsnorm")
    return out_sum, normed


def silu_mul(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """``silu(gate) * up`` in the 16-bit dtype with torch's rounding points (the SiLU's
    result rounded, then the product): the MLP's act_fn(gate_proj(x)) * up_proj(x)
    (modeling.py:164). gate, up of one shape, bf16 / fp16, numel a multiple of 8."""
    if gate.shape != up.shape or gate.dtype != up.dtype:
        raise RuntimeError("silu_mul: gate and up must share shape and dtype")
    dev = _require_gpu(gate, up)
    if gate.dtype not in (torch.bfloat16, torch.float16):
        raise RuntimeError("silu_mul: dtype must be bf16 or fp16")
    gate, up = gate.contiguous(), up.contiguous()
    out = torch.empty_like(gate)
    rc = _ffi.lib().fdllm_silu_mul(gate.data_ptr(), up.data_ptr(), out.data_ptr(), gate.numel(),
                                   _ffi.dtype_code(gate.dtype), _ffi.stream_ptr(dev))
    _ffi.check(rc, "fdllm_silu_mul")
    return out


def scatter_rows(values: torch.Tensor, indices: torch.Tensor,
                 cache: torch.Tensor, current: Optional[torch.Tensor] = None) -> Optional[torch.Tensor]:
    """cache[b, indices[b,t]] = values[b, t] (and current[b, indices[b,t]] when given).

    Indices that repeat within a sequence race, as in the reference kernel: each element
    of such a row ends with that element of one of the rows aimed at it (which one is
    unspecified, and may differ between the two destinations).

    Returns ``current`` (None when it is not given)."""
    dests = [cache] + ([current] if current is not None else [])
    if values.dim() != 3 or indices.dim() != 2 or any(d.dim() != 3 for d in dests):
        raise RuntimeError("scatter_rows: expected values/cache/current [B,*,H] and indices [B,T]")
    dev = _require_gpu(values, indices, *dests)
    if any(d.dtype != values.dtype for d in dests):
        raise RuntimeError("scatter_rows: values, cache and current must share a dtype")
    if cache.shape[0] != values.shape[0] or cache.shape[2] != values.shape[2] or \
            (current is not None and current.shape != cache.shape):
        raise RuntimeError("scatter_rows: shape mismatch")
    if any(d.stride(-1) != 1 for d in dests):
        raise RuntimeError("scatter_rows: cache/current last dim must be contiguous (written in place)")
    if indices.shape[0] != values.shape[0] or indices.shape[1] != values.shape[1]:
        raise RuntimeError("scatter_rows: indices must be [B, T] for values [B, T, H]")
    values = values.contiguous()
    if indices.dtype != torch.int64 or indices.stride(-1) != 1:
        indices = indices.to(torch.int64).contiguous()
    B, T, H = values.shape
    S = cache.shape[1]
    rc = _ffi.lib().fdllm_scatter_rows(
        values.data_ptr(), indices.data_ptr(), indices.stride(0),
        cache.data_ptr(), cache.stride(0), cache.stride(1),
        _ptr(current), current.stride(0) if current is not None else 0,
        current.stride(1) if current is not None else 0,
        B, S, T, H, _ffi.dtype_code(values.dtype), _ffi.stream_ptr(dev))
    _ffi.check(rc, "fdllm_scatter_rows")
    return current


# ---------------------------------------------------------------------------
# attention
# ---------------------------------------------------------------------------

def _attn_desc(q, k_cache, v_cache, seqlens, out, scale, mask_mode, mask_block,
               q_start, page_table, page_size, kv_split, flags=0, k_new=None, v_new=None) -> _ffi.KVAttnDesc:
    B, Sq, Hq, D = q.shape
    d = _ffi.KVAttnDesc()
    d.q = q.data_ptr()
    d.q_stride_b, d.q_stride_s, d.q_stride_h = q.stride(0), q.stride(1), q.stride(2)
    d.k = k_cache.data_ptr()
    d.k_stride_page, d.k_stride_slot, d.k_stride_h = k_cache.stride(0), k_cache.stride(1), k_cache.stride(2)
    d.v = v_cache.data_ptr()
    d.v_stride_page, d.v_stride_slot, d.v_stride_h = v_cache.stride(0), v_cache.stride(1), v_cache.stride(2)
    d.out = out.data_ptr()
    d.out_stride_b, d.out_stride_s, d.out_stride_h = out.stride(0), out.stride(1), out.stride(2)
    d.seqlens = seqlens.data_ptr()
    d.q_start = _ptr(q_start)
    if page_table is not None:
        d.page_table = page_table.data_ptr()
        d.max_pages = page_table.shape[1]
        d.page_size = int(page_size)
        d.max_seqlen = page_table.shape[1] * int(page_size)
    else:
        d.page_table = None
        d.max_pages = 0
        d.page_size = 0
        d.max_seqlen = k_cache.shape[1]
    d.batch, d.q_len, d.num_q_heads, d.num_kv_heads, d.head_dim = B, Sq, Hq, k_cache.shape[2], D
    d.mask_mode = int(mask_mode)
    d.mask_block = int(mask_block)
    d.dtype = _ffi.dtype_code(q.dtype)
    d.kv_split = int(kv_split)
    d.softmax_scale = float(scale)
    d.flags = int(flags)
    if k_new is not None:
        d.k_new = k_new.data_ptr()
        d.v_new = v_new.data_ptr()
        d.new_stride_b, d.new_stride_s, d.new_stride_h = k_new.stride(0), k_new.stride(1), k_new.stride(2)
    return d


def block_attn(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    cache_seqlens: torch.Tensor,
    softmax_scale: Optional[float] = None,
    mask_mode: int = _ffi.MASK_SEQLEN,
    mask_block: int = 32,
    q_start: Optional[torch.Tensor] = None,
    page_table: Optional[torch.Tensor] = None,
    page_size: int = 0,
    out: Optional[torch.Tensor] = None,
    kv_split: int = 0,
    decode_kernel: bool = True,
    all_heads_decode: bool = False,
    k_new: Optional[torch.Tensor] = None,
    v_new: Optional[torch.Tensor] = None,
    cache_write_kernel: bool = False,
    balanced_splits: bool = False,
) -> torch.Tensor:
    """Attention of BSHD queries over a (paged) BSHD KV cache.

    q            [B, Sq, Hq, D] bf16/fp16, or fp32 (computed in fp32 throughout by a
                 general kernel; head_dim contiguous)
    k/v_cache    [B, max_S, Hkv, D] without a page table, or the page pool
                 [num_pages, page_size, Hkv, D] with ``page_table`` [B, max_pages] int32
    cache_seqlens [B] visible key count per sequence (int32; other ints converted)
    Returns a new [B, Sq, Hq, D] tensor (or fills ``out``).
    decode_kernel=False forces the general kernel where a decode kernel would
    apply; all_heads_decode=True picks the all-KV-heads decode kernel instead of
    the split-KV one (all compute the same function).
    k_new / v_new [B, Sq, Hkv, D]: the K / V rows of the query tokens, stored into
    the cache at positions q_start[b] + t (cache_seqlens[b] - Sq + t without q_start)
    as part of the call, before any key is read (StaticKVCache.update followed by the
    attention, static_kv_cache.py:132-160): inside the prefill kernels, otherwise (and
    with cache_write_kernel=True) by a copy kernel ahead of the attention (same results).
    balanced_splits=True deals all sequences' keys evenly over the sub-block decode
    workgroups (runs that cross sequence boundaries) instead of splitting each sequence
    on its own.
    """
    if q.dim() != 4 or k_cache.dim() != 4 or v_cache.dim() != 4:
        raise RuntimeError("block_attn: q, k_cache and v_cache must be 4-D (BSHD)")
    tensors = [q, k_cache, v_cache, cache_seqlens]
    if (k_new is None) != (v_new is None):
        raise RuntimeError("block_attn: give k_new and v_new together")
    if k_new is not None:
        if k_new.shape != (q.shape[0], q.shape[1], k_cache.shape[2], q.shape[3]) or v_new.shape != k_new.shape:
            raise RuntimeError(f"block_attn: k_new / v_new must be [B, Sq, Hkv, D]; got {tuple(k_new.shape)}")
        if k_new.dtype != q.dtype or v_new.dtype != q.dtype:
            raise RuntimeError("block_attn: k_new / v_new must have q's dtype")
        if k_new.stride() != v_new.stride() or k_new.stride(-1) != 1:
            k_new, v_new = k_new.contiguous(), v_new.contiguous()
        tensors += [k_new, v_new]
    if q_start is not None:
        tensors.append(q_start)
    if page_table is not None:
        tensors.append(page_table)
    dev = _require_gpu(*tensors)
    if not (q.dtype == k_cache.dtype == v_cache.dtype) or \
            q.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise RuntimeError(f"block_attn: q/k/v must share dtype bf16, fp16 or fp32 "
                           f"(got {q.dtype}, {k_cache.dtype}, {v_cache.dtype})")
    if q.dtype == torch.float32 and k_new is not None:
        raise RuntimeError("block_attn: the cache write (k_new / v_new) takes bf16 or fp16 only")
    if k_cache.shape != v_cache.shape:
        raise RuntimeError("block_attn: k_cache and v_cache shapes differ")
    B, Sq, Hq, D = q.shape
    if k_cache.shape[3] != D:
        raise RuntimeError("block_attn: head_dim mismatch between q and the cache")
    if Hq % k_cache.shape[2] != 0:
        raise RuntimeError("block_attn: num_q_heads must be a multiple of num_kv_heads")
    if page_table is None and k_cache.shape[0] != B:
        raise RuntimeError("block_attn: cache batch dim must equal q batch dim without a page table")
    if q.stride(-1) != 1:
        q = q.contiguous()
    if k_cache.stride(-1) != 1 or v_cache.stride(-1) != 1:
        raise RuntimeError("block_attn: cache head_dim must be contiguous")
    if cache_seqlens.dtype != torch.int32 or not cache_seqlens.is_contiguous():
        cache_seqlens = cache_seqlens.to(torch.int32).contiguous()
    if q_start is not None and (q_start.dtype != torch.int32 or not q_start.is_contiguous()):
        q_start = q_start.to(torch.int32).contiguous()
    if page_table is not None:
        if page_table.dtype != torch.int32 or not page_table.is_contiguous():
            page_table = page_table.to(torch.int32).contiguous()
        if page_size <= 0 or k_cache.shape[1] != page_size:
            raise RuntimeError("block_attn: page pool dim 1 must equal page_size")
    if out is None:
        out = torch.empty((B, Sq, Hq, D), dtype=q.dtype, device=dev)
    elif out.shape != (B, Sq, Hq, D) or out.dtype != q.dtype or out.stride(-1) != 1:
        raise RuntimeError("block_attn: bad `out` tensor")
    if softmax_scale is None:
        softmax_scale = D ** -0.5
    desc = _attn_desc(q, k_cache, v_cache, cache_seqlens, out, softmax_scale, mask_mode,
                      mask_block, q_start, page_table, page_size, kv_split,
                      (0 if decode_kernel else _ffi.ATTN_NO_DECODE_KERNEL)
                      | (_ffi.ATTN_ALL_HEADS_DECODE if all_heads_decode else 0)
                      | (_ffi.ATTN_CACHE_WRITE_KERNEL if cache_write_kernel else 0)
                      | (_ffi.ATTN_BALANCED_SPLITS if balanced_splits else 0), k_new, v_new)
    L = _ffi.lib()
    need = ctypes.c_size_t(0)
    _ffi.check(L.fdllm_kv_attn_workspace_size(ctypes.byref(desc), ctypes.byref(need)),
               "fdllm_kv_attn_workspace_size")
    ws_ptr, ws_bytes = None, 0
    if need.value:
        ws = _WORKSPACE.get(need.value, dev)
        ws_ptr, ws_bytes = ws.data_ptr(), ws.numel()
    rc = L.fdllm_kv_attn_fwd(ctypes.byref(desc), ws_ptr, ws_bytes, _ffi.stream_ptr(dev))
    _ffi.check(rc, "fdllm_kv_attn_fwd")
    return out


def _rope_dest_desc(d, B, S, Hq, Hkv, D, dtype, dev, cos, sin, k_cache, v_cache, write_start, write_offset,
                    k_block, v_block, block_offset, q_out, kv_out):
    """Validate the RoPE / cache-write arguments shared by rope_kv_write and
    qkv_rope_kv_write and fill those fields of ``d`` (a RopeKVDesc); returns
    (q_out, (k_out, v_out) or (None, None), keep): ``keep`` holds the tensors the
    descriptor points to that this function made, for the caller to hold until the
    launch."""
    if cos.dim() == 2:
        cos, sin = cos[None], sin[None]
    if cos.shape != sin.shape or cos.dim() != 3 or cos.shape[1] != S or cos.shape[2] != D or \
            cos.shape[0] not in (1, B):
        raise RuntimeError("rope_kv_write: cos / sin must be [1 or B, S, D]")
    if (k_cache is None) != (v_cache is None) or (k_block is None) != (v_block is None):
        raise RuntimeError("rope_kv_write: give k and v destinations together")
    _require_gpu(cos, sin, *[t for t in (k_cache, v_cache, k_block, v_block, write_start, q_out) if t is not None])
    if any(t.dtype != dtype for t in (cos, sin, k_cache, v_cache, k_block, v_block, q_out) if t is not None):
        raise RuntimeError("rope_kv_write: all tensors must share one 16-bit dtype")

    def last_contig(t):
        return t if t.stride(-1) == 1 and all(st % 8 == 0 for st in t.stride()[:-1]) else t.contiguous()
    cos, sin = last_contig(cos), last_contig(sin)
    for name, c in (("k_cache", k_cache), ("v_cache", v_cache), ("k_block", k_block), ("v_block", v_block)):
        if c is not None and (c.dim() != 4 or c.shape[0] != B or c.shape[2] != Hkv or c.shape[3] != D or
                              c.stride(-1) != 1):
            raise RuntimeError(f"rope_kv_write: {name} must be [B, L, Hkv, D] with a contiguous last dim")
    if k_cache is not None and k_cache.stride() != v_cache.stride():
        raise RuntimeError("rope_kv_write: k_cache and v_cache strides differ")
    if k_block is not None and k_block.stride() != v_block.stride():
        raise RuntimeError("rope_kv_write: k_block and v_block strides differ")
    if write_start is not None and (write_start.dtype != torch.int32 or not write_start.is_contiguous()):
        write_start = write_start.to(torch.int32).contiguous()
    if q_out is None:
        q_out = torch.empty((B, S, Hq, D), dtype=dtype, device=dev)
    kv_o = (torch.empty((B, S, Hkv, D), dtype=dtype, device=dev),
            torch.empty((B, S, Hkv, D), dtype=dtype, device=dev)) if kv_out else (None, None)
    if sin.stride()[:2] != cos.stride()[:2]:
        cos, sin = cos.contiguous(), sin.contiguous()
    d.cos, d.sin = cos.data_ptr(), sin.data_ptr()
    d.cs_stride_b = cos.stride(0) if cos.shape[0] == B and B > 1 else 0
    d.cs_stride_s = cos.stride(1)
    d.q_out, (d.qo_stride_b, d.qo_stride_s, d.qo_stride_h) = q_out.data_ptr(), q_out.stride()[:3]
    if kv_out:
        d.k_out, d.v_out = kv_o[0].data_ptr(), kv_o[1].data_ptr()
        d.ko_stride_b, d.ko_stride_s, d.ko_stride_h = kv_o[0].stride()[:3]
    if k_cache is not None:
        d.k_cache, d.v_cache = k_cache.data_ptr(), v_cache.data_ptr()
        d.c_stride_b, d.c_stride_s, d.c_stride_h = k_cache.stride()[:3]
        d.cache_len = k_cache.shape[1]
        d.write_start = _ptr(write_start)
        d.write_offset = int(write_offset)
    if k_block is not None:
        d.k_block, d.v_block = k_block.data_ptr(), v_block.data_ptr()
        d.bc_stride_b, d.bc_stride_s, d.bc_stride_h = k_block.stride()[:3]
        d.block_len = k_block.shape[1]
        d.block_offset = int(block_offset)
    d.batch, d.seq_len, d.num_q_heads, d.num_kv_heads, d.head_dim = B, S, Hq, Hkv, D
    d.dtype = _ffi.dtype_code(dtype)
    return q_out, kv_o, (cos, sin, write_start)


def rope_kv_write(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    k_cache: Optional[torch.Tensor] = None,
    v_cache: Optional[torch.Tensor] = None,
    write_start: Optional[torch.Tensor] = None,
    write_offset: int = 0,
    k_block: Optional[torch.Tensor] = None,
    v_block: Optional[torch.Tensor] = None,
    block_offset: int = 0,
    q_out: Optional[torch.Tensor] = None,
    kv_out: bool = False,
):
    """RoPE of q and k fused with the cache writes (one kernel).

    q [B, S, Hq, D], k / v [B, S, Hkv, D] (last dim contiguous), cos / sin [B or 1, S, D]
    (or [S, D]) in the same 16-bit dtype. Returns ``q_rot`` (and ``(k_rot, v)`` copies
    when ``kv_out``). The rotated k rows and the v rows go to ``k_cache``/``v_cache``
    [B, L, Hkv, D] at ``write_start[b] + write_offset + t`` (``write_offset + t`` without
    ``write_start``) and to ``k_block``/``v_block`` [B, Lb, Hkv, D] at ``block_offset + t``;
    rows past a buffer's length are skipped. Rounding as the eager expression
    ``q * cos + rotate_half(q) * sin`` (utils/attention_backends.py:777-788).
    """
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4 or k.shape != v.shape:
        raise RuntimeError("rope_kv_write: q [B,S,Hq,D], k / v [B,S,Hkv,D] expected")
    B, S, Hq, D = q.shape
    if k.shape[0] != B or k.shape[1] != S or k.shape[3] != D:
        raise RuntimeError("rope_kv_write: q and k/v disagree in batch, length or head_dim")
    Hkv = k.shape[2]
    dev = _require_gpu(q, k, v)
    if q.dtype not in (torch.bfloat16, torch.float16) or k.dtype != q.dtype or v.dtype != q.dtype:
        raise RuntimeError("rope_kv_write: all tensors must share one 16-bit dtype")

    def last_contig(t):
        return t if t.stride(-1) == 1 and all(st % 8 == 0 for st in t.stride()[:-1]) else t.contiguous()
    q, k, v = (last_contig(t) for t in (q, k, v))
    d = _ffi.RopeKVDesc()
    q_out, kv_o, keep = _rope_dest_desc(d, B, S, Hq, Hkv, D, q.dtype, dev, cos, sin, k_cache, v_cache,
                                        write_start, write_offset, k_block, v_block, block_offset, q_out, kv_out)
    d.q, (d.q_stride_b, d.q_stride_s, d.q_stride_h) = q.data_ptr(), q.stride()[:3]
    d.k, (d.k_stride_b, d.k_stride_s, d.k_stride_h) = k.data_ptr(), k.stride()[:3]
    d.v, (d.v_stride_b, d.v_stride_s, d.v_stride_h) = v.data_ptr(), v.stride()[:3]
    rc = _ffi.lib().fdllm_rope_kv_write(ctypes.byref(d), _ffi.stream_ptr(dev))
    del keep  # launched: the stream orders any reuse of that memory after the kernel
    _ffi.check(rc, "fdllm_rope_kv_write")
    return (q_out, kv_o) if kv_out else q_out


def qkv_rope_kv_write(
    x: torch.Tensor,
    wq: torch.Tensor, bq: Optional[torch.Tensor],
    wk: torch.Tensor, bk: Optional[torch.Tensor],
    wv: torch.Tensor, bv: Optional[torch.Tensor],
    cos: torch.Tensor,
    sin: torch.Tensor,
    k_cache: Optional[torch.Tensor] = None,
    v_cache: Optional[torch.Tensor] = None,
    write_start: Optional[torch.Tensor] = None,
    write_offset: int = 0,
    k_block: Optional[torch.Tensor] = None,
    v_block: Optional[torch.Tensor] = None,
    block_offset: int = 0,
    q_out: Optional[torch.Tensor] = None,
    kv_out: bool = False,
    head_dim: int = 128,
):
    """The q / k / v projections of ``x`` [B, S, hidden] (nn.Linear weights [heads * D,
    hidden] and biases), then what ``rope_kv_write`` does with them, in one kernel
    (utils/attention_backends.py:837-842). The projections sum in fp32 and round once
    after the bias, as a 16-bit linear layer does, in a different order than a library
    GEMM. head_dim 128, hidden a multiple of 64."""
    if x.dim() != 3:
        raise RuntimeError("qkv_rope_kv_write: x must be [B, S, hidden]")
    B, S, H = x.shape
    D = head_dim
    if wq.dim() != 2 or wk.dim() != 2 or wk.shape != wv.shape or wq.shape[1] != H or wk.shape[1] != H or \
            wq.shape[0] % D or wk.shape[0] % D:
        raise RuntimeError("qkv_rope_kv_write: weights must be [heads * head_dim, hidden]")
    Hq, Hkv = wq.shape[0] // D, wk.shape[0] // D
    for name, b_, w_ in (("bq", bq, wq), ("bk", bk, wk), ("bv", bv, wv)):
        if b_ is not None and (b_.dim() != 1 or b_.shape[0] != w_.shape[0]):
            raise RuntimeError(f"qkv_rope_kv_write: {name} must be [{w_.shape[0]}]")
    ts = [x, wq, wk, wv] + [b_ for b_ in (bq, bk, bv) if b_ is not None]
    dev = _require_gpu(*ts)
    if x.dtype not in (torch.bfloat16, torch.float16) or any(t.dtype != x.dtype for t in ts):
        raise RuntimeError("qkv_rope_kv_write: all tensors must share one 16-bit dtype")
    if x.stride(-1) != 1 or x.stride(1) % 8 or (B > 1 and x.stride(0) != S * x.stride(1)):
        x = x.contiguous()
    wq, wk, wv = (w_.contiguous() for w_ in (wq, wk, wv))
    bq, bk, bv = (b_.contiguous() if b_ is not None else None for b_ in (bq, bk, bv))
    d = _ffi.QkvRopeDesc()
    q_out, kv_o, keep = _rope_dest_desc(d.rope, B, S, Hq, Hkv, D, x.dtype, dev, cos, sin, k_cache, v_cache,
                                        write_start, write_offset, k_block, v_block, block_offset, q_out, kv_out)
    d.x, d.x_stride_row, d.hidden = x.data_ptr(), x.stride(1), H
    d.wq, d.wk, d.wv = wq.data_ptr(), wk.data_ptr(), wv.data_ptr()
    d.bq, d.bk, d.bv = _ptr(bq), _ptr(bk), _ptr(bv)
    rc = _ffi.lib().fdllm_qkv_rope_kv_write(ctypes.byref(d), _ffi.stream_ptr(dev))
    del keep  # launched: the stream orders any reuse of that memory after the kernel
    _ffi.check(rc, "fdllm_qkv_rope_kv_write")
    return (q_out, kv_o) if kv_out else q_out


class UnmaskScratch:
    """Device buffers of one sampler (greedy token and confidence per position, four
    counters), allocated once per (batch, positions, device)."""

    def __init__(self, batch: int, positions: int, device):
        self.row_tok = torch.empty((batch, positions), dtype=torch.int64, device=device)
        self.row_conf = torch.empty((batch, positions), dtype=torch.float32, device=device)
        self.counts = torch.zeros(4, dtype=torch.int32, device=device)


def unmask_step(logits: torch.Tensor, tokens: torch.Tensor, mask_id: int, threshold: float,
                row_offset: int = 0, shift: int = 1, finished: Optional[torch.Tensor] = None,
                stop_token: Optional[int] = None, scratch: Optional[UnmaskScratch] = None) -> UnmaskScratch:
    """Greedy sampling + threshold unmasking of one sub-block step, on the GPU.

    logits [B, R, V] (16-bit, vocab contiguous); position i of the sub-block reads row
    max(row_offset + i - shift, 0). tokens [B, L] int64 (positions contiguous) is
    updated in place; finished [B] bool / uint8 (or None) too. Returns the scratch
    whose ``counts`` = [unmasked, masked left in unfinished rows, rows with position 0
    still masked, finished rows] and ``row_tok`` / ``row_conf`` hold the greedy token
    and its probability per position (generation_functions.py:784-807,
    modeling.py:2263-2270)."""
    if logits.dim() != 3 or tokens.dim() != 2 or tokens.shape[0] != logits.shape[0]:
        raise RuntimeError("unmask_step: logits [B, R, V] and tokens [B, L] expected")
    dev = _require_gpu(logits, tokens, *([finished] if finished is not None else []))
    if logits.dtype not in (torch.bfloat16, torch.float16):
        raise RuntimeError("unmask_step: logits must be bf16 or fp16")
    if logits.stride(-1) != 1:
        logits = logits.contiguous()
    if tokens.dtype != torch.int64 or tokens.stride(-1) != 1:
        raise RuntimeError("unmask_step: tokens must be int64 with contiguous positions (updated in place)")
    B, L = tokens.shape
    if finished is not None and (finished.dtype not in (torch.bool, torch.uint8) or not finished.is_contiguous()
                                 or finished.numel() != B):
        raise RuntimeError("unmask_step: finished must be a contiguous bool / uint8 [B]")
    if scratch is None or scratch.row_tok.shape != (B, L) or scratch.row_tok.device != dev:
        scratch = UnmaskScratch(B, L, dev)
    rc = _ffi.lib().fdllm_unmask_step(
        logits.data_ptr(), logits.stride(0), logits.stride(1), logits.shape[2], int(row_offset), int(shift),
        tokens.data_ptr(), tokens.stride(0), _ptr(finished), int(mask_id), float(threshold),
        -1 if stop_token is None else int(stop_token),
        scratch.row_tok.data_ptr(), scratch.row_conf.data_ptr(), scratch.counts.data_ptr(),
        B, L, _ffi.dtype_code(logits.dtype), _ffi.stream_ptr(dev))
    _ffi.check(rc, "fdllm_unmask_step")
    return scratch


def kv_cache_write(
    k_new: torch.Tensor,
    v_new: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    write_offset: int = 0,
    write_start: Optional[torch.Tensor] = None,
    positions: Optional[torch.Tensor] = None,
    page_table: Optional[torch.Tensor] = None,
    page_size: int = 0,
) -> None:
    """Write new BSHD K/V rows [B, T, Hkv, D] into the cache in place.

    Row t of sequence b goes to position ``positions[b, t]`` if given, else
    ``write_start[b] + t`` if given, else ``write_offset + t``.
    """
    if k_new.dim() != 4 or k_new.shape != v_new.shape:
        raise RuntimeError("kv_cache_write: k_new / v_new must be matching [B, T, Hkv, D]")
    tensors = [k_new, v_new, k_cache, v_cache]
    for t in (write_start, positions, page_table):
        if t is not None:
            tensors.append(t)
    dev = _require_gpu(*tensors)
    if not (k_new.dtype == v_new.dtype == k_cache.dtype == v_cache.dtype):
        raise RuntimeError("kv_cache_write: dtype mismatch")
    if k_cache.shape != v_cache.shape or k_cache.stride() != v_cache.stride():
        raise RuntimeError("kv_cache_write: k_cache and v_cache must have the same shape and strides")
    B, T, Hkv, D = k_new.shape
    if k_cache.shape[2] != Hkv or k_cache.shape[3] != D or k_cache.stride(-1) != 1:
        raise RuntimeError("kv_cache_write: cache shape mismatch")
    if page_table is None and k_cache.shape[0] != B:
        raise RuntimeError("kv_cache_write: cache batch dim must equal the batch without a page table")
    if k_new.stride() != v_new.stride() or k_new.stride(-1) != 1:
        k_new = k_new.contiguous()
        v_new = v_new.contiguous()
    if write_start is not None and (write_start.dtype != torch.int32 or not write_start.is_contiguous()):
        write_start = write_start.to(torch.int32).contiguous()
    if positions is not None and (positions.dtype != torch.int64 or not positions.is_contiguous()):
        positions = positions.to(torch.int64).contiguous()
    if page_table is not None and (page_table.dtype != torch.int32 or not page_table.is_contiguous()):
        page_table = page_table.to(torch.int32).contiguous()
    rc = _ffi.lib().fdllm_kv_cache_write(
        k_new.data_ptr(), v_new.data_ptr(), k_new.stride(0), k_new.stride(1), k_new.stride(2),
        k_cache.data_ptr(), v_cache.data_ptr(), k_cache.stride(0), k_cache.stride(1), k_cache.stride(2),
        _ptr(page_table), page_table.shape[1] if page_table is not None else 0, int(page_size),
        k_cache.shape[1] if page_table is None else page_table.shape[1] * int(page_size),
        _ptr(write_start), int(write_offset), _ptr(positions),
        B, T, Hkv, D, _ffi.dtype_code(k_new.dtype), _ffi.stream_ptr(dev))
    _ffi.check(rc, "fdllm_kv_cache_write")


# ---------------------------------------------------------------------------
# torch.library registration
# ---------------------------------------------------------------------------

_LIB = torch.library.Library("fdllm", "DEF")
_LIB.define(
    "flash_kvcache(Tensor q, Tensor k_cache, Tensor v_cache, Tensor cache_seqlens, "
    "float softmax_scale, bool causal) -> Tensor")
_LIB.define(
    "block_attn(Tensor q, Tensor k_cache, Tensor v_cache, Tensor cache_seqlens, "
    "float softmax_scale, int mask_mode, int mask_block, Tensor? q_start, "
    "Tensor? page_table, int page_size) -> Tensor")
_LIB.define(
    "gather_rmsnorm(Tensor hidden, Tensor indices, Tensor? weight, float eps, "
    "int norm_mode, bool with_gathered) -> (Tensor, Tensor)")
# the cache write mutates k_cache / v_cache in place: the (a!) / (b!) annotations let
# torch.compile and functionalization see the mutation (the reference's compiled
# forward writes with a traceable scatter_, static_kv_cache.py:218-229)
_LIB.define(
    "kv_cache_write(Tensor k_new, Tensor v_new, Tensor(a!) k_cache, Tensor(b!) v_cache, "
    "Tensor? write_start, int write_offset, Tensor? positions) -> ()")


def _flash_kvcache_impl(q, k_cache, v_cache, cache_seqlens, softmax_scale, causal):
    # causal=True follows flash_attn_with_kvcache: the mask is aligned to the
    # bottom-right corner, i.e. query i sits at position seqlen - Sq + i.
    mode = _ffi.MASK_CAUSAL if causal else _ffi.MASK_SEQLEN
    return block_attn(q, k_cache, v_cache, cache_seqlens, softmax_scale, mask_mode=mode)


def _flash_kvcache_meta(q, k_cache, v_cache, cache_seqlens, softmax_scale, causal):
    return torch.empty_like(q)


def _block_attn_impl(q, k_cache, v_cache, cache_seqlens, softmax_scale, mask_mode, mask_block,
                     q_start, page_table, page_size):
    return block_attn(q, k_cache, v_cache, cache_seqlens, softmax_scale, mask_mode, mask_block,
                      q_start, page_table, page_size)


def _block_attn_meta(q, k_cache, v_cache, cache_seqlens, softmax_scale, mask_mode, mask_block,
                     q_start, page_table, page_size):
    return torch.empty_like(q)


def _gather_rmsnorm_impl(hidden, indices, weight, eps, norm_mode, with_gathered):
    normed, gathered = gather_rmsnorm(hidden, indices, weight, eps, norm_mode, with_gathered)
    if gathered is None:
        gathered = hidden.new_empty((0,))
    return normed, gathered


def _gather_rmsnorm_meta(hidden, indices, weight, eps, norm_mode, with_gathered):
    B, _, H = hidden.shape
    T = indices.shape[1]
    normed = hidden.new_empty((B, T, H))
    gathered = hidden.new_empty((B, T, H)) if with_gathered else hidden.new_empty((0,))
    return normed, gathered


def _kv_cache_write_impl(k_new, v_new, k_cache, v_cache, write_start, write_offset, positions):
    kv_cache_write(k_new, v_new, k_cache, v_cache, write_offset=write_offset, write_start=write_start,
                   positions=positions)


def _kv_cache_write_meta(k_new, v_new, k_cache, v_cache, write_start, write_offset, positions):
    return None


_LIB.impl("kv_cache_write", _kv_cache_write_impl, "CUDA")
_LIB.impl("kv_cache_write", _kv_cache_write_meta, "Meta")
_LIB.impl("flash_kvcache", _flash_kvcache_impl, "CUDA")
_LIB.impl("flash_kvcache", _flash_kvcache_meta, "Meta")
_LIB.impl("block_attn", _block_attn_impl, "CUDA")
_LIB.impl("block_attn", _block_attn_meta, "Meta")
_LIB.impl("gather_rmsnorm", _gather_rmsnorm_impl, "CUDA")
_LIB.impl("gather_rmsnorm", _gather_rmsnorm_meta, "Meta")

flash_kvcache = torch.ops.fdllm.flash_kvcache

LOG2E = 1.0 / math.log(2.0)
