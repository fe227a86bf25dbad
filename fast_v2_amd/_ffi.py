"""ctypes binding of libfdllm_hip.so (the C ABI declared in include/fdllm_hip.h).

The library is loaded after ``import torch`` so that it binds to the HIP runtime
torch already mapped (both carry the soname libamdhip64.so.7): device pointers
and hipStream_t handles from torch are then valid inside the library.

There is no fallback: if the library is missing or fails to load, every entry
point raises ``RuntimeError``.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch  # noqa: F401  (must precede the library load, see above)

import os

# FDLLM_HIP_LIB overrides the location of the library (default: the in-tree build).
LIB_PATH = Path(os.environ.get("FDLLM_HIP_LIB") or (Path(__file__).resolve().parent / "lib" / "libfdllm_hip.so"))

ABI_VERSION = 2  # FDLLM_ABI_VERSION

FDLLM_OK = 0
FDLLM_ERR_INVALID_ARGUMENT = -1
FDLLM_ERR_UNSUPPORTED = -2
FDLLM_ERR_WORKSPACE = -3

DTYPE_F32 = 0
DTYPE_BF16 = 1
DTYPE_F16 = 2

NORM_PLAIN = 0
NORM_WEIGHT_FP32 = 1
NORM_WEIGHT_AFTER_CAST = 2

MASK_SEQLEN = 0
MASK_CAUSAL = 1
MASK_BLOCK_CAUSAL = 2

_c_i32 = ctypes.c_int32
_c_i64 = ctypes.c_int64
_c_int = ctypes.c_int
_c_float = ctypes.c_float
_c_vp = ctypes.c_void_p
_c_sz = ctypes.c_size_t


class KVAttnDesc(ctypes.Structure):
    """Mirror of ``fdllm_kv_attn_desc`` (include/fdllm_hip.h)."""

    _fields_ = [
        ("q", _c_vp), ("q_stride_b", _c_i64), ("q_stride_s", _c_i64), ("q_stride_h", _c_i64),
        ("k", _c_vp), ("k_stride_page", _c_i64), ("k_stride_slot", _c_i64), ("k_stride_h", _c_i64),
        ("v", _c_vp), ("v_stride_page", _c_i64), ("v_stride_slot", _c_i64), ("v_stride_h", _c_i64),
        ("out", _c_vp), ("out_stride_b", _c_i64), ("out_stride_s", _c_i64), ("out_stride_h", _c_i64),
        ("page_table", _c_vp), ("seqlens", _c_vp), ("q_start", _c_vp),
        ("max_pages", _c_i32), ("page_size", _c_i32), ("max_seqlen", _c_i32),
        ("batch", _c_i32), ("q_len", _c_i32), ("num_q_heads", _c_i32), ("num_kv_heads", _c_i32),
        ("head_dim", _c_i32),
        ("mask_mode", _c_i32), ("mask_block", _c_i32), ("dtype", _c_i32), ("kv_split", _c_i32),
        ("softmax_scale", _c_float),
        ("flags", _c_i32),
        ("k_new", _c_vp), ("v_new", _c_vp),
        ("new_stride_b", _c_i64), ("new_stride_s", _c_i64), ("new_stride_h", _c_i64),
    ]


ATTN_NO_DECODE_KERNEL = 1
ATTN_ALL_HEADS_DECODE = 2
ATTN_CACHE_WRITE_KERNEL = 4
ATTN_BALANCED_SPLITS = 8

KV_ATTN_SCRATCH_BYTES = 48 * 1024 * 1024  # FDLLM_KV_ATTN_SCRATCH_BYTES


class RopeKVDesc(ctypes.Structure):
    """Mirror of ``fdllm_rope_kv_desc`` (include/fdllm_hip.h)."""

    _fields_ = [
        ("q", _c_vp), ("q_stride_b", _c_i64), ("q_stride_s", _c_i64), ("q_stride_h", _c_i64),
        ("k", _c_vp), ("k_stride_b", _c_i64), ("k_stride_s", _c_i64), ("k_stride_h", _c_i64),
        ("v", _c_vp), ("v_stride_b", _c_i64), ("v_stride_s", _c_i64), ("v_stride_h", _c_i64),
        ("cos", _c_vp), ("sin", _c_vp), ("cs_stride_b", _c_i64), ("cs_stride_s", _c_i64),
        ("q_out", _c_vp), ("qo_stride_b", _c_i64), ("qo_stride_s", _c_i64), ("qo_stride_h", _c_i64),
        ("k_out", _c_vp), ("v_out", _c_vp), ("ko_stride_b", _c_i64), ("ko_stride_s", _c_i64),
        ("ko_stride_h", _c_i64),
        ("k_cache", _c_vp), ("v_cache", _c_vp), ("c_stride_b", _c_i64), ("c_stride_s", _c_i64),
        ("c_stride_h", _c_i64), ("cache_len", _c_i32), ("write_start", _c_vp), ("write_offset", _c_i32),
        ("k_block", _c_vp), ("v_block", _c_vp), ("bc_stride_b", _c_i64), ("bc_stride_s", _c_i64),
        ("bc_stride_h", _c_i64), ("block_len", _c_i32), ("block_offset", _c_i32),
        ("batch", _c_i32), ("seq_len", _c_i32), ("num_q_heads", _c_i32), ("num_kv_heads", _c_i32),
        ("head_dim", _c_i32), ("dtype", _c_i32),
    ]


class QkvRopeDesc(ctypes.Structure):
    """Mirror of ``fdllm_qkv_rope_desc`` (include/fdllm_hip.h)."""

    _fields_ = [
        ("x", _c_vp), ("x_stride_row", _c_i64), ("wq", _c_vp), ("wk", _c_vp), ("wv", _c_vp),
        ("bq", _c_vp), ("bk", _c_vp), ("bv", _c_vp), ("hidden", _c_i32), ("rope", RopeKVDesc),
    ]


# name -> (restype, argtypes); every symbol of include/fdllm_hip.h
SIGNATURES = {
    "fdllm_abi_version": (_c_int, []),
    "fdllm_last_error": (ctypes.c_char_p, []),
    "fdllm_gather_rmsnorm": (_c_int, [
        _c_vp, _c_i64, _c_i64,          # hidden, batch stride, row stride
        _c_vp, _c_i64,                  # indices, batch stride
        _c_vp, _c_int,                  # weight, weight dtype
        _c_vp, _c_vp,                   # normed, gathered
        _c_int, _c_int, _c_int, _c_int,  # B, S, T, H
        _c_float, _c_int, _c_int, _c_vp,  # eps, dtype, norm mode, stream
    ]),
    "fdllm_scatter_rows": (_c_int, [
        _c_vp, _c_vp, _c_i64,           # values, indices, indices batch stride
        _c_vp, _c_i64, _c_i64,          # cache, strides
        _c_vp, _c_i64, _c_i64,          # current, strides
        _c_int, _c_int, _c_int, _c_int,  # B, S, T, H
        _c_int, _c_vp,                  # dtype, stream
    ]),
    "fdllm_add_rmsnorm": (_c_int, [
        _c_vp, _c_vp, _c_vp, _c_int,    # x, residual, weight, weight dtype
        _c_vp, _c_vp, _c_int, _c_int,   # sum out, normed out, rows, hidden size
        ctypes.c_float, _c_int, _c_int, _c_vp,  # eps, dtype, norm mode, stream
    ]),
    "fdllm_silu_mul": (_c_int, [_c_vp, _c_vp, _c_vp, _c_i64, _c_int, _c_vp]),  # gate, up, out, n, dtype, stream
    "fdllm_kv_attn_workspace_size": (_c_int, [ctypes.POINTER(KVAttnDesc), ctypes.POINTER(_c_sz)]),
    "fdllm_kv_attn_fwd": (_c_int, [ctypes.POINTER(KVAttnDesc), _c_vp, _c_sz, _c_vp]),
    "fdllm_kv_attn_fwd_noalloc": (_c_int, [ctypes.POINTER(KVAttnDesc), _c_vp]),
    "fdllm_kv_cache_write": (_c_int, [
        _c_vp, _c_vp, _c_i64, _c_i64, _c_i64,   # k_new, v_new, strides
        _c_vp, _c_vp, _c_i64, _c_i64, _c_i64,   # k_cache, v_cache, strides
        _c_vp, _c_i32, _c_i32, _c_i32,          # page table, max_pages, page_size, max_seqlen
        _c_vp, _c_i32, _c_vp,                   # write_start, write_offset, positions
        _c_int, _c_int, _c_int, _c_int,         # B, T, Hkv, D
        _c_int, _c_vp,                          # dtype, stream
    ]),
    "fdllm_rope_kv_write": (_c_int, [ctypes.POINTER(RopeKVDesc), _c_vp]),
    "fdllm_qkv_rope_kv_write": (_c_int, [ctypes.POINTER(QkvRopeDesc), _c_vp]),
    "fdllm_unmask_step": (_c_int, [
        _c_vp, _c_i64, _c_i64, _c_int,          # logits, batch stride, row stride, vocab
        _c_int, _c_int,                         # row_offset, shift
        _c_vp, _c_i64,                          # tokens (int64), batch stride
        _c_vp, _c_i64, _c_float, _c_i64,        # finished (uint8), mask_id, threshold, stop_token
        _c_vp, _c_vp, _c_vp,                    # row_tok, row_conf, counts
        _c_int, _c_int, _c_int, _c_vp,          # batch, positions, dtype, stream
    ]),
}

_lib = None
_lock = threading.Lock()


def lib() -> ctypes.CDLL:
    """Load (once) and return the library; raises RuntimeError if it is unavailable."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is not built; run `python -m fast_v2_amd.build` "
                "(or __graft_entry__.build()) first")
        try:
            handle = ctypes.CDLL(str(LIB_PATH))
        except OSError as exc:
            raise RuntimeError(f"failed to load {LIB_PATH}: {exc}") from exc
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        if handle.fdllm_abi_version() != ABI_VERSION:
            raise RuntimeError("libfdllm_hip.so ABI version mismatch")
        _lib = handle
    return _lib


def check(rc: int, what: str) -> None:
    if rc != FDLLM_OK:
        msg = lib().fdllm_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed (code {rc}): {msg}")


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.bfloat16:
        return DTYPE_BF16
    if dt == torch.float16:
        return DTYPE_F16
    if dt == torch.float32:
        return DTYPE_F32
    raise RuntimeError(f"dtype {dt} is not supported by libfdllm_hip")


def stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream
