"""Gather + RMSNorm oracle (CPU) — test infrastructure only; never imported by the product.

ref_gather_input_rmsnorm   cuda_bench/test_correctness.py:33-50: gather in fp32,
                           var = mean(g*g), inv = rsqrt(var + eps),
                           normed = weight * (g*inv).to(dtype)  — the rounding order of
                           Fast_dLLM_QwenRMSNorm.forward (modeling.py:427-432) and of
                           fused_sparse_extension.fused_gather_input_rmsnorm_pair
                           (cuda_bench/fused_sparse_extension.py:80-87).
ref_gather_rmsnorm_fp32w   gather_rmsnorm_cuda / fused_select_norm
                           (cuda_bench/fused_gather_norm.cu:21-73, :177-190):
                           out = g * inv * w in fp32 (weight applied before rounding).
ref_gather_pair_plain      fused_gather_input_rmsnorm_pair host fn (fused_gather_norm.cu:193-209):
                           returns (g, g*inv) without a weight.
gather_rmsnorm_np          the same three modes in float64 numpy, with explicit
                           round-to-nearest-even to bf16/fp16 where the reference rounds.
scatter_rows_np            scatter_and_return_cuda (fused_gather_norm.cu:79-119): the
                           rows written back to two [B, S, H] destinations.
"""
from __future__ import annotations

import numpy as np
import torch

NORM_PLAIN = 0
NORM_WEIGHT_FP32 = 1
NORM_WEIGHT_AFTER_CAST = 2


def ref_gather_input_rmsnorm(hidden: torch.Tensor, token_indices: torch.Tensor,
                             weight: torch.Tensor, eps: float):
    h = hidden.float().contiguous()
    b, _, dim = h.shape
    t = token_indices.shape[1]
    idx = token_indices.unsqueeze(-1).expand(b, t, dim)
    gathered_f = h.gather(1, idx)
    var = (gathered_f * gathered_f).mean(dim=-1, keepdim=True)
    inv = torch.rsqrt(var + eps)
    normed_pre = gathered_f * inv
    dt = hidden.dtype
    normed = weight * normed_pre.to(dt)
    return gathered_f.to(dt), normed


def ref_gather_rmsnorm_fp32w(hidden: torch.Tensor, token_indices: torch.Tensor,
                             weight: torch.Tensor, eps: float) -> torch.Tensor:
    h = hidden.float()
    b, _, dim = h.shape
    idx = token_indices.long().unsqueeze(-1).expand(b, token_indices.shape[1], dim)
    g = h.gather(1, idx)
    inv = torch.rsqrt((g * g).mean(-1, keepdim=True) + eps)
    return (g * inv * weight.float()).to(hidden.dtype)


def ref_gather_pair_plain(hidden: torch.Tensor, token_indices: torch.Tensor, eps: float):
    h = hidden.float()
    b, _, dim = h.shape
    idx = token_indices.long().unsqueeze(-1).expand(b, token_indices.shape[1], dim)
    g = h.gather(1, idx)
    inv = torch.rsqrt((g * g).mean(-1, keepdim=True) + eps)
    return g.to(hidden.dtype), (g * inv).to(hidden.dtype)


# ---------------------------------------------------------------------------
# numpy float64 restatement
# ---------------------------------------------------------------------------

def round_f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """Round float32 values to the nearest bfloat16 (ties to even); returns float32."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    out = rounded.astype(np.uint32).view(np.float32)
    return np.where(np.isnan(x), x, out)


def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "bf16":
        return round_f32_to_bf16(np.asarray(x, dtype=np.float32))
    if dtype == "f16":
        return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)
    return np.asarray(x, dtype=np.float32)


def gather_rmsnorm_np(hidden: np.ndarray, indices: np.ndarray, weight, eps: float,
                      mode: int = NORM_WEIGHT_AFTER_CAST, dtype: str = "bf16"):
    """hidden [B,S,H] (values already representable in `dtype`), indices [B,T] -> (gathered, normed).

    Arithmetic in float64; results rounded to `dtype` where the reference rounds.
    """
    h = np.asarray(hidden, dtype=np.float64)
    idx = np.asarray(indices).astype(np.int64)
    B = h.shape[0]
    g = np.stack([h[b, idx[b]] for b in range(B)])  # [B, T, H]
    inv = 1.0 / np.sqrt((g * g).mean(axis=-1, keepdims=True) + eps)
    n = g * inv
    if mode == NORM_PLAIN:
        normed = round_to(n, dtype)
    elif mode == NORM_WEIGHT_FP32:
        normed = round_to(n * np.asarray(weight, dtype=np.float64), dtype)
    elif mode == NORM_WEIGHT_AFTER_CAST:
        nb = round_to(n, dtype).astype(np.float64)
        normed = round_to(np.asarray(weight, dtype=np.float64) * nb, dtype)
    else:
        raise ValueError(mode)
    return round_to(g, dtype), normed


def scatter_rows_np(values: np.ndarray, indices: np.ndarray, cache: np.ndarray,
                    current: np.ndarray | None = None):
    """scatter_and_return_kernel / scatter_and_return_cuda (cuda_bench/fused_gather_norm.cu:79-119):
    cache[b, indices[b, t]] = values[b, t] and the same into current, which is returned.
    The reference's PyTorch statement of the same step is the scatter_ of
    cuda_bench/bench_sparse_cuda.py:88-96 (pytorch_roundtrip). Indices outside [0, S) leave both destinations
    untouched (the reference kernel does not check them). Works on copies; returns
    (cache, current)."""
    v = np.asarray(values)
    idx = np.asarray(indices).astype(np.int64)
    c = np.array(cache, copy=True)
    u = None if current is None else np.array(current, copy=True)
    S = c.shape[1]
    for b in range(v.shape[0]):
        for t in range(v.shape[1]):
            r = idx[b, t]
            if 0 <= r < S:
                c[b, r] = v[b, t]
                if u is not None:
                    u[b, r] = v[b, t]
    return c, u
