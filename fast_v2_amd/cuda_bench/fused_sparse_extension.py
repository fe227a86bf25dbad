"""HIP (gfx950) drop-in for cuda_bench/fused_sparse_extension.py.

Same surface as the reference module:

  get_fused_ops()                         -> object exposing the four entry points of
                                             fused_gather_norm.cu:215-221
  fused_gather_input_rmsnorm_pair(hidden_states, token_indices, input_layernorm)
                                          -> (selected_hidden, selected_norm) or None

Differences, by design:
  * The kernels live in libfdllm_hip.so (hand-written HIP for gfx950), loaded
    through ctypes; there is no JIT build and no CUDA toolchain.
  * bf16 / fp16 hidden states are consumed directly: the reference upcasts the
    whole [B, S, H] tensor to fp32 before gathering
    (fused_sparse_extension.py:81); here only the selected rows are read, once.
  * The model-path wrapper computes weight * normalized.to(dtype) inside the
    kernel (the Fast_dLLM_QwenRMSNorm order, modeling.py:427-432), one launch.
  * Load failure keeps the reference's contract (fused_sparse_extension.py:17-48):
    ``get_fused_ops()`` logs the reason once at ERROR level, latches the failure
    and returns ``None`` on this and every later call, and
    ``fused_gather_input_rmsnorm_pair`` then returns ``None`` so the caller takes
    its PyTorch path (modeling.py:879-890). Nothing in this module computes on
    the CPU; the ops of ``ops`` itself still raise without the library.
"""
from __future__ import annotations

import logging
from typing import Optional, Tuple

import torch

from .. import _ffi, ops


class _FusedOps:
    """The four pybind entry points of fused_gather_norm.cu:215-221."""

    @staticmethod
    def gather_rmsnorm_cuda(input: torch.Tensor, indices: torch.Tensor, weight: torch.Tensor,
                            eps: float) -> torch.Tensor:
        """out[b,t] = x * rsqrt(mean(x^2)+eps) * weight, x = input[b, indices[b,t]] (fp32 math)."""
        normed, _ = ops.gather_rmsnorm(input, indices, weight, eps, _ffi.NORM_WEIGHT_FP32,
                                       with_gathered=False)
        return normed

    @staticmethod
    def scatter_and_return_cuda(sparse_values: torch.Tensor, indices: torch.Tensor,
                                global_cache: torch.Tensor, current_hidden: torch.Tensor) -> torch.Tensor:
        """global_cache[b, idx] = current_hidden[b, idx] = sparse_values[b, t]; returns current_hidden."""
        return ops.scatter_rows(sparse_values, indices, global_cache, current_hidden)

    @staticmethod
    def fused_select_norm(hidden: torch.Tensor, indices: torch.Tensor, weight: torch.Tensor,
                          eps: float) -> torch.Tensor:
        normed, _ = ops.gather_rmsnorm(hidden, indices, weight, eps, _ffi.NORM_WEIGHT_FP32,
                                       with_gathered=False)
        return normed

    @staticmethod
    def fused_gather_input_rmsnorm_pair(hidden: torch.Tensor, indices: torch.Tensor, eps: float):
        """[gathered, x * rsqrt(mean(x^2)+eps)] with no weight (fused_gather_norm.cu:193-209)."""
        normed, gathered = ops.gather_rmsnorm(hidden, indices, None, eps, _ffi.NORM_PLAIN,
                                              with_gathered=True)
        return [gathered, normed]


_LOG = logging.getLogger(__name__)
_OPS: Optional[_FusedOps] = None
_OPS_FAILED = False


def get_fused_ops() -> Optional[_FusedOps]:
    """Load libfdllm_hip.so once and return the op table, or None if it cannot load.

    The first failure is logged with its reason and latched: later calls return
    None without trying again (fused_sparse_extension.py:25-48)."""
    global _OPS, _OPS_FAILED
    if _OPS_FAILED:
        return None
    if _OPS is None:
        try:
            _ffi.lib()
        except Exception as exc:  # a missing or unloadable library: the caller falls back
            _OPS_FAILED = True
            _LOG.error("fused gather+RMSNorm ops unavailable, callers fall back to PyTorch: %s", exc)
            return None
        _OPS = _FusedOps()
    return _OPS


def fused_gather_input_rmsnorm_pair(
    hidden_states: torch.Tensor,
    token_indices: torch.Tensor,
    input_layernorm: torch.nn.Module,
) -> Optional[Tuple[torch.Tensor, torch.Tensor]]:
    """Gather rows and apply Fast_dLLM_QwenRMSNorm to them in one kernel.

    hidden_states (B, S, H); token_indices (B, T); input_layernorm has .weight and
    .variance_epsilon (default 1e-6). Returns (selected_hidden, selected_norm) in
    hidden_states' dtype, or None when hidden_states is not on a GPU, the library
    cannot load, or the module has no weight (the reference's contract,
    fused_sparse_extension.py:70-78).
    """
    if not hidden_states.is_cuda:
        return None
    if get_fused_ops() is None:
        return None
    w = getattr(input_layernorm, "weight", None)
    if w is None:
        return None
    eps = getattr(input_layernorm, "variance_epsilon", 1e-6)
    eps = float(eps.item() if isinstance(eps, torch.Tensor) else eps)
    dt = hidden_states.dtype
    if w.dtype == dt:
        normed, gathered = ops.gather_rmsnorm(hidden_states, token_indices, w.detach(), eps,
                                              _ffi.NORM_WEIGHT_AFTER_CAST, with_gathered=True)
        return gathered, normed
    # Mixed precision (weight dtype != activations): the kernel rounds x*rsqrt to
    # `dt`, the product follows torch's type promotion exactly as the reference's
    # `w * normed_pre.to(dt)` does.
    normed_pre, gathered = ops.gather_rmsnorm(hidden_states, token_indices, None, eps,
                                              _ffi.NORM_PLAIN, with_gathered=True)
    return gathered, w * normed_pre
