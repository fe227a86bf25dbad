"""Drop-in for utils/dynamic_block_kv.py: the current block's key/value rows of
each deep layer, BHSD ``[B, num_kv_heads, block_size, head_dim]``.

``write`` (the selected-token scatter along the sequence dim,
dynamic_block_kv.py:39-43) runs the HIP KV-write kernel with per-token
positions: the BHSD buffer is handed over as a strided BSHD view, so no
``[B, Hkv, n, D]`` index tensor is built.
"""
from __future__ import annotations

import torch

from .. import ops


class DynamicBlockKV:
    def __init__(self, deep_layer_start, num_layers, batch_size, num_kv_heads, block_size, head_dim, dtype,
                 device):
        self.deep_layer_start = deep_layer_start
        self.num_layers = num_layers
        self.num_kv_heads = num_kv_heads
        self.block_size = block_size
        self.head_dim = head_dim
        self.dtype = dtype
        self.device = torch.device(device)
        self.k = {L: torch.zeros(batch_size, num_kv_heads, block_size, head_dim, dtype=dtype, device=self.device)
                  for L in range(deep_layer_start, num_layers)}
        self.v = {L: torch.zeros(batch_size, num_kv_heads, block_size, head_dim, dtype=dtype, device=self.device)
                  for L in range(deep_layer_start, num_layers)}
        self.batch_size = batch_size

    def write_full(self, layer_idx, k, v) -> None:
        """Replace every row of ``layer_idx``'s block with ``k`` / ``v`` (both BHSD, all
        ``block_size`` positions), as the dense seed step of a block does."""
        self.k[layer_idx].copy_(k)
        self.v[layer_idx].copy_(v)

    def write(self, layer_idx, k, v, token_indices) -> None:
        """Store ``n`` recomputed rows per sequence: row ``i`` of ``k`` / ``v`` (BHSD, length
        ``n``) lands at block position ``token_indices[b, i]``; positions not listed keep
        their previous contents."""
        if k.dim() != 4 or k.shape != v.shape or token_indices.shape != (k.shape[0], k.shape[2]):
            raise RuntimeError("DynamicBlockKV.write: expected k, v [B, Hkv, n, D] and token_indices [B, n]")
        ops.kv_cache_write(k.transpose(1, 2), v.transpose(1, 2),
                           self.k[layer_idx].transpose(1, 2), self.v[layer_idx].transpose(1, 2),
                           positions=token_indices)

    def get(self, layer_idx):
        """The (k, v) buffers of ``layer_idx`` themselves, not copies."""
        return self.k[layer_idx], self.v[layer_idx]

    def reset(self) -> None:
        """No-op: each block opens with a dense write that covers every position."""

    def compact_batch(self, active_indices) -> None:
        """Keep only the sequences in ``active_indices`` (in that order)."""
        for L in self.k:
            self.k[L] = self.k[L][active_indices].contiguous()
            self.v[L] = self.v[L][active_indices].contiguous()
        self.batch_size = active_indices.numel()


__all__ = ["DynamicBlockKV"]
