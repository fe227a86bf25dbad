"""Drop-in for utils/block_sparse_cache.py: per-block stacked caches of the
token-sparse forward, ``[num_layers, batch, block_size, hidden]`` each.

The two scatter methods (the writes that follow a sparse attention or MLP step,
block_sparse_cache.py:112-132) run the HIP row-scatter kernel
(``fdllm_scatter_rows`` with one destination) instead of building a
``[B, T, hidden]`` int64 index for ``scatter_``; whole-layer writes are plain
device copies.
"""
from __future__ import annotations

import torch

from .. import ops


class BlockSparseCache:
    """layer_input / attn_output / mlp_input / mlp_output, each [L, B, block_size, hidden]
    (block_sparse_cache.py:18-147). Layer output = mlp_input + mlp_output."""

    def __init__(self, num_layers: int, batch_size: int, block_size: int, hidden_size: int,
                 dtype: torch.dtype, device: torch.device):
        self.num_layers = num_layers
        self.batch_size = batch_size
        self.block_size = block_size
        self.hidden_size = hidden_size
        self.dtype = dtype
        self.device = torch.device(device)
        shape = (num_layers, batch_size, block_size, hidden_size)
        self.layer_input = torch.zeros(shape, dtype=dtype, device=self.device)
        self.attn_output = torch.zeros(shape, dtype=dtype, device=self.device)
        self.mlp_input = torch.zeros(shape, dtype=dtype, device=self.device)
        self.mlp_output = torch.zeros(shape, dtype=dtype, device=self.device)

    # ---- writes
    def cache_layer_input(self, layer_idx: int, hidden_states: torch.Tensor) -> None:
        self.layer_input.select(0, layer_idx).copy_(hidden_states)

    def cache_attn_output(self, layer_idx: int, attn_out: torch.Tensor) -> None:
        self.attn_output.select(0, layer_idx).copy_(attn_out)

    def cache_mlp_input(self, layer_idx: int, mid: torch.Tensor) -> None:
        self.mlp_input.select(0, layer_idx).copy_(mid)

    def cache_mlp_output(self, layer_idx: int, mlp_out: torch.Tensor) -> None:
        self.mlp_output.select(0, layer_idx).copy_(mlp_out)

    # ---- reads
    def get_layer_input(self, layer_idx: int) -> torch.Tensor:
        return self.layer_input.select(0, layer_idx)

    def get_attn_output(self, layer_idx: int) -> torch.Tensor:
        return self.attn_output.select(0, layer_idx)

    def get_mlp_input(self, layer_idx: int) -> torch.Tensor:
        return self.mlp_input.select(0, layer_idx)

    def get_mlp_output(self, layer_idx: int) -> torch.Tensor:
        return self.mlp_output.select(0, layer_idx)

    # ---- sparse scatters: row t of values goes to block position token_indices[b, t]
    def scatter_attn_output(self, layer_idx: int, token_indices: torch.Tensor, values: torch.Tensor) -> None:
        ops.scatter_rows(values, token_indices, self.attn_output.select(0, layer_idx))

    def scatter_mlp_output(self, layer_idx: int, token_indices: torch.Tensor, values: torch.Tensor) -> None:
        ops.scatter_rows(values, token_indices, self.mlp_output.select(0, layer_idx))

    def reset(self) -> None:
        """Nothing to clear: the first (dense) step of each block overwrites every row."""

    def compact_batch(self, active_indices: torch.Tensor) -> None:
        active_indices = active_indices.to(device=self.device, dtype=torch.long)
        self.layer_input = self.layer_input[:, active_indices].contiguous()
        self.attn_output = self.attn_output[:, active_indices].contiguous()
        self.mlp_input = self.mlp_input[:, active_indices].contiguous()
        self.mlp_output = self.mlp_output[:, active_indices].contiguous()
        self.batch_size = active_indices.numel()


__all__ = ["BlockSparseCache"]
