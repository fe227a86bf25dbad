"""Drop-in for utils/static_kv_cache.py: the cross-block KV cache and the
within-block sub-block cache, with every KV write done by the HIP cache-write
kernel (libfdllm_hip.so, ``fdllm_kv_cache_write``).

Layout. Each cache owns ONE device allocation per tensor kind,
``[num_layers, batch, max_seq_len, num_kv_heads, head_dim]`` (BSHD per layer);
``key_cache[layer]`` / ``value_cache[layer]`` are views into it, so callers see
the reference's per-layer list of ``[B, max_S, Hkv, D]`` buffers
(static_kv_cache.py:55-69) while the memory stays one contiguous stretch of HBM
that the attention kernel walks with plain strides. At 7B geometry with the
default max_seq_len 4096 and batch 16 that is 28 x 2 x 16 x 4096 x 4 x 128 x 2 B
= 3.76 GB, about 1.3 % of one MI355X's HBM.

Writes. The reference builds a ``[B, S, Hkv, D]`` int64 scatter index for every
compiled step (prepare_write_idx, :180-216) and scatters through it; here the
write kernel computes each destination row from the int32 start position, so
``prepare_write_idx`` only refreshes that position and no index tensor exists.

Control signals keep the reference's names, dtypes and meaning:
``cache_seqlens`` int32 [B] committed length, ``scratch_seqlens`` int32 [B]
committed + current block (the attention's ``cache_seqlens``), ``kv_write_start``
int64 scalar. Buffer addresses are stable between compaction calls, so the
write and attention launches can be captured in a HIP graph.

CPU tensors: the bookkeeping (lengths, masks, compaction) works on any device;
the KV writes need the GPU and raise ``RuntimeError`` elsewhere.
"""
from __future__ import annotations

import torch

from .. import ops


def _mark_static(t: torch.Tensor) -> None:
    # torch.compile: buffer addresses never change (static_kv_cache.py:110-126)
    try:
        torch._dynamo.mark_static_address(t)
    except Exception:  # pragma: no cover - dynamo unavailable
        pass


class StaticKVCache:
    """Static KV cache for cross-block context (static_kv_cache.py:19-398)."""

    def __init__(self, batch_size: int, max_seq_len: int, num_layers: int, num_kv_heads: int,
                 head_dim: int, dtype: torch.dtype, device: torch.device):
        self.batch_size = batch_size
        self.max_batch_size = batch_size
        self.max_seq_len = max_seq_len
        self.num_layers = num_layers
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.dtype = dtype
        self.device = torch.device(device)
        self._alloc_buffers(batch_size)
        self._seq_len = 0
        self.kv_write_start = torch.zeros((), dtype=torch.int64, device=self.device)
        self._arange = torch.arange(max_seq_len, dtype=torch.int64, device=self.device)
        self._kv_indices = torch.arange(max_seq_len, dtype=torch.int32, device=self.device)
        self._write_len = 0
        self._mark_static_addresses()

    # ------------------------------------------------------------------
    def _alloc_buffers(self, bs: int) -> None:
        shape = (self.num_layers, bs, self.max_seq_len, self.num_kv_heads, self.head_dim)
        self._k_pool = torch.zeros(shape, dtype=self.dtype, device=self.device)
        self._v_pool = torch.zeros(shape, dtype=self.dtype, device=self.device)
        self.key_cache = list(self._k_pool.unbind(0))
        self.value_cache = list(self._v_pool.unbind(0))
        self.cache_seqlens = torch.zeros(bs, dtype=torch.int32, device=self.device)
        self.scratch_seqlens = torch.zeros(bs, dtype=torch.int32, device=self.device)
        # per-sequence copy of kv_write_start in the write kernel's int32 form
        self._write_start = torch.zeros(bs, dtype=torch.int32, device=self.device)
        self._attn_mask_buffer = torch.zeros(bs, 1, 1, self.max_seq_len, dtype=self.dtype, device=self.device)

    def _mark_static_addresses(self) -> None:
        for t in (self._k_pool, self._v_pool, self.cache_seqlens, self.scratch_seqlens, self.kv_write_start,
                  self._write_start, self._arange, self._attn_mask_buffer, self._kv_indices):
            _mark_static(t)

    def _check_states(self, key_states: torch.Tensor, value_states: torch.Tensor) -> None:
        if key_states.dim() != 4 or key_states.shape != value_states.shape:
            raise RuntimeError("StaticKVCache: key/value states must be matching BSHD [B, S, Hkv, D] tensors")
        if key_states.shape[0] != self.batch_size or key_states.shape[2] != self.num_kv_heads \
                or key_states.shape[3] != self.head_dim:
            raise RuntimeError(
                f"StaticKVCache: states {tuple(key_states.shape)} do not match the cache "
                f"[B={self.batch_size}, *, {self.num_kv_heads}, {self.head_dim}]")

    # ------------------------------------------------------------------
    # DynamicCache-compatible interface (eager prefill / commit)
    # ------------------------------------------------------------------
    def update(self, key_states, value_states, layer_idx, cache_kwargs=None):
        """Write at the committed position; the pointer advances after the last layer
        (static_kv_cache.py:132-160). Returns BSHD views up to the new end."""
        self._check_states(key_states, value_states)
        seq_len = key_states.shape[1]
        start = self._seq_len
        if start + seq_len > self.max_seq_len:
            raise RuntimeError(f"StaticKVCache.update: {start} + {seq_len} exceeds max_seq_len {self.max_seq_len}")
        ops.kv_cache_write(key_states, value_states, self.key_cache[layer_idx], self.value_cache[layer_idx],
                           write_offset=start)
        return self.note_update(seq_len, layer_idx)

    def note_update(self, seq_len: int, layer_idx: int):
        """The bookkeeping of ``update`` for rows a fused kernel already wrote at the
        committed position: advance after the last layer; returns the views ``update``
        returns."""
        start = self._seq_len
        if start + seq_len > self.max_seq_len:
            raise RuntimeError(f"StaticKVCache.update: {start} + {seq_len} exceeds max_seq_len {self.max_seq_len}")
        if layer_idx == self.num_layers - 1:
            self._seq_len += seq_len
            self.cache_seqlens.fill_(self._seq_len)
        end = start + seq_len
        return self.key_cache[layer_idx][:, :end], self.value_cache[layer_idx][:, :end]

    def commit_written(self, seq_len: int) -> None:
        """Commit the ``seq_len`` rows every layer already holds at ``kv_write_start``
        (written there by a diffusion-step forward over the final tokens of the block,
        which is what the commit forward computes): advance the committed length as
        ``update`` does after the last layer (static_kv_cache.py:132-160), without a
        forward that carries the write position on the host. The caller keeps
        ``kv_write_start`` at the committed length while the block is open."""
        if self._seq_len + seq_len > self.max_seq_len:
            raise RuntimeError(f"StaticKVCache.commit_written: {self._seq_len} + {seq_len} exceeds "
                               f"max_seq_len {self.max_seq_len}")
        self._seq_len += seq_len
        self.cache_seqlens.fill_(self._seq_len)

    def __getitem__(self, layer_idx):
        end = self._seq_len
        return self.key_cache[layer_idx][:, :end], self.value_cache[layer_idx][:, :end]

    def __len__(self):
        return self.num_layers if self._seq_len > 0 else 0

    def get_seq_length(self, layer_idx: int = 0) -> int:
        return self._seq_len

    # ------------------------------------------------------------------
    # Graph-friendly methods (device tensors only, no host-side positions)
    # ------------------------------------------------------------------
    def prepare_write_idx(self, seq_len: int) -> None:
        """Refresh the write position from ``kv_write_start`` before a captured step
        (static_kv_cache.py:180-216). No scatter index is built: the write kernel
        derives each row's destination from the start position."""
        self._write_len = int(seq_len)
        self._write_start.copy_(self.kv_write_start.to(torch.int32).expand(self.batch_size))

    def write_scratch_compiled(self, key_states, value_states, layer_idx) -> None:
        """Write at ``kv_write_start`` without advancing the pointer (:218-229).

        Goes through the ``fdllm::kv_cache_write`` op (in-place mutation of the layer's
        buffers declared in its schema), so torch.compile traces it without a break."""
        self._check_states(key_states, value_states)
        torch.ops.fdllm.kv_cache_write(key_states, value_states, self.key_cache[layer_idx],
                                       self.value_cache[layer_idx], self._write_start, 0, None)

    def write_sparse(self, key_states, value_states, layer_idx, write_positions) -> None:
        """Write token t of sequence b at position ``write_positions[b, t]`` (:231-247)."""
        self._check_states(key_states, value_states)
        if write_positions.shape != key_states.shape[:2]:
            raise RuntimeError("StaticKVCache.write_sparse: write_positions must be [B, num_tokens]")
        ops.kv_cache_write(key_states, value_states, self.key_cache[layer_idx], self.value_cache[layer_idx],
                           positions=write_positions)

    def get_full_kv(self, layer_idx):
        """The full static buffers, constant shape [B, max_seq_len, Hkv, D] (:249-254)."""
        return self.key_cache[layer_idx], self.value_cache[layer_idx]

    def set_scratch_seqlens(self, total_valid_len: int) -> None:
        """Every row gets the same effective length (:256-258)."""
        self.scratch_seqlens.fill_(total_valid_len)

    def set_kv_write_start(self, offset: int) -> None:
        self.kv_write_start.fill_(offset)
        self._write_start.fill_(offset)

    # ------------------------------------------------------------------
    # Eager helpers
    # ------------------------------------------------------------------
    def write_scratch(self, key_states, value_states, layer_idx, position) -> None:
        self._check_states(key_states, value_states)
        ops.kv_cache_write(key_states, value_states, self.key_cache[layer_idx], self.value_cache[layer_idx],
                           write_offset=int(position))

    def get_kv_up_to(self, layer_idx, length):
        return self.key_cache[layer_idx][:, :length], self.value_cache[layer_idx][:, :length]

    def get_seqused_mask(self, total_valid_len: int):
        """Additive SDPA mask: 0 below ``total_valid_len``, -inf from there (:286-293)."""
        self._attn_mask_buffer.fill_(0.0)
        invalid = self._kv_indices[None, :] >= total_valid_len
        self._attn_mask_buffer.masked_fill_(invalid[:, None, None, :], float("-inf"))
        return self._attn_mask_buffer

    def get_seqused_mask_batched(self, seqused: torch.Tensor):
        self._attn_mask_buffer.fill_(0.0)
        invalid = self._kv_indices[None, :] >= seqused[:, None]
        self._attn_mask_buffer.masked_fill_(invalid[:, None, None, :], float("-inf"))
        return self._attn_mask_buffer

    def reset(self) -> None:
        """Reset the committed length; the buffers keep their contents (:304-307)."""
        self._seq_len = 0
        self.cache_seqlens.fill_(0)

    def zero_and_reset(self) -> None:
        self._k_pool.zero_()
        self._v_pool.zero_()
        self._seq_len = 0
        self.cache_seqlens.fill_(0)
        self.scratch_seqlens.fill_(0)
        self.kv_write_start.fill_(0)
        self._write_start.fill_(0)

    def restore_full_batch(self) -> None:
        """Re-allocate at max_batch_size after compaction; contents are stale (:319-348)."""
        if self.batch_size == self.max_batch_size:
            return
        self._alloc_buffers(self.max_batch_size)
        self._seq_len = 0
        self.kv_write_start.fill_(0)
        self.batch_size = self.max_batch_size
        self._mark_static_addresses()

    def compact_batch(self, active_indices: torch.Tensor) -> None:
        """Keep only the sequences in ``active_indices`` (eager, block boundaries; :350-398)."""
        active_indices = active_indices.to(device=self.device, dtype=torch.long)
        self._k_pool = self._k_pool[:, active_indices].contiguous()
        self._v_pool = self._v_pool[:, active_indices].contiguous()
        self.key_cache = list(self._k_pool.unbind(0))
        self.value_cache = list(self._v_pool.unbind(0))
        self.cache_seqlens = self.cache_seqlens[active_indices].contiguous()
        self.scratch_seqlens = self.scratch_seqlens[active_indices].contiguous()
        self._write_start = self._write_start[active_indices].contiguous()
        n = active_indices.numel()
        self._attn_mask_buffer = torch.zeros(n, 1, 1, self.max_seq_len, dtype=self.dtype, device=self.device)
        self.batch_size = n


class StaticBlockCache:
    """Within-block sub-block cache, [B, block_size, Hkv, D] per layer
    (static_kv_cache.py:401-491). ``reset`` clears the initialised-layer count,
    not the data."""

    def __init__(self, batch_size: int, block_size: int, num_layers: int, num_kv_heads: int, head_dim: int,
                 dtype: torch.dtype, device: torch.device):
        self.batch_size = batch_size
        self.block_size = block_size
        self.num_layers = num_layers
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.dtype = dtype
        self.device = torch.device(device)
        shape = (num_layers, batch_size, block_size, num_kv_heads, head_dim)
        self._k_pool = torch.zeros(shape, dtype=dtype, device=self.device)
        self._v_pool = torch.zeros(shape, dtype=dtype, device=self.device)
        self.key_cache = list(self._k_pool.unbind(0))
        self.value_cache = list(self._v_pool.unbind(0))
        self._num_initialized = 0
        _mark_static(self._k_pool)
        _mark_static(self._v_pool)

    def update(self, key_states, value_states, layer_idx, cache_kwargs=None):
        """Write rows [0, S) of the layer's block buffer; returns the full buffers."""
        if key_states.shape[1] > self.block_size:
            raise RuntimeError("StaticBlockCache.update: more tokens than the block holds")
        self.write(key_states, value_states, layer_idx, 0)
        return self.note_update(layer_idx)

    def note_update(self, layer_idx: int):
        """The bookkeeping of ``update`` for rows a fused kernel already wrote."""
        if layer_idx >= self._num_initialized:
            self._num_initialized = layer_idx + 1
        return self.key_cache[layer_idx], self.value_cache[layer_idx]

    def write(self, key_states, value_states, layer_idx, offset: int) -> None:
        """Copy S new rows to block positions offset .. offset + S (the sub-block write of
        utils/attention_backends.py:847-866)."""
        ops.kv_cache_write(key_states, value_states, self.key_cache[layer_idx], self.value_cache[layer_idx],
                           write_offset=int(offset))

    def __getitem__(self, layer_idx):
        return self.key_cache[layer_idx], self.value_cache[layer_idx]

    def __len__(self):
        return self._num_initialized

    def get_seq_length(self, layer_idx: int = 0) -> int:
        return 0 if self._num_initialized == 0 else self.block_size

    def reset(self) -> None:
        self._num_initialized = 0

    def compact_batch(self, active_indices: torch.Tensor) -> None:
        active_indices = active_indices.to(device=self.device, dtype=torch.long)
        self._k_pool = self._k_pool[:, active_indices].contiguous()
        self._v_pool = self._v_pool[:, active_indices].contiguous()
        self.key_cache = list(self._k_pool.unbind(0))
        self.value_cache = list(self._v_pool.unbind(0))
        self.batch_size = active_indices.numel()


__all__ = ["StaticKVCache", "StaticBlockCache"]
