"""Seeded synthetic inputs for the hot-path workloads (generated on the CPU).

Every generator draws from its own ``torch.Generator`` seeded with ``seed`` in a
fixed order, so the CPU baseline and the GPU run see identical inputs.

  kv_decode_fp32_small   block-decode attention, fp32, batch 1, 12/2 heads, D 128,
                         512 cached prefix keys + a 32-token block, all visible
  gather_rmsnorm_rows    bf16 hidden [4096 x 3584] with 1% x20 outliers, 1024 distinct
                         rows, RMSNorm weight ~ N(1, 0.02), eps 1e-6
  kv_decode_paged        7B geometry block decode: batch 16, 28/4 heads, D 128,
                         prefixes uniform in {1024..4096} step 32, 32-token pages,
                         an 8-token active sub-block of the current 32-token block
  block_prefill          block-causal prefill at 7B geometry: batch 4, 4096 tokens
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch


def _gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


# ---------------------------------------------------------------------------
@dataclass
class KVDecodeSmall:
    q: torch.Tensor          # [1, 32, 12, 128]
    k_cache: torch.Tensor    # [1, 544, 2, 128]
    v_cache: torch.Tensor
    seqlens: torch.Tensor    # [1] int32 (= 544)
    scale: float


def kv_decode_fp32_small(seed: int = 0, dtype=torch.float32) -> KVDecodeSmall:
    g = _gen(seed)
    q = torch.randn(1, 32, 12, 128, generator=g)
    k = torch.randn(1, 544, 2, 128, generator=g)
    v = torch.randn(1, 544, 2, 128, generator=g)
    return KVDecodeSmall(q.to(dtype), k.to(dtype), v.to(dtype),
                         torch.tensor([544], dtype=torch.int32), 128 ** -0.5)


# ---------------------------------------------------------------------------
@dataclass
class GatherRows:
    hidden: torch.Tensor   # [1, S, H] bf16
    indices: torch.Tensor  # [1, T] int64, distinct
    weight: torch.Tensor   # [H] bf16
    eps: float


def gather_rmsnorm_rows(seed: int = 0, seq_len: int = 4096, hidden: int = 3584, rows: int = 1024,
                        outlier_frac: float = 0.01, outlier_scale: float = 20.0,
                        dtype=torch.bfloat16) -> GatherRows:
    g = _gen(seed)
    h = torch.randn(1, seq_len, hidden, generator=g)
    mask = torch.rand(1, seq_len, hidden, generator=g) < outlier_frac
    h = torch.where(mask, h * outlier_scale, h).to(dtype)
    idx = torch.randperm(seq_len, generator=g)[:rows].unsqueeze(0).contiguous()
    w = (1.0 + 0.02 * torch.randn(hidden, generator=g)).to(dtype)
    return GatherRows(h, idx, w, 1e-6)


def gather_bytes(rows: int, hidden: int, elem: int = 2, with_gathered: bool = False,
                 index_bytes: int = 8) -> int:
    """Algorithmic HBM bytes of one gather+RMSNorm call: read the selected rows,
    write the normalised rows (and the gathered copy), read the weight and the indices."""
    per_row = hidden * elem
    return rows * per_row * (3 if with_gathered else 2) + hidden * elem + rows * index_bytes


def scatter_bytes(rows: int, hidden: int, elem: int = 2, destinations: int = 2, index_bytes: int = 8) -> int:
    """Algorithmic HBM bytes of one row scatter: read each value row once, write it to every
    destination, read the indices."""
    return rows * hidden * elem * (1 + destinations) + rows * index_bytes


# ---------------------------------------------------------------------------
@dataclass
class PagedDecode:
    q: torch.Tensor           # [B, Sq, Hq, D]
    k_pool: torch.Tensor      # [num_pages, page_size, Hkv, D]
    v_pool: torch.Tensor
    page_table: torch.Tensor  # [B, max_pages] int32
    seqlens: torch.Tensor     # [B] int32 = prefix + block
    prefix: torch.Tensor      # [B] int64 committed prefix lengths
    page_size: int
    sub_block: int            # index of the active sub-block within the current block
    scale: float


def kv_decode_paged(seed: int = 0, batch: int = 16, num_q_heads: int = 28, num_kv_heads: int = 4,
                    head_dim: int = 128, min_prefix: int = 1024, max_prefix: int = 4096,
                    block: int = 32, active: int = 8, page_size: int = 32, step: int = 0,
                    dtype=torch.bfloat16, shuffle_pages: bool = True,
                    layers: int = 1, head_major: bool = False) -> PagedDecode:
    """Paged block-decode attention inputs. With layers > 1 the pools carry a leading
    layer dimension [layers, num_pages, page_size, Hkv, D] (one pool per layer, same
    page table), the layout a 28-layer model step walks through. head_major=True stores
    each page [Hkv, page_size, D] (one KV head's page is one contiguous run) and returns
    the pools as [.., num_pages, page_size, Hkv, D] views of that storage; the values
    are the same draws as the token-major pools."""
    g = _gen(seed)
    lo, hi = min_prefix // block, max_prefix // block
    prefix = block * torch.randint(lo, hi + 1, (batch,), generator=g)
    seqlens = (prefix + block).to(torch.int32)
    pages_per = [(int(s) + page_size - 1) // page_size for s in seqlens]
    num_pages = sum(pages_per)
    max_pages = max(pages_per)
    perm = torch.randperm(num_pages, generator=g) if shuffle_pages else torch.arange(num_pages)
    table = torch.zeros(batch, max_pages, dtype=torch.int32)
    off = 0
    for b, n in enumerate(pages_per):
        table[b, :n] = perm[off:off + n].to(torch.int32)
        off += n
    shape = (num_pages, page_size, num_kv_heads, head_dim)
    if layers > 1:
        shape = (layers,) + shape
    k = torch.randn(*shape, generator=g).to(dtype)
    v = torch.randn(*shape, generator=g).to(dtype)
    q = torch.randn(batch, active, num_q_heads, head_dim, generator=g).to(dtype)
    if head_major:
        k = k.transpose(-3, -2).contiguous().transpose(-3, -2)
        v = v.transpose(-3, -2).contiguous().transpose(-3, -2)
    return PagedDecode(q, k, v, table, seqlens, prefix, page_size, step % max(1, block // active),
                       head_dim ** -0.5)


def decode_bytes(seqlens, num_q_heads: int, num_kv_heads: int, head_dim: int, q_len: int,
                 elem: int = 2) -> int:
    """Algorithmic HBM bytes of one block-decode attention call: every visible K and V
    row of every KV head once, plus Q in and O out."""
    keys = int(torch.as_tensor(seqlens).to(torch.int64).sum())
    batch = int(torch.as_tensor(seqlens).numel())
    return keys * num_kv_heads * head_dim * elem * 2 + 2 * batch * q_len * num_q_heads * head_dim * elem


def decode_flops(seqlens, num_q_heads: int, head_dim: int, q_len: int) -> int:
    keys = int(torch.as_tensor(seqlens).to(torch.int64).sum())
    return 4 * q_len * num_q_heads * head_dim * keys


# ---------------------------------------------------------------------------
@dataclass
class Prefill:
    q: torch.Tensor  # [B, S, Hq, D]
    k: torch.Tensor  # [B, S, Hkv, D]
    v: torch.Tensor
    block: int
    scale: float


def block_prefill(seed: int = 0, batch: int = 4, seq_len: int = 4096, num_q_heads: int = 28,
                  num_kv_heads: int = 4, head_dim: int = 128, block: int = 32,
                  dtype=torch.bfloat16) -> Prefill:
    g = _gen(seed)
    q = torch.randn(batch, seq_len, num_q_heads, head_dim, generator=g).to(dtype)
    k = torch.randn(batch, seq_len, num_kv_heads, head_dim, generator=g).to(dtype)
    v = torch.randn(batch, seq_len, num_kv_heads, head_dim, generator=g).to(dtype)
    return Prefill(q, k, v, block, head_dim ** -0.5)


def prefill_flops(batch: int, seq_len: int, num_q_heads: int, head_dim: int, block: int) -> int:
    """QK^T and PV over the visible (block-causal) key set: sum over query blocks j of
    block * (j+1) * block keys, 2 products x 2 flops each."""
    nblk = seq_len // block
    visible = sum(block * block * (j + 1) for j in range(nblk))
    return 4 * head_dim * num_q_heads * batch * visible


def prefill_bytes(batch: int, seq_len: int, num_q_heads: int, num_kv_heads: int, head_dim: int,
                  elem: int = 2) -> int:
    """Q read, O write, K/V read once and written once into the cache."""
    qo = 2 * batch * seq_len * num_q_heads * head_dim * elem
    kv = 2 * 2 * batch * seq_len * num_kv_heads * head_dim * elem
    return qo + kv
