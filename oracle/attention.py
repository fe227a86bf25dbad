"""Attention oracle (CPU) — test infrastructure only; never imported by the product.

Three restatements of the reference's attention semantics:

sdpa_kvcache        the reference's only CPU statement of kv-cache attention, the
                    SDPA shim of tests/test_focus.py:205-228 (== the SDPA backend,
                    utils/attention_backends.py:362-383, with the seqused mask of
                    utils/static_kv_cache.py:295-302): GQA expand, -inf for key
                    positions >= cache_seqlens[b], non-causal, BSHD in and out.
                    This is also the timed "reference CPU path" of bench.py.
sdpa_block_causal   the eager prefill / commit attention of
                    Fast_dLLM_QwenAttention.forward (modeling.py:385-411) with the
                    bool mask of eval_block_diff_mask / eval_mask
                    (modeling.py:145-150, :585-593) and repeat_kv (:202-211).
cache_write_np      StaticKVCache.update's write (utils/static_kv_cache.py:132-160:
                    rows t of the new K / V land at position start + t of the
                    layer's buffer) generalised to per-sequence starts and the
                    paged layout, with positions outside [0, capacity) skipped.
attention_np        an independent float64 numpy brute force of
                    softmax(q k^T * scale + M) v covering every mask mode of the
                    HIP kernel and the paged KV layout. Rows with no visible key
                    give 0, the flash_attn_with_kvcache convention (SDPA gives NaN).
"""
from __future__ import annotations

from typing import Optional

import numpy as np
import torch
import torch.nn.functional as F

MASK_SEQLEN = 0
MASK_CAUSAL = 1
MASK_BLOCK_CAUSAL = 2


def sdpa_kvcache(query: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                 cache_seqlens: torch.Tensor, is_causal: bool = False,
                 scaling: Optional[float] = None) -> torch.Tensor:
    """tests/test_focus.py:205-228: query [B,Sq,H,D], k/v_cache [B,max_S,Hkv,D] -> [B,Sq,H,D]."""
    B, Sq, H, D = query.shape
    max_S = k_cache.shape[1]
    Hkv = k_cache.shape[2]
    scale = scaling if scaling is not None else D ** -0.5
    q = query.transpose(1, 2)
    k = k_cache.transpose(1, 2)
    v = v_cache.transpose(1, 2)
    if H != Hkv:
        n_rep = H // Hkv
        k = k[:, :, None].expand(-1, -1, n_rep, -1, -1).reshape(B, H, max_S, D)
        v = v[:, :, None].expand(-1, -1, n_rep, -1, -1).reshape(B, H, max_S, D)
    pos = torch.arange(max_S, device=query.device)
    valid = pos[None, :] < cache_seqlens.to(torch.long)[:, None]
    attn_mask = torch.zeros(B, 1, 1, max_S, device=query.device, dtype=q.dtype)
    attn_mask.masked_fill_(~valid[:, None, None, :], float("-inf"))
    out = F.scaled_dot_product_attention(q, k, v, attn_mask=attn_mask, is_causal=is_causal, scale=scale)
    return out.transpose(1, 2).contiguous()


def block_causal_mask(q_len: int, kv_len: int, block_size: int, past_len: int = 0) -> torch.Tensor:
    """eval_block_diff_mask over q_idx = arange(q_len) + past_len, kv_idx = arange(kv_len)
    (modeling.py:145-150, :585-593): True where block(q) >= block(kv)."""
    q_idx = torch.arange(q_len) + past_len
    kv_idx = torch.arange(kv_len)
    return (q_idx[:, None] // block_size) >= (kv_idx[None, :] // block_size)


def repeat_kv(x: torch.Tensor, n_rep: int) -> torch.Tensor:
    """modeling.py:202-211 on BHSD tensors: KV head j serves query heads j*n_rep .. j*n_rep+n_rep-1."""
    b, hkv, s, d = x.shape
    if n_rep == 1:
        return x
    return x[:, :, None, :, :].expand(b, hkv, n_rep, s, d).reshape(b, hkv * n_rep, s, d)


def sdpa_block_causal(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, block_size: int = 32,
                      past_len: int = 0, scaling: Optional[float] = None) -> torch.Tensor:
    """Eager block-causal attention: q [B,S,H,D] for positions past_len.., k/v [B,past_len+S,Hkv,D]."""
    B, S, H, D = q.shape
    Hkv = k.shape[2]
    scale = scaling if scaling is not None else D ** -0.5
    qh = q.transpose(1, 2)
    kh = repeat_kv(k.transpose(1, 2), H // Hkv)
    vh = repeat_kv(v.transpose(1, 2), H // Hkv)
    mask = block_causal_mask(S, k.shape[1], block_size, past_len).to(q.device)
    out = F.scaled_dot_product_attention(qh, kh, vh, attn_mask=mask, is_causal=False, scale=scale)
    return out.transpose(1, 2).contiguous()


def cache_write_np(cache: np.ndarray, new: np.ndarray, starts, page_table=None,
                   page_size: Optional[int] = None, capacity: Optional[int] = None) -> np.ndarray:
    """A copy of ``cache`` ([B, max_S, Hkv, D], or a page pool with ``page_table``)
    with row t of ``new`` [B, T, Hkv, D] stored at position starts[b] + t, the
    StaticKVCache.update write (utils/static_kv_cache.py:132-160) per sequence.
    Positions < 0 or >= capacity (default: the buffer length, or pages x page_size)
    are skipped."""
    out = np.array(cache, copy=True)
    new = np.asarray(new)
    starts = np.asarray(starts).astype(np.int64)
    B, T = new.shape[:2]
    pt = None if page_table is None else np.asarray(page_table).astype(np.int64)
    if capacity is None:
        capacity = out.shape[1] if pt is None else pt.shape[1] * page_size
    for b in range(B):
        for t in range(T):
            pos = int(starts[b]) + t
            if pos < 0 or pos >= capacity:
                continue
            if pt is None:
                out[b, pos] = new[b, t]
            else:
                out[pt[b, pos // page_size], pos % page_size] = new[b, t]
    return out


def gather_kv_np(cache: np.ndarray, b: int, length: int, page_table: Optional[np.ndarray],
                 page_size: Optional[int]) -> np.ndarray:
    """Keys/values 0..length-1 of sequence b as [length, Hkv, D]."""
    if page_table is None:
        return cache[b, :length]
    pos = np.arange(length)
    pages = page_table[b, pos // page_size]
    return cache[pages, pos % page_size]


def attention_np(q, k_cache, v_cache, seqlens, scale: Optional[float] = None,
                 mask_mode: int = MASK_SEQLEN, mask_block: int = 32, q_start=None,
                 page_table=None, page_size: Optional[int] = None) -> np.ndarray:
    """float64 brute force. q [B,Sq,H,D]; k/v_cache [B,max_S,Hkv,D] (or a page pool with
    page_table [B,max_pages]); seqlens [B]; returns [B,Sq,H,D] float64.

    Query t of sequence b sits at position qpos = q_start[b] + t (default
    seqlens[b] - Sq). Key j is visible iff j < seqlens[b] and
      MASK_SEQLEN:        always
      MASK_CAUSAL:        j <= qpos
      MASK_BLOCK_CAUSAL:  j // mask_block <= qpos // mask_block
    """
    q = np.asarray(q, dtype=np.float64)
    kc = np.asarray(k_cache, dtype=np.float64)
    vc = np.asarray(v_cache, dtype=np.float64)
    seqlens = np.asarray(seqlens).astype(np.int64)
    B, Sq, H, D = q.shape
    Hkv = kc.shape[2]
    G = H // Hkv
    scale = D ** -0.5 if scale is None else scale
    out = np.zeros((B, Sq, H, D), dtype=np.float64)
    pt = None if page_table is None else np.asarray(page_table).astype(np.int64)
    for b in range(B):
        L = int(seqlens[b])
        if L <= 0:
            continue
        K = gather_kv_np(kc, b, L, pt, page_size)  # [L, Hkv, D]
        V = gather_kv_np(vc, b, L, pt, page_size)
        head_kv = np.arange(H) // G
        Kh = K[:, head_kv, :]  # [L, H, D]
        Vh = V[:, head_kv, :]
        s = np.einsum("thd,lhd->htl", q[b], Kh) * scale  # [H, Sq, L]
        qs = (L - Sq) if q_start is None else int(np.asarray(q_start)[b])
        qpos = qs + np.arange(Sq)
        j = np.arange(L)
        if mask_mode == MASK_SEQLEN:
            vis = np.ones((Sq, L), dtype=bool)
        elif mask_mode == MASK_CAUSAL:
            vis = j[None, :] <= qpos[:, None]
        elif mask_mode == MASK_BLOCK_CAUSAL:
            vis = (j[None, :] // mask_block) <= np.where(qpos >= 0, qpos // mask_block, -1)[:, None]
        else:
            raise ValueError(mask_mode)
        s = np.where(vis[None], s, -np.inf)
        m = s.max(axis=-1, keepdims=True)
        m = np.where(np.isfinite(m), m, 0.0)
        p = np.exp(s - m)
        l = p.sum(axis=-1, keepdims=True)
        o = np.einsum("htl,lhd->thd", p, Vh)  # [Sq, H, D]
        lt = np.transpose(l[..., 0])[:, :, None]  # [Sq, H, 1]
        out[b] = np.where(lt > 0, o / np.where(lt > 0, lt, 1.0), 0.0)
    return out
