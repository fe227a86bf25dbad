"""Static-KV block-diffusion sampler: batch_sample_dynamo
(generation_functions.py:243-954) in eager execution with a fixed batch.

Per block of ``block_size`` tokens (generation_functions.py:586-700):
  * the block is filled with ``mask_id`` and the cache's control signals are set
    (kv_write_start = committed length, scratch_seqlens = committed + block);
  * for each sub-block of ``small_block_size`` tokens, repeat until none of its
    tokens is masked: run the model (the full block, or only the sub-block when the
    block cache holds the block's K/V and the sub-block's first token is known,
    :723-756), shift the logits by one position (:774), take the greedy token and
    its probability, unmask every masked token whose probability exceeds
    ``threshold`` (strict ``>``, :791) and at least the most probable one per row
    (:792-794);
  * commit: run the block once more with update_past_key_values=True, which writes
    its K/V at the committed position and advances it, and append the argmax of the
    last position as the first token of the next block (:685-696).
The prompt is prefilled the same way (:557-575); on this static path the prefill
attention sees the whole prompt (the patched forward ignores the block mask).

Attention and KV caching come from an ``impl`` object, so the same loop runs on
the HIP kernels (``HipStaticAttention``, the product) or on any other
implementation of the same cache interface.
"""
from __future__ import annotations

import time
from dataclasses import dataclass, field
from typing import Optional

import torch

from .. import ops
from ..utils import attention_backends as ab
from ..utils.attention_backends import get_attention_backend, patch_attention_layers, unpatch_attention_layers
from ..utils.static_kv_cache import StaticBlockCache, StaticKVCache
from .model import set_fused_norms


class HipStaticAttention:
    """StaticKVCache / StaticBlockCache with HIP writes + the 'hip' attention backend,
    the model's RMSNorms on the fused gather + RMSNorm kernel, and the diffusion-step
    forwards replayed from HIP graphs (``graphs=False`` runs them eagerly)."""

    name = "hip"

    def __init__(self, graphs: bool = True, fused_norm: bool = True, fused_sampler: bool = True,
                 fused_qkv: bool = False):
        self.graphs = graphs
        self.fused_norm = fused_norm
        self.fused_sampler = fused_sampler
        # the q / k / v projections in the RoPE + cache-write kernel (attention_backends.FUSED_QKV_PROJECTION)
        self.fused_qkv = fused_qkv
        self._saved_qkv = None

    def make_caches(self, batch, max_seq_len, cfg, dtype, device, use_block_cache):
        cache = StaticKVCache(batch, max_seq_len, cfg.num_hidden_layers, cfg.num_key_value_heads, cfg.head_dim,
                              dtype, device)
        block = (StaticBlockCache(batch, cfg.bd_size, cfg.num_hidden_layers, cfg.num_key_value_heads, cfg.head_dim,
                                  dtype, device) if use_block_cache else None)
        return cache, block

    def patch(self, model, block_cache):
        if self.fused_norm:
            set_fused_norms(model, True)
        self._saved_qkv = ab.FUSED_QKV_PROJECTION
        ab.FUSED_QKV_PROJECTION = self.fused_qkv
        return patch_attention_layers(model, get_attention_backend("hip"), block_cache)

    def unpatch(self, model, originals):
        unpatch_attention_layers(model, originals)
        set_fused_norms(model, False)
        if self._saved_qkv is not None:
            ab.FUSED_QKV_PROJECTION = self._saved_qkv


class ForwardGraphs:
    """One HIP graph per kind of diffusion-step forward (the full block, and the
    sub-block at each offset), captured on first use and replayed after that.

    Everything that changes between blocks reaches the captured kernels through
    device memory: the token ids and positions are copied into the graph's static
    inputs before each replay, and the static cache's write position and visible
    lengths live in device tensors (StaticKVCache.kv_write_start / scratch_seqlens).
    Commits are a kind of their own (the full block without the block cache); the host
    only advances the committed length after the replay. (The prompt prefill runs
    eagerly in the same form: it runs once per generation.) The first use of a kind runs
    it eagerly once (on the capture stream, so allocations and the attention
    workspace exist before capture), captures it, and replays it; the eager run and
    the replay write the same cache rows."""

    def __init__(self):
        self._graphs = {}
        self._stream = None

    def __call__(self, key, fn, ids: torch.Tensor, pos: torch.Tensor) -> torch.Tensor:
        ent = self._graphs.get(key)
        if ent is None:
            if self._stream is None:
                self._stream = torch.cuda.Stream(ids.device)
            s = self._stream
            sid, spos = ids.clone(), pos.clone()
            s.wait_stream(torch.cuda.current_stream(ids.device))
            with torch.cuda.stream(s):
                fn(sid, spos)
            torch.cuda.current_stream(ids.device).wait_stream(s)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=s):
                out = fn(sid, spos)
            ent = (graph, sid, spos, out)
            self._graphs[key] = ent
        graph, sid, spos, out = ent
        sid.copy_(ids)
        spos.copy_(pos)
        graph.replay()
        return out


@dataclass
class GenerationStats:
    forwards: int = 0
    commits: int = 0
    blocks: int = 0
    seconds: float = 0.0
    generated_tokens: int = 0
    step_tokens: list = field(default_factory=list)

    @property
    def tokens_per_second(self) -> float:
        return self.generated_tokens / self.seconds if self.seconds > 0 else 0.0


def greedy_with_confidence(logits: torch.Tensor):
    """sample_with_top_p at temperature 0 (modeling.py:2263-2270): softmax in the
    logits' dtype, argmax token and its probability."""
    p = torch.softmax(logits, dim=-1)
    x = p.argmax(dim=-1)
    return x, torch.gather(p, -1, x.unsqueeze(-1)).squeeze(-1)


def threshold_unmask(tok: torch.Tensor, conf: torch.Tensor, masked: torch.Tensor, threshold: float):
    """Unmask every masked position whose confidence exceeds ``threshold`` and the
    most confident masked position of each row (generation_functions.py:784-795)."""
    conf = torch.where(masked, conf, torch.full_like(conf, float("-inf")))
    unmask = conf > threshold
    unmask[torch.arange(conf.shape[0], device=conf.device), conf.argmax(dim=-1)] = True
    return unmask & masked


@torch.no_grad()
def generate(model, input_ids: torch.Tensor, max_new_tokens: int = 1024, block_size: int = 32,
             small_block_size: int = 8, mask_id: int = 152063, threshold: float = 0.9,
             use_block_cache: bool = True, stop_token: Optional[int] = None, pad_token: int = 0,
             impl=None, max_seq_len: Optional[int] = None, sync_timing: bool = True, policy=None,
             bridge_policy=None, progress=None):
    """Generate for a batch of equal-length prompts [B, P]; returns (tokens [B, P + N + 1], stats).

    Equal prompt lengths are the config of the end-to-end workload; the reference's
    per-row bookkeeping for ragged prompts (BatchBucket) is not needed for it.
    ``policy(step, tok, conf, masked) -> (tok, unmask)`` replaces the greedy threshold
    rule when given (``step`` counts sampling steps from 0); ``bridge_policy(i, tok) ->
    tok`` likewise replaces the argmax token that opens each block (i = 0 after the
    prefill, then one per commit). ``progress(stats)`` is called on the host after every
    forward is issued (it must not synchronise the device if timing matters)."""
    n_bridge = [0]

    def bridge(tok):
        if bridge_policy is not None:
            tok = bridge_policy(n_bridge[0], tok)
        n_bridge[0] += 1
        return tok

    impl = impl or HipStaticAttention()
    graphs = ForwardGraphs() if getattr(impl, "graphs", False) else None
    fused = getattr(impl, "fused_sampler", False) and policy is None
    scratch = None
    cfg = model.config
    B, P = input_ids.shape
    dev = input_ids.device
    dtype = model.lm_head.weight.dtype
    if max_seq_len is None:
        need = P + max_new_tokens + block_size
        max_seq_len = (need + 255) // 256 * 256
    cache, block_cache = impl.make_caches(B, max_seq_len, cfg, dtype, dev, use_block_cache)
    originals = impl.patch(model, block_cache)
    stats = GenerationStats()
    try:
        if sync_timing:
            torch.cuda.synchronize(dev)
        t0 = time.perf_counter()
        x = input_ids.clone()
        min_len = P
        # ---- prefill (generation_functions.py:557-575)
        if min_len > block_size:
            prefill_len = min_len // block_size * block_size
            if graphs is not None and isinstance(cache, StaticKVCache) and cache.get_seq_length() == 0:
                # the commits' form of the forward (the prompt's rows written at
                # kv_write_start = 0, every prompt key visible as in the update path, the last
                # position's logits kept, the only ones read; the committed length then
                # advances on the host), run eagerly: it runs once per generation, where a
                # graph would cost an eager run and a capture for a single replay
                cache.set_kv_write_start(0)
                cache.set_scratch_seqlens(prefill_len)
                cache.prepare_write_idx(prefill_len)
                logits = model(x[:, :prefill_len], cache, cache_position=torch.arange(prefill_len, device=dev),
                               logits_to_keep=1)
                cache.commit_written(prefill_len)
            else:
                logits = model(x[:, :prefill_len], cache, update_past_key_values=True)
            stats.forwards += 1
            if progress is not None:
                progress(stats)
            if min_len % block_size == 0:
                x = torch.cat([x, bridge(logits[:, -1:].argmax(dim=-1))], dim=1)
        num_blocks = max_new_tokens // block_size + P // block_size
        finished = torch.zeros(B, dtype=torch.bool, device=dev)
        for block_idx in range(min_len // block_size, num_blocks):
            if x.shape[1] < (block_idx + 1) * block_size:
                pad_len = (block_idx + 1) * block_size - x.shape[1]
                x = torch.cat([x, torch.full((B, pad_len), mask_id, dtype=x.dtype, device=dev)], dim=1)
            if block_cache is not None:
                block_cache.reset()
            past_len = cache.get_seq_length()
            cache.set_kv_write_start(past_len)
            cache.set_scratch_seqlens(past_len + block_size)
            cache.prepare_write_idx(block_size)
            cache_pos = torch.arange(past_len, past_len + block_size, device=dev)
            stats.blocks += 1
            blk = slice(block_idx * block_size, (block_idx + 1) * block_size)
            for sb in range(block_size // small_block_size):
                s0, s1 = sb * small_block_size, (sb + 1) * small_block_size
                # sub-block state: masked positions left (unfinished rows) and whether
                # position s0 is still masked in some row; the fused sampler reports both
                # after each step, the torch rule recomputes them from x
                mask = x[:, blk] == mask_id
                left = bool((mask[:, s0:s1] & ~finished[:, None]).any())
                first_masked = bool(mask[:, s0].any())
                sub_steps = 0
                while left:
                    # every step unmasks at least one position of each unfinished row unless
                    # the sampled token is the mask token itself, so a sub-block needs at most
                    # small_block_size steps; far more means the model keeps predicting the
                    # mask token (the reference loop would not end either)
                    sub_steps += 1
                    if sub_steps > 8 * small_block_size:
                        raise RuntimeError(
                            f"block {block_idx}, sub-block {sb}: no progress after {sub_steps - 1} steps "
                            f"(the model keeps predicting the mask token {mask_id})")
                    if use_block_cache and len(block_cache) > 0 and not first_masked:
                        def sub_fwd(ids, pos, s0=s0):
                            return model(ids, cache, use_block_cache=True, block_past_key_values=block_cache,
                                         replace_position=s0, cache_position=pos, logits_to_keep=small_block_size)
                        ids = x[:, blk][:, s0:s1]
                        pos = cache_pos[s0:s1]
                        raw = graphs(("sub", s0), sub_fwd, ids, pos) if graphs else sub_fwd(ids, pos)
                        row_offset = 0
                    else:
                        def full_fwd(ids, pos):
                            return model(ids, cache, use_block_cache=use_block_cache,
                                         block_past_key_values=block_cache, cache_position=pos,
                                         logits_to_keep=block_size)
                        if graphs:
                            raw = graphs(("full",), full_fwd, x[:, blk], cache_pos)
                            if block_cache is not None:
                                # the replay wrote every layer's block rows (StaticBlockCache.update)
                                block_cache._num_initialized = cfg.num_hidden_layers
                        else:
                            raw = full_fwd(x[:, blk], cache_pos)
                        row_offset = s0
                    stats.forwards += 1
                    if progress is not None:
                        progress(stats)
                    if fused:
                        # logits shifted by one position (:774): position i reads raw row
                        # max(row_offset + i - 1, 0)
                        scratch = ops.unmask_step(raw, x[:, blk.start + s0:blk.start + s1], mask_id, threshold,
                                                  row_offset=row_offset, shift=1, finished=finished,
                                                  stop_token=stop_token, scratch=scratch)
                        n_unmasked, n_left, n_first, n_finished = scratch.counts.tolist()
                        if n_unmasked == 0 and n_finished < B:
                            # the rule unmasks at least one position of every unfinished row
                            # with a finite confidence: no progress means non-finite logits
                            raise RuntimeError(
                                f"sampling step {len(stats.step_tokens)} (block {block_idx}, sub-block {sb}) "
                                f"unmasked nothing with {n_left} masked positions left: non-finite logits?")
                        stats.step_tokens.append(n_unmasked)
                        left, first_masked = n_left > 0, n_first > 0
                        if n_finished == B:
                            break
                        continue
                    logits = torch.cat([raw[:, :1], raw[:, :-1]], dim=1)[:, row_offset:row_offset + small_block_size]
                    tok, conf = greedy_with_confidence(logits)
                    m = mask[:, s0:s1] & ~finished[:, None]
                    if policy is None:
                        unmask = threshold_unmask(tok, conf, m, threshold)
                    else:
                        tok, unmask = policy(len(stats.step_tokens), tok, conf, m)
                    sub = x[:, blk][:, s0:s1]
                    x[:, blk.start + s0:blk.start + s1] = torch.where(unmask, tok, sub)
                    if stop_token is not None:
                        finished |= ((tok == stop_token) & unmask).any(dim=1)
                    stats.step_tokens.append(int(unmask.sum()))
                    if bool(finished.all()):
                        break
                    mask = x[:, blk] == mask_id
                    left = bool((mask[:, s0:s1] & ~finished[:, None]).any())
                    first_masked = bool(mask[:, s0].any())
            # ---- commit (generation_functions.py:685-696). With graphs, the commit is the
            # full-block forward over the final tokens without the block cache, replayed
            # from its own graph: it writes the block's rows at kv_write_start (the
            # committed length while the block is open) and attends over the same keys
            # as the eager commit; the committed length then advances on the host.
            if graphs is not None and isinstance(cache, StaticKVCache):
                def commit_fwd(ids, pos):
                    return model(ids, cache, cache_position=pos, logits_to_keep=block_size)
                logits = graphs(("commit",), commit_fwd, x[:, blk], cache_pos)
                cache.commit_written(block_size)
            else:
                logits = model(x[:, blk], cache, update_past_key_values=True)
            stats.forwards += 1
            if progress is not None:
                progress(stats)
            stats.commits += 1
            nxt = bridge(logits[:, -1:].argmax(dim=-1))
            nxt[finished] = pad_token
            x = torch.cat([x, nxt], dim=1)
            if bool(finished.all()):
                break
        if sync_timing:
            torch.cuda.synchronize(dev)
        stats.seconds = time.perf_counter() - t0
        gen = x[:, P:P + max_new_tokens]
        stats.generated_tokens = int((gen != mask_id).sum())
        return x, stats
    finally:
        impl.unpatch(model, originals)


__all__ = ["generate", "greedy_with_confidence", "threshold_unmask", "HipStaticAttention", "ForwardGraphs",
           "GenerationStats"]
