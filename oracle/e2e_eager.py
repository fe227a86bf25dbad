"""Eager torch attention + KV caches for the end-to-end generation check — TEST
INFRASTRUCTURE ONLY (imported by tests/, never by the product).

Restates, with plain torch indexing and the SDPA shim of tests/test_focus.py:205-228
(``oracle.attention.sdpa_kvcache``), what the static-KV path of the reference does
per attention layer (utils/attention_backends.py:814-898):
  q/k/v projections -> RoPE (rotate_half form, modeling.py:168-200) ->
  sub-block cache (rows [rp, rp + S) of a [B, 32, Hkv, D] buffer, :847-866) ->
  static cache write (commit: at the committed length, pointer advanced after the
  last layer, static_kv_cache.py:132-160; diffusion step: at kv_write_start,
  :218-229) -> attention over the full buffer with keys j < scratch_seqlens[b]
  -> o_proj.
``EagerStaticAttention`` plugs into fast_v2_amd.e2e.sampler.generate in place of
the HIP implementation, so both runs share the sampler and the model weights and
differ only in attention and KV caching.
"""
from __future__ import annotations

import torch

from .attention import sdpa_kvcache


class TorchKVCache:
    def __init__(self, batch, max_seq_len, num_layers, num_kv_heads, head_dim, dtype, device):
        self.num_layers = num_layers
        self.max_seq_len = max_seq_len
        shape = (batch, max_seq_len, num_kv_heads, head_dim)
        self.key_cache = [torch.zeros(shape, dtype=dtype, device=device) for _ in range(num_layers)]
        self.value_cache = [torch.zeros(shape, dtype=dtype, device=device) for _ in range(num_layers)]
        self._seq_len = 0
        self.scratch_seqlens = torch.zeros(batch, dtype=torch.int32, device=device)
        self.write_start = 0

    def get_seq_length(self, layer_idx: int = 0) -> int:
        return self._seq_len

    def __len__(self):
        return self.num_layers if self._seq_len > 0 else 0

    def update(self, k, v, layer_idx):
        n = k.shape[1]
        self.key_cache[layer_idx][:, self._seq_len:self._seq_len + n] = k
        self.value_cache[layer_idx][:, self._seq_len:self._seq_len + n] = v
        if layer_idx == self.num_layers - 1:
            self._seq_len += n

    def write_scratch_compiled(self, k, v, layer_idx):
        n = k.shape[1]
        self.key_cache[layer_idx][:, self.write_start:self.write_start + n] = k
        self.value_cache[layer_idx][:, self.write_start:self.write_start + n] = v

    def get_full_kv(self, layer_idx):
        return self.key_cache[layer_idx], self.value_cache[layer_idx]

    def set_scratch_seqlens(self, n):
        self.scratch_seqlens.fill_(n)

    def set_kv_write_start(self, n):
        self.write_start = int(n)

    def prepare_write_idx(self, n):
        pass


class TorchBlockCache:
    def __init__(self, batch, block_size, num_layers, num_kv_heads, head_dim, dtype, device):
        shape = (batch, block_size, num_kv_heads, head_dim)
        self.key_cache = [torch.zeros(shape, dtype=dtype, device=device) for _ in range(num_layers)]
        self.value_cache = [torch.zeros(shape, dtype=dtype, device=device) for _ in range(num_layers)]
        self.block_size = block_size
        self._n = 0

    def __len__(self):
        return self._n

    def __getitem__(self, layer_idx):
        return self.key_cache[layer_idx], self.value_cache[layer_idx]

    def update(self, k, v, layer_idx):
        self.write(k, v, layer_idx, 0)
        self._n = max(self._n, layer_idx + 1)
        return self[layer_idx]

    def write(self, k, v, layer_idx, offset):
        n = k.shape[1]
        self.key_cache[layer_idx][:, offset:offset + n] = k
        self.value_cache[layer_idx][:, offset:offset + n] = v

    def reset(self):
        self._n = 0


def _rotate_half(x):
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


def kvcache_attention_f32(q, k_cache, v_cache, seqlens, scale, p_bf16: bool):
    """softmax(q k^T * scale + M) v in float32 over keys j < seqlens[b] (GQA h -> h // G).

    p_bf16=True rounds the unnormalised probabilities exp(s - max) to bf16 before the
    PV product while the row sums stay in fp32 — the rounding points of a flash-style
    kernel with bf16 P operands (the HIP kernel, and flash-attn's kv-cache kernel)."""
    B, Sq, H, D = q.shape
    Hkv = k_cache.shape[2]
    qh = q.float().transpose(1, 2)                                       # [B, H, Sq, D]
    kh = k_cache.float().transpose(1, 2).repeat_interleave(H // Hkv, dim=1).contiguous()
    vh = v_cache.float().transpose(1, 2).repeat_interleave(H // Hkv, dim=1).contiguous()
    s = torch.matmul(qh, kh.transpose(-1, -2).contiguous()) * scale   # [B, H, Sq, S]
    valid = torch.arange(k_cache.shape[1], device=q.device)[None, :] < seqlens.long()[:, None]
    s = s.masked_fill(~valid[:, None, None, :], float("-inf"))
    p = torch.exp(s - s.amax(-1, keepdim=True))
    l = p.sum(-1, keepdim=True)
    if p_bf16:
        p = p.to(torch.bfloat16).float()
    return (torch.matmul(p, vh) / l).transpose(1, 2)                     # [B, Sq, H, D]


def eager_attention_forward(attn_module, p_bf16: bool = False):
    layer_idx = attn_module.layer_idx
    head_dim = attn_module.head_dim
    scaling = attn_module.scaling

    def forward(hidden_states, position_embeddings, attention_mask=None, past_key_value=None, cache_position=None,
                update_past_key_values=False, block_past_key_values=None, replace_position=None, **kw):
        shape = (*hidden_states.shape[:-1], -1, head_dim)
        q = attn_module.q_proj(hidden_states).view(shape)
        k = attn_module.k_proj(hidden_states).view(shape)
        v = attn_module.v_proj(hidden_states).view(shape)
        cos, sin = position_embeddings
        cos, sin = cos.unsqueeze(2), sin.unsqueeze(2)
        q = q * cos + _rotate_half(q) * sin
        k = k * cos + _rotate_half(k) * sin
        if block_past_key_values is not None:
            if len(block_past_key_values) <= layer_idx:
                k, v = block_past_key_values.update(k, v, layer_idx)
            else:
                rp = 0 if replace_position is None else int(replace_position)
                block_past_key_values.write(k, v, layer_idx, rp)
                k, v = block_past_key_values[layer_idx]
        if update_past_key_values:
            past = past_key_value.get_seq_length()
            past_key_value.update(k, v, layer_idx)
            past_key_value.set_scratch_seqlens(past + k.shape[1])
        else:
            past_key_value.write_scratch_compiled(k, v, layer_idx)
        kc, vc = past_key_value.get_full_kv(layer_idx)
        # float32 products: the reference attention is never run as a bf16 batched product here
        if p_bf16:
            out = kvcache_attention_f32(q, kc, vc, past_key_value.scratch_seqlens, scaling, True)
        else:
            out = sdpa_kvcache(q.float(), kc.float(), vc.float(), past_key_value.scratch_seqlens, scaling=scaling)
        return attn_module.o_proj(out.to(q.dtype).reshape(*hidden_states.shape[:-1], -1))

    return forward


class EagerStaticAttention:
    """p_bf16=False: the SDPA shim in float32 (exact softmax); True: the same product with
    the probabilities rounded to bf16 before PV (flash-style rounding points)."""

    name = "eager-torch"

    def __init__(self, p_bf16: bool = False):
        self.p_bf16 = p_bf16

    def make_caches(self, batch, max_seq_len, cfg, dtype, device, use_block_cache):
        cache = TorchKVCache(batch, max_seq_len, cfg.num_hidden_layers, cfg.num_key_value_heads, cfg.head_dim,
                             dtype, device)
        block = (TorchBlockCache(batch, cfg.bd_size, cfg.num_hidden_layers, cfg.num_key_value_heads, cfg.head_dim,
                                 dtype, device) if use_block_cache else None)
        return cache, block

    def patch(self, model, block_cache):
        originals = {}
        for i, layer in enumerate(model.model.layers):
            originals[i] = layer.self_attn.forward
            layer.self_attn.forward = eager_attention_forward(layer.self_attn, self.p_bf16)
        return originals

    def unpatch(self, model, originals):
        for i, layer in enumerate(model.model.layers):
            if i in originals:
                layer.self_attn.forward = originals[i]
