"""Qwen2.5-layout block-diffusion LM (the Fast-dLLM v2 7B architecture) for the
end-to-end generation workload, with random weights (no checkpoint is available).

Layout follows the reference model (models/.../modeling.py): RMSNorm with the
Fast_dLLM_QwenRMSNorm rounding order (:427-432), q/k/v projections with bias and
o_proj without (:314-325), SiLU-gated MLP (:153-166), RoPE with theta 1e6
computed in fp32 and cast to the activation dtype (:544-556), weights initialised
as in _init_weights (:511-522): Linear / Embedding ~ N(0, 0.02), biases 0, norm
weights 1.

The attention modules carry the attributes the layer patching of
utils/attention_backends.py reads (layer_idx, head_dim, scaling, q/k/v/o_proj);
their own forward refuses to run, so the model is used with
``patch_attention_layers`` as batch_sample_dynamo does
(generation_functions.py:382-385).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch
import torch.nn as nn
import torch.nn.functional as F


@dataclass
class BlockDiffusionConfig:
    vocab_size: int = 152064
    hidden_size: int = 3584
    intermediate_size: int = 18944
    num_hidden_layers: int = 28
    num_attention_heads: int = 28
    num_key_value_heads: int = 4
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1_000_000.0
    initializer_range: float = 0.02
    bd_size: int = 32
    # the diffusion mask token (the last vocabulary id in the end-to-end workload)
    mask_token_id: int = 152063

    @property
    def head_dim(self) -> int:
        return self.hidden_size // self.num_attention_heads


_IDENTITY_ROWS: dict = {}


def _identity_rows(n: int, device) -> torch.Tensor:
    """int64 [1, n] = 0 .. n-1, cached per (n, device) (the gather index of a plain norm)."""
    key = (n, str(device))
    t = _IDENTITY_ROWS.get(key)
    if t is None:
        t = torch.arange(n, dtype=torch.int64, device=device)[None]
        _IDENTITY_ROWS[key] = t
    return t


class RMSNorm(nn.Module):
    """w * (x.f32 * rsqrt(mean(x.f32^2) + eps)).to(dtype) (modeling.py:427-432).

    With ``fused`` set (the HIP implementation sets it while the model is patched),
    the norm runs as one gather + RMSNorm kernel over all rows in the same rounding
    order (the model-path mode of fused_sparse_extension.py:51-87), instead of the
    eight elementwise and reduction kernels of the torch statement."""

    def __init__(self, hidden_size: int, eps: float):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(hidden_size))
        self.variance_epsilon = eps
        self.fused = False

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.fused:
            from .. import _ffi, ops
            shape = x.shape
            rows = x.reshape(1, -1, shape[-1])
            normed, _ = ops.gather_rmsnorm(rows, _identity_rows(rows.shape[1], x.device), self.weight,
                                           self.variance_epsilon, _ffi.NORM_WEIGHT_AFTER_CAST, with_gathered=False)
            return normed.view(shape)
        dt = x.dtype
        h = x.float()
        h = h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + self.variance_epsilon)
        return self.weight * h.to(dt)

    def add_norm(self, h: torch.Tensor, a: torch.Tensor):
        """(h + a, norm(h + a)): the residual add that precedes the norm in the decoder
        layer (modeling.py:475-484). Fused, one kernel reads h and a once and writes the
        rounded sum and its norm; the sum is the 16-bit add's, bit for bit, and the norm
        that of ``forward`` on it."""
        if self.fused:
            from .. import _ffi, ops
            return ops.add_rmsnorm(h, a, self.weight, self.variance_epsilon, _ffi.NORM_WEIGHT_AFTER_CAST)
        s = h + a
        return s, self(s)


def set_fused_norms(model: nn.Module, on: bool) -> None:
    """Switch every RMSNorm of ``model`` to the fused kernels, and the MLPs' SiLU-gated
    product to its kernel (or both back to torch)."""
    for mod in model.modules():
        if isinstance(mod, RMSNorm):
            mod.fused = on
        elif isinstance(mod, MLP):
            mod.fused = on


class Attention(nn.Module):
    def __init__(self, cfg: BlockDiffusionConfig, layer_idx: int):
        super().__init__()
        self.layer_idx = layer_idx
        self.head_dim = cfg.head_dim
        self.scaling = self.head_dim ** -0.5
        self.q_proj = nn.Linear(cfg.hidden_size, cfg.num_attention_heads * self.head_dim, bias=True)
        self.k_proj = nn.Linear(cfg.hidden_size, cfg.num_key_value_heads * self.head_dim, bias=True)
        self.v_proj = nn.Linear(cfg.hidden_size, cfg.num_key_value_heads * self.head_dim, bias=True)
        self.o_proj = nn.Linear(cfg.num_attention_heads * self.head_dim, cfg.hidden_size, bias=False)

    def forward(self, *args, **kwargs):
        raise RuntimeError("attention layers run through patch_attention_layers "
                           "(fast_v2_amd.utils.attention_backends)")


class MLP(nn.Module):
    def __init__(self, cfg: BlockDiffusionConfig):
        super().__init__()
        self.gate_proj = nn.Linear(cfg.hidden_size, cfg.intermediate_size, bias=False)
        self.up_proj = nn.Linear(cfg.hidden_size, cfg.intermediate_size, bias=False)
        self.down_proj = nn.Linear(cfg.intermediate_size, cfg.hidden_size, bias=False)
        self.fused = False

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.fused:
            from .. import ops
            return self.down_proj(ops.silu_mul(self.gate_proj(x), self.up_proj(x)))
        return self.down_proj(F.silu(self.gate_proj(x)) * self.up_proj(x))


class DecoderLayer(nn.Module):
    def __init__(self, cfg: BlockDiffusionConfig, layer_idx: int):
        super().__init__()
        self.self_attn = Attention(cfg, layer_idx)
        self.mlp = MLP(cfg)
        self.input_layernorm = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps)
        self.post_attention_layernorm = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps)

    def forward(self, h, position_embeddings, past_key_value, update_past_key_values, block_past_key_values,
                replace_position, pending: Optional[torch.Tensor] = None):
        """Returns (h, m) with the layer's output h + m (modeling.py:465-488). The MLP's
        residual add is left to the caller so that it runs together with the next norm
        (the next layer's input norm, or the final norm); ``pending`` is the previous
        layer's m, added to h before this layer's input norm. The sums are the same 16-bit
        adds as ``h = residual + h`` in the reference layer, in the same order."""
        if pending is None:
            x = self.input_layernorm(h)
        else:
            h, x = self.input_layernorm.add_norm(h, pending)
        a = self.self_attn(x, position_embeddings, None, past_key_value, None,
                           update_past_key_values, block_past_key_values, replace_position)
        h, x = self.post_attention_layernorm.add_norm(h, a)
        return h, self.mlp(x)


class Backbone(nn.Module):
    def __init__(self, cfg: BlockDiffusionConfig):
        super().__init__()
        self.embed_tokens = nn.Embedding(cfg.vocab_size, cfg.hidden_size)
        self.layers = nn.ModuleList(DecoderLayer(cfg, i) for i in range(cfg.num_hidden_layers))
        self.norm = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps)
        d = cfg.head_dim
        self.register_buffer("inv_freq", 1.0 / (cfg.rope_theta ** (torch.arange(0, d, 2, dtype=torch.float32) / d)),
                             persistent=False)

    def rotary(self, positions: torch.Tensor, dtype: torch.dtype):
        """cos / sin [1, S, D] for absolute positions [S] (fp32, then cast)."""
        freqs = positions.float()[:, None] * self.inv_freq.float()[None, :]
        emb = torch.cat((freqs, freqs), dim=-1)
        return emb.cos().to(dtype)[None], emb.sin().to(dtype)[None]


class BlockDiffusionLM(nn.Module):
    """Embedding -> decoder layers -> norm -> lm_head, over a static KV cache."""

    def __init__(self, cfg: BlockDiffusionConfig):
        super().__init__()
        self.config = cfg
        self.model = Backbone(cfg)
        self.lm_head = nn.Linear(cfg.hidden_size, cfg.vocab_size, bias=False)

    @torch.no_grad()
    def init_weights(self, seed: int = 0) -> None:
        """_init_weights (modeling.py:511-522), drawn on the module's device."""
        dev = self.lm_head.weight.device
        gen = torch.Generator(device=dev).manual_seed(seed)
        std = self.config.initializer_range
        for mod in self.modules():
            if isinstance(mod, nn.Linear):
                mod.weight.normal_(0.0, std, generator=gen)
                if mod.bias is not None:
                    mod.bias.zero_()
            elif isinstance(mod, nn.Embedding):
                mod.weight.normal_(0.0, std, generator=gen)
            elif isinstance(mod, RMSNorm):
                mod.weight.fill_(1.0)
        # A trained model never predicts its mask token. A random one can, and then the
        # unmask rule writes the mask token back (generation_functions.py:789-799): the
        # position stays masked and the block never completes. Its output row is zero, so
        # its logit is 0 and never the argmax of ~N(0, 1) logits over the vocabulary.
        mid = self.config.mask_token_id
        if 0 <= mid < self.config.vocab_size:
            self.lm_head.weight[mid].zero_()

    @torch.no_grad()
    def forward(self, input_ids: torch.Tensor, past_key_values, update_past_key_values: bool = False,
                use_block_cache: bool = False, block_past_key_values=None, replace_position: Optional[int] = None,
                cache_position: Optional[torch.Tensor] = None, logits_to_keep: int = 0) -> torch.Tensor:
        """Logits [B, logits_to_keep or S, vocab] for ``input_ids`` [B, S].

        Positions (forward_dynamo, modeling.py:715-733): ``cache_position`` if given,
        else the committed length (plus ``replace_position`` for a sub-block step)
        onwards."""
        h = self.model.embed_tokens(input_ids)
        S = input_ids.shape[1]
        if cache_position is None:
            start = past_key_values.get_seq_length()
            if use_block_cache and replace_position is not None:
                start += int(replace_position)
            cache_position = torch.arange(start, start + S, device=input_ids.device)
        pe = self.model.rotary(cache_position, h.dtype)
        bpkv = block_past_key_values if use_block_cache else None
        m = None
        for layer in self.model.layers:
            h, m = layer(h, pe, past_key_values, update_past_key_values, bpkv, replace_position, m)
        h = self.model.norm(h) if m is None else self.model.norm.add_norm(h, m)[1]
        if logits_to_keep:
            h = h[:, -logits_to_keep:]
        return self.lm_head(h)


def build_model(cfg: BlockDiffusionConfig, device, dtype=torch.bfloat16, seed: int = 0) -> BlockDiffusionLM:
    """Allocate the model directly on ``device`` in ``dtype`` (no host copy, no default
    initialisation pass) and initialise it with ``init_weights``."""
    old = torch.get_default_dtype()
    torch.set_default_dtype(dtype)
    try:
        with torch.device("meta"):
            model = BlockDiffusionLM(cfg)
    finally:
        torch.set_default_dtype(old)
    model = model.to_empty(device=device)
    d = cfg.head_dim
    model.model.inv_freq = 1.0 / (cfg.rope_theta ** (torch.arange(0, d, 2, dtype=torch.float32, device=device) / d))
    model.init_weights(seed)
    model.eval()
    return model


def param_count(cfg: BlockDiffusionConfig) -> int:
    h, i, v, L = cfg.hidden_size, cfg.intermediate_size, cfg.vocab_size, cfg.num_hidden_layers
    kv = cfg.num_key_value_heads * cfg.head_dim
    per_layer = h * h + h + 2 * (h * kv + kv) + h * h + 3 * h * i + 2 * h
    return v * h * 2 + L * per_layer + h


__all__ = ["BlockDiffusionConfig", "BlockDiffusionLM", "build_model", "param_count", "RMSNorm", "set_fused_norms"]
