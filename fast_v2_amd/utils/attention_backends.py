"""Drop-in for utils/attention_backends.py with a HIP (gfx950) backend.

Surface kept from the reference:
  AttentionBackend(name, impl)           names sdpa / flash2 / flash3 / flash4 / flashinfer,
                                         plus ``hip`` (this build)            (:293-682)
    .attention(q, k, v, attn_mask, scaling, is_causal, dropout)   BHSD     (:332-360)
    .flash_kvcache_attention(query, k_cache, v_cache, cache_seqlens,
                             is_causal=False, scaling=None)        BSHD     (:588-640)
    .plan_flashinfer(...), .mark_dispatch_logged()                  no-ops here
  get_attention_backend(preference="auto")   lru-cached singleton            (:685-770)
  patch_attention_layers / patch_attention_layers_compiled / unpatch_attention_layers
                                                                             (:977-1019)

The ``hip`` backend calls the block-attention kernel of libfdllm_hip.so through
the torch op ``fdllm::flash_kvcache`` (CUDA + Meta implementations, as the
reference's ``_wrap_flash_kvcache_as_custom_op`` registers, :73-120).
Selection: ``auto`` picks ``hip`` when a gfx950 device is visible; on such a
device a library that fails to load raises instead of falling back. Without a
GPU ``auto`` returns ``sdpa``, whose ``flash_kvcache_attention`` raises
``RuntimeError`` exactly as the reference's does (:637-640). The flash / FlashInfer
names need CUDA-only packages; requesting them falls back along the reference's
chain.
"""
from __future__ import annotations

import logging
from functools import lru_cache
from typing import Optional

import torch
import torch.nn.functional as F

from .. import _ffi, ops
from .static_kv_cache import StaticKVCache

logger = logging.getLogger(__name__)


def _device_arch() -> Optional[str]:
    if not torch.cuda.is_available():
        return None
    return torch.cuda.get_device_properties(torch.cuda.current_device()).gcnArchName.split(":")[0]


class AttentionBackend:
    """Unified interface for attention backends (attention_backends.py:293-682)."""

    SDPA = "sdpa"
    FLASH2 = "flash2"
    FLASH3 = "flash3"
    FLASH4 = "flash4"
    FLASHINFER = "flashinfer"
    HIP = "hip"

    def __init__(self, name: str, impl=None):
        self.name = name
        self._impl = impl
        self._kvcache_dispatch_logged = False

    def mark_dispatch_logged(self) -> None:
        self._kvcache_dispatch_logged = True

    def plan_flashinfer(self, batch_size, query_len, max_seq_len, num_qo_heads, num_kv_heads, head_dim,
                        kv_seqlens, dtype, device) -> None:
        """FlashInfer planning; nothing to plan for the other backends (:511-512)."""
        return None

    # ------------------------------------------------------------------
    def attention(self, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                  attn_mask: Optional[torch.Tensor] = None, scaling: Optional[float] = None,
                  is_causal: bool = False, dropout: float = 0.0) -> torch.Tensor:
        """BHSD attention without a cache; returns [B, H, S_q, D]."""
        if self.name == self.SDPA:
            return self._sdpa_attention(query, key, value, attn_mask, scaling, is_causal, dropout)
        if self.name == self.HIP:
            return self._hip_attention(query, key, value, attn_mask, scaling, is_causal, dropout)
        raise ValueError(f"Unknown attention backend: {self.name}")

    def _sdpa_attention(self, q, k, v, attn_mask, scaling, is_causal, dropout):
        """torch SDPA after the GQA expand (:362-383)."""
        hq, hk = q.shape[1], k.shape[1]
        if hq != hk:
            n_rep = hq // hk
            k = k[:, :, None].expand(-1, -1, n_rep, -1, -1).reshape(k.shape[0], hq, k.shape[2], k.shape[3])
            v = v[:, :, None].expand(-1, -1, n_rep, -1, -1).reshape(v.shape[0], hq, v.shape[2], v.shape[3])
        scale = scaling if scaling is not None else q.shape[-1] ** -0.5
        return F.scaled_dot_product_attention(q, k, v, attn_mask=attn_mask, dropout_p=dropout,
                                              is_causal=is_causal, scale=scale)

    def _hip_attention(self, q, k, v, attn_mask, scaling, is_causal, dropout):
        """The HIP kernel on BHSD tensors, read in place through BSHD strides.

        Masks are arithmetic only: none (every key) or causal. Causal follows the
        flash-attn convention of the reference's flash backends (:385-422): query i
        of S_q sits at key position S_kv - S_q + i (the same as SDPA's when
        S_q == S_kv). An explicit mask tensor or dropout is rejected."""
        if attn_mask is not None:
            raise RuntimeError("hip attention: explicit attn_mask tensors are not supported "
                               "(masks are computed from lengths and block indices)")
        if dropout:
            raise RuntimeError("hip attention: dropout is not supported (inference kernel)")
        B, Hq, Sq, D = q.shape
        Skv = k.shape[2]
        out = torch.empty((B, Hq, Sq, D), dtype=q.dtype, device=q.device)
        seqlens = torch.full((B,), Skv, dtype=torch.int32, device=q.device)
        ops.block_attn(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), seqlens, scaling,
                       mask_mode=_ffi.MASK_CAUSAL if is_causal else _ffi.MASK_SEQLEN,
                       out=out.transpose(1, 2))
        return out

    # ------------------------------------------------------------------
    def flash_kvcache_attention(self, query: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                                cache_seqlens: torch.Tensor, is_causal: bool = False,
                                scaling: Optional[float] = None) -> torch.Tensor:
        """Attention of BSHD queries [B, S_q, Hq, D] over the static cache buffers
        [B, max_S, Hkv, D], keys j < cache_seqlens[b] visible; returns a new
        [B, S_q, Hq, D] tensor in the query's dtype."""
        scale = scaling if scaling is not None else query.shape[-1] ** -0.5
        if not self._kvcache_dispatch_logged and not torch.compiler.is_compiling():
            logger.info("[flash_kvcache_attention] backend=%r query=%s kv_cache=%s", self.name,
                        tuple(query.shape), tuple(k_cache.shape))
            self._kvcache_dispatch_logged = True
        if self.name == self.HIP:
            return ops.flash_kvcache(query, k_cache, v_cache, cache_seqlens, float(scale), bool(is_causal))
        raise RuntimeError(
            f"flash_kvcache_attention requires the hip backend (a gfx950 GPU and libfdllm_hip.so), "
            f"but current backend is {self.name!r}.")


@lru_cache(maxsize=1)
def get_attention_backend(preference: str = "auto") -> AttentionBackend:
    """Return the attention backend (attention_backends.py:685-770).

    preference: "auto" | "hip" | "sdpa" | "flash4" | "flash3" | "flash2" | "flashinfer".
    """
    arch = _device_arch()
    if preference == "sdpa":
        return AttentionBackend(AttentionBackend.SDPA)
    if preference in ("auto", "hip"):
        if arch == "gfx950":
            _ffi.lib()  # raises RuntimeError if the library is missing: no silent fallback
            logger.info("[attention_backend] SELECTED: hip (gfx950)")
            return AttentionBackend(AttentionBackend.HIP)
        if preference == "hip":
            raise RuntimeError(f"hip attention backend needs a gfx950 GPU (found {arch or 'no GPU'})")
    if preference in ("flash4", "flash3", "flash2", "flashinfer"):
        logger.warning("%s is a CUDA-only package; not available here", preference)
        if arch == "gfx950":
            _ffi.lib()
            return AttentionBackend(AttentionBackend.HIP)
    logger.info("[attention_backend] SELECTED: sdpa (no gfx950 GPU)")
    return AttentionBackend(AttentionBackend.SDPA)


# ---------------------------------------------------------------------------
# Attention-layer patching for the static KV cache
# ---------------------------------------------------------------------------

def _apply_rotary_pos_emb(q, k, cos, sin):
    """RoPE on BSHD q/k with cos/sin [B, S, D] (attention_backends.py:777-788)."""
    cos = cos.unsqueeze(2)
    sin = sin.unsqueeze(2)
    half = q.shape[-1] // 2
    q_rot = torch.cat((-q[..., half:], q[..., :half]), dim=-1)
    k_rot = torch.cat((-k[..., half:], k[..., :half]), dim=-1)
    return q * cos + q_rot * sin, k * cos + k_rot * sin


# The patched forward uses ops.rope_kv_write where it applies (False: RoPE in torch
# and separate cache writes, the statement of the reference's code).
FUSED_ROPE_CACHE_WRITE = True
# True: with the fused RoPE + cache write, the q / k / v projections run in the same
# kernel (ops.qkv_rope_kv_write) where head_dim is 128, hidden a multiple of 64 and the
# call has at most FUSED_QKV_MAX_TOKENS token rows. Off by default: the projections are
# then three nn.Linear calls, as in the reference's code, and bit-identical to them; the
# fused kernel sums in another order, so its projections differ from a library GEMM's
# in the last bit of about 1 % of the values. On the 7B layout it takes 40 us against
# 53 us for three hipBLASLt GEMMs + the RoPE kernel at 512 rows and 29 against 53 us at
# 128 rows, but 117 against 99 us at 2048 rows, where the library GEMMs' larger tiles win.
FUSED_QKV_PROJECTION = False
FUSED_QKV_MAX_TOKENS = 1024


def _fused_rope_cache_write(rope, S, cos, layer_idx, cache, update, block_cache, replace_position):
    """RoPE + the cache writes of the patched forward in one kernel; ``rope(k_cache,
    v_cache, **destinations)`` launches it (ops.rope_kv_write on projected q / k / v, or
    ops.qkv_rope_kv_write with the projections included) and returns the rotated q.
    Returns None (nothing launched) where the call is not one of the three forms below,
    which then take the unfused path.

    * commit (update_past_key_values, no block cache): rows at the committed length;
    * diffusion step, no block cache: rows at kv_write_start (write_scratch_compiled);
    * diffusion step with the block cache: rows at block offset rp and at
      kv_write_start + rp. The unfused path copies all block rows to the static cache
      at kv_write_start after each write; every earlier write of this block already put
      the other rows there, so writing the new rows alone leaves the same cache. The
      first forward of a block (the block cache's update) must cover the whole block.
    Writes through ops.kv_cache_write and the attention are unchanged."""
    if not isinstance(cache, StaticKVCache) or cos.dim() != 3:
        return None
    kc, vc = cache.key_cache[layer_idx], cache.value_cache[layer_idx]
    if update:
        if block_cache is not None:
            return None
        start = cache.get_seq_length()
        q_rot = rope(kc, vc, write_offset=start)
        cache.note_update(S, layer_idx)
        cache.set_scratch_seqlens(start + S)
        return q_rot
    if block_cache is None:
        return rope(kc, vc, write_start=cache._write_start)
    kb, vb = block_cache[layer_idx]
    if len(block_cache) <= layer_idx:
        if S != kb.shape[1]:
            return None
        rp = 0
    else:
        rp = 0 if replace_position is None else int(replace_position)
    q_rot = rope(kc, vc, write_start=cache._write_start, write_offset=rp, k_block=kb, v_block=vb, block_offset=rp)
    if len(block_cache) <= layer_idx:
        block_cache.note_update(layer_idx)
    return q_rot


def _fusable(attn_module, hidden_states, head_dim):
    """The 16-bit shapes the fused kernels take: RoPE + cache write need head_dim a
    multiple of 16; the fused projections need head_dim 128, hidden a multiple of 64 and
    16-bit nn.Linear weights."""
    dt = hidden_states.dtype
    rope_ok = dt in (torch.bfloat16, torch.float16) and head_dim % 16 == 0
    proj_ok = (rope_ok and FUSED_QKV_PROJECTION and head_dim == 128 and hidden_states.shape[-1] % 64 == 0 and
               hidden_states[..., 0].numel() <= FUSED_QKV_MAX_TOKENS and
               all(getattr(attn_module, n).weight.dtype == dt for n in ("q_proj", "k_proj", "v_proj")))
    return rope_ok, proj_ok


def _create_patched_attention_forward(attn_module, attn_backend, static_block_cache=None):
    """Attention forward over the static cache (attention_backends.py:791-898):
    q/k/v projections -> RoPE -> sub-block cache -> KV write -> block attention
    -> o_proj. Diffusion steps write at kv_write_start without advancing the
    committed length; commit steps (update_past_key_values=True) write at the
    committed position and advance it after the last layer."""
    original_forward = attn_module.forward
    layer_idx = attn_module.layer_idx
    head_dim = attn_module.head_dim
    scaling = attn_module.scaling

    def patched_forward(hidden_states, position_embeddings, attention_mask=None, past_key_value=None,
                        cache_position=None, update_past_key_values=False, block_past_key_values=None,
                        replace_position=None, **kwargs):
        if not isinstance(past_key_value, StaticKVCache):
            return original_forward(hidden_states, position_embeddings, attention_mask, past_key_value,
                                    cache_position, update_past_key_values, block_past_key_values,
                                    replace_position, **kwargs)
        input_shape = hidden_states.shape[:-1]
        hidden_shape = (*input_shape, -1, head_dim)
        cos, sin = position_embeddings
        fused = attn_backend.name == AttentionBackend.HIP and FUSED_ROPE_CACHE_WRITE
        rope_ok, proj_ok = _fusable(attn_module, hidden_states, head_dim) if fused else (False, False)
        if proj_ok and hidden_states.dim() == 3:
            qp, kp, vp = attn_module.q_proj, attn_module.k_proj, attn_module.v_proj

            def rope(kc, vc, **dst):
                return ops.qkv_rope_kv_write(hidden_states, qp.weight, qp.bias, kp.weight, kp.bias, vp.weight,
                                             vp.bias, cos, sin, kc, vc, head_dim=head_dim, **dst)
            q = _fused_rope_cache_write(rope, hidden_states.shape[1], cos, layer_idx, past_key_value,
                                        update_past_key_values, block_past_key_values, replace_position)
            if q is not None:
                full_k, full_v = past_key_value.get_full_kv(layer_idx)
                out = attn_backend.flash_kvcache_attention(q, full_k, full_v,
                                                           cache_seqlens=past_key_value.scratch_seqlens,
                                                           is_causal=False, scaling=scaling)
                return attn_module.o_proj(out.reshape(*input_shape, -1))
        q = attn_module.q_proj(hidden_states).view(hidden_shape)
        k = attn_module.k_proj(hidden_states).view(hidden_shape)
        v = attn_module.v_proj(hidden_states).view(hidden_shape)

        if rope_ok:
            def rope(kc, vc, **dst):
                return ops.rope_kv_write(q, k, v, cos, sin, kc, vc, **dst)
            q_rot = _fused_rope_cache_write(rope, k.shape[1], cos, layer_idx, past_key_value,
                                            update_past_key_values, block_past_key_values, replace_position)
            if q_rot is not None:
                full_k, full_v = past_key_value.get_full_kv(layer_idx)
                out = attn_backend.flash_kvcache_attention(q_rot, full_k, full_v,
                                                           cache_seqlens=past_key_value.scratch_seqlens,
                                                           is_causal=False, scaling=scaling)
                return attn_module.o_proj(out.reshape(*input_shape, -1))
        q, k = _apply_rotary_pos_emb(q, k, cos, sin)

        if block_past_key_values is not None:
            if len(block_past_key_values) <= layer_idx:
                k, v = block_past_key_values.update(k, v, layer_idx)
            else:
                rp = 0 if replace_position is None else int(replace_position)
                block_past_key_values.write(k, v, layer_idx, rp)
                k, v = block_past_key_values[layer_idx]

        if update_past_key_values:
            past_len = past_key_value.get_seq_length()
            seq_len = k.shape[1]
            past_key_value.update(k, v, layer_idx)
            past_key_value.set_scratch_seqlens(past_len + seq_len)
        else:
            past_key_value.write_scratch_compiled(k, v, layer_idx)

        full_k, full_v = past_key_value.get_full_kv(layer_idx)
        out = attn_backend.flash_kvcache_attention(q, full_k, full_v, cache_seqlens=past_key_value.scratch_seqlens,
                                                   is_causal=False, scaling=scaling)
        out = out.reshape(*input_shape, -1)
        return attn_module.o_proj(out)

    return patched_forward


def _create_compiled_attention_forward(attn_module, attn_backend):
    """Branch-free diffusion-step forward (attention_backends.py:901-974): always the
    static cache, never a commit, no sub-block cache."""
    layer_idx = attn_module.layer_idx
    head_dim = attn_module.head_dim
    scaling = attn_module.scaling

    def compiled_forward(hidden_states, position_embeddings, attention_mask=None, past_key_value=None,
                         cache_position=None, update_past_key_values=False, block_past_key_values=None,
                         replace_position=None, **kwargs):
        input_shape = hidden_states.shape[:-1]
        hidden_shape = (*input_shape, -1, head_dim)
        q = attn_module.q_proj(hidden_states).view(hidden_shape)
        k = attn_module.k_proj(hidden_states).view(hidden_shape)
        v = attn_module.v_proj(hidden_states).view(hidden_shape)
        cos, sin = position_embeddings
        q, k = _apply_rotary_pos_emb(q, k, cos, sin)
        past_key_value.write_scratch_compiled(k, v, layer_idx)
        full_k, full_v = past_key_value.get_full_kv(layer_idx)
        out = attn_backend.flash_kvcache_attention(q, full_k, full_v, cache_seqlens=past_key_value.scratch_seqlens,
                                                   is_causal=False, scaling=scaling)
        return attn_module.o_proj(out.reshape(*input_shape, -1))

    return compiled_forward


def patch_attention_layers(model, attn_backend, static_block_cache=None):
    """Replace every ``layer.self_attn.forward``; returns the original forwards."""
    original = {}
    for i, layer in enumerate(model.model.layers):
        original[i] = layer.self_attn.forward
        layer.self_attn.forward = _create_patched_attention_forward(layer.self_attn, attn_backend,
                                                                    static_block_cache)
    return original


def patch_attention_layers_compiled(model, attn_backend):
    original = {}
    for i, layer in enumerate(model.model.layers):
        original[i] = layer.self_attn.forward
        layer.self_attn.forward = _create_compiled_attention_forward(layer.self_attn, attn_backend)
    return original


def unpatch_attention_layers(model, original_forwards):
    for i, layer in enumerate(model.model.layers):
        if i in original_forwards:
            layer.self_attn.forward = original_forwards[i]


__all__ = ["AttentionBackend", "get_attention_backend", "patch_attention_layers",
           "patch_attention_layers_compiled", "unpatch_attention_layers"]
