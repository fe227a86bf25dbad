"""Drop-in mirrors of the reference's utils/ surfaces on the HIP kernels:
attention_backends, static_kv_cache, block_sparse_cache, dynamic_block_kv."""
from .attention_backends import (AttentionBackend, get_attention_backend, patch_attention_layers,
                                 patch_attention_layers_compiled, unpatch_attention_layers)
from .block_sparse_cache import BlockSparseCache
from .dynamic_block_kv import DynamicBlockKV
from .static_kv_cache import StaticBlockCache, StaticKVCache

__all__ = ["AttentionBackend", "get_attention_backend", "patch_attention_layers",
           "patch_attention_layers_compiled", "unpatch_attention_layers", "StaticKVCache",
           "StaticBlockCache", "BlockSparseCache", "DynamicBlockKV"]
