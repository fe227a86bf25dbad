"""fast_v2_amd — MI355X (gfx950) block-diffusion hot path.

HIP kernels behind a C ABI (libfdllm_hip.so, include/fdllm_hip.h) for
  * block attention over the static / paged block KV cache, and
  * fused row gather + RMSNorm (and the sibling row scatter),
with drop-in mirrors of the reference's Python surfaces:
  fast_v2_amd.utils.attention_backends   (utils/attention_backends.py)
  fast_v2_amd.utils.static_kv_cache      (utils/static_kv_cache.py)
  fast_v2_amd.utils.block_sparse_cache   (utils/block_sparse_cache.py)
  fast_v2_amd.utils.dynamic_block_kv     (utils/dynamic_block_kv.py)
  fast_v2_amd.cuda_bench.fused_sparse_extension (cuda_bench/fused_sparse_extension.py)
"""
__version__ = "0.1.0"
