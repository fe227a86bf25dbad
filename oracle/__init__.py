"""CPU oracle for the block-diffusion hot path — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this package, and only as the checker (or the timed CPU baseline). The product
(fast_v2_amd) never calls into it.

Modules
  attention       kv-cache / block-causal attention: the reference's SDPA shim
                  restated in torch, plus an independent float64 numpy brute force,
                  and the static / paged KV-cache write
  gather_rmsnorm  row gather + RMSNorm in the reference's rounding order, in torch
                  and in float64 numpy with explicit bf16/fp16 rounding; the row
                  scatter to two destinations
  e2e_eager       the reference's eager static-KV attention layer (projections,
                  RoPE, sub-block cache, static cache write, SDPA shim), plugged
                  into the generation loop for the end-to-end comparison

Pinning status (what checks each function; see tests/test_oracle_*.py):
  attention.sdpa_kvcache            pinned: fp64 brute force, committed golden
                                    vectors (torch CPU SDPA), closed forms
                                    (single key -> v, equal keys -> mean v),
                                    masked-key independence, key permutation,
                                    G=1 == per-head MHA
  attention.attention_np            pinned: same checks, plus a planted-mistake
                                    test (a wrong GQA map fails)
  attention.block_causal_mask       pinned: hand-enumerated 4x4 / 64-token cases
  attention.sdpa_block_causal       pinned: last block == kv-cache attention with
                                    L = S - 32; fp64 brute force
  attention.cache_write_np          pinned: contiguous write == slice assignment,
                                    paged write read back through the page table,
                                    out-of-range rows skipped
  gather_rmsnorm.ref_gather_input_rmsnorm
                                    pinned: exact gather vs numpy take, closed
                                    forms (zero row, constant row, unit RMS),
                                    rounding-order planted-mistake vector
  gather_rmsnorm.ref_gather_rmsnorm_fp32w / ref_gather_pair_plain
                                    pinned: agree with gather_rmsnorm_np in the
                                    fp32-weight and plain modes (<= 1 bf16 ulp)
  gather_rmsnorm.gather_rmsnorm_np  pinned: agrees with the torch restatement,
                                    closed forms
  gather_rmsnorm.scatter_rows_np    pinned: torch's scatter_ (a library routine),
                                    gather-after-scatter round trip, untouched
                                    rows unchanged, out-of-range rows skipped
  e2e_eager                         pinned through its parts: its float32
                                    attention equals attention.sdpa_kvcache (and
                                    the one-key closed form); its caches' writes
                                    equal cache_write_np; its RoPE equals the
                                    explicit pairwise rotation (identity at
                                    position 0, norms kept, relative positions).
                                    The projections are the model's own nn.Linear
                                    modules, applied in the reference's order
There are no golden vectors in the reference (its tests generate inputs from
seeds on CUDA), and no function here needed an import of the reference.
"""
