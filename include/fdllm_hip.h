/*
 * libfdllm_hip.so — C ABI of the MI355X (gfx950) block-diffusion hot path.
 *
 * Two operator families, each a drop-in for one surface of navneet-13/fast_v2:
 *
 *   1. Row gather + RMSNorm (and the sibling row scatter), replacing the
 *      pybind entry points of cuda_bench/fused_gather_norm.cu:215-221.
 *   2. Block attention over the static / paged block KV cache, replacing the
 *      flash_attn_with_kvcache call behind
 *      AttentionBackend.flash_kvcache_attention (utils/attention_backends.py:588-640)
 *      and the eager block-causal SDPA of the prefill/commit forward
 *      (modeling.py:385-411 with eval_block_diff_mask, modeling.py:145-150).
 *
 * Conventions shared by every entry point:
 *   - Plain device pointers, element strides and sizes; no framework types.
 *   - `stream` is a hipStream_t passed as void* (NULL = the null stream).
 *     Every launch is asynchronous on that stream; no entry point synchronises
 *     the host or allocates device memory.
 *   - Return value: FDLLM_OK (0) on success, a negative FDLLM_ERR_* for a
 *     rejected argument (nothing was launched), or a positive hipError_t when
 *     the launch itself failed. fdllm_last_error() describes the last failure
 *     of the calling thread.
 *   - The last dimension of every tensor is contiguous (stride 1).
 */
#ifndef FDLLM_HIP_H_
#define FDLLM_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------- */
#define FDLLM_OK 0
#define FDLLM_ERR_INVALID_ARGUMENT (-1)
#define FDLLM_ERR_UNSUPPORTED (-2)
#define FDLLM_ERR_WORKSPACE (-3)

/* ---- element types ------------------------------------------------------ */
#define FDLLM_DTYPE_F32 0
#define FDLLM_DTYPE_BF16 1
#define FDLLM_DTYPE_F16 2

/* ---- how the RMSNorm weight is applied ---------------------------------- */
/* out = x * rsqrt(mean(x^2) + eps)               (fused_gather_norm.cu:166-174, weight == nullptr) */
#define FDLLM_NORM_PLAIN 0
/* out = (x * rsqrt(mean(x^2) + eps)) * w, in fp32, one rounding  (fused_gather_norm.cu:53-57) */
#define FDLLM_NORM_WEIGHT_FP32 1
/* out = w * to_dtype(x * rsqrt(mean(x^2) + eps)), the Fast_dLLM_QwenRMSNorm
 * order (modeling.py:427-432; fused_sparse_extension.py:80-87)                    */
#define FDLLM_NORM_WEIGHT_AFTER_CAST 2

/* ---- attention masks ---------------------------------------------------- */
/* key j visible iff j < seqlens[b]  (flash_attn_with_kvcache, causal=False;
 * the seqused mask of static_kv_cache.py:295-302)                               */
#define FDLLM_MASK_SEQLEN 0
/* key j visible iff j < seqlens[b] and j <= qpos(i)  (causal, query i at
 * absolute position qpos(i) = q_start[b] + i)                                    */
#define FDLLM_MASK_CAUSAL 1
/* key j visible iff j < seqlens[b] and j / mask_block <= qpos(i) / mask_block
 * (eval_block_diff_mask, modeling.py:145-150)                                    */
#define FDLLM_MASK_BLOCK_CAUSAL 2

/* Library identification: returns FDLLM_ABI_VERSION. */
#define FDLLM_ABI_VERSION 2
int fdllm_abi_version(void);

/* Human-readable description of the calling thread's last failure ("" if none). */
const char* fdllm_last_error(void);

/* -------------------------------------------------------------------------
 * Row gather + RMSNorm.
 *
 *   for b < batch, t < num_tokens:
 *     s = indices[b * indices_batch_stride + t]
 *     x = hidden[b * hidden_batch_stride + s * hidden_row_stride + 0 .. hidden_size)
 *     gathered[b, t, :] = x                                  (bit-exact; optional)
 *     normed[b, t, :]   = rmsnorm(x) per norm_mode, fp32 arithmetic
 *
 * hidden / normed / gathered share `dtype`; weight has `weight_dtype` and may be
 * NULL only with FDLLM_NORM_PLAIN. normed and gathered are contiguous
 * [batch, num_tokens, hidden_size]. An index outside [0, seq_len) yields a zero
 * row in both outputs (the input is never read out of bounds).
 *
 * Replaces: gather_rmsnorm_cuda (fused_gather_norm.cu:60-73, NORM_WEIGHT_FP32),
 * fused_select_norm (:177-190, NORM_WEIGHT_FP32),
 * fused_gather_input_rmsnorm_pair (:193-209, NORM_PLAIN + gathered), and the
 * model-path wrapper fused_sparse_extension.fused_gather_input_rmsnorm_pair
 * (fused_sparse_extension.py:51-87, NORM_WEIGHT_AFTER_CAST + gathered).
 * ------------------------------------------------------------------------- */
int fdllm_gather_rmsnorm(const void* hidden, int64_t hidden_batch_stride, int64_t hidden_row_stride,
                         const int64_t* indices, int64_t indices_batch_stride,
                         const void* weight, int weight_dtype,
                         void* normed, void* gathered,
                         int batch, int seq_len, int num_tokens, int hidden_size,
                         float eps, int dtype, int norm_mode, void* stream);

/* -------------------------------------------------------------------------
 * Row scatter to two destinations.
 *
 *   for b < batch, t < num_tokens:
 *     s = indices[b * indices_batch_stride + t]
 *     cache[b, s, :] = current[b, s, :] = values[b, t, :]
 *
 * values is contiguous [batch, num_tokens, hidden_size]; cache and current are
 * [batch, seq_len, hidden_size] with the given strides. current may be NULL
 * (one destination: BlockSparseCache.scatter_attn_output / scatter_mlp_output,
 * utils/block_sparse_cache.py:112-132). Out-of-range indices are skipped.
 * Duplicate indices within a row race, as in the reference: each element of such a
 * destination row ends with that element of one of the rows aimed at it; which one
 * is unspecified and may differ between the two destinations.
 *
 * Replaces: scatter_and_return_cuda (fused_gather_norm.cu:79-119).
 * ------------------------------------------------------------------------- */
int fdllm_scatter_rows(const void* values, const int64_t* indices, int64_t indices_batch_stride,
                       void* cache, int64_t cache_batch_stride, int64_t cache_row_stride,
                       void* current, int64_t current_batch_stride, int64_t current_row_stride,
                       int batch, int seq_len, int num_tokens, int hidden_size,
                       int dtype, void* stream);

/* -------------------------------------------------------------------------
 * Residual add + RMSNorm of contiguous rows (the decoder layer around the path):
 *
 *   sum[r, :]    = to_dtype(x[r, :] + residual[r, :])
 *   normed[r, :] = the norm of sum[r, :] in `norm_mode` (as fdllm_gather_rmsnorm)
 *
 * x, residual, sum_out, normed: [rows, hidden_size] in `dtype` (bf16 or fp16),
 * contiguous and 16-byte aligned; hidden_size a multiple of 8, at most 4096; the
 * weight in fp32 or `dtype`.
 *
 * Replaces: hidden_states = residual + hidden_states followed by the next RMSNorm
 * (modeling.py:465-488, 427-432 of the Fast_dLLM_v2_7B snapshot).
 * ------------------------------------------------------------------------- */
int fdllm_add_rmsnorm(const void* x, const void* residual, const void* weight, int weight_dtype,
                      void* sum_out, void* normed, int rows, int hidden_size, float eps, int dtype,
                      int norm_mode, void* stream);

/* -------------------------------------------------------------------------
 * SiLU-gated product of the MLP:
 *
 *   out[i] = to_dtype(to_dtype(silu(gate[i])) * up[i]),  silu(g) = g / (1 + exp(-g)) in fp32
 *
 * gate, up, out: n elements of `dtype` (bf16 or fp16), n a multiple of 8, 16-byte aligned.
 *
 * Replaces: act_fn(gate_proj(x)) * up_proj(x) (modeling.py:164 of the snapshot).
 * ------------------------------------------------------------------------- */
int fdllm_silu_mul(const void* gate, const void* up, void* out, int64_t n, int dtype, void* stream);

/* -------------------------------------------------------------------------
 * Block attention over a (paged) KV cache.
 *
 * Query row (b, i, h) attends to the keys j of sequence b that the mask allows,
 * using KV head h / (num_q_heads / num_kv_heads) (GQA), with
 *   out = softmax(q . k^T * softmax_scale) . v      (fp32 softmax and accumulation)
 * A row with no visible key produces zeros.
 *
 * KV addressing: element (j, kv_head, d) of sequence b lives at
 *   base + page * stride_page + slot * stride_slot + kv_head * stride_head + d
 * with (page, slot) = (page_table[b * max_pages + j / page_size], j % page_size)
 * when page_table != NULL, else (b, j): the contiguous [batch, max_S, Hkv, D]
 * static cache of static_kv_cache.py:55-69 is the page-table-free case.
 * page_size must be a power of two, at least 16 for head_dim 128 and at least
 * 32 for head_dim 64.
 * ------------------------------------------------------------------------- */
typedef struct fdllm_kv_attn_desc {
  const void* q; /* [batch, q_len, num_q_heads, head_dim] */
  int64_t q_stride_b, q_stride_s, q_stride_h;
  const void* k; /* key pool */
  int64_t k_stride_page, k_stride_slot, k_stride_h;
  const void* v; /* value pool */
  int64_t v_stride_page, v_stride_slot, v_stride_h;
  void* out; /* [batch, q_len, num_q_heads, head_dim] */
  int64_t out_stride_b, out_stride_s, out_stride_h;
  const int32_t* page_table; /* [batch, max_pages] or NULL */
  const int32_t* seqlens;    /* [batch] visible KV length */
  const int32_t* q_start;    /* [batch] absolute position of query 0, or NULL: seqlens[b] - q_len */
  int32_t max_pages;         /* page-table row length (ignored without a page table) */
  int32_t page_size;         /* tokens per page (ignored without a page table) */
  int32_t max_seqlen;        /* upper bound on every seqlens[b]; sizes the grid */
  int32_t batch, q_len, num_q_heads, num_kv_heads, head_dim;
  int32_t mask_mode;  /* FDLLM_MASK_* */
  int32_t mask_block; /* block length for FDLLM_MASK_BLOCK_CAUSAL */
  int32_t dtype;      /* FDLLM_DTYPE_BF16 or FDLLM_DTYPE_F16 (q, k, v, out); FDLLM_DTYPE_F32 runs a
                         general fp32 kernel (k_new / v_new not accepted; a workspace, as
                         fdllm_kv_attn_workspace_size reports, when it splits the keys) */
  int32_t kv_split;   /* keys per split-KV work item (multiple of 64), 0 = automatic */
  float softmax_scale;
  int32_t flags;      /* FDLLM_ATTN_* bits, 0 = defaults */
  /* Optional cache write fused into the call (both NULL: none). k_new / v_new hold
   * the key / value rows of the q_len query tokens, [batch, q_len, num_kv_heads,
   * head_dim] with the strides below; row t of sequence b is stored into the cache
   * (k / v, addressed as above) at position q_start[b] + t (seqlens[b] - q_len + t
   * without q_start) before any key is read, positions outside [0, capacity) being
   * skipped (capacity = max_pages * page_size with a page table, else max_seqlen).
   * Replaces StaticKVCache.update (static_kv_cache.py:132-160) followed by the
   * attention of the prefill / commit forward (modeling.py:385-411): without q_start
   * the prefill kernels read these rows from k_new / v_new and store them from
   * registers as they stage them, so the write costs no second read; other shapes,
   * and every call with an explicit q_start (whose visible keys may run past the last
   * new row), launch the cache write kernel before the attention. */
  const void* k_new;
  const void* v_new;
  int64_t new_stride_b, new_stride_s, new_stride_h;
} fdllm_kv_attn_desc;

/* Use the general kernel (one KV head per workgroup) even where the decode
 * kernel (all KV heads of a key range per workgroup) applies. */
#define FDLLM_ATTN_NO_DECODE_KERNEL 1
/* Decode shapes: use the all-KV-heads-per-workgroup kernel instead of the
 * split-KV kernel with one KV head per workgroup. */
#define FDLLM_ATTN_ALL_HEADS_DECODE 2
/* With k_new / v_new: store the new rows into the cache by a copy kernel launched
 * before the attention, also for prefill shapes, whose kernels otherwise store them
 * themselves (each row by the one workgroup that owns it). Same results, bit for bit;
 * the in-kernel write is the default (the 4 x 4096-token prefill: 473-475 us against
 * 479-480 us with the copy kernel, timed in rotation). */
#define FDLLM_ATTN_CACHE_WRITE_KERNEL 4
/* Sub-block decode shapes (at most 64 sequences, a page table of at most 4096 entries or
 * none): deal the keys of all sequences evenly over the workgroups, in runs of 128-key
 * quads that cross from one sequence into the next, instead of splitting each sequence's
 * keys on its own. Results agree within rounding (the splits differ). Off by default: on
 * the 16-sequence 7B step it measured slower (a workgroup whose run crosses a sequence
 * boundary loses about one quad's time). */
#define FDLLM_ATTN_BALANCED_SPLITS 8

/* Bytes of device workspace fdllm_kv_attn_fwd needs for `desc` (0 when the call
 * is not split over several workgroups per KV head). The workspace starts with
 * 64 KiB of arrival counters (one int per (sequence, KV head)), followed by the
 * per-split partial results (running max, sum and unnormalised output rows). The
 * split-KV decode kernel (the default for at most 64 query rows per KV head)
 * merges them in the last workgroup of a (sequence, KV head) to finish; the other
 * kernels leave them to a second kernel on the same stream. The workspace must be
 * zero-filled once when it is
 * allocated: every call leaves the counters at zero again and writes every
 * partial it reads, so one workspace then serves any sequence of calls of any
 * sizes. Calls that may overlap in time (different streams) need separate
 * workspaces. */
int fdllm_kv_attn_workspace_size(const fdllm_kv_attn_desc* desc, size_t* bytes);

/* Launch the attention described by `desc` on `stream`. */
int fdllm_kv_attn_fwd(const fdllm_kv_attn_desc* desc, void* workspace, size_t workspace_bytes,
                      void* stream);

/* Bytes of the library's own attention scratch on each device (48 MiB). */
#define FDLLM_KV_ATTN_SCRATCH_BYTES (48u * 1024u * 1024u)

/* fdllm_kv_attn_fwd without a workspace argument and without any allocation: the
 * split partials and arrival counters live in a device array of
 * FDLLM_KV_ATTN_SCRATCH_BYTES that the library holds on every device it runs on
 * until the process ends. Same kernels, same results as fdllm_kv_attn_fwd.
 *
 * No counterpart in the reference: it is for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). It calls no hipMalloc / hipFree.
 *   - A call whose fdllm_kv_attn_workspace_size exceeds FDLLM_KV_ATTN_SCRATCH_BYTES
 *     is rejected with FDLLM_ERR_WORKSPACE (nothing launched). At head_dim 128 with
 *     the automatic split (kv_split 0), in the default build, the scratch holds any sub-block decode
 *     (<= 64 query rows per KV head) of up to 64 sequences of at most 5120 keys
 *     with <= 8 KV heads, and any full-block decode (<= 256 rows per KV head) of up
 *     to 64 sequences of at most 10240 keys with <= 4 KV heads; calls that need no
 *     workspace (prefill) always fit.
 *   - The first call on a device resolves the scratch, clears its counters on
 *     `stream` and waits for that clear (so later calls from any stream or thread
 *     start after it); it must not be made under stream capture
 *     (FDLLM_ERR_UNSUPPORTED).
 *   - Every call on one device shares that device's scratch, and each call leaves
 *     its counters at zero: calls on one stream run in order, but calls that overlap
 *     in time on one device (other streams, other threads) race. */
int fdllm_kv_attn_fwd_noalloc(const fdllm_kv_attn_desc* desc, void* stream);

/* -------------------------------------------------------------------------
 * KV cache write: copy `num_tokens` new key/value rows of every sequence into
 * the (paged) cache at positions write_start[b] + t (or `write_offset` + t when
 * write_start is NULL).
 *
 *   k_cache[b, pos, h, :] = k_new[b, t, h, :];  v_cache likewise
 *
 * Positions are mapped to (page, slot) exactly as in fdllm_kv_attn_fwd.
 * Positions at or beyond max_pages * page_size (or max_seqlen without a page
 * table) are skipped.
 *
 * Replaces: StaticKVCache.update (static_kv_cache.py:132-160),
 * write_scratch_compiled (:218-229) and write_sparse (:231-247, with
 * `positions` = per-token absolute positions [batch, num_tokens]).
 * ------------------------------------------------------------------------- */
int fdllm_kv_cache_write(const void* k_new, const void* v_new,
                         int64_t new_stride_b, int64_t new_stride_s, int64_t new_stride_h,
                         void* k_cache, void* v_cache,
                         int64_t cache_stride_page, int64_t cache_stride_slot, int64_t cache_stride_h,
                         const int32_t* page_table, int32_t max_pages, int32_t page_size,
                         int32_t max_seqlen,
                         const int32_t* write_start, int32_t write_offset,
                         const int64_t* positions,
                         int batch, int num_tokens, int num_kv_heads, int head_dim,
                         int dtype, void* stream);

/* -------------------------------------------------------------------------
 * RoPE of the new queries and keys fused with the KV cache write (the step
 * between the q/k/v projections and the attention).
 *
 *   for b < batch, t < seq_len:
 *     q_out[b, t, h]  = rope(q[b, t, h])                 h < num_q_heads
 *     kr              = rope(k[b, t, g])                 g < num_kv_heads
 *     k_cache[b, write_start[b] + write_offset + t, g] = kr   (write_start may
 *     v_cache[b, write_start[b] + write_offset + t, g] = v[b, t, g]      be NULL)
 *     k_block[b, block_offset + t, g] = kr;  v_block likewise    (if k_block)
 *     k_out[b, t, g] = kr;  v_out[b, t, g] = v[b, t, g]           (if k_out)
 *
 *   rope(x)[i] = x[i] * cos[i] + rotate_half(x)[i] * sin[i],
 *   rotate_half(x) = (-x[D/2 .. D), x[0 .. D/2)),
 * rounded to `dtype` after each product and after the sum: the arithmetic of the
 * eager 16-bit expression q * cos + rotate_half(q) * sin, so the result equals it
 * bit for bit. cos / sin are [cs_batch (1 or batch), seq_len, head_dim] in `dtype`
 * (the model's position embeddings). The caches are contiguous-row
 * [batch, len, heads, head_dim] buffers with the given strides; rows at or
 * beyond cache_len / block_len are skipped. q_out may alias q.
 *
 * Replaces: apply_rotary_pos_emb + the static / block cache writes of the
 * patched attention forward (utils/attention_backends.py:777-788, :843-878;
 * static_kv_cache.py:218-229 write_scratch_compiled, :451-457 StaticBlockCache.update).
 * ------------------------------------------------------------------------- */
typedef struct fdllm_rope_kv_desc {
  const void* q; /* [batch, seq_len, num_q_heads, head_dim] */
  int64_t q_stride_b, q_stride_s, q_stride_h;
  const void* k; /* [batch, seq_len, num_kv_heads, head_dim] */
  int64_t k_stride_b, k_stride_s, k_stride_h;
  const void* v;
  int64_t v_stride_b, v_stride_s, v_stride_h;
  const void* cos; /* [cs_batch, seq_len, head_dim] */
  const void* sin;
  int64_t cs_stride_b, cs_stride_s; /* cs_stride_b = 0 broadcasts one table */
  void* q_out;
  int64_t qo_stride_b, qo_stride_s, qo_stride_h;
  void* k_out; /* optional [batch, seq_len, num_kv_heads, head_dim], with v_out */
  void* v_out;
  int64_t ko_stride_b, ko_stride_s, ko_stride_h;
  void* k_cache; /* optional destination 1 (the static cache of this layer) */
  void* v_cache;
  int64_t c_stride_b, c_stride_s, c_stride_h;
  int32_t cache_len;
  const int32_t* write_start; /* [batch] or NULL */
  int32_t write_offset;
  void* k_block; /* optional destination 2 (the within-block cache of this layer) */
  void* v_block;
  int64_t bc_stride_b, bc_stride_s, bc_stride_h;
  int32_t block_len;
  int32_t block_offset;
  int batch, seq_len, num_q_heads, num_kv_heads, head_dim;
  int dtype; /* FDLLM_DTYPE_BF16 or FDLLM_DTYPE_F16 */
} fdllm_rope_kv_desc;

int fdllm_rope_kv_write(const fdllm_rope_kv_desc* desc, void* stream);

/* -------------------------------------------------------------------------
 * The q / k / v projections of the new tokens fused with the RoPE + KV cache
 * write above: the projection GEMMs with RoPE and the cache write as their
 * epilogue.
 *
 *   for token row r = b * seq_len + t (r < batch * seq_len):
 *     q[b, t, h] = round(x[r] . wq[h * D + i] + bq[h * D + i])   i < D (= 128)
 *     k[b, t, g], v[b, t, g] likewise with wk / bk, wv / bv
 *   then everything fdllm_rope_kv_write does with q, k, v (outputs, caches,
 *   positions and rounding as there).
 *
 * x is [batch * seq_len, hidden] with row stride x_stride_row (elements, a
 * multiple of 8, at least hidden); wq is [num_q_heads * D, hidden] and wk / wv
 * [num_kv_heads * D, hidden], rows contiguous (nn.Linear weights); biases are
 * [heads * D] or NULL. Products are summed in fp32 (MFMA), the bias added in
 * fp32 and the sum rounded once to `dtype`, as a 16-bit linear layer with bias
 * does; the summation order differs from a library GEMM's, so q / k / v agree
 * with separate projections to within the rounding of their last bit. In
 * `rope`, q / k / v and their strides are not read; head_dim must be 128 and
 * hidden a multiple of 64.
 *
 * Replaces: the q_proj / k_proj / v_proj calls of the patched attention forward
 * (utils/attention_backends.py:837-839, :946-948; the layers of modeling.py:321-323)
 * together with the RoPE and cache writes that fdllm_rope_kv_write replaces.
 * ------------------------------------------------------------------------- */
typedef struct fdllm_qkv_rope_desc {
  const void* x;
  int64_t x_stride_row;
  const void* wq;
  const void* wk;
  const void* wv;
  const void* bq; /* or NULL */
  const void* bk;
  const void* bv;
  int hidden;
  fdllm_rope_kv_desc rope;
} fdllm_qkv_rope_desc;

int fdllm_qkv_rope_kv_write(const fdllm_qkv_rope_desc* desc, void* stream);

/* -------------------------------------------------------------------------
 * One greedy sampling + threshold unmasking step of a sub-block.
 *
 *   for b < batch, i < num_positions (<= 64):
 *     row    = logits[b, max(row_offset + i - shift, 0), :]   (shift 1: the one-
 *              position shift of the diffusion logits)
 *     p      = softmax(row), rounded to the logits' dtype
 *     tok    = first index of max(p);   conf = p[tok]
 *     row_tok[b, i] = tok;  row_conf[b, i] = conf
 *     masked = tokens[b, i] == mask_id and not finished[b]
 *     unmask = masked and (conf > threshold or i is the first position of
 *              max(conf over masked positions of b))
 *     if unmask: tokens[b, i] = tok;   finished[b] |= unmask and tok == stop_token
 *   counts[0] = positions unmasked, counts[1] = masked positions left in rows not
 *   finished, counts[2] = rows whose position 0 is still masked, counts[3] =
 *   finished rows (all after the step).
 *
 * tokens is int64 with the positions of a row contiguous; finished is a byte per
 * row or NULL; stop_token < 0 disables the stop rule. row_tok / row_conf are
 * [batch, num_positions] outputs, counts an int32[4] output. Two kernels on
 * `stream`; the caller reads counts to decide the next step.
 *
 * Replaces: sample_with_top_p at temperature 0 (modeling.py:2263-2270 of the
 * model snapshot) and the unmask rule of batch_sample_dynamo
 * (generation_functions.py:784-807).
 * ------------------------------------------------------------------------- */
int fdllm_unmask_step(const void* logits, int64_t logits_stride_b, int64_t logits_stride_row, int vocab,
                      int row_offset, int shift, int64_t* tokens, int64_t tokens_stride_b,
                      uint8_t* finished, int64_t mask_id, float threshold, int64_t stop_token,
                      int64_t* row_tok, float* row_conf, int32_t* counts,
                      int batch, int num_positions, int dtype, void* stream);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* FDLLM_HIP_H_ */
