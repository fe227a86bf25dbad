// Host-side planning of fdllm_kv_attn_fwd: which kernel family a descriptor takes, the
// workspace it needs, the grid of every kernel the call launches, and the argument
// checks made before any launch. Plain C++ with no HIP dependency: block_attn.hip
// includes it and launches exactly the grids computed here, and a host-only test builds
// it with AddressSanitizer and UndefinedBehaviorSanitizer and sweeps descriptors out to
// the limits of every field.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include <algorithm>

#include "../../include/fdllm_hip.h"
#include "host_errors.h"

#ifndef FDLLM_F32_ROWS_PER_WAVE
#define FDLLM_F32_ROWS_PER_WAVE 1  // query rows per wave of the fp32 kernel
#endif

namespace fdllm {

constexpr int kKT = 64;                // keys per tile of the general kernel
constexpr int kThreads = 256;          // threads of the general kernel (4 waves)
constexpr int kMaxDecodeSplits = 16;   // key splits per (sequence, KV head) with a fixed chunk
constexpr int kDecodeMaxTiles = 160;   // 32-key tiles per split: page ids staged in LDS
constexpr int kBalMaxPages = 4096;     // page-table entries the cross-sequence decode kernel stages
constexpr int kPrefillWaves = 8;       // waves (x 32 query rows) per prefill workgroup
constexpr int kSplitTargetWG = 256;    // MI355X compute units
// Teams of 4 waves per split decode workgroup: two (512 threads, one workgroup per compute
// unit; the default) or one (256 threads, two workgroups per compute unit and twice the
// slots). One team was measured slower on the bs16 7B sub-block step, 31.4 against
// 25.5 us: no split is longer than the median any more, but the loop is bound by HBM and
// ends no earlier, and folding a unit's 8 splits in one 256-thread workgroup takes 6.8
// against 2.4 us.
#ifndef FDLLM_DECODE_TEAMS
#define FDLLM_DECODE_TEAMS 2
#endif
constexpr int kDecodeTeams = FDLLM_DECODE_TEAMS;
static_assert(kDecodeTeams == 1 || kDecodeTeams == 2, "one or two teams per split decode workgroup");
constexpr int kDecodeSlotsTarget = kSplitTargetWG * (kDecodeTeams == 1 ? 2 : 1);
constexpr int kSplitMaxChunk = kDecodeMaxTiles * 32;  // keys per split: page ids staged in LDS
constexpr int kBalancedMaxBatch = 64;  // one wave lane per sequence in the partition search
// fp32 kernel: key splits up to about two workgroups per CU. On a batch-1, 12 / 2-head block
// of 32 queries over 544 keys (96 row blocks): 3 splits 16.4 us, 5 (this target) 13.8 us,
// 9 splits 15.5 us, no split 27.4 us.
constexpr int kF32TargetWG = 512;
// 1: the fp32 kernel's key splits are merged by the last workgroup of each row block to
// arrive (one arrival counter per row block), where the counters suffice; 0: by a second
// kernel.
#ifndef FDLLM_F32_MERGE_IN_KERNEL
#define FDLLM_F32_MERGE_IN_KERNEL 1
#endif
constexpr int kF32MaxSplits = 16;      // fp32 kernel: key splits per row block at most
constexpr size_t kCounterBytes = 64 * 1024;  // arrival counters at the head of the workspace
constexpr uint32_t kMaxGridX = 0x7fffffffu;  // grid limits of a launch
constexpr uint32_t kMaxGridYZ = 65535u;

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

// Kernel families a call can take (make_plan picks one per descriptor).
enum PlanKind {
  kPlanGeneral = 0,
  kPlanAllHeads = 1,
  kPlanSplitDecode = 2,
  kPlanPrefill = 3,
  kPlanSplitPrefill = 4,
  kPlanF32 = 5,
  kPlanBalancedDecode = 6
};

struct Plan {
  int kind;     // PlanKind
  bool decode;  // all-heads decode kernel (kv_decode_kernel)
  int MT, rows_per_wg, n_rb, n_splits, chunk, R;
  size_t ws_o_bytes, ws_ml_bytes;
  size_t ws_unit_off;  // split prefill: byte offset of the unit table in the (m, l) region
};

// Longest key range a call can read: max_seqlen, capped by the pages' capacity.
inline int64_t plan_max_keys(const fdllm_kv_attn_desc* d) {
  return d->page_table ? std::min<int64_t>(d->max_seqlen, static_cast<int64_t>(d->max_pages) * d->page_size)
                       : d->max_seqlen;
}

// Split-KV decode: by default the kernel partitions the keys itself from the device-side
// lengths over S slots per KV head (S * Hkv ~ one workgroup per CU); a caller-given
// kv_split fixes the keys per split instead.
inline int make_plan(const fdllm_kv_attn_desc* d, Plan* pl) {
  FDLLM_CHECK_ARG(d != nullptr, "fdllm_kv_attn: null descriptor");
  pl->ws_unit_off = 0;
  FDLLM_CHECK_ARG(d->dtype == FDLLM_DTYPE_BF16 || d->dtype == FDLLM_DTYPE_F16 || d->dtype == FDLLM_DTYPE_F32,
                  "fdllm_kv_attn: dtype %d unsupported (bf16, fp16 or fp32)", d->dtype);
  FDLLM_CHECK_ARG(d->head_dim == 64 || d->head_dim == 128, "fdllm_kv_attn: head_dim %d unsupported (64 or 128)",
                  d->head_dim);
  FDLLM_CHECK_ARG(d->batch >= 0 && d->q_len >= 0 && d->num_q_heads > 0 && d->num_kv_heads > 0,
                  "fdllm_kv_attn: bad sizes");
  FDLLM_CHECK_ARG(d->num_q_heads % d->num_kv_heads == 0, "fdllm_kv_attn: num_q_heads %d not a multiple of %d",
                  d->num_q_heads, d->num_kv_heads);
  FDLLM_CHECK_ARG(d->max_seqlen >= 0, "fdllm_kv_attn: max_seqlen < 0");
  FDLLM_CHECK_ARG(d->mask_mode >= FDLLM_MASK_SEQLEN && d->mask_mode <= FDLLM_MASK_BLOCK_CAUSAL,
                  "fdllm_kv_attn: unknown mask_mode %d", d->mask_mode);
  FDLLM_CHECK_ARG(d->mask_mode != FDLLM_MASK_BLOCK_CAUSAL || d->mask_block > 0,
                  "fdllm_kv_attn: block-causal mask needs mask_block > 0");
  // every kernel holds key positions and capacities in 32-bit ints with room for a tile
  // of look-ahead: 2^30 keys at most
  FDLLM_CHECK_ARG(d->max_seqlen <= (1 << 30), "fdllm_kv_attn: max_seqlen %d above 2^30", d->max_seqlen);
  // every family puts the (sequence, KV head) pairs, or one of the two, on a grid
  // dimension of at most 65535
  FDLLM_CHECK_ARG(static_cast<int64_t>(d->batch) * d->num_kv_heads <= static_cast<int64_t>(kMaxGridYZ),
                  "fdllm_kv_attn: batch x num_kv_heads = %lld above %u",
                  static_cast<long long>(d->batch) * d->num_kv_heads, kMaxGridYZ);
  if (d->dtype == FDLLM_DTYPE_F32) {
    // fp32: kv_attn_f32_kernel; pages of any power of two. Keys are split (chunk keys
    // per split, a multiple of the kernel's 64-key chunk) when the row blocks alone give
    // fewer than kF32TargetWG workgroups; kv_attn_combine_kernel then folds the partials.
    FDLLM_CHECK_ARG(d->page_table == nullptr ||
                        (d->page_size > 0 && (d->page_size & (d->page_size - 1)) == 0 && d->max_pages > 0),
                    "fdllm_kv_attn: page table needs a power-of-two page_size and max_pages > 0");
    FDLLM_CHECK_ARG(d->k_new == nullptr && d->v_new == nullptr,
                    "fdllm_kv_attn: the cache write (k_new / v_new) takes bf16 or fp16 only");
    const int64_t rows = static_cast<int64_t>(d->q_len) * (d->num_q_heads / d->num_kv_heads);
    FDLLM_CHECK_ARG(rows < (int64_t{1} << 30), "fdllm_kv_attn: q_len * group too large");
    pl->kind = kPlanF32;
    pl->decode = false;
    pl->MT = 0;
    pl->rows_per_wg = 4 * FDLLM_F32_ROWS_PER_WAVE;
    pl->R = static_cast<int>(rows);
    pl->n_rb = static_cast<int>((rows + pl->rows_per_wg - 1) / pl->rows_per_wg);
    const int64_t chunks = std::max<int64_t>(1, (plan_max_keys(d) + 63) / 64);  // 64-key chunks of the longest
    const int64_t units = static_cast<int64_t>(d->batch) * d->num_kv_heads * pl->n_rb;
    int64_t per;  // chunks per split
    if (d->kv_split > 0) {
      per = (static_cast<int64_t>(d->kv_split) + 63) / 64;
    } else if (units >= kF32TargetWG || units == 0) {  // units == 0: an empty call (nothing launches)
      per = chunks;
    } else {
      const int64_t splits = (kF32TargetWG + units - 1) / std::max<int64_t>(units, 1);
      per = (chunks + splits - 1) / splits;
    }
    per = std::max<int64_t>(per, (chunks + kF32MaxSplits - 1) / kF32MaxSplits);  // at most kF32MaxSplits splits
    per = std::max<int64_t>(1, std::min(per, chunks));
    pl->chunk = static_cast<int>(per * 64);
    pl->n_splits = static_cast<int>((chunks + per - 1) / per);
    if (pl->n_splits > 1) {
      FDLLM_CHECK_ARG(units * pl->n_splits * pl->rows_per_wg < (int64_t{1} << 31) / 128,
                      "fdllm_kv_attn: too many fp32 split slots");
      pl->ws_o_bytes = static_cast<size_t>(units) * pl->n_splits * pl->rows_per_wg * d->head_dim * sizeof(float);
      pl->ws_ml_bytes = static_cast<size_t>(units) * pl->n_splits * pl->rows_per_wg * 2 * sizeof(float);
    } else {
      pl->ws_o_bytes = pl->ws_ml_bytes = 0;
    }
    return FDLLM_OK;
  }
  // Each thread stages aligned groups of 2048 / head_dim keys from one page.
  FDLLM_CHECK_ARG(d->page_table == nullptr ||
                      (d->page_size >= kThreads * 8 / d->head_dim && (d->page_size & (d->page_size - 1)) == 0 &&
                       d->max_pages > 0),
                  "fdllm_kv_attn: page table needs a power-of-two page_size >= %d (got %d) and max_pages > 0",
                  kThreads * 8 / d->head_dim, d->page_size);
  FDLLM_CHECK_ARG(d->kv_split >= 0 && d->kv_split % kKT == 0, "fdllm_kv_attn: kv_split %d not a multiple of %d",
                  d->kv_split, kKT);
  const int G = d->num_q_heads / d->num_kv_heads;
  const int64_t R64 = static_cast<int64_t>(d->q_len) * G;
  FDLLM_CHECK_ARG(R64 < (1 << 30), "fdllm_kv_attn: q_len * group too large");
  pl->R = static_cast<int>(R64);
  const int hkv = d->num_kv_heads;
  const int64_t max_len = plan_max_keys(d);  // <= 2^30
  const bool decode_shape = !(d->flags & FDLLM_ATTN_NO_DECODE_KERNEL) && d->head_dim == 128 && pl->R <= 64 &&
                            (d->page_table == nullptr || d->page_size >= 32) &&
                            d->k_stride_slot >= d->head_dim && d->v_stride_slot >= d->head_dim &&
                            d->k_stride_slot < (1 << 24) && d->v_stride_slot < (1 << 24);
  pl->kind = kPlanGeneral;
  if (decode_shape && !(d->flags & FDLLM_ATTN_ALL_HEADS_DECODE)) {
    const int64_t len = std::max<int64_t>(1, max_len);
    const int64_t max_t = (len + 31) / 32;  // tiles of the longest sequence
    // every split holds at most kDecodeMaxTiles tiles and a sequence at most kMaxDecodeSplits splits
    if (max_t <= static_cast<int64_t>(kDecodeMaxTiles) * kMaxDecodeSplits &&
        static_cast<int64_t>(d->batch) * hkv <= static_cast<int64_t>(kCounterBytes / sizeof(int))) {
      const int64_t B = std::max(d->batch, 1);
      const int64_t min_splits = (max_t + kDecodeMaxTiles - 1) / kDecodeMaxTiles;  // of the longest sequence
      pl->kind = kPlanSplitDecode;
      pl->decode = false;
      pl->MT = 1;
      pl->rows_per_wg = 64;
      pl->n_rb = 1;
      int64_t slots;  // partial slots per KV head
      bool split_possible;
      const bool pages_fit = d->page_table == nullptr || B * d->max_pages <= kBalMaxPages;
      if (d->kv_split == 0 && B <= kBalancedMaxBatch && pages_fit && (d->flags & FDLLM_ATTN_BALANCED_SPLITS)) {
        // pairs of 32-key tiles dealt evenly over S slots per KV head (S * Hkv ~ one
        // workgroup per CU, S a multiple of 8 for the XCD-major slot order); partial
        // slots S + batch per head (piece (s, b) owns slot s + b)
        pl->kind = kPlanBalancedDecode;
        pl->chunk = 0;
        const int64_t s8 = std::max<int64_t>(8, (kSplitTargetWG / hkv + 7) / 8 * 8);
        pl->n_splits = static_cast<int>(s8);
        const int64_t pslots = s8 + B;
        FDLLM_CHECK_ARG(pslots * hkv < (int64_t{1} << 31) / 64, "fdllm_kv_attn: too many split slots");
        pl->ws_o_bytes = static_cast<size_t>(pslots) * hkv * 64 * d->head_dim * sizeof(float);
        pl->ws_ml_bytes = static_cast<size_t>(pslots) * hkv * 64 * 2 * sizeof(float);
        return FDLLM_OK;
      }
      if (d->kv_split == 0 && B <= kBalancedMaxBatch) {
        pl->chunk = 0;
        slots = std::max<int64_t>((kDecodeSlotsTarget + hkv - 1) / hkv, B * min_splits);
        pl->n_splits = static_cast<int>(slots);
        split_possible = slots > B;
      } else {
        int64_t chunk = d->kv_split > 0 ? d->kv_split : kSplitMaxChunk;
        chunk = std::max<int64_t>(chunk, (max_t + kMaxDecodeSplits - 1) / kMaxDecodeSplits * 32);
        chunk = std::min<int64_t>(chunk, kSplitMaxChunk);
        pl->chunk = static_cast<int>(chunk);
        pl->n_splits = static_cast<int>((max_t * 32 + chunk - 1) / chunk);  // per sequence
        slots = B * pl->n_splits;
        split_possible = pl->n_splits > 1;
      }
      FDLLM_CHECK_ARG(slots * hkv < (int64_t{1} << 31) / 64, "fdllm_kv_attn: too many split slots");
      if (split_possible) {
        pl->ws_o_bytes = static_cast<size_t>(slots) * hkv * 64 * d->head_dim * sizeof(float);
        pl->ws_ml_bytes = static_cast<size_t>(slots) * hkv * 64 * 2 * sizeof(float);
      } else {
        pl->ws_o_bytes = pl->ws_ml_bytes = 0;
      }
      return FDLLM_OK;
    }
  }
  pl->decode = decode_shape && (hkv == 1 || hkv == 2 || hkv == 4 || hkv == 8) && d->k_stride_h == 128 &&
               d->v_stride_h == 128;
  if (pl->decode) {
    pl->kind = kPlanAllHeads;
    const int64_t max_t32 = std::max<int64_t>(1, (max_len + 31) / 32);
    int64_t chunk_t32;
    if (d->kv_split > 0) {
      chunk_t32 = d->kv_split / 32;
    } else {
      // ~320 workgroups when every sequence is full length, >= 128 keys each
      const int64_t splits = (320 + std::max(d->batch, 1) - 1) / std::max(d->batch, 1);
      chunk_t32 = std::max<int64_t>(4, (max_t32 + splits - 1) / splits);
    }
    chunk_t32 = std::max<int64_t>(1, std::min(chunk_t32, max_t32));
    pl->MT = 0;
    pl->rows_per_wg = 64;
    pl->n_rb = 1;
    pl->chunk = static_cast<int>(chunk_t32 * 32);
    pl->n_splits = static_cast<int>((max_t32 + chunk_t32 - 1) / chunk_t32);
    const int64_t units = static_cast<int64_t>(d->batch) * hkv;
    if (pl->n_splits > 1) {
      pl->ws_o_bytes = static_cast<size_t>(units) * pl->n_splits * 64 * d->head_dim * sizeof(float);
      pl->ws_ml_bytes = static_cast<size_t>(units) * pl->n_splits * 64 * 2 * sizeof(float);
    } else {
      pl->ws_o_bytes = pl->ws_ml_bytes = 0;
    }
    return FDLLM_OK;
  }
  // Block decode shapes (64 < rows per KV head <= 256, e.g. a whole 32-token block at
  // GQA 7): the prefill kernel's math on one row block, keys split and merged as in the
  // split decode kernel (64-key tiles)
  const bool split_prefill_shape = !(d->flags & FDLLM_ATTN_NO_DECODE_KERNEL) && d->head_dim == 128 &&
                                   pl->R > 64 && pl->R <= 256 && (d->kv_split == 0 || d->kv_split % 64 == 0) &&
                                   (d->page_table == nullptr || d->page_size >= 32) &&
                                   d->k_stride_slot < (1 << 24) && d->v_stride_slot < (1 << 24);
  if (split_prefill_shape) {
    const int64_t max_t = (std::max<int64_t>(1, max_len) + 63) / 64;  // 64-key tiles of the longest sequence
    if (max_t <= static_cast<int64_t>(kDecodeMaxTiles) * kMaxDecodeSplits &&
        static_cast<int64_t>(d->batch) * hkv <= static_cast<int64_t>(kCounterBytes / sizeof(int))) {
      const int64_t B = std::max(d->batch, 1);
      const int64_t min_splits = (max_t + kDecodeMaxTiles - 1) / kDecodeMaxTiles;
      pl->kind = kPlanSplitPrefill;
      pl->decode = false;
      pl->MT = 4;
      pl->rows_per_wg = 256;
      pl->n_rb = 1;
      int64_t slots;
      bool split_possible;
      if (d->kv_split == 0 && B <= kBalancedMaxBatch) {
        pl->chunk = 0;
        slots = std::max<int64_t>((kSplitTargetWG + hkv - 1) / hkv, B * min_splits);
        pl->n_splits = static_cast<int>(slots);
        split_possible = slots > B;
      } else {
        int64_t chunk = d->kv_split > 0 ? d->kv_split : static_cast<int64_t>(kDecodeMaxTiles) * 64;
        chunk = std::max<int64_t>(chunk, (max_t + kMaxDecodeSplits - 1) / kMaxDecodeSplits * 64);
        chunk = std::min<int64_t>(chunk, static_cast<int64_t>(kDecodeMaxTiles) * 64);
        pl->chunk = static_cast<int>(chunk);
        pl->n_splits = static_cast<int>((max_t * 64 + chunk - 1) / chunk);
        slots = B * pl->n_splits;
        split_possible = pl->n_splits > 1;
      }
      FDLLM_CHECK_ARG(slots * hkv < (int64_t{1} << 31) / 256, "fdllm_kv_attn: too many split slots");
      if (split_possible) {
        pl->ws_o_bytes = static_cast<size_t>(slots) * hkv * 256 * d->head_dim * sizeof(float);
        pl->ws_unit_off = static_cast<size_t>(slots) * hkv * 256 * 2 * sizeof(float);
        pl->ws_ml_bytes = pl->ws_unit_off + static_cast<size_t>(B) * hkv * 2 * sizeof(int32_t);
      } else {
        pl->ws_o_bytes = pl->ws_ml_bytes = 0;
      }
      return FDLLM_OK;
    }
  }
  // Prefill shapes: at least 8 row blocks of 256 per KV head, pages of >= 32 keys
  const bool prefill_shape = !(d->flags & FDLLM_ATTN_NO_DECODE_KERNEL) && d->head_dim == 128 &&
                             pl->R >= 8 * 256 && d->kv_split == 0 &&
                             (d->page_table == nullptr || d->page_size >= 32) && d->k_stride_slot < (1 << 24) &&
                             d->v_stride_slot < (1 << 24) && (pl->R + 255) / 256 < 65536;
  if (prefill_shape) {
    pl->kind = kPlanPrefill;
    pl->MT = 4;
    pl->rows_per_wg = 32 * kPrefillWaves;
    pl->n_rb = (pl->R + pl->rows_per_wg - 1) / pl->rows_per_wg;
    pl->n_splits = 1;
    pl->chunk = 1 << 30;
    pl->ws_o_bytes = pl->ws_ml_bytes = 0;
    return FDLLM_OK;
  }
  const int mtiles = (pl->R + 15) / 16;
  pl->MT = mtiles <= 4 ? 1 : (mtiles <= 8 ? 2 : 4);
  pl->rows_per_wg = 64 * pl->MT;
  pl->n_rb = (pl->R + pl->rows_per_wg - 1) / pl->rows_per_wg;
  const int64_t max_tiles = std::max<int64_t>(1, (max_len + kKT - 1) / kKT);
  int64_t chunk_tiles;
  const int64_t units = static_cast<int64_t>(d->batch) * d->num_kv_heads * pl->n_rb;
  if (d->kv_split > 0) {
    chunk_tiles = d->kv_split / kKT;
  } else {
    // Aim for ~2 workgroups per CU (256 CUs) when every sequence is full length.
    const int64_t target = 512;
    if (units >= target) {
      chunk_tiles = max_tiles;
    } else {
      const int64_t splits = (target + units - 1) / std::max<int64_t>(units, 1);
      chunk_tiles = (max_tiles + splits - 1) / splits;
      chunk_tiles = std::max<int64_t>(chunk_tiles, 4);  // >= 256 keys per split keeps partial traffic small
    }
  }
  chunk_tiles = std::max<int64_t>(1, std::min(chunk_tiles, max_tiles));
  pl->chunk = static_cast<int>(chunk_tiles * kKT);
  pl->n_splits = static_cast<int>((max_tiles + chunk_tiles - 1) / chunk_tiles);
  if (pl->n_splits > 1) {
    // the merge kernel has one workgroup row per (sequence, KV head, row block)
    FDLLM_CHECK_ARG(units <= static_cast<int64_t>(kMaxGridYZ),
                    "fdllm_kv_attn: %lld (sequence, KV head, row block) units with %d key splits exceed the merge "
                    "grid; pass kv_split = 0 or a larger kv_split",
                    static_cast<long long>(units), pl->n_splits);
    pl->ws_o_bytes = static_cast<size_t>(units) * pl->n_splits * pl->rows_per_wg * d->head_dim * sizeof(float);
    pl->ws_ml_bytes = static_cast<size_t>(units) * pl->n_splits * pl->rows_per_wg * 2 * sizeof(float);
  } else {
    pl->ws_o_bytes = pl->ws_ml_bytes = 0;
  }
  return FDLLM_OK;
}

// Workspace layout: a fixed 64 KiB of arrival counters (one int per (sequence,
// KV head)), the (m, l) pairs of every split partial (for the split prefill kernel
// followed by its table of (first slot, splits) per (sequence, KV head)), then the
// partial rows. The counter region has the same place and size for every call, so
// partials of one call never land where a later call with more sequences keeps its
// counters.
inline size_t plan_workspace_bytes(const fdllm_kv_attn_desc*, const Plan& pl) {
  return pl.ws_o_bytes > 0 ? kCounterBytes + align256(pl.ws_ml_bytes) + pl.ws_o_bytes : 0;
}

// The rows of k_new / v_new are stored from inside the prefill kernels (plan kinds
// prefill and split prefill, no explicit q_start, no FDLLM_ATTN_CACHE_WRITE_KERNEL);
// otherwise a copy kernel stores them ahead of the attention.
// The prefill kernels read every key at or past the query start from the new rows,
// which is exact only when no visible key lies past the last new row. Without q_start
// that holds by construction (query start = visible length - q_len); an explicit
// q_start may leave visible cache rows past q_start + q_len, so such calls take the
// copy kernel, which stores the rows before the attention reads the cache.
inline bool plan_fuses_cache_write(const fdllm_kv_attn_desc* d, const Plan& pl) {
  return d->k_new != nullptr && d->q_start == nullptr && !(d->flags & FDLLM_ATTN_CACHE_WRITE_KERNEL) &&
         (pl.kind == kPlanPrefill || pl.kind == kPlanSplitPrefill);
}

// The fp32 plan merges its key splits in the kernel (one counter per row block unit).
inline bool plan_f32_merge_in_kernel(const Plan& pl, int64_t batch, int64_t hkv) {
  return FDLLM_F32_MERGE_IN_KERNEL && pl.kind == kPlanF32 && pl.n_splits > 1 &&
         batch * hkv * pl.n_rb <= static_cast<int64_t>(kCounterBytes / sizeof(int));
}

struct GridDims {
  uint32_t x, y, z;
};

// Every kernel one call launches, in launch order: the cache-write copy kernel (if any),
// the attention kernel, and the merge / combine kernel of the split partials (if any).
struct LaunchSet {
  bool write;
  GridDims write_grid;  // kv_write_kernel, 256 threads
  GridDims main_grid;
  uint32_t main_block;
  bool second;
  GridDims second_grid;  // 256 threads
};

inline bool grid_fits(const GridDims& g) {
  return g.x >= 1 && g.y >= 1 && g.z >= 1 && g.x <= kMaxGridX && g.y <= kMaxGridYZ && g.z <= kMaxGridYZ;
}

// Grids of the kernels a validated, non-empty call launches (batch and q_len > 0).
inline int plan_launches(const fdllm_kv_attn_desc* d, const Plan& pl, LaunchSet* ls) {
  const int64_t B = d->batch, hkv = d->num_kv_heads;
  const int64_t grid_z = B * hkv;
  FDLLM_CHECK_ARG(B > 0 && d->q_len > 0, "fdllm_kv_attn_fwd: empty call has no launches");
  FDLLM_CHECK_ARG(grid_z <= kMaxGridYZ && pl.n_rb <= static_cast<int>(kMaxGridYZ),
                  "fdllm_kv_attn_fwd: grid too large (batch x KV heads %lld, row blocks %d)",
                  static_cast<long long>(grid_z), pl.n_rb);
  ls->write = d->k_new != nullptr && !plan_fuses_cache_write(d, pl);
  ls->write_grid = GridDims{1, 1, 1};
  if (ls->write) {
    const int64_t n = B * d->q_len * hkv * (d->head_dim / 8);  // 16-byte vectors
    const int64_t blocks = (n + 255) / 256;
    FDLLM_CHECK_ARG(blocks <= static_cast<int64_t>(kMaxGridX), "fdllm_kv_attn_fwd: cache write too large");
    ls->write_grid = GridDims{static_cast<uint32_t>(blocks), 1, 1};
  }
  ls->second = false;
  ls->second_grid = GridDims{1, 1, 1};
  switch (pl.kind) {
    case kPlanF32: {
      // x = row block + n_rb * split
      ls->main_grid = GridDims{static_cast<uint32_t>(static_cast<int64_t>(pl.n_rb) * pl.n_splits),
                               static_cast<uint32_t>(hkv), static_cast<uint32_t>(B)};
      ls->main_block = 256;
      if (pl.n_splits > 1 && !plan_f32_merge_in_kernel(pl, B, hkv)) {
        // combine: one workgroup row per (sequence, KV head, row block)
        const int rpb = 256 / (d->head_dim / 8);
        const int64_t units = static_cast<int64_t>(B) * hkv * pl.n_rb;
        FDLLM_CHECK_ARG(units <= static_cast<int64_t>(kMaxGridYZ),
                        "fdllm_kv_attn_fwd: %lld split units exceed the merge grid; pass a larger kv_split",
                        static_cast<long long>(units));
        ls->second = true;
        ls->second_grid = GridDims{static_cast<uint32_t>((pl.rows_per_wg + rpb - 1) / rpb),
                                   static_cast<uint32_t>(units), 1};
      }
      break;
    }
    case kPlanBalancedDecode:
      ls->main_grid = GridDims{static_cast<uint32_t>(pl.n_splits), static_cast<uint32_t>(hkv), 1};
      ls->main_block = 512;
      break;
    case kPlanSplitDecode:
      ls->main_grid = GridDims{static_cast<uint32_t>(pl.n_splits), static_cast<uint32_t>(hkv),
                               static_cast<uint32_t>(pl.chunk > 0 ? B : 1)};
      ls->main_block = 512;
      break;
    case kPlanPrefill:
      ls->main_grid = GridDims{static_cast<uint32_t>(grid_z), static_cast<uint32_t>(pl.n_rb), 1};
      ls->main_block = 64 * kPrefillWaves;
      break;
    case kPlanSplitPrefill:
      ls->main_grid = GridDims{static_cast<uint32_t>(pl.n_splits), static_cast<uint32_t>(hkv),
                               static_cast<uint32_t>(pl.chunk > 0 ? B : 1)};
      ls->main_block = 512;
      if (pl.ws_o_bytes > 0) {  // merge: 32 rows per workgroup, one workgroup row per (sequence, KV head)
        ls->second = true;
        ls->second_grid = GridDims{static_cast<uint32_t>((pl.R + 31) / 32), static_cast<uint32_t>(grid_z), 1};
      }
      break;
    case kPlanAllHeads: {
      ls->main_grid = GridDims{static_cast<uint32_t>(pl.n_splits), static_cast<uint32_t>(B), 1};
      ls->main_block = static_cast<uint32_t>(128 * hkv);
      if (pl.n_splits > 1) {
        const int rpb = 256 / (d->head_dim / 8);
        ls->second = true;
        ls->second_grid = GridDims{static_cast<uint32_t>((pl.rows_per_wg + rpb - 1) / rpb),
                                   static_cast<uint32_t>(grid_z), 1};
      }
      break;
    }
    default: {  // kPlanGeneral
      ls->main_grid = GridDims{static_cast<uint32_t>(pl.n_splits), static_cast<uint32_t>(pl.n_rb),
                               static_cast<uint32_t>(grid_z)};
      ls->main_block = kThreads;
      if (pl.n_splits > 1) {
        // combine: one workgroup row per (sequence, KV head, row block)
        const int rpb = 256 / (d->head_dim / 8);
        const int64_t units = grid_z * pl.n_rb;
        FDLLM_CHECK_ARG(units <= static_cast<int64_t>(kMaxGridYZ),
                        "fdllm_kv_attn_fwd: %lld split units exceed the merge grid; pass kv_split = 0 or a "
                        "larger kv_split",
                        static_cast<long long>(units));
        ls->second = true;
        ls->second_grid = GridDims{static_cast<uint32_t>((pl.rows_per_wg + rpb - 1) / rpb),
                                   static_cast<uint32_t>(units), 1};
      }
      break;
    }
  }
  FDLLM_CHECK_ARG(grid_fits(ls->main_grid) && (!ls->second || grid_fits(ls->second_grid)) &&
                      (!ls->write || grid_fits(ls->write_grid)),
                  "fdllm_kv_attn_fwd: grid out of range");
  return FDLLM_OK;
}

// Checks of a call's pointers, strides and workspace against its plan, made before any
// launch (batch and q_len > 0).
inline int validate_call(const fdllm_kv_attn_desc* d, const Plan& pl, const void* workspace, size_t workspace_bytes) {
  FDLLM_CHECK_ARG(d->q && d->k && d->v && d->out && d->seqlens, "fdllm_kv_attn_fwd: null pointer");
  FDLLM_CHECK_ARG(aligned16(d->q) && aligned16(d->k) && aligned16(d->v) && aligned16(d->out),
                  "fdllm_kv_attn_fwd: q/k/v/out must be 16-byte aligned");
  FDLLM_CHECK_ARG(d->q_stride_b % 8 == 0 && d->q_stride_s % 8 == 0 && d->q_stride_h % 8 == 0 &&
                      d->k_stride_page % 8 == 0 && d->k_stride_slot % 8 == 0 && d->k_stride_h % 8 == 0 &&
                      d->v_stride_page % 8 == 0 && d->v_stride_slot % 8 == 0 && d->v_stride_h % 8 == 0 &&
                      d->out_stride_b % 8 == 0 && d->out_stride_s % 8 == 0 && d->out_stride_h % 8 == 0,
                  "fdllm_kv_attn_fwd: strides must be multiples of 8 elements");
  const size_t need = plan_workspace_bytes(d, pl);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need || !aligned16(workspace))) {
    set_last_error("fdllm_kv_attn_fwd: workspace of %zu bytes required (got %zu)", need, workspace_bytes);
    return FDLLM_ERR_WORKSPACE;
  }
  FDLLM_CHECK_ARG((d->k_new == nullptr) == (d->v_new == nullptr),
                  "fdllm_kv_attn_fwd: k_new and v_new must both be given or both be NULL");
  if (d->k_new != nullptr) {
    FDLLM_CHECK_ARG(aligned16(d->k_new) && aligned16(d->v_new) && d->new_stride_b % 8 == 0 &&
                        d->new_stride_s % 8 == 0 && d->new_stride_h % 8 == 0,
                    "fdllm_kv_attn_fwd: k_new / v_new must be 16-byte aligned with strides in multiples of 8");
    FDLLM_CHECK_ARG(d->new_stride_s < (1 << 24), "fdllm_kv_attn_fwd: new_stride_s too large");
    if (!plan_fuses_cache_write(d, pl)) {
      FDLLM_CHECK_ARG(d->k_stride_page == d->v_stride_page && d->k_stride_slot == d->v_stride_slot &&
                          d->k_stride_h == d->v_stride_h,
                      "fdllm_kv_attn_fwd: a cache write with this shape needs equal K and V cache strides");
    }
  }
  return FDLLM_OK;
}

}  // namespace fdllm
