// Block attention over the static / paged block KV cache, gfx950.
//
// Semantics: out = softmax(q k^T * scale + M) v per query row, GQA head map
// h -> h / G (repeat_kv, modeling.py:202-211), with the masks of
// fdllm_hip.h (seqused: static_kv_cache.py:295-302 and tests/test_focus.py:220-224;
// block-causal: modeling.py:145-150). This is the operation that
// AttentionBackend.flash_kvcache_attention (utils/attention_backends.py:588-640)
// dispatches to flash_attn_with_kvcache.
//
// Kernel design (one workgroup = 4 wavefronts = 256 threads):
//   * Rows. The Sq query tokens x G query heads that share one KV head form the
//     M dimension: row r = t * G + hh. For the 8-token sub-block decode that is
//     56 rows (padded to 64); for a 32-token block 224 rows. Each wave owns MT
//     16-row M-tiles, so a workgroup covers 64 * MT rows and every K/V byte
//     fetched from HBM serves all G heads of the group.
//   * Keys. Each workgroup streams one split of the sequence's keys in tiles of
//     64. Tiles are fetched two ahead into registers with coalesced 16-byte
//     loads (page ids one step further ahead, issued before the tile loads so
//     the in-order vmcnt counter never drains the prefetch), then written to
//     LDS: K row-major with a 16-byte row pad, V transposed ([d][key]) with an
//     8-byte row pad, so both MFMA operands are read as contiguous LDS vectors
//     without bank conflicts. Workgroup barriers fence LDS only, so global
//     loads stay in flight across them.
//   * Math. S^T = K Q^T with v_mfma_f32_16x16x32_bf16 (keys along M, query rows
//     along N, so each lane owns one query row), online softmax in the base-2
//     domain with a 4-lane-group max reduction, then O^T = V^T P^T with the
//     same instruction; P is re-packed to bf16 straight from the S^T
//     accumulators (the key order inside one 32-key MFMA step is permuted
//     consistently for P and V, which leaves the sum unchanged).
//   * Masks are arithmetic: key < row limit, where the limit per row comes from
//     seqlens / q_start / mask_block. Keys past the limit are never loaded.
//   * Split-KV. When one (sequence, KV head) is split over several workgroups,
//     each writes an unnormalised partial (O, m, l) to the workspace and a
//     second, fully parallel kernel merges them (16 threads per row, all
//     splits' loads in flight). The kernel boundary orders the two, so no
//     device-scope fence or counter is needed.
#include <algorithm>
#include <climits>
#include <mutex>

#include "fdllm_common.h"
#include "attn_plan.h"

namespace fdllm {
namespace {

constexpr int kSlcNt = 2;      // buffer-load cache policy: streaming (no reuse expected)
// Buffer load/store cache policy "sc1": coherent at device scope. With 8 XCDs the L2
// caches are per XCD; sc1 stores write through to memory and sc1 loads do not hit
// another XCD's stale copy, which is all a cross-workgroup handoff of a few KiB needs
// (the agent-scope fences of the HIP memory model write back and invalidate whole L2s).
constexpr int kSc1 = 16;
#ifndef FDLLM_DECODE_STAGES
#define FDLLM_DECODE_STAGES 2
#endif
// tiles in flight per team in the split decode kernel: 2, or 3 (slower on the bs16 step:
// 25.9 against 25.35 us, more loads in flight slow the phase in which every workgroup streams)
constexpr int kDecodeStages = FDLLM_DECODE_STAGES;
// 1: the balanced split kernels number their slots XCD-major (decode_partition); on the
// bs16 sub-block decode step 27.27 us against 27.75 us in slot order.
// 1: the split prefill (full-block) shapes also take kv_prefill_ring_kernel (bs16
// full-block step 47.14 us against 47.7 us with kv_prefill_kernel).
#ifndef FDLLM_TIMELINE
#define FDLLM_TIMELINE 0
#endif
#ifndef FDLLM_PREFILL_RING_SPLIT
#define FDLLM_PREFILL_RING_SPLIT 1
#endif
#ifndef FDLLM_XCD_SLOTS
#define FDLLM_XCD_SLOTS 1
#endif
// Prefill workgroups have kPrefillWaves = 8 waves (x 32 query rows). Measured and not
// kept: 4 waves (two independent workgroups per CU, so that their softmax and MFMA phases
// drift apart): 549 us against 516-523 us for the 4 x 4096 prefill, the doubled K/V
// staging per thread pushed it to 256 VGPRs with spills.

struct AttnParams {
  const uint16_t* q;
  int64_t q_sb, q_ss, q_sh;
  const uint16_t* k;
  int64_t k_sp, k_ss, k_sh;
  const uint16_t* v;
  int64_t v_sp, v_ss, v_sh;
  uint16_t* out;
  int64_t o_sb, o_ss, o_sh;
  const int32_t* page_table;
  const int32_t* seqlens;
  const int32_t* q_start;
  int max_pages, page_size, page_shift, max_seqlen;  // page_size == 1 << page_shift
  int B, Sq, Hq, Hkv, G;
  int R;            // rows per (b, kv head) = Sq * G
  int rows_per_wg;  // 64 * MT
  int n_rb;         // row blocks per (b, kv head)
  int n_splits;     // split slots per row block (grid x); split decode: partial slots per KV head
  int chunk;        // keys per split, multiple of kKT; split decode: 0 = balanced partition
  int mask_mode, mask_block;
  float scale_log2;  // softmax_scale * log2(e)
  float* ws_o;       // [units, n_splits, rows_per_wg, D]
  float2* ws_ml;     // [units, n_splits, rows_per_wg]
  int* ws_cnt;       // [units] arrival counters of the split decode kernel (zero between calls)
  int2* ws_unit;     // [units] (first slot, splits) written by the split prefill kernel for its merge
  // fused cache write (prefill kernels): K / V rows of the Sq query tokens, [B, Sq, Hkv, D]
  // with strides (n_sb, n_ss, n_sh), stored into the cache at positions qs + t below `cap`
  const uint16_t* kn;
  const uint16_t* vn;
  int64_t n_sb, n_ss, n_sh;
  int cap;
#if FDLLM_TIMELINE
  uint64_t* tl;  // per-workgroup phase stamps (kTimelineStamps each), or null
#endif
};

// Phase stamps of the instrumented build (FDLLM_TIMELINE, built as a library of its
// own): thread 0 of each workgroup of the split decode kernel (and of the ring prefill
// kernel) writes the device's constant 100 MHz clock (s_memrealtime) at the ends of its
// phases into the buffer given to fdllm_timeline_attach, kTimelineStamps words per
// workgroup, indexed by the linear workgroup id. The production library has none of
// this code.
constexpr int kTimelineStamps = 8;
#if FDLLM_TIMELINE
#define FDLLM_STAMP(i, value)                                                                              \
  do {                                                                                                     \
    if (threadIdx.x == 0 && p.tl != nullptr)                                                               \
      p.tl[(blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z)) * kTimelineStamps + (i)] = (value); \
  } while (0)
#else
#define FDLLM_STAMP(i, value) \
  do {                        \
  } while (0)
#endif

template <bool F16>
__device__ __forceinline__ f32x4 mfma16x16x32(const u32x4& a, const u32x4& b, const f32x4& c) {
  if constexpr (F16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0,
                                                  0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                   0, 0);
  }
}

template <bool F16>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  if constexpr (F16) {
    return Elt<f16_t>::pack(a, b);
  } else {
    return Elt<bf16_t>::pack(a, b);
  }
}

// 2^x with the hardware transcendental (v_exp_f32): no denormal range fix-up;
// exp2(-inf) = 0, the softmax's masked value.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// ds_read_b64_tr_b16: transposing LDS read of four 16-bit values (see kv_decode_kernel).
__device__ __forceinline__ s16x4 lds_read_tr16(const uint16_t* lds_ptr) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(lds_ptr));
}

// Exclusive key bound for query token t of sequence b.
__device__ __forceinline__ int row_key_limit(const AttnParams& p, int seqlen, int qs, int t) {
  if (p.mask_mode == FDLLM_MASK_SEQLEN) return seqlen;
  const int qpos = qs + t;
  int lim;
  if (p.mask_mode == FDLLM_MASK_CAUSAL) {
    lim = qpos + 1;
  } else {
    lim = qpos >= 0 ? (qpos / p.mask_block + 1) * p.mask_block : 0;
  }
  return lim < seqlen ? lim : seqlen;
}

// Per (sequence, row block) facts shared by the attention and combine kernels.
struct SeqInfo {
  int seqlen;  // visible KV length after clamping to the cache capacity
  int qs;      // absolute position of query token 0
  int kv_end;  // keys any row of the row block may see
  int n_act;   // splits that hold at least one of those keys
};

// The arguments a kernel's first loads need (lengths, query starts, page table, and the
// batch and page-table sizes that bound those loads), passed ahead of AttnParams as
// scalars: with kernel-argument preloading they are in SGPRs when the waves start, so
// these loads go out without waiting for the argument segment to be read.
struct Lead {
  const int* seqlens;
  const int* q_start;
  const int32_t* page_table;
  int B;
  int max_pages;
};
#define FDLLM_LEAD_PARAMS \
  const int *lead_seqlens, const int *lead_q_start, const int32_t *lead_page_table, int lead_B, int lead_max_pages
#define FDLLM_LEAD_ARGS(p) (p).seqlens, (p).q_start, (p).page_table, (p).B, (p).max_pages
#define FDLLM_LEAD_LOCAL const Lead ld{lead_seqlens, lead_q_start, lead_page_table, lead_B, lead_max_pages}

__device__ __forceinline__ Lead lead_of(const AttnParams& p) {
  return Lead{p.seqlens, p.q_start, p.page_table, p.B, p.max_pages};
}

template <bool PAGED>
__device__ __forceinline__ SeqInfo seq_info(const AttnParams& p, const Lead& ld, int b, int rb) {
  SeqInfo si;
  // both loads issue before either is waited for (q_start falls back to a dummy read)
  int seqlen = ld.seqlens[b];
  const int qs_raw = (ld.q_start ? ld.q_start : ld.seqlens)[b];
  if (seqlen > p.max_seqlen) seqlen = p.max_seqlen;
  if (PAGED && seqlen > p.max_pages * p.page_size) seqlen = p.max_pages * p.page_size;
  if (seqlen < 0) seqlen = 0;
  si.seqlen = seqlen;
  si.qs = ld.q_start ? qs_raw : seqlen - p.Sq;
  const int row0 = rb * p.rows_per_wg;
  const int row_last = min(p.R, row0 + p.rows_per_wg) - 1;  // limits grow with t
  si.kv_end = max(0, row_key_limit(p, seqlen, si.qs, row_last / p.G));
  si.n_act = p.chunk > 0 ? (si.kv_end + p.chunk - 1) / p.chunk : 1;
  return si;
}

template <bool PAGED>
__device__ __forceinline__ SeqInfo seq_info(const AttnParams& p, int b, int rb) {
  return seq_info<PAGED>(p, lead_of(p), b, rb);
}

template <int D, int MT, bool F16, bool PAGED>
__global__ __launch_bounds__(kThreads, MT <= 2 ? 2 : 1) void kv_attn_kernel(const AttnParams p) {
  constexpr int KS = D + 8;      // K row stride in LDS (elements), 16-byte pad
  constexpr int VS = kKT + 4;    // V^T row stride in LDS (elements), 8-byte pad
  constexpr int NKS = D / 32;    // MFMA k-steps over d for S
  constexpr int NDT = D / 16;    // 16-wide d tiles of O
  constexpr int KCH = D / 8;     // 16-byte chunks per key row
  constexpr int KLD = kKT * KCH / kThreads;  // K 16-byte loads per thread per tile
  static_assert(KLD >= 1, "tile too small");
  __shared__ __attribute__((aligned(16))) uint16_t sK[kKT * KS];
  __shared__ __attribute__((aligned(16))) uint16_t sVt[D * VS];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int l16 = lane & 15;
  const int g = lane >> 4;

  const int split = blockIdx.x;
  const int rb = p.n_rb - 1 - static_cast<int>(blockIdx.y);  // heaviest row blocks first under causal masks
  const int bh = blockIdx.z;
  const int b = bh / p.Hkv;
  const int kvh = bh - b * p.Hkv;
  const int unit = bh * p.n_rb + rb;

  const SeqInfo si = seq_info<PAGED>(p, b, rb);
  if (split >= max(si.n_act, 1)) return;
  const int row0 = rb * p.rows_per_wg;
  const int k_lo = split * p.chunk;
  const int k_hi = min(si.kv_end, k_lo + p.chunk);
  const int ntiles = k_hi > k_lo ? (k_hi - k_lo + kKT - 1) / kKT : 0;

  // ---- per-lane query rows, Q fragments (B operand of S^T = K Q^T), row limits
  u32x4 qf[MT][NKS];
  int lim[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int r = row0 + (wave * MT + mt) * 16 + l16;
    const int rc = min(r, p.R - 1);  // padding rows read a valid row; their limit is 0
    const int t = rc / p.G;
    const int hh = rc - t * p.G;
    // padding rows (r >= R) reuse a valid row's query and limit: finite, never written
    lim[mt] = row_key_limit(p, si.seqlen, si.qs, t);
    const uint16_t* qrow = p.q + b * p.q_sb + t * p.q_ss + (kvh * p.G + hh) * p.q_sh;
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) qf[mt][ks] = *reinterpret_cast<const u32x4*>(qrow + ks * 32 + g * 8);
  }

  // tiles wholly below every row limit of this wave need no mask
  int lim_min = lim[0];
#pragma unroll
  for (int mt = 1; mt < MT; ++mt) lim_min = min(lim_min, lim[mt]);
  lim_min = __builtin_amdgcn_readfirstlane(-static_cast<int>(wave_allreduce_max(-static_cast<float>(lim_min))));

  f32x4 acc[MT][NDT];
  float m_run[MT], l_run[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    m_run[mt] = -INFINITY;
    l_run[mt] = 0.f;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) acc[mt][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // ---- global -> register staging. Loads are unconditional: keys at or past
  // k_hi are clamped to k_hi - 1, a valid key whose score is masked to -inf
  // (p = 0 against finite data), so no branch separates a tile's loads.
  constexpr bool kVAll = (kThreads / 16) == KCH;  // every thread stages V (D == 128)
  const int v_kq = tid & 15;  // key quad
  const int v_dq = tid >> 4;  // d octet
  const bool v_active = kVAll || v_dq < KCH;
  const int32_t* pt_row = PAGED ? p.page_table + static_cast<int64_t>(b) * p.max_pages : nullptr;

  struct Stage {
    u32x4 k[KLD];
    u32x4 v[4];
  };
  // Pages of the keys this thread stages for one tile (paged pools). Page sizes
  // are powers of two >= 16, so each aligned 16-key group of K lives in one page
  // (the same for the whole workgroup: scalar loads) and each aligned 4-key group
  // of V in one page (one id per lane). Clamping stays inside the group.
  struct Rows {
    int kpg[KLD];
    int vpg;
  };
  Stage st0;
  Stage st1;  // unused (and removed by the compiler) when kDepth == 1
  Rows rs0, rs1;  // unused without a page table

  auto kkey = [&](int kb, int i) { return min(kb + (tid + kThreads * i) / KCH, k_hi - 1); };
  auto vkey = [&](int kb, int r) { return min(kb + v_kq * 4 + r, k_hi - 1); };
  auto resolve = [&](Rows& rs, int kb) {
    if constexpr (PAGED) {
#pragma unroll
      for (int i = 0; i < KLD; ++i) {
        // keys kb + i * (kThreads / KCH) + tid / KCH: one aligned group of kThreads / KCH
        // keys per i (16 for D == 128, 32 for D == 64); the host requires
        // page_size >= kThreads / KCH so the group sits in one page
        const int k0 = min(kb + i * (kThreads / KCH), k_hi - 1);
        rs.kpg[i] = pt_row[k0 >> p.page_shift];
      }
      rs.vpg = pt_row[min(kb + v_kq * 4, k_hi - 1) >> p.page_shift];
    }
  };
  auto row_off = [&](int key, int page, int64_t sp, int64_t ss) -> int64_t {
    if constexpr (PAGED) {
      return static_cast<int64_t>(page) * sp + (key & (p.page_size - 1)) * ss;
    } else {
      return b * sp + key * ss;
    }
  };
  auto load_tile = [&](Stage& st, const Rows& rs, int kb) {
#pragma unroll
    for (int i = 0; i < KLD; ++i) {
      const int dc = (tid + kThreads * i) % KCH;
      st.k[i] = *reinterpret_cast<const u32x4*>(p.k + row_off(kkey(kb, i), rs.kpg[i], p.k_sp, p.k_ss) +
                                                kvh * p.k_sh + dc * 8);
    }
    if (v_active) {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        st.v[r] = *reinterpret_cast<const u32x4*>(p.v + row_off(vkey(kb, r), rs.vpg, p.v_sp, p.v_ss) +
                                                  kvh * p.v_sh + v_dq * 8);
    }
  };
  auto store_tile = [&](const Stage& st) {
#pragma unroll
    for (int i = 0; i < KLD; ++i) {
      const int c = tid + kThreads * i;
      *reinterpret_cast<u32x4*>(&sK[(c / KCH) * KS + (c % KCH) * 8]) = st.k[i];
    }
    if (v_active) {
      // 4 keys x 8 d  ->  8 rows of V^T, 4 consecutive keys each (8 bytes)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int w = e >> 1;
        uint32_t lo, hi;
        if (e & 1) {
          lo = (st.v[0][w] >> 16) | (st.v[1][w] & 0xffff0000u);
          hi = (st.v[2][w] >> 16) | (st.v[3][w] & 0xffff0000u);
        } else {
          lo = (st.v[0][w] & 0xffffu) | (st.v[1][w] << 16);
          hi = (st.v[2][w] & 0xffffu) | (st.v[3][w] << 16);
        }
        *reinterpret_cast<u32x2*>(&sVt[(v_dq * 8 + e) * VS + v_kq * 4]) = u32x2{lo, hi};
      }
    }
  };

  // ---- one 64-key tile from LDS: S^T = K Q^T, online softmax, O^T += V^T P^T
  auto compute_tile = [&](int kb) {
    f32x4 s[MT][4];
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      u32x4 kf[NKS];
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks)
        kf[ks] = *reinterpret_cast<const u32x4*>(&sK[(st * 16 + l16) * KS + ks * 32 + g * 8]);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        f32x4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) c = mfma16x16x32<F16>(kf[ks], qf[mt][ks], c);
        s[mt][st] = c;
      }
    }
    // lane owns query row l16 of each M-tile; its 16 scores sit at keys kb + 16st + 4g + j.
    // Scores stay unscaled; scale * log2(e) is folded into the exponent's FMA.
    const bool full_tile = kb + kKT <= lim_min;  // wave-uniform
    u32x4 pf[MT][2];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      if (!full_tile) {
#pragma unroll
        for (int st = 0; st < 4; ++st)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (kb + st * 16 + g * 4 + j >= lim[mt]) s[mt][st][j] = -INFINITY;
      }
      float tmax = -INFINITY;
#pragma unroll
      for (int st = 0; st < 4; ++st)
#pragma unroll
        for (int j = 0; j < 4; ++j) tmax = fmaxf(tmax, s[mt][st][j]);
      tmax = group4_allreduce_max(tmax);
      const float m_new = fmaxf(m_run[mt], tmax);
      // Rescale the accumulators only when some lane's running max moved; alpha is
      // exactly 1 for every other lane, so skipping is exact.
      if (__builtin_amdgcn_ballot_w64(m_new > m_run[mt]) != 0) {
        const float alpha = m_new == -INFINITY ? 1.f : fast_exp2((m_run[mt] - m_new) * p.scale_log2);
        l_run[mt] *= alpha;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) acc[mt][dt] *= alpha;
        m_run[mt] = m_new;
      }
      const float mc = m_new == -INFINITY ? 0.f : m_new * p.scale_log2;
      float lsum = 0.f;
#pragma unroll
      for (int st = 0; st < 4; ++st) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float e = fast_exp2(fmaf(s[mt][st][j], p.scale_log2, -mc));
          s[mt][st][j] = e;
          lsum += e;
        }
      }
      l_run[mt] += lsum;
      // B operand of O^T = V^T P^T for key steps kk = 0, 1:
      // k-index 8g + j <-> key 32kk + 4g + j (j < 4), 32kk + 16 + 4g + (j - 4) (j >= 4)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        pf[mt][kk][0] = pack2<F16>(s[mt][2 * kk][0], s[mt][2 * kk][1]);
        pf[mt][kk][1] = pack2<F16>(s[mt][2 * kk][2], s[mt][2 * kk][3]);
        pf[mt][kk][2] = pack2<F16>(s[mt][2 * kk + 1][0], s[mt][2 * kk + 1][1]);
        pf[mt][kk][3] = pack2<F16>(s[mt][2 * kk + 1][2], s[mt][2 * kk + 1][3]);
      }
    }
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        const uint16_t* vrow = &sVt[(dt * 16 + l16) * VS + kk * 32 + g * 4];
        const u32x2 lo = *reinterpret_cast<const u32x2*>(vrow);
        const u32x2 hi = *reinterpret_cast<const u32x2*>(vrow + 16);
        const u32x4 vf = {lo[0], lo[1], hi[0], hi[1]};
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[mt][dt] = mfma16x16x32<F16>(vf, pf[mt][kk], acc[mt][dt]);
      }
    }
  };

  // Prefetch depth: decode-shaped workgroups (MT <= 2) keep two tiles in flight;
  // MT == 4 (prefill) has 4x the math per tile, which hides a one-tile prefetch,
  // and not the registers for a second stage.
  constexpr int kDepth = MT <= 2 ? 2 : 1;
  // At step t the page ids of tile t + kDepth + 1 are requested first, then the
  // loads of tile t + kDepth, so waiting for the page ids one step later never
  // waits for those tile loads (vmcnt retires in issue order). Every step issues
  // the same loads whether or not the tiles exist (keys clamp to k_hi - 1, so
  // surplus loads re-read one cached row): the number of loads in flight is the
  // same on every path, which lets the compiler wait for exactly the stage it
  // needs instead of draining the prefetch. Only the LDS math is conditional.
  auto step = [&](Stage& st, Rows& rs_load, Rows& rs_resolve, int t) {
    lds_barrier();  // every wave is done reading the previous tile
    store_tile(st);
    lds_barrier();
    resolve(rs_resolve, k_lo + (t + kDepth + 1) * kKT);
    load_tile(st, rs_load, k_lo + (t + kDepth) * kKT);
    if (t < ntiles) compute_tile(k_lo + t * kKT);
  };

  if (ntiles > 0) {
    if constexpr (kDepth == 2) {
      // tile t in stage t % 2; pages of tile t + 2 in rs[t % 2]
      resolve(rs0, k_lo);
      resolve(rs1, k_lo + kKT);
      load_tile(st0, rs0, k_lo);
      load_tile(st1, rs1, k_lo + kKT);
      resolve(rs0, k_lo + 2 * kKT);
      for (int t = 0; t < ntiles; t += 2) {
        step(st0, rs0, rs1, t);
        step(st1, rs1, rs0, t + 1);
      }
    } else {
      // one stage; pages of tile t + 1 in rs[(t + 1) % 2]
      resolve(rs0, k_lo);
      load_tile(st0, rs0, k_lo);
      resolve(rs1, k_lo + kKT);
      for (int t = 0; t < ntiles; t += 2) {
        step(st0, rs1, rs0, t);
        step(st0, rs0, rs1, t + 1);
      }
    }
  }

  // ---- epilogue
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) l_run[mt] = group4_allreduce_sum(l_run[mt]);

  if (si.n_act <= 1) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int r = row0 + (wave * MT + mt) * 16 + l16;
      if (r >= p.R) continue;
      const int t = r / p.G;
      const int hh = r - t * p.G;
      const float inv = l_run[mt] > 0.f ? 1.f / l_run[mt] : 0.f;
      uint16_t* orow = p.out + b * p.o_sb + t * p.o_ss + (kvh * p.G + hh) * p.o_sh;
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        const f32x4 o = acc[mt][dt] * inv;
        *reinterpret_cast<u32x2*>(orow + dt * 16 + g * 4) = u32x2{pack2<F16>(o[0], o[1]), pack2<F16>(o[2], o[3])};
      }
    }
    return;
  }

  // split: publish this workgroup's unnormalised partial for the combine kernel
  const int64_t slot = static_cast<int64_t>(unit) * p.n_splits + split;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int rl = (wave * MT + mt) * 16 + l16;
    float* po = p.ws_o + (slot * p.rows_per_wg + rl) * D;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) *reinterpret_cast<f32x4*>(po + dt * 16 + g * 4) = acc[mt][dt];
    if (g == 0) p.ws_ml[slot * p.rows_per_wg + rl] = make_float2(m_run[mt], l_run[mt]);
  }
}

// ---------------------------------------------------------------------------
// Decode-shaped attention: every KV head of a key range in one workgroup.
//
// For q_len * G <= 64 rows per KV head and head_dim 128 with the heads of one
// key stored next to each other (the [.., Hkv, D] cache rows of
// static_kv_cache.py, or a page pool [pages, page_size, Hkv, D]), a workgroup of
// 2 * HKV waves streams whole key rows (HKV * 256 bytes) of its split: each
// 16-byte load instruction of a wave covers one contiguous row, which is what
// HBM serves best, and every byte feeds the G query heads of its KV head.
//   * Tiles of 32 keys; K and V land in LDS row-major with plain 16-byte stores.
//   * Wave w works on KV head w / 2, query rows 32 * (w % 2) .. +32 (2 M-tiles).
//   * S^T = K Q^T as in kv_attn_kernel; the V^T operand of O^T = V^T P^T is read
//     with ds_read_b64_tr_b16 (gfx950 LDS transpose read): in each 16-lane group,
//     lane j receives element j % 4 of lanes 4k + j / 4 (k = 0..3), so a lane
//     addressing V[kb + l16 / 4][16 dt + 4 (l16 % 4)] receives the four keys
//     kb .. kb + 3 at d = 16 dt + l16.
//   * Partials use the layout of kv_attn_kernel with rows_per_wg = 64, so the
//     same combine kernel merges the splits.
template <int HKV, bool F16, bool PAGED>
__global__ __launch_bounds__(128 * HKV) void kv_decode_kernel(const AttnParams p) {
  constexpr int D = 128;
  constexpr int NT = 128 * HKV;
  constexpr int KT = 32;
  constexpr int ROWE = HKV * D;       // elements of one key row (all heads)
  constexpr int KS = ROWE + 8;        // K row stride in LDS: +16 bytes (conflict-free b128 reads)
  constexpr int VS = ROWE + 16;       // V row stride in LDS: +32 bytes (conflict-free transpose reads)
  constexpr int CPR = ROWE / 8;       // 16-byte chunks per key row
  constexpr int LPT = KT * CPR / NT;  // 16-byte loads per thread per tile, per tensor
  constexpr int NDT = D / 16;
  static_assert(LPT == 4, "tile shape");
  __shared__ __attribute__((aligned(16))) uint16_t sK[KT * KS];
  __shared__ __attribute__((aligned(16))) uint16_t sV[KT * VS];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int l16 = lane & 15;
  const int g = lane >> 4;
  const int h = wave >> 1;
  const int half = wave & 1;

  const int split = blockIdx.x;
  const int b = blockIdx.y;
  const SeqInfo si = seq_info<PAGED>(p, b, 0);
  if (split >= max(si.n_act, 1)) return;
  const int k_lo = split * p.chunk;
  const int k_hi = min(si.kv_end, k_lo + p.chunk);
  const int ntiles = k_hi > k_lo ? (k_hi - k_lo + KT - 1) / KT : 0;

  // ---- query fragments of this wave's 32 rows (2 M-tiles) of head h
  u32x4 qf[2][4];
  int lim[2];
#pragma unroll
  for (int mt = 0; mt < 2; ++mt) {
    const int r = half * 32 + mt * 16 + l16;
    const int rc = min(r, p.R - 1);  // padding rows reuse a valid row: finite, never written
    const int t = rc / p.G;
    const int hh = rc - t * p.G;
    lim[mt] = row_key_limit(p, si.seqlen, si.qs, t);
    const uint16_t* qrow = p.q + b * p.q_sb + t * p.q_ss + (h * p.G + hh) * p.q_sh;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) qf[mt][ks] = *reinterpret_cast<const u32x4*>(qrow + ks * 32 + g * 8);
  }
  int lim_min = min(lim[0], lim[1]);
  lim_min = __builtin_amdgcn_readfirstlane(-static_cast<int>(wave_allreduce_max(-static_cast<float>(lim_min))));
  const float rescale_thr = 8.f / p.scale_log2;  // raw-score distance of a 2^8 factor

  f32x4 acc[2][NDT];
  float m_run[2], l_run[2];
#pragma unroll
  for (int mt = 0; mt < 2; ++mt) {
    m_run[mt] = -INFINITY;
    l_run[mt] = 0.f;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) acc[mt][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // ---- staging: chunk c = tid + NT * i of the tile -> key c / CPR, column (c % CPR) * 8.
  // Buffer loads: the descriptor (scalar) points at the tile's first key and covers
  // only the keys below k_hi, so keys past the end read as zero with no clamping;
  // each thread's byte offsets inside a tile are the same for every tile.
  struct Stage {
    u32x4 k[LPT];
    u32x4 v[LPT];
  };
  Stage st0, st1;
  const int32_t* pt_row = PAGED ? p.page_table + static_cast<int64_t>(b) * p.max_pages : nullptr;
  const int krow_bytes = static_cast<int>(p.k_ss) * 2;
  const int vrow_bytes = static_cast<int>(p.v_ss) * 2;
  int koff[LPT], voff[LPT];
#pragma unroll
  for (int i = 0; i < LPT; ++i) {
    const int c = tid + NT * i;
    koff[i] = (c / CPR) * krow_bytes + (c % CPR) * 16;
    voff[i] = (c / CPR) * vrow_bytes + (c % CPR) * 16;
  }
  auto load_tile = [&](Stage& st, int kb) {
    // every value the descriptors are built from is wave-uniform; readfirstlane
    // states it, so the descriptors live in scalar registers
    const int valid = __builtin_amdgcn_readfirstlane(max(0, min(KT, k_hi - kb)));
    const uint16_t* kt;
    const uint16_t* vt;
    if constexpr (PAGED) {
      // a 32-key tile lies in one page (page_size is a power of two >= 32)
      const int page = __builtin_amdgcn_readfirstlane(pt_row[min(kb, k_hi - 1) >> p.page_shift]);
      const int slot0 = kb & (p.page_size - 1);
      kt = p.k + static_cast<int64_t>(page) * p.k_sp + static_cast<int64_t>(slot0) * p.k_ss;
      vt = p.v + static_cast<int64_t>(page) * p.v_sp + static_cast<int64_t>(slot0) * p.v_ss;
    } else {
      kt = p.k + b * p.k_sp + static_cast<int64_t>(kb) * p.k_ss;
      vt = p.v + b * p.v_sp + static_cast<int64_t>(kb) * p.v_ss;
    }
    const __amdgpu_buffer_rsrc_t kr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(kt), 0, valid * krow_bytes, kBufferFlags);
    const __amdgpu_buffer_rsrc_t vr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(vt), 0, valid * vrow_bytes, kBufferFlags);
#pragma unroll
    for (int i = 0; i < LPT; ++i) {
      st.k[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(kr, koff[i], 0, 0));
      st.v[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(vr, voff[i], 0, 0));
    }
  };
  auto store_tile = [&](const Stage& st) {
#pragma unroll
    for (int i = 0; i < LPT; ++i) {
      const int c = tid + NT * i;
      *reinterpret_cast<u32x4*>(&sK[(c / CPR) * KS + (c % CPR) * 8]) = st.k[i];
      *reinterpret_cast<u32x4*>(&sV[(c / CPR) * VS + (c % CPR) * 8]) = st.v[i];
    }
  };

  auto compute_tile = [&](int kb) {
    // S^T for two 16-key sub-tiles
    f32x4 s[2][2];
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      u32x4 kf[4];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
        kf[ks] = *reinterpret_cast<const u32x4*>(&sK[(st * 16 + l16) * KS + h * D + ks * 32 + g * 8]);
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        f32x4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) c = mfma16x16x32<F16>(kf[ks], qf[mt][ks], c);
        s[mt][st] = c;
      }
    }
    const bool full_tile = kb + KT <= lim_min;  // wave-uniform
    u32x4 pf[2];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      if (!full_tile) {
#pragma unroll
        for (int st = 0; st < 2; ++st)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (kb + st * 16 + g * 4 + j >= lim[mt]) s[mt][st][j] = -INFINITY;
      }
      float tmax = -INFINITY;
#pragma unroll
      for (int st = 0; st < 2; ++st)
#pragma unroll
        for (int j = 0; j < 4; ++j) tmax = fmaxf(tmax, s[mt][st][j]);
      tmax = group4_allreduce_max(tmax);
      // The reference max m_run only moves when a score exceeds it by more than
      // 2^8 in the exponent (or on the first visible key): exponentials stay <= 256,
      // far from fp32 / bf16 overflow, and the result is the same function.
      if (__builtin_amdgcn_ballot_w64(tmax > m_run[mt] + rescale_thr) != 0) {
        const float m_new = fmaxf(m_run[mt], tmax);
        const float alpha = m_run[mt] == -INFINITY ? 0.f : fast_exp2((m_run[mt] - m_new) * p.scale_log2);
        l_run[mt] *= alpha;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) acc[mt][dt] *= alpha;
        m_run[mt] = m_new;
      }
      const float mc = m_run[mt] == -INFINITY ? 0.f : m_run[mt] * p.scale_log2;
      float lsum = 0.f;
#pragma unroll
      for (int st = 0; st < 2; ++st) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float e = fast_exp2(fmaf(s[mt][st][j], p.scale_log2, -mc));
          s[mt][st][j] = e;
          lsum += e;
        }
      }
      l_run[mt] += lsum;
      // k-index 8g + j <-> key 4g + j (j < 4), 16 + 4g + (j - 4) (j >= 4)
      pf[mt][0] = pack2<F16>(s[mt][0][0], s[mt][0][1]);
      pf[mt][1] = pack2<F16>(s[mt][0][2], s[mt][0][3]);
      pf[mt][2] = pack2<F16>(s[mt][1][0], s[mt][1][1]);
      pf[mt][3] = pack2<F16>(s[mt][1][2], s[mt][1][3]);
    }
    // O^T += V^T P^T; V^T fragments by LDS transpose reads of row-major V
    const int vrow = 4 * g + (l16 >> 2);
    const int vcol = h * D + 4 * (l16 & 3);
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      const s16x4 lo = lds_read_tr16(&sV[vrow * VS + vcol + dt * 16]);
      const s16x4 hi = lds_read_tr16(&sV[(vrow + 16) * VS + vcol + dt * 16]);
      const u32x2 lo2 = __builtin_bit_cast(u32x2, lo);
      const u32x2 hi2 = __builtin_bit_cast(u32x2, hi);
      const u32x4 vf = {lo2[0], lo2[1], hi2[0], hi2[1]};
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) acc[mt][dt] = mfma16x16x32<F16>(vf, pf[mt], acc[mt][dt]);
    }
  };

  // Two tiles in flight (see kv_attn_kernel): every step issues the same loads,
  // zero-filled past k_hi, so the waits stay exact; only the math is conditional.
  auto step = [&](Stage& st, int t) {
    lds_barrier();
    store_tile(st);
    lds_barrier();
    load_tile(st, k_lo + (t + 2) * KT);
    if (t < ntiles) compute_tile(k_lo + t * KT);
  };
  if (ntiles > 0) {
    load_tile(st0, k_lo);
    load_tile(st1, k_lo + KT);
    for (int t = 0; t < ntiles; t += 2) {
      step(st0, t);
      step(st1, t + 1);
    }
  }

  // ---- epilogue
#pragma unroll
  for (int mt = 0; mt < 2; ++mt) l_run[mt] = group4_allreduce_sum(l_run[mt]);
  if (si.n_act <= 1) {
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      const int r = half * 32 + mt * 16 + l16;
      if (r >= p.R) continue;
      const int t = r / p.G;
      const int hh = r - t * p.G;
      const float inv = l_run[mt] > 0.f ? 1.f / l_run[mt] : 0.f;
      uint16_t* orow = p.out + b * p.o_sb + t * p.o_ss + (h * p.G + hh) * p.o_sh;
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        const f32x4 o = acc[mt][dt] * inv;
        *reinterpret_cast<u32x2*>(orow + dt * 16 + g * 4) = u32x2{pack2<F16>(o[0], o[1]), pack2<F16>(o[2], o[3])};
      }
    }
    return;
  }
  const int64_t slot = static_cast<int64_t>(b * p.Hkv + h) * p.n_splits + split;
#pragma unroll
  for (int mt = 0; mt < 2; ++mt) {
    const int rl = half * 32 + mt * 16 + l16;
    if (rl >= p.R) continue;  // padding rows are never read
    float* po = p.ws_o + (slot * 64 + rl) * D;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) *reinterpret_cast<f32x4*>(po + dt * 16 + g * 4) = acc[mt][dt];
    if (g == 0) p.ws_ml[slot * 64 + rl] = make_float2(m_run[mt], l_run[mt]);
  }
}

// Inclusive prefix sum over the 64 lanes of a wave with DPP moves: shifts by 1,
// 2, 4 and 8 within each 16-lane row, then the running totals of rows 0 and 1
// broadcast into the rows above them (row_bcast:15 into rows 1 and 3, row_bcast:31
// into rows 2 and 3). Lanes whose DPP source lies outside the row add 0.
__device__ __forceinline__ int wave_incl_scan_i32(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false);  // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);  // row_bcast:15
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);  // row_bcast:31
  return v;
}
__device__ __forceinline__ int wave_sum_i32(int v) {
  return __builtin_amdgcn_readlane(wave_incl_scan_i32(v), 63);
}

// ceil(a / b) for 0 <= a < 2^20 and 1 <= b < 2^20: the float quotient is within
// 0.25 of a / b, its truncation at most one below floor(a / b), and two exact
// integer corrections reach the ceiling.
__device__ __forceinline__ int ceil_div_small(int a, int b) {
  int q = static_cast<int>(static_cast<float>(a) * __builtin_amdgcn_rcpf(static_cast<float>(b)));
  q += q * b < a;
  q += q * b < a;
  return q;
}

// Key range of one workgroup of the split decode kernel.
struct DecodePart {
  int b;       // sequence, -1 for an idle workgroup
  int split;   // index of the split within the sequence
  int n_act;   // splits of the sequence (1: the workgroup writes the output itself)
  int first;   // partial slot of split 0 of the sequence for this workgroup's KV head
  int seqlen, qs, kv_end;
  int k_lo, k_hi;
};

// Sequence of t tiles in n splits of equal size: the splits that hold keys.
__device__ __forceinline__ int active_splits(int t, int n) {
  if (t <= 0) return 1;
  return ceil_div_small(t, ceil_div_small(t, n));
}

// Partition of every sequence's keys into splits of equal size (whole TILE-key tiles).
//   * Fixed (chunk > 0, grid (n_splits, Hkv, B)): sequence b gets
//     n = ceil(tiles / chunk tiles) splits, capped at kMaxDecodeSplits.
//   * Balanced (chunk == 0, B <= 64, grid (S, Hkv, 1)): sequence b gets
//     n_b = min(kMaxDecodeSplits, ceil(t_b / C)) splits, with C the smallest tile
//     count per split (>= 4) for which the splits of all sequences fit in the S
//     slots; the slots are handed out in sequence order. The cost of one workgroup
//     is then at most C tiles whatever the mix of lengths, where a per-sequence
//     chunk gives the short sequences half-empty workgroups. Every workgroup
//     evaluates the same integer search (binary, on one wave's lanes, one lane per
//     sequence), so all of them agree on the partition.
template <bool PAGED, int TILE = 32>
__device__ __forceinline__ DecodePart decode_partition(const AttnParams& p, const Lead& ld) {
  DecodePart dp;
  if (p.chunk > 0) {
    dp.b = blockIdx.z;
    dp.split = blockIdx.x;
    const SeqInfo si = seq_info<PAGED>(p, ld, dp.b, 0);
    const int t = (si.kv_end + TILE - 1) / TILE;
    const int ct = p.chunk / TILE;
    const int n = max(1, min(kMaxDecodeSplits, (t + ct - 1) / ct));
    const int size = (t + n - 1) / n;
    dp.n_act = active_splits(t, n);
    dp.first = (blockIdx.y * p.B + dp.b) * p.n_splits;  // n_splits slots per (KV head, sequence)
    dp.seqlen = si.seqlen;
    dp.qs = si.qs;
    dp.kv_end = si.kv_end;
    dp.k_lo = dp.split * size * TILE;
    dp.k_hi = min(si.kv_end, dp.k_lo + size * TILE);
    if (dp.split >= dp.n_act) dp.b = -1;
    return dp;
  }
  const int lane = threadIdx.x & 63;
  const bool has = lane < ld.B;
  SeqInfo sl;
  sl.seqlen = sl.qs = sl.kv_end = 0;
  if (has) sl = seq_info<PAGED>(p, ld, lane, 0);
  const int t = (sl.kv_end + TILE - 1) / TILE;
  const int S = p.n_splits;
  // splits of a sequence for C tiles per split (an empty sequence still takes one
  // slot); the count over-estimates only where the cap of kMaxDecodeSplits bites
  auto splits_of = [&](int C) { return max(1, min(kMaxDecodeSplits, ceil_div_small(t, C))); };
  auto count = [&](int C) { return wave_sum_i32(has ? splits_of(C) : 0); };
  const int T = wave_sum_i32(t);
  // C = ceil(T / S) is a lower bound; ceil(T / (S - B)) fits, as each sequence
  // rounds up by less than one split (the host sizes S so that C = 160 fits).
  const int nb = min(ld.B, 64);
  int lo = min(kDecodeMaxTiles, max(4, ceil_div_small(T, S)));
  int hi = S > nb ? min(kDecodeMaxTiles, max(lo, ceil_div_small(T, S - nb))) : kDecodeMaxTiles;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (count(mid) <= S) hi = mid;
    else lo = mid + 1;
  }
  const int n_split = splits_of(lo);
  const int n_l = has ? active_splits(t, n_split) : 0;
  const int size_l = t > 0 ? ceil_div_small(t, n_split) : 0;
  const int incl = wave_incl_scan_i32(n_l);
#if FDLLM_XCD_SLOTS
  // slots in XCD-major order: workgroups are dealt to the 8 XCDs round-robin by linear
  // id (x + S y here), so with S a multiple of 8 the workgroups of XCD j take slots
  // j S / 8 .. (j + 1) S / 8 - 1, and the consecutive splits of one sequence share an
  // L2 (their query rows are fetched from memory once)
  const int slot = (S & 7) == 0 ? static_cast<int>(blockIdx.x & 7) * (S >> 3) + static_cast<int>(blockIdx.x >> 3)
                                : static_cast<int>(blockIdx.x);
#else
  const int slot = blockIdx.x;
#endif
  const uint64_t mine = __builtin_amdgcn_ballot_w64(has && incl > slot);
  if (mine == 0) {
    dp.b = -1;
    return dp;
  }
  const int b = static_cast<int>(__builtin_ctzll(mine));
  dp.b = b;
  dp.n_act = __builtin_amdgcn_readlane(n_l, b);
  const int first = __builtin_amdgcn_readlane(incl, b) - dp.n_act;
  dp.split = slot - first;
  dp.first = blockIdx.y * S + first;  // S slots per KV head
  dp.seqlen = __builtin_amdgcn_readlane(sl.seqlen, b);
  dp.qs = __builtin_amdgcn_readlane(sl.qs, b);
  dp.kv_end = __builtin_amdgcn_readlane(sl.kv_end, b);
  const int size = __builtin_amdgcn_readlane(size_l, b);
  dp.k_lo = dp.split * size * TILE;
  dp.k_hi = min(dp.kv_end, dp.k_lo + size * TILE);
  return dp;
}

// Merge of the split partials of one (sequence, KV head) unit. One work item per
// (row, 16 columns), so the 64-row worst case takes one pass of 512 threads; the
// splits are folded in groups of GS whose loads are all issued before any is used
// (one memory round trip per group), with the running maximum moved between groups.
// merge_splits_n picks GS = n_act up to eight (equal groups beyond): loads of splits past
// n_act would read zero without memory traffic, but each still takes the texture unit's
// address cycles.
template <bool F16, int RS = 64, int AUX = kSc1, int GS = 8>  // RS: partial rows per slot; AUX: load cache policy
__device__ __forceinline__ void merge_splits(const AttnParams& p, int b, int kvh, int64_t slot0, int n_act, int tid,
                                             int nthreads, int item_end = -1) {
  constexpr int D = 128;
  const int iend = item_end < 0 ? p.R * 8 : item_end;
  const auto orsrc = __builtin_amdgcn_make_buffer_rsrc(p.ws_o + slot0 * RS * D, 0, n_act * RS * D * 4, kBufferFlags);
  const auto mrsrc = __builtin_amdgcn_make_buffer_rsrc(p.ws_ml + slot0 * RS, 0, n_act * RS * 8, kBufferFlags);
  for (int item = tid; item < iend; item += nthreads) {
    // columns 4 c8 + 32 j + (0..3), j = 0..3: the eight threads of a row read 128
    // contiguous bytes per load
    const int r = item >> 3;
    const int c8 = (item & 7) * 4;
    float m = -INFINITY, l = 0.f;
    f32x4 o[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) o[j] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int s0 = 0; s0 < n_act; s0 += GS) {
      float2 ml[GS];
      f32x4 x[GS][4];
#pragma unroll
      for (int u = 0; u < GS; ++u) {
        // splits past n_act read as zero (outside the descriptor) and weigh nothing
        const int row = (s0 + u) * RS + r;
        ml[u] = __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(mrsrc, row * 8, 0, AUX));
#pragma unroll
        for (int j = 0; j < 4; ++j)
          x[u][j] = __builtin_bit_cast(
              f32x4, __builtin_amdgcn_raw_buffer_load_b128(orsrc, (row * D + c8 + 32 * j) * 4, 0, AUX));
      }
      float mg = m;
#pragma unroll
      for (int u = 0; u < GS; ++u)
        if (s0 + u < n_act) mg = fmaxf(mg, ml[u].x);
      if (mg == -INFINITY) continue;  // nothing seen yet
      const float a = m == -INFINITY ? 0.f : fast_exp2((m - mg) * p.scale_log2);
      l *= a;
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] *= a;
#pragma unroll
      for (int u = 0; u < GS; ++u) {
        const float w = (s0 + u < n_act && ml[u].x != -INFINITY) ? fast_exp2((ml[u].x - mg) * p.scale_log2) : 0.f;
        l += w * ml[u].y;
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] += w * x[u][j];
      }
      m = mg;
    }
    const float inv = l > 0.f ? 1.f / l : 0.f;
    const int t = r / p.G;
    const int hh = r - t * p.G;
    uint16_t* orow = p.out + b * p.o_sb + t * p.o_ss + (kvh * p.G + hh) * p.o_sh + c8;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      *reinterpret_cast<u32x2*>(orow + 32 * j) =
          u32x2{pack2<F16>(o[j][0] * inv, o[j][1] * inv), pack2<F16>(o[j][2] * inv, o[j][3] * inv)};
  }
}

template <bool F16, int RS = 64, int AUX = kSc1>
__device__ __forceinline__ void merge_splits_n(const AttnParams& p, int b, int kvh, int64_t slot0, int n_act,
                                               int tid, int nthreads, int item_end = -1) {
  // groups of equal size, at most eight: 9 splits take two groups of five, not 8 + 1
  const int groups = (n_act + 7) >> 3;
  switch ((n_act + groups - 1) / groups) {  // uniform over the workgroup
    case 2: merge_splits<F16, RS, AUX, 2>(p, b, kvh, slot0, n_act, tid, nthreads, item_end); break;
    case 3: merge_splits<F16, RS, AUX, 3>(p, b, kvh, slot0, n_act, tid, nthreads, item_end); break;
    case 4: merge_splits<F16, RS, AUX, 4>(p, b, kvh, slot0, n_act, tid, nthreads, item_end); break;
    case 5: merge_splits<F16, RS, AUX, 5>(p, b, kvh, slot0, n_act, tid, nthreads, item_end); break;
    case 6: merge_splits<F16, RS, AUX, 6>(p, b, kvh, slot0, n_act, tid, nthreads, item_end); break;
    case 7: merge_splits<F16, RS, AUX, 7>(p, b, kvh, slot0, n_act, tid, nthreads, item_end); break;
    default: merge_splits<F16, RS, AUX, 8>(p, b, kvh, slot0, n_act, tid, nthreads, item_end); break;
  }
}

// ---------------------------------------------------------------------------
// Split-KV decode attention, one (sequence, KV head, key range) per workgroup.
//
// The shape of the sub-block decode step: q_len * G <= 64 query rows share one
// KV head, head_dim 128. Each sequence's keys are split over several workgroups
// per KV head, which gives a grid of a few hundred workgroups whose partial
// results are only the 64 rows of one KV head.
//   * Workgroup = 8 waves in two teams of 4. Team tm takes the 32-key tiles
//     t = 2j + tm of the range, so a workgroup keeps 8 waves busy without a
//     second split of the keys; wave w of a team owns query rows 16w .. 16w + 15.
//     The two teams' running results are merged through LDS at the end.
//   * The keys of each sequence are cut into equal splits of whole 32-key tiles
//     (decode_partition): balanced over the grid's slots from the device-side
//     lengths by default, or a fixed number of keys per split; slots without a
//     split exit at once.
//   * Staging: each thread owns 2 K and 2 V 16-byte chunks of its team's tile,
//     fetched NS tiles ahead into registers with buffer loads whose descriptor
//     covers only the keys below k_hi: rows past the end read as zero without
//     touching memory, so every step issues the same loads and the compiler's
//     waits stay exact. Page ids of the range are read once into LDS.
//   * LDS is double-buffered per team (K row-major with a 16-byte row pad; V
//     row-major with a 32-byte pad for the transposing reads), so one barrier per
//     step orders both the stores of tile t and the reads of tile t - 2.
//   * Math as in kv_decode_kernel, one 16-row M-tile per wave: S^T = K Q^T with
//     v_mfma_f32_16x16x32_bf16, online softmax with a lazily moved reference max,
//     O^T += V^T P^T with the V^T operand from ds_read_b64_tr_b16.
//   * A single-split unit writes its output rows. Otherwise each workgroup
//     writes its unnormalised partial (O, m, l) to the workspace with
//     device-coherent stores, waits for them to complete and counts its arrival
//     with one atomic; the last workgroup of the unit merges all partials
//     (merge_splits) and resets the counter, so no second kernel is launched.
template <int NS, bool F16, bool PAGED>
__global__ __launch_bounds__(256 * kDecodeTeams, 2) void kv_split_decode_kernel(FDLLM_LEAD_PARAMS, const AttnParams p) {
  FDLLM_LEAD_LOCAL;
  FDLLM_STAMP(0, __builtin_amdgcn_s_memrealtime());  // start
  constexpr int D = 128;
  constexpr int NT = 256 * kDecodeTeams;  // threads
  constexpr int KT = 32;
  constexpr int KS = D + 8;
  constexpr int VS = D + 16;
  constexpr int NDT = D / 16;
  constexpr int kMaxPages = kDecodeMaxTiles;
  constexpr int KBUF = KT * KS;
  constexpr int VBUF = KT * VS;
  // [team][buffer] K then V tiles; reused for the team merge at the end
  __shared__ __attribute__((aligned(16))) uint16_t sKV[kDecodeTeams][2][KBUF + VBUF];
  __shared__ int sPage[kMaxPages];
  // the whole page table when it is small: read together with the lengths, so the
  // page ids of the workgroup's range need no second round trip after the partition
  constexpr int kPrefetchPages = 4096;
  __shared__ int sAllPages[kPrefetchPages];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  // wave-uniform by construction; readfirstlane lets the compiler keep the
  // per-team buffer descriptors in scalar registers
  const int team = kDecodeTeams == 2 ? __builtin_amdgcn_readfirstlane(wave >> 2) : 0;
  const int wt = wave & 3;
  const int ttid = tid & 255;  // thread index within the team
  const int l16 = lane & 15;
  const int g = lane >> 4;

  const int kvh = blockIdx.y;
  const int n_pt = PAGED ? ld.B * ld.max_pages : 0;
  const bool pt_prefetch = PAGED && n_pt <= kPrefetchPages;  // uniform
  int pf[kPrefetchPages / NT];
  if (pt_prefetch) {
#pragma unroll
    for (int u = 0; u < kPrefetchPages / NT; ++u) {
      const int idx = tid + NT * u;
      pf[u] = idx < n_pt ? ld.page_table[idx] : 0;
    }
  }
  const DecodePart dp = decode_partition<PAGED>(p, ld);
  FDLLM_STAMP(1, __builtin_amdgcn_s_memrealtime());  // partition known
  if (dp.b < 0) return;  // idle slot (uniform over the workgroup)
  const int b = __builtin_amdgcn_readfirstlane(dp.b);
  const int split = __builtin_amdgcn_readfirstlane(dp.split);
  const int n_act = __builtin_amdgcn_readfirstlane(dp.n_act);
  const int k_lo = __builtin_amdgcn_readfirstlane(dp.k_lo);
  const int k_hi = __builtin_amdgcn_readfirstlane(dp.k_hi);
  SeqInfo si;
  si.seqlen = dp.seqlen;
  si.qs = dp.qs;
  si.kv_end = dp.kv_end;
  // at most kMaxPages tiles by construction of the partition (the min keeps LDS indexing in bounds)
  const int ntiles = min(kMaxPages, k_hi > k_lo ? (k_hi - k_lo + KT - 1) / KT : 0);
  const int nsteps = (ntiles + kDecodeTeams - 1) / kDecodeTeams;  // tiles per team, rounded up (every team runs every step)

  // ---- query fragments and row limits of this wave's 16 rows
  u32x4 qf[4];
  int lim;
  {
    const int r = wt * 16 + l16;
    const int rc = min(r, p.R - 1);  // padding rows reuse a valid row: finite, never written
    const int t = rc / p.G;
    const int hh = rc - t * p.G;
    lim = min(row_key_limit(p, si.seqlen, si.qs, t), k_hi);
    const uint16_t* qrow = p.q + b * p.q_sb + t * p.q_ss + (kvh * p.G + hh) * p.q_sh;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) qf[ks] = *reinterpret_cast<const u32x4*>(qrow + ks * 32 + g * 8);
  }
  const int lim_min =
      __builtin_amdgcn_readfirstlane(-static_cast<int>(wave_allreduce_max(-static_cast<float>(lim))));
  const float rescale_thr = 8.f / p.scale_log2;

  if constexpr (PAGED) {
    if (pt_prefetch) {
#pragma unroll
      for (int u = 0; u < kPrefetchPages / NT; ++u) {
        const int idx = tid + NT * u;
        if (idx < n_pt) sAllPages[idx] = pf[u];
      }
    } else {
      const int32_t* pt_row = ld.page_table + static_cast<int64_t>(b) * ld.max_pages;
      for (int i = tid; i < ntiles; i += NT) sPage[i] = pt_row[(k_lo + i * KT) >> p.page_shift];
    }
  }

  f32x4 acc[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) acc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;

  // chunk c = ttid + 256 i of a tile: key c / 16, 16-byte column c % 16
  const int krow_bytes = static_cast<int>(p.k_ss) * 2;
  const int vrow_bytes = static_cast<int>(p.v_ss) * 2;
  int koff[2], voff[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int c = ttid + 256 * i;
    koff[i] = (c >> 4) * krow_bytes + (c & 15) * 16;
    voff[i] = (c >> 4) * vrow_bytes + (c & 15) * 16;
  }
  // per-workgroup bases: the KV head of this unit, sequence b (static cache)
  const uint16_t* kbase = p.k + kvh * p.k_sh + (PAGED ? 0 : b * p.k_sp);
  const uint16_t* vbase = p.v + kvh * p.v_sh + (PAGED ? 0 : b * p.v_sp);
  struct Stage {
    u32x4 k[2];
    u32x4 v[2];
  };
  static_assert(NS == 2 || NS == 3, "two or three register stages (named, so both paths into the loop agree on registers)");
  Stage st0, st1, st2;

  if constexpr (PAGED) __syncthreads();  // sPage visible

  // tile j of this team = tile kDecodeTeams j + team of the range
  auto load_tile = [&](Stage& sg, int j) {
    const int t = kDecodeTeams * j + team;
    const int kb = k_lo + t * KT;
    const int valid = __builtin_amdgcn_readfirstlane(max(0, min(KT, k_hi - kb)));
    int64_t koffs, voffs;
    if constexpr (PAGED) {
      const int tc = min(t, max(ntiles - 1, 0));
      const int page = __builtin_amdgcn_readfirstlane(
          pt_prefetch ? sAllPages[b * p.max_pages + min((k_lo + tc * KT) >> p.page_shift, p.max_pages - 1)]
                      : sPage[tc]);
      const int slot0 = kb & (p.page_size - 1);
      koffs = static_cast<int64_t>(page) * p.k_sp + slot0 * p.k_ss;
      voffs = static_cast<int64_t>(page) * p.v_sp + slot0 * p.v_ss;
    } else {
      koffs = static_cast<int64_t>(kb) * p.k_ss;
      voffs = static_cast<int64_t>(kb) * p.v_ss;
    }
    const __amdgpu_buffer_rsrc_t kr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(kbase + koffs), 0, valid * krow_bytes, kBufferFlags);
    const __amdgpu_buffer_rsrc_t vr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(vbase + voffs), 0, valid * vrow_bytes, kBufferFlags);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      sg.k[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(kr, koff[i], 0, kSlcNt));
      sg.v[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(vr, voff[i], 0, kSlcNt));
    }
  };
  auto store_tile = [&](const Stage& sg, int buf) {
    uint16_t* sk = sKV[team][buf];
    uint16_t* sv = sk + KBUF;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int c = ttid + 256 * i;
      *reinterpret_cast<u32x4*>(&sk[(c >> 4) * KS + (c & 15) * 8]) = sg.k[i];
      *reinterpret_cast<u32x4*>(&sv[(c >> 4) * VS + (c & 15) * 8]) = sg.v[i];
    }
  };
  auto compute_tile = [&](int buf, int kb) {
    const uint16_t* sk = sKV[team][buf];
    const uint16_t* sv = sk + KBUF;
    f32x4 s[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int st2 = 0; st2 < 2; ++st2) {
        const u32x4 kf = *reinterpret_cast<const u32x4*>(&sk[(st2 * 16 + l16) * KS + ks * 32 + g * 8]);
        s[st2] = mfma16x16x32<F16>(kf, qf[ks], s[st2]);
      }
    if (!(kb + KT <= lim_min)) {  // wave-uniform: some row of the wave sees only part of the tile
#pragma unroll
      for (int st2 = 0; st2 < 2; ++st2)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (kb + st2 * 16 + g * 4 + j >= lim) s[st2][j] = -INFINITY;
    }
    float tmax = -INFINITY;
#pragma unroll
    for (int st2 = 0; st2 < 2; ++st2)
#pragma unroll
      for (int j = 0; j < 4; ++j) tmax = fmaxf(tmax, s[st2][j]);
    tmax = group4_allreduce_max(tmax);
    if (__builtin_amdgcn_ballot_w64(tmax > m_run + rescale_thr) != 0) {
      const float m_new = fmaxf(m_run, tmax);
      const float alpha = m_run == -INFINITY ? 0.f : fast_exp2((m_run - m_new) * p.scale_log2);
      l_run *= alpha;
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) acc[dt] *= alpha;
      m_run = m_new;
    }
    const float mc = m_run == -INFINITY ? 0.f : m_run * p.scale_log2;
    float lsum = 0.f;
#pragma unroll
    for (int st2 = 0; st2 < 2; ++st2)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float e = fast_exp2(fmaf(s[st2][j], p.scale_log2, -mc));
        s[st2][j] = e;
        lsum += e;
      }
    l_run += lsum;
    u32x4 pf;
    pf[0] = pack2<F16>(s[0][0], s[0][1]);
    pf[1] = pack2<F16>(s[0][2], s[0][3]);
    pf[2] = pack2<F16>(s[1][0], s[1][1]);
    pf[3] = pack2<F16>(s[1][2], s[1][3]);
    const int vrow = 4 * g + (l16 >> 2);
    const int vcol = 4 * (l16 & 3);
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      const s16x4 lo = lds_read_tr16(&sv[vrow * VS + vcol + dt * 16]);
      const s16x4 hi = lds_read_tr16(&sv[(vrow + 16) * VS + vcol + dt * 16]);
      const u32x2 lo2 = __builtin_bit_cast(u32x2, lo);
      const u32x2 hi2 = __builtin_bit_cast(u32x2, hi);
      acc[dt] = mfma16x16x32<F16>(u32x4{lo2[0], lo2[1], hi2[0], hi2[1]}, pf, acc[dt]);
    }
  };

  // Every step stores, synchronises and issues its loads, whether or not its
  // tile exists (loads past the range are zero-filled without memory traffic),
  // so the number of loads in flight is the same on every path and each wait
  // covers exactly the stage it needs; only the math is conditional.
  auto step = [&](Stage& sg, int j) {
    store_tile(sg, j & 1);
    lds_barrier();
    if (FDLLM_TIMELINE && j == 0) FDLLM_STAMP(2, __builtin_amdgcn_s_memrealtime());  // first tiles in LDS
    load_tile(sg, j + NS);
    const int t = kDecodeTeams * j + team;
    if (t < ntiles) compute_tile(j & 1, k_lo + t * KT);  // wave-uniform
  };
  if (nsteps > 0) {
    load_tile(st0, 0);
    load_tile(st1, 1);
    if constexpr (NS == 3) load_tile(st2, 2);
    for (int j = 0; j < nsteps; j += NS) {
      step(st0, j);
      step(st1, j + 1);
      if constexpr (NS == 3) step(st2, j + 2);
    }
  }

  FDLLM_STAMP(3, __builtin_amdgcn_s_memrealtime());  // key loop done
  FDLLM_STAMP(6, (static_cast<uint64_t>(b) << 48) | (static_cast<uint64_t>(split) << 32) |
                     (static_cast<uint64_t>(n_act) << 16) | static_cast<uint64_t>(ntiles));
  // ---- merge the two teams: team 1 hands (m, l, O) to team 0 through LDS
  float* xfer = reinterpret_cast<float*>(&sKV[0][0][0]);  // [4 waves][64 lanes][NDT * 4 + 2]
  constexpr int XS = NDT * 4 + 2;
  if constexpr (kDecodeTeams == 1) {
    l_run = group4_allreduce_sum(l_run);
  } else {
  lds_barrier();  // every wave is done with the tiles
  if (team == 1) {
    float* x = xfer + (wt * 64 + lane) * XS;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int j = 0; j < 4; ++j) x[dt * 4 + j] = acc[dt][j];
    x[NDT * 4] = m_run;
    x[NDT * 4 + 1] = l_run;
  }
  lds_barrier();
  if (team == 0) {
    const float* x = xfer + (wt * 64 + lane) * XS;
    const float m1 = x[NDT * 4];
    const float l1 = x[NDT * 4 + 1];
    const float m_new = fmaxf(m_run, m1);
    const float a0 = m_run == -INFINITY ? 0.f : fast_exp2((m_run - m_new) * p.scale_log2);
    const float a1 = m1 == -INFINITY ? 0.f : fast_exp2((m1 - m_new) * p.scale_log2);
    l_run = l_run * a0 + l1 * a1;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[dt][j] = acc[dt][j] * a0 + x[dt * 4 + j] * a1;
    m_run = m_new;
    l_run = group4_allreduce_sum(l_run);
  }
  }

  // ---- epilogue (team 0 holds the workgroup's result): rows r = 16 wt + l16,
  // columns d = 16 dt + 4 g + j
  const int r = wt * 16 + l16;
  if (n_act <= 1) {
    if (team == 0 && r < p.R) {
      const int t = r / p.G;
      const int hh = r - t * p.G;
      const float inv = l_run > 0.f ? 1.f / l_run : 0.f;
      uint16_t* orow = p.out + b * p.o_sb + t * p.o_ss + (kvh * p.G + hh) * p.o_sh;
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        const f32x4 o = acc[dt] * inv;
        *reinterpret_cast<u32x2*>(orow + dt * 16 + g * 4) = u32x2{pack2<F16>(o[0], o[1]), pack2<F16>(o[2], o[3])};
      }
    }
    FDLLM_STAMP(4, __builtin_amdgcn_s_memrealtime());  // output written (single split)
    return;
  }
  const int unit = b * p.Hkv + kvh;
  const int64_t slot0 = dp.first;  // partial slot of split 0 of this unit
  if (team == 0 && r < p.R) {  // padding rows are never read
    const int64_t slot = slot0 + split;
    const auto orsrc = __builtin_amdgcn_make_buffer_rsrc(p.ws_o + slot * 64 * D, 0, 64 * D * 4, kBufferFlags);
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc[dt]), orsrc, (r * D + dt * 16 + g * 4) * 4,
                                             0, kSc1);
    if (g == 0) {
      const auto mrsrc = __builtin_amdgcn_make_buffer_rsrc(p.ws_ml + slot * 64, 0, 64 * 8, kBufferFlags);
      __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, make_float2(m_run, l_run)), mrsrc, r * 8, 0,
                                            kSc1);
    }
  }
  // The last workgroup of the unit to arrive merges every split. The partials were
  // written with device-coherent stores; waiting for their acknowledgement before the
  // arrival is counted (one device-scope atomic) publishes them, and the merge reads
  // them back with device-coherent loads.
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  __shared__ int s_last;
  if (tid == 0)
    s_last = __hip_atomic_fetch_add(&p.ws_cnt[unit], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == n_act - 1;
  __syncthreads();
  FDLLM_STAMP(4, __builtin_amdgcn_s_memrealtime());  // partial stored, arrival counted
  if (!s_last) return;
  merge_splits_n<F16>(p, b, kvh, slot0, n_act, tid, NT);
  if (tid == 0) __hip_atomic_store(&p.ws_cnt[unit], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // next call
  FDLLM_STAMP(5, __builtin_amdgcn_s_memrealtime());  // merge written (last arrival)
}

// ---------------------------------------------------------------------------
// Balanced split-KV decode (opt-in, FDLLM_ATTN_BALANCED_SPLITS): the keys of all sequences
// of one KV head, in quads of four 32-key tiles, are dealt to the S slots of the head as
// equal runs of quads regardless of where one sequence ends and the next begins, so every
// workgroup streams the same number of bytes (to one quad) whatever the mix of lengths.
//   * Quads. Sequence b holds Q_b = max(1, ceil(tiles_b / 4)) quads (two steps of one tile
//     per team), at offset off_b of the head's quad list; slot s takes quads
//     [s P / S, (s + 1) P / S) (S <= P, so no run is empty). Every piece therefore starts
//     on an even step, so one code path with fixed stage registers runs every piece (a
//     piece starting on an odd step, or stage registers exchanged between pieces, made
//     the compiler drain the loads in flight at each boundary). The run crosses from one
//     sequence into the next ("pieces"): the load pipeline goes on across the boundary
//     (the load cursor moves to the next sequence's pages), and at the boundary the two
//     teams merge through the LDS of the tile buffer they just finished and both start
//     over with the next sequence's query block.
//   * Query blocks. The query rows of the first kBalQSlots pieces are loaded together
//     with the first tiles and kept in LDS; a later piece (a run over many short
//     sequences) loads its block at its boundary.
//   * Partials. Piece (s, b) owns partial slot s + b of the head: along the runs, each
//     new piece moves to the next slot or the next sequence, so the ids are distinct,
//     and the pieces of sequence b occupy consecutive slots from first_slot(b) + b.
//     A piece that is the whole of its sequence writes the output rows itself.
//   * Arrivals. No partial is stored inside the loop (a store there makes the next
//     steps' waits for their tiles also wait for the store's acknowledgement): the first
//     finished piece is parked in registers; after its last step the workgroup writes
//     its pieces, waits once for the stores, adds one arrival per stored piece to that
//     sequence's counter, and merges the sequences whose last arrival it was, side by
//     side.
// Measured on the bs16 7B sub-block step (head-major pages): 30.45 us against 25.25 us
// for the per-sequence splits of kv_split_decode_kernel; a workgroup whose run crosses a
// sequence boundary finishes its loop about 2.5 us after one that does not, which more
// than eats the balance gained. Hence opt-in.
// Conditions (host): batch <= 64 (one wave lane per sequence in the partition), the
// whole page table in LDS (batch * max_pages <= kBalMaxPages) or a contiguous cache,
// head_dim 128, at most 64 query rows per KV head.
constexpr int kBalQSlots = 3;
// LDS placement of the balanced decode kernel's regions (byte offsets in one arena): team
// 0's two tile buffers, team 1's, the query blocks, the page table, the per-sequence
// facts. (Five placements of the team buffers relative to the query blocks and the 80 KB
// mark ran alike.)
struct BalLds {
  static constexpr int kTile = 2 * (32 * (128 + 8) + 32 * (128 + 16)) * 2;  // two buffers of one team
  static constexpr int kQRow = 128 + 8;  // query row in LDS, padded: the 16 rows of one read hit distinct banks
  static constexpr int kQBytes = kBalQSlots * 64 * kQRow * 2;
  static constexpr int kPagesBytes = kBalMaxPages * 4;
  static constexpr int kSmallBytes = (65 + 8 * 64) * 4;
  static constexpr int kTeam0 = 0, kTeam1 = kTile, kQ = 2 * kTile, kPages = kQ + kQBytes, kSmall = kPages + kPagesBytes;
  static constexpr int kBytes = kSmall + kSmallBytes;  // the regions in this order, end to end
};
static_assert(BalLds::kBytes <= 160 * 1024, "balanced decode LDS fits one CU");

template <bool F16, bool PAGED>
__global__ __launch_bounds__(512, 2) void kv_balanced_decode_kernel(FDLLM_LEAD_PARAMS, const AttnParams p) {
  FDLLM_LEAD_LOCAL;
  FDLLM_STAMP(0, __builtin_amdgcn_s_memrealtime());  // start
  constexpr int D = 128;
  constexpr int KT = 32;
  constexpr int KS = D + 8;
  constexpr int VS = D + 16;
  constexpr int NDT = D / 16;
  constexpr int KBUF = KT * KS;
  constexpr int VBUF = KT * VS;
  // One LDS arena with placed regions (BalLds): each team's two tile buffers (K then V),
  // the query blocks, the page table and the per-sequence facts.
  __shared__ __attribute__((aligned(16))) unsigned char smem[BalLds::kBytes];
  uint16_t(*const sKVt)[2][KBUF + VBUF] = reinterpret_cast<uint16_t(*)[2][KBUF + VBUF]>(smem);  // unused base
  auto sKV_of = [&](int buf, int tm) {
    return reinterpret_cast<uint16_t*>(smem + (tm ? BalLds::kTeam1 : BalLds::kTeam0) + buf * (KBUF + VBUF) * 2);
  };
  (void)sKVt;
  int* const sAllPages = reinterpret_cast<int*>(smem + BalLds::kPages);
  uint16_t(*const sQ)[64 * BalLds::kQRow] = reinterpret_cast<uint16_t(*)[64 * BalLds::kQRow]>(smem + BalLds::kQ);
  int* const sOff = reinterpret_cast<int*>(smem + BalLds::kSmall);  // [65] pair offset of each sequence; sOff[B] = P
  int* const sLen = sOff + 65;     // [64] visible length
  int* const sQs = sLen + 64;      // [64] query start
  int* const sEnd = sQs + 64;      // [64] key bound
  int* const sNs = sEnd + 64;      // [64] pieces of each sequence
  int* const sFirst = sNs + 64;    // [64] first partial slot
  int* const sArr = sFirst + 64;   // [64] sequences this workgroup stored a partial for
  int* const sLast = sArr + 64;    // [64]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int team = __builtin_amdgcn_readfirstlane(wave >> 2);
  const int wt = wave & 3;
  const int ttid = tid & 255;
  const int l16 = lane & 15;
  const int g = lane >> 4;
  const int kvh = blockIdx.y;

  // the whole page table, read together with the lengths
  const int n_pt = PAGED ? ld.B * ld.max_pages : 0;
  int pf[kBalMaxPages / 512];
  if constexpr (PAGED) {
#pragma unroll
    for (int u = 0; u < kBalMaxPages / 512; ++u) {
      const int idx = tid + 512 * u;
      pf[u] = idx < n_pt ? ld.page_table[idx] : 0;
    }
  }
  // ---- partition (every wave evaluates it; lane b holds sequence b)
  const bool has = lane < ld.B;
  SeqInfo sl;
  sl.seqlen = sl.qs = sl.kv_end = 0;
  if (has) sl = seq_info<PAGED>(p, ld, lane, 0);
  const int tiles = (sl.kv_end + KT - 1) / KT;
  const int quads = has ? max(1, (tiles + 3) >> 2) : 0;  // two steps of two tiles
  const int incl = wave_incl_scan_i32(quads);
  const int off = incl - quads;
  const int P = __builtin_amdgcn_readlane(incl, 63);
  const int S = min(p.n_splits, P);  // active slots, each with at least one quad
  const int x = blockIdx.x;
  const int slot = (p.n_splits & 7) == 0 ? (x & 7) * (p.n_splits >> 3) + (x >> 3) : x;
  if (slot >= S) return;  // uniform
  const int qlo = static_cast<int>(static_cast<int64_t>(slot) * P / S);
  const int qhi = static_cast<int>(static_cast<int64_t>(slot + 1) * P / S);
  // slot holding quad y: the largest s with floor(s P / S) <= y
  auto slot_of = [&](int y) { return static_cast<int>((static_cast<int64_t>(y + 1) * S + P - 1) / P) - 1; };
  if (wave == 0) {
    if (has) {
      sOff[lane] = 2 * off;  // in steps
      sLen[lane] = sl.seqlen;
      sQs[lane] = sl.qs;
      sEnd[lane] = sl.kv_end;
      const int s0 = slot_of(off);
      sNs[lane] = slot_of(off + quads - 1) - s0 + 1;
      sFirst[lane] = s0 + lane;
    }
    if (lane == 0) sOff[ld.B] = 2 * P;
  }
  const int b0 = static_cast<int>(__builtin_ctzll(__builtin_amdgcn_ballot_w64(has && off <= qlo && qlo < incl)));
  const int b_last = static_cast<int>(__builtin_ctzll(__builtin_amdgcn_ballot_w64(has && off < qhi && qhi <= incl)));
  const int lo = 2 * qlo, hi = 2 * qhi;  // the run in steps (pairs of tiles)
  FDLLM_STAMP(1, __builtin_amdgcn_s_memrealtime());  // partition known
  if constexpr (PAGED) {
#pragma unroll
    for (int u = 0; u < kBalMaxPages / 512; ++u) {
      const int idx = tid + 512 * u;
      if (idx < n_pt) sAllPages[idx] = pf[u];
    }
  }
  __syncthreads();  // page table and sequence facts visible
  const int n = hi - lo;  // steps of this workgroup (even)

  f32x4 acc[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) acc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;

  // chunk c = ttid + 256 i of a tile: key c / 16, 16-byte column c % 16
  const int krow_bytes = static_cast<int>(p.k_ss) * 2;
  const int vrow_bytes = static_cast<int>(p.v_ss) * 2;
  int koff[2], voff[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int c = ttid + 256 * i;
    koff[i] = (c >> 4) * krow_bytes + (c & 15) * 16;
    voff[i] = (c >> 4) * vrow_bytes + (c & 15) * 16;
  }
  const uint16_t* kbase = p.k + kvh * p.k_sh;
  const uint16_t* vbase = p.v + kvh * p.v_sh;
  struct Stage {
    u32x4 k[2];
    u32x4 v[2];
  };
  Stage st0, st1;

  // load cursor: the sequence of the pair being loaded (moves forward only)
  int lb = b0;
  int l_off = sOff[lb];
  int l_end = sOff[lb + 1];
  int l_kv = sEnd[lb];
  auto load_tile = [&](Stage& sg, int j) {
    const int gq = lo + j;
    if (gq < hi) {
      while (gq >= l_end) {  // uniform; at most once per step for sequences of >= 1 pair
        ++lb;
        l_off = l_end;
        l_end = sOff[lb + 1];
        l_kv = sEnd[lb];
      }
    }
    const int kb = (min(gq, hi - 1) - l_off) * 64 + 32 * team;
    const int valid = __builtin_amdgcn_readfirstlane(gq < hi ? max(0, min(KT, l_kv - kb)) : 0);
    int64_t koffs, voffs;
    if constexpr (PAGED) {
      const int page = __builtin_amdgcn_readfirstlane(
          sAllPages[lb * p.max_pages + min(kb >> p.page_shift, p.max_pages - 1)]);
      const int slot0 = kb & (p.page_size - 1);
      koffs = static_cast<int64_t>(page) * p.k_sp + slot0 * p.k_ss;
      voffs = static_cast<int64_t>(page) * p.v_sp + slot0 * p.v_ss;
    } else {
      koffs = static_cast<int64_t>(lb) * p.k_sp + static_cast<int64_t>(kb) * p.k_ss;
      voffs = static_cast<int64_t>(lb) * p.v_sp + static_cast<int64_t>(kb) * p.v_ss;
    }
    const __amdgpu_buffer_rsrc_t kr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(kbase + koffs), 0, valid * krow_bytes, kBufferFlags);
    const __amdgpu_buffer_rsrc_t vr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(vbase + voffs), 0, valid * vrow_bytes, kBufferFlags);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      sg.k[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(kr, koff[i], 0, kSlcNt));
      sg.v[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(vr, voff[i], 0, kSlcNt));
    }
  };
  auto store_tile = [&](const Stage& sg, int buf) {
    uint16_t* sk = sKV_of(buf, team);
    uint16_t* sv = sk + KBUF;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int c = ttid + 256 * i;
      *reinterpret_cast<u32x4*>(&sk[(c >> 4) * KS + (c & 15) * 8]) = sg.k[i];
      *reinterpret_cast<u32x4*>(&sv[(c >> 4) * VS + (c & 15) * 8]) = sg.v[i];
    }
  };
  // query rows of sequence b: chunk c = tid + 512 i is row c / 16 (padding rows repeat
  // the last row: finite, never written), 16-byte column c % 16
  auto q_chunk = [&](int b, int i) {
    const int c = tid + 512 * i;
    const int rc = min(c >> 4, p.R - 1);
    const int t = rc / p.G;
    const int hh = rc - t * p.G;
    return *reinterpret_cast<const u32x4*>(p.q + b * p.q_sb + t * p.q_ss + (kvh * p.G + hh) * p.q_sh + (c & 15) * 8);
  };
  auto q_store = [&](int qslot, int i, const u32x4& v) {
    const int c = tid + 512 * i;
    *reinterpret_cast<u32x4*>(&sQ[qslot][(c >> 4) * BalLds::kQRow + (c & 15) * 8]) = v;
  };

  load_tile(st0, 0);
  // query blocks of the first pieces (a piece past b_last loads b_last's block again)
  u32x4 qpre[kBalQSlots][2];
#pragma unroll
  for (int u = 0; u < kBalQSlots; ++u)
#pragma unroll
    for (int i = 0; i < 2; ++i) qpre[u][i] = q_chunk(min(b0 + u, b_last), i);
  load_tile(st1, 1);

  // compute cursor: the sequence of the piece being computed
  int cb = b0;
  int piece = 0;
  int narr = 0;  // partials stored by this workgroup (uniform)
  u32x4 qf[4];
  int lim = 0, lim_min = 0;
  const float rescale_thr = 8.f / p.scale_log2;

  auto compute_tile = [&](int buf, int kb) {
    const uint16_t* sk = sKV_of(buf, team);
    const uint16_t* sv = sk + KBUF;
    f32x4 s[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int st2 = 0; st2 < 2; ++st2) {
        const u32x4 kf = *reinterpret_cast<const u32x4*>(&sk[(st2 * 16 + l16) * KS + ks * 32 + g * 8]);
        s[st2] = mfma16x16x32<F16>(kf, qf[ks], s[st2]);
      }
    if (!(kb + KT <= lim_min)) {  // wave-uniform: some row of the wave sees only part of the tile
#pragma unroll
      for (int st2 = 0; st2 < 2; ++st2)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (kb + st2 * 16 + g * 4 + j >= lim) s[st2][j] = -INFINITY;
    }
    float tmax = -INFINITY;
#pragma unroll
    for (int st2 = 0; st2 < 2; ++st2)
#pragma unroll
      for (int j = 0; j < 4; ++j) tmax = fmaxf(tmax, s[st2][j]);
    tmax = group4_allreduce_max(tmax);
    if (__builtin_amdgcn_ballot_w64(tmax > m_run + rescale_thr) != 0) {
      const float m_new = fmaxf(m_run, tmax);
      const float alpha = m_run == -INFINITY ? 0.f : fast_exp2((m_run - m_new) * p.scale_log2);
      l_run *= alpha;
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) acc[dt] *= alpha;
      m_run = m_new;
    }
    const float mc = m_run == -INFINITY ? 0.f : m_run * p.scale_log2;
    float lsum = 0.f;
#pragma unroll
    for (int st2 = 0; st2 < 2; ++st2)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float e = fast_exp2(fmaf(s[st2][j], p.scale_log2, -mc));
        s[st2][j] = e;
        lsum += e;
      }
    l_run += lsum;
    u32x4 pk;
    pk[0] = pack2<F16>(s[0][0], s[0][1]);
    pk[1] = pack2<F16>(s[0][2], s[0][3]);
    pk[2] = pack2<F16>(s[1][0], s[1][1]);
    pk[3] = pack2<F16>(s[1][2], s[1][3]);
    const int vrow = 4 * g + (l16 >> 2);
    const int vcol = 4 * (l16 & 3);
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      const s16x4 lo4 = lds_read_tr16(&sv[vrow * VS + vcol + dt * 16]);
      const s16x4 hi4 = lds_read_tr16(&sv[(vrow + 16) * VS + vcol + dt * 16]);
      const u32x2 lo2 = __builtin_bit_cast(u32x2, lo4);
      const u32x2 hi2 = __builtin_bit_cast(u32x2, hi4);
      acc[dt] = mfma16x16x32<F16>(u32x4{lo2[0], lo2[1], hi2[0], hi2[1]}, pk, acc[dt]);
    }
  };

  // Output rows (a piece that is its whole sequence) or the partial of piece (slot, b),
  // from team 0's merged state.
  const int r = wt * 16 + l16;  // this lane's query row
  auto emit = [&](int b, const f32x4 (&a)[NDT], float m, float l) {
    if (team != 0 || r >= p.R) return;  // padding rows are never read
    if (sNs[b] <= 1) {
      const int t = r / p.G;
      const int hh = r - t * p.G;
      const float inv = l > 0.f ? 1.f / l : 0.f;
      uint16_t* orow = p.out + b * p.o_sb + t * p.o_ss + (kvh * p.G + hh) * p.o_sh;
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        const f32x4 o = a[dt] * inv;
        *reinterpret_cast<u32x2*>(orow + dt * 16 + g * 4) = u32x2{pack2<F16>(o[0], o[1]), pack2<F16>(o[2], o[3])};
      }
      return;
    }
    const int64_t pslot = static_cast<int64_t>(kvh) * (p.n_splits + p.B) + slot + b;
    const auto orsrc = __builtin_amdgcn_make_buffer_rsrc(p.ws_o + pslot * 64 * D, 0, 64 * D * 4, kBufferFlags);
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, a[dt]), orsrc, (r * D + dt * 16 + g * 4) * 4, 0,
                                             kSc1);
    if (g == 0) {
      const auto mrsrc = __builtin_amdgcn_make_buffer_rsrc(p.ws_ml + pslot * 64, 0, 64 * 8, kBufferFlags);
      __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, make_float2(m, l)), mrsrc, r * 8, 0, kSc1);
    }
  };
  // A piece that ends before the run does is parked in registers (one such piece) and
  // written after the loop: stores issued inside the loop would make the next steps'
  // waits for their tiles also wait for the stores' acknowledgement.
  f32x4 hacc[NDT];
  float hm = -INFINITY, hl = 0.f;
  int hb = -1;  // sequence of the parked piece (uniform), -1: none

  // End of a piece (workgroup-uniform): the teams merge through buffer `buf` of both
  // teams (idle until the tile two steps on is stored there, after the next barrier),
  // team 0 parks or writes the result, and both teams start over.
  constexpr int XS = NDT * 4 + 2;
  static_assert(2 * 64 * XS * 4 <= (KBUF + VBUF) * 2, "half of the team merge fits one buffer of one team");
  // waves 0-1 of team 1 hand over through team 0's buffer `buf`, waves 2-3 through team 1's
  float* const xwave = reinterpret_cast<float*>(sKV_of(0, wt >> 1)) + ((wt & 1) * 64 + lane) * XS;
  auto finalize = [&](int buf, bool last_piece) {
    float* xs_base = xwave + buf * (KBUF + VBUF) / 2;  // (KBUF + VBUF) 16-bit words = half as many floats
    lds_barrier();  // both teams are done with the tiles in `buf`
    if (team == 1) {
      float* xs = xs_base;
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int j = 0; j < 4; ++j) xs[dt * 4 + j] = acc[dt][j];
      xs[NDT * 4] = m_run;
      xs[NDT * 4 + 1] = l_run;
    }
    lds_barrier();
    if (team == 0) {
      const float* xs = xs_base;
      const float m1 = xs[NDT * 4];
      const float l1 = xs[NDT * 4 + 1];
      const float m_new = fmaxf(m_run, m1);
      const float a0 = m_run == -INFINITY ? 0.f : fast_exp2((m_run - m_new) * p.scale_log2);
      const float a1 = m1 == -INFINITY ? 0.f : fast_exp2((m1 - m_new) * p.scale_log2);
      l_run = l_run * a0 + l1 * a1;
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[dt][j] = acc[dt][j] * a0 + xs[dt * 4 + j] * a1;
      m_run = m_new;
      l_run = group4_allreduce_sum(l_run);
    }
    if (last_piece) {
      emit(cb, acc, m_run, l_run);
    } else if (hb < 0) {
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) hacc[dt] = acc[dt];
      hm = m_run;
      hl = l_run;
      hb = cb;
    } else {
      emit(cb, acc, m_run, l_run);  // a run over several short sequences: written now
    }
    if (sNs[cb] > 1) {
      if (tid == 0) sArr[narr] = cb;
      ++narr;
    }
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) acc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    m_run = -INFINITY;
    l_run = 0.f;
  };

  // One step: the pair of tiles of step j into LDS, the loads of step j + 2 issued,
  // then this team's tile of step j (the piece's keys start at pair c_off, end at c_kv).
  auto step = [&](Stage& sg, int j, int c_off, int c_kv) {
    store_tile(sg, j & 1);
    lds_barrier();
    load_tile(sg, j + 2);
    const int kb = (lo + j - c_off) * 64 + 32 * team;
    if (kb < c_kv) compute_tile(j & 1, kb);  // wave-uniform
  };
  // Steps [j, e) of one piece (j and e even): even steps' tiles are in st0, odd steps' in
  // st1, on every path (a stage register set copied while its loads are in flight would
  // make the copy wait for them, and a piece starting on an odd step would leave the
  // compiler's wait counts at the piece loop conservative: full drains).
  auto run_steps = [&](int& j, int e, int c_off, int c_kv) {
    for (; j < e; j += 2) {
      step(st0, j, c_off, c_kv);
      step(st1, j + 1, c_off, c_kv);
    }
  };

  // The query blocks of the first pieces into LDS: their wait also covers the first
  // tile (loaded before them); the second tile stays in flight.
#pragma unroll
  for (int u = 0; u < kBalQSlots; ++u)
#pragma unroll
    for (int i = 0; i < 2; ++i) q_store(u, i, qpre[u][i]);
  lds_barrier();
  FDLLM_STAMP(2, __builtin_amdgcn_s_memrealtime());  // first tile and query blocks landed
  int j = 0;  // next step (pair of the run)
  while (true) {  // one iteration per piece (workgroup-uniform)
    const int c_off = sOff[cb];
    const int e = min(sOff[cb + 1], hi) - lo;  // the piece's steps end before e
    const int c_kv = sEnd[cb];
    {
      const uint16_t* qrow = &sQ[piece % kBalQSlots][r * BalLds::kQRow];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) qf[ks] = *reinterpret_cast<const u32x4*>(qrow + ks * 32 + g * 8);
      const int rc = min(r, p.R - 1);  // padding rows take a valid row's limit
      lim = min(row_key_limit(p, sLen[cb], sQs[cb], rc / p.G), c_kv);
      lim_min = __builtin_amdgcn_readfirstlane(-static_cast<int>(wave_allreduce_max(-static_cast<float>(lim))));
    }
    run_steps(j, e, c_off, c_kv);
    finalize((j - 1) & 1, j == n);
    if (j == n) break;
    if (piece == 0) FDLLM_STAMP(7, __builtin_amdgcn_s_memrealtime());  // first boundary passed
    ++cb;
    ++piece;
    if (piece >= kBalQSlots) {
      // a run over many short sequences: this piece's query block loads now into the
      // slot of piece - kBalQSlots (finished)
#pragma unroll
      for (int i = 0; i < 2; ++i) q_store(piece % kBalQSlots, i, q_chunk(cb, i));
      lds_barrier();
    }
  }
  if (hb >= 0) emit(hb, hacc, hm, hl);  // uniform: the parked piece
  FDLLM_STAMP(3, __builtin_amdgcn_s_memrealtime());  // key loop done (every piece finalized)
  FDLLM_STAMP(6, (static_cast<uint64_t>(b0) << 48) | (static_cast<uint64_t>(b_last - b0 + 1) << 32) |
                     static_cast<uint64_t>(2 * n));
  if (narr == 0) return;  // uniform: every piece wrote its output rows
  // Publish the stored partials (device-coherent stores, acknowledged), then count one
  // arrival per stored piece; the workgroup that brings a sequence's counter to its
  // piece count merges that sequence's partials.
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid < narr) {
    const int b = sArr[tid];
    sLast[tid] = __hip_atomic_fetch_add(&p.ws_cnt[b * p.Hkv + kvh], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                 sNs[b] - 1;
  }
  __syncthreads();
  FDLLM_STAMP(4, __builtin_amdgcn_s_memrealtime());  // arrivals counted
  // the sequences this workgroup merges, run side by side (one group of threads each:
  // the merge is bound by its loads' round trip, not by the threads)
  int nm = 0;
  for (int i = 0; i < narr; ++i) nm += sLast[i] ? 1 : 0;  // uniform
  if (nm == 0) return;
  const int groups = min(nm, 4);
  const int gsize = 512 / groups;  // 512, 256 or 128 threads (3 merges: 128 each, one group idle)
  const int grp = tid / (groups == 3 ? 128 : gsize);
  for (int i = 0, k = 0; i < narr; ++i) {
    if (!sLast[i]) continue;  // uniform
    if (k % groups == grp) {
      const int b = sArr[i];
      const int64_t slot0 = static_cast<int64_t>(kvh) * (p.n_splits + p.B) + sFirst[b];
      const int gtid = tid - grp * (groups == 3 ? 128 : gsize);
      merge_splits_n<F16>(p, b, kvh, slot0, sNs[b], gtid, groups == 3 ? 128 : gsize);
      if (gtid == 0) __hip_atomic_store(&p.ws_cnt[b * p.Hkv + kvh], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    ++k;
  }
  FDLLM_STAMP(5, __builtin_amdgcn_s_memrealtime());  // merges written
}


// max / sum of the values of lanes l and l ^ 32 (v_permlane32_swap_b32: both
// results hold lanes 0-31 of one operand and lanes 32-63 of the other, so each
// lane ends up with its own value and its partner's)
__device__ __forceinline__ float halves_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float halves_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// fp32 attention: fp32 inputs, fp32 output, fp32 arithmetic throughout (the reference's
// CPU path runs the SDPA shim in fp32, e.g. a 12 / 2-head, 128-dim block of 32 queries over
// 544 keys; tests/test_focus.py:205-228). Every mask mode, contiguous or paged, any GQA.
// Workgroup = 4 query rows of one (sequence, KV head) (rows r = t G + g of its Sq x G
// rows), one per wave. Each 64-key chunk of K and V is loaded once per workgroup,
// coalesced, into LDS (K rows padded to D + 4 floats, so the 16 lanes of a read phase hit
// distinct banks), the next chunk's loads in flight in registers meanwhile. Scores: lane
// = key, a full dot product (four partial sums) from its K row in LDS against the wave's
// query row (broadcast from LDS); output: lane = head dimension (DPL of them), the chunk's
// probabilities written to LDS and read back as broadcasts, V rows read from LDS. Online softmax in
// base 2 (scores pre-multiplied by scale * log2 e), rescaled whenever the chunk maximum
// moves it. The workgroup runs to the largest key bound of its rows; each row masks the
// keys past its own.
// Key splits: a row block's keys are cut into splits of p.chunk keys (a multiple of the
// 64-key chunk) over x = row block + n_rb * split; a row block whose keys fit one split
// writes its rows directly, otherwise each split writes unnormalised (O, m, l) partials
// (m in base-2 score units), which the row block's last split to arrive folds (MERGE), or
// kv_attn_combine_kernel<..., true> after the kernel. On the 12 / 2-head block of 32
// queries over 544 keys: 27.4 us unsplit, 13.8 us in 5 splits with the combine kernel,
// 12.9 us merged in the kernel.
// query rows per wave of kv_attn_f32_kernel, unsplit: 1: 27.8 us, 2: 36.2 us, 4: 72.9 us
// (fewer rows per workgroup, more workgroups in flight; the previous one-wave-per-row form
// without staging: 85 us). The PV products run over every key of a chunk, unrolled,
// instead of a loop to the chunk's last visible key: 27.8 -> 26.9 us, the same sums bit for
// bit; the query row held in registers instead of broadcast reads from LDS was slower
// (36.1 us).
// (FDLLM_F32_ROWS_PER_WAVE, the rows per wave, is set in attn_plan.h: the plan sizes the
// grid from it.)
template <int DPL, bool PAGED, bool MERGE>
__global__ __launch_bounds__(256) void kv_attn_f32_kernel(const AttnParams p) {
  constexpr int D = 64 * DPL;
  constexpr int KS = D + 4;   // K row stride in LDS (floats)
  constexpr int RW = FDLLM_F32_ROWS_PER_WAVE;  // rows per wave
  constexpr int RWG = 4 * RW; // rows per workgroup
  constexpr int CK = 64;      // keys per chunk
  constexpr int PER = CK * D / 4 / 256;  // 16-byte loads per thread per chunk and tensor
  __shared__ __attribute__((aligned(16))) float sK[CK * KS];
  __shared__ __attribute__((aligned(16))) float sV[CK * D];
  __shared__ __attribute__((aligned(16))) float sQ[RWG][D];
  __shared__ __attribute__((aligned(16))) float sP[RWG][CK];  // the chunk's probabilities of each row
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int b = blockIdx.z;
  const int kvh = blockIdx.y;
  const int R = p.Sq * p.G;
  // x = row block + n_rb * split
  const int split = static_cast<int>(blockIdx.x) / p.n_rb;
  const int rb = static_cast<int>(blockIdx.x) - split * p.n_rb;
  const int r0 = rb * RWG;
  int seqlen = p.seqlens[b];
  if (seqlen > p.max_seqlen) seqlen = p.max_seqlen;
  if (PAGED && seqlen > p.max_pages * p.page_size) seqlen = p.max_pages * p.page_size;
  if (seqlen < 0) seqlen = 0;
  const int qs = p.q_start ? p.q_start[b] : seqlen - p.Sq;
  // key bounds never decrease with the query token, so the workgroup's last row has the largest
  const int kv_end = __builtin_amdgcn_readfirstlane(row_key_limit(p, seqlen, qs, (min(r0 + RWG, R) - 1) / p.G));
  // this workgroup's keys: split `split` of p.chunk keys (the row block's splits with keys;
  // a row block without keys still has split 0, which writes its zero rows)
  const int n_act = max(1, (kv_end + p.chunk - 1) / p.chunk);
  if (split >= n_act) return;  // uniform
  const int k_lo = split * p.chunk;  // < kv_end, or 0
  const int k_hi = static_cast<int>(min<int64_t>(kv_end, static_cast<int64_t>(k_lo) + p.chunk));

  int lim[RW], tq[RW], hq[RW];
  bool live[RW];
#pragma unroll
  for (int i = 0; i < RW; ++i) {
    const int r = r0 + w * RW + i;
    live[i] = r < R;  // wave-uniform
    const int rc = live[i] ? r : R - 1;
    tq[i] = rc / p.G;
    hq[i] = kvh * p.G + (rc - tq[i] * p.G);
    lim[i] = __builtin_amdgcn_readfirstlane(min(row_key_limit(p, seqlen, qs, tq[i]), k_hi));
    const float* q = reinterpret_cast<const float*>(p.q) + b * p.q_sb + tq[i] * p.q_ss + hq[i] * p.q_sh;
    for (int d = lane; d < D; d += 64) sQ[w * RW + i][d] = q[d];
  }
  const float* kb = reinterpret_cast<const float*>(p.k) + kvh * p.k_sh;
  const float* vb = reinterpret_cast<const float*>(p.v) + kvh * p.v_sh;
  auto row_off = [&](int key, bool kcache) -> int64_t {
    const int64_t ss = kcache ? p.k_ss : p.v_ss;
    if constexpr (PAGED) {
      const int page = p.page_table[static_cast<int64_t>(b) * p.max_pages + (key >> p.page_shift)];
      return static_cast<int64_t>(page) * (kcache ? p.k_sp : p.v_sp) + (key & (p.page_size - 1)) * ss;
    } else {
      return static_cast<int64_t>(b) * (kcache ? p.k_sp : p.v_sp) + static_cast<int64_t>(key) * ss;
    }
  };
  // load e of a thread: f32x4 index tid + 256 e of the chunk = key idx / (D / 4), column
  // 4 (idx % (D / 4)); keys at or past k_hi read as zero
  f32x4 kr[PER], vr[PER];
  auto load_chunk = [&](int k0) {
#pragma unroll
    for (int e = 0; e < PER; ++e) {
      const int idx = tid + 256 * e;
      const int key = k0 + idx / (D / 4);
      const int c = 4 * (idx % (D / 4));
      if (key < k_hi) {
        kr[e] = *reinterpret_cast<const f32x4*>(kb + row_off(key, true) + c);
        vr[e] = *reinterpret_cast<const f32x4*>(vb + row_off(key, false) + c);
      } else {
        kr[e] = f32x4{0.f, 0.f, 0.f, 0.f};
        vr[e] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
    }
  };
  float o[RW][DPL], m[RW], l[RW];
#pragma unroll
  for (int i = 0; i < RW; ++i) {
    m[i] = -INFINITY;
    l[i] = 0.f;
#pragma unroll
    for (int j = 0; j < DPL; ++j) o[i][j] = 0.f;
  }
  if (k_hi > k_lo) load_chunk(k_lo);
  for (int k0 = k_lo; k0 < k_hi; k0 += CK) {
    __syncthreads();  // every wave is done with the previous chunk (and sQ is written)
#pragma unroll
    for (int e = 0; e < PER; ++e) {
      const int idx = tid + 256 * e;
      const int key = idx / (D / 4);
      const int c = 4 * (idx % (D / 4));
      *reinterpret_cast<f32x4*>(&sK[key * KS + c]) = kr[e];
      *reinterpret_cast<f32x4*>(&sV[key * D + c]) = vr[e];
    }
    __syncthreads();
    if (k0 + CK < k_hi) load_chunk(k0 + CK);  // in flight during this chunk's math
    const int key = k0 + lane;
    // four partial sums per row (independent FMA chains), added at the end
    float acc[RW][4];
#pragma unroll
    for (int i = 0; i < RW; ++i)
#pragma unroll
      for (int u = 0; u < 4; ++u) acc[i][u] = 0.f;
#pragma unroll 8
    for (int d = 0; d < D; d += 4) {
      const f32x4 kv = *reinterpret_cast<const f32x4*>(&sK[lane * KS + d]);
#pragma unroll
      for (int i = 0; i < RW; ++i) {
        const f32x4 qv = *reinterpret_cast<const f32x4*>(&sQ[w * RW + i][d]);
#pragma unroll
        for (int u = 0; u < 4; ++u) acc[i][u] = fmaf(qv[u], kv[u], acc[i][u]);
      }
    }
#pragma unroll
    for (int i = 0; i < RW; ++i) {
      const float dot = (acc[i][0] + acc[i][1]) + (acc[i][2] + acc[i][3]);
      const float sc = key < lim[i] ? dot * p.scale_log2 : -INFINITY;
      const float m_new = fmaxf(m[i], wave_allreduce_max(sc));
      const float alpha = m[i] == -INFINITY ? 0.f : fast_exp2(m[i] - m_new);
      const float pk = key < lim[i] ? fast_exp2(sc - m_new) : 0.f;
      sP[w * RW + i][lane] = pk;  // read back by this wave only, as broadcasts
      l[i] = l[i] * alpha + wave_allreduce_sum(pk);
#pragma unroll
      for (int j = 0; j < DPL; ++j) o[i][j] *= alpha;
      m[i] = m_new;
    }
    // every key of the chunk in order, unrolled: keys past k_hi hold p = 0 and V rows of
    // zeros (never loaded), so they add exactly nothing
#pragma unroll
    for (int kk = 0; kk < CK; kk += 4) {
      f32x4 pp[RW];
#pragma unroll
      for (int i = 0; i < RW; ++i) pp[i] = *reinterpret_cast<const f32x4*>(&sP[w * RW + i][kk]);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        float v[DPL];
#pragma unroll
        for (int j = 0; j < DPL; ++j) v[j] = sV[(kk + u) * D + lane + 64 * j];
#pragma unroll
        for (int i = 0; i < RW; ++i)
#pragma unroll
          for (int j = 0; j < DPL; ++j) o[i][j] = fmaf(pp[i][u], v[j], o[i][j]);
      }
    }
  }
  if (n_act > 1) {
    // unnormalised partial (O, m, l) of each row, m in the base-2 score units of this
    // kernel, at slot (unit, split, row in block)
    const int64_t unit = (static_cast<int64_t>(b) * p.Hkv + kvh) * p.n_rb + rb;
    if constexpr (!MERGE) {  // for kv_attn_combine_kernel<..., true>, which follows
#pragma unroll
      for (int i = 0; i < RW; ++i) {
        if (live[i]) {
          const int64_t slot = (unit * p.n_splits + split) * p.rows_per_wg + w * RW + i;
#pragma unroll
          for (int j = 0; j < DPL; ++j) p.ws_o[slot * D + lane + 64 * j] = o[i][j];
          if (lane == 0) p.ws_ml[slot] = make_float2(m[i], l[i]);
        }
      }
      return;
    } else {
      // The last workgroup of the row block to arrive merges its splits: the partials
      // are written with device-coherent stores (relaxed agent-scope atomic stores: the
      // sc1 bit, no fence) and acknowledged before the arrival is counted with one
      // device-scope atomic; the merging workgroup reads them back the same way.
      float* const po = p.ws_o;
      float* const pml = reinterpret_cast<float*>(p.ws_ml);
#pragma unroll
      for (int i = 0; i < RW; ++i) {
        if (live[i]) {
          const int64_t slot = (unit * p.n_splits + split) * p.rows_per_wg + w * RW + i;
#pragma unroll
          for (int j = 0; j < DPL; ++j)
            __hip_atomic_store(po + slot * D + lane + 64 * j, o[i][j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          if (lane < 2)
            __hip_atomic_store(pml + 2 * slot + lane, lane == 0 ? m[i] : l[i], __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        }
      }
      __builtin_amdgcn_s_waitcnt(0);  // this wave's partial stores acknowledged
      __syncthreads();
      __shared__ int s_last;
      if (tid == 0)
        s_last = __hip_atomic_fetch_add(&p.ws_cnt[unit], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == n_act - 1;
      __syncthreads();
      if (!s_last) return;
      // each wave merges its own rows over the splits, eight splits' loads in flight at once
#pragma unroll
      for (int i = 0; i < RW; ++i) {
        if (!live[i]) continue;
        const int64_t slot0 = unit * p.n_splits * p.rows_per_wg + w * RW + i;  // split s at + s rows_per_wg
        float mm = -INFINITY, ll = 0.f, oo[DPL];
#pragma unroll
        for (int j = 0; j < DPL; ++j) oo[j] = 0.f;
        for (int s0 = 0; s0 < n_act; s0 += 8) {
          float sm[8], sl[8], so[8][DPL];
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            const int64_t slot = slot0 + static_cast<int64_t>(min(s0 + u, n_act - 1)) * p.rows_per_wg;
            sm[u] = __hip_atomic_load(pml + 2 * slot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            sl[u] = __hip_atomic_load(pml + 2 * slot + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
            for (int j = 0; j < DPL; ++j)
              so[u][j] = __hip_atomic_load(po + slot * D + lane + 64 * j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          }
          float mg = mm;
#pragma unroll
          for (int u = 0; u < 8; ++u)
            if (s0 + u < n_act) mg = fmaxf(mg, sm[u]);
          if (mg == -INFINITY) continue;  // no visible key yet
          const float a = mm == -INFINITY ? 0.f : fast_exp2(mm - mg);
          ll *= a;
#pragma unroll
          for (int j = 0; j < DPL; ++j) oo[j] *= a;
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            const float wt = (s0 + u < n_act && sm[u] != -INFINITY) ? fast_exp2(sm[u] - mg) : 0.f;
            ll += wt * sl[u];
#pragma unroll
            for (int j = 0; j < DPL; ++j) oo[j] += wt * so[u][j];
          }
          mm = mg;
        }
        float* out = reinterpret_cast<float*>(p.out) + b * p.o_sb + tq[i] * p.o_ss + hq[i] * p.o_sh;
        const float inv = ll > 0.f ? 1.f / ll : 0.f;
#pragma unroll
        for (int j = 0; j < DPL; ++j) out[lane + 64 * j] = oo[j] * inv;
      }
      if (tid == 0) __hip_atomic_store(&p.ws_cnt[unit], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // next call
      return;
    }
  }
#pragma unroll
  for (int i = 0; i < RW; ++i) {
    if (live[i]) {
      float* out = reinterpret_cast<float*>(p.out) + b * p.o_sb + tq[i] * p.o_ss + hq[i] * p.o_sh;
      const float inv = l[i] > 0.f ? 1.f / l[i] : 0.f;
#pragma unroll
      for (int j = 0; j < DPL; ++j) out[lane + 64 * j] = o[i][j] * inv;
    }
  }
}

// Partial (O, m, l) of one split of the split prefill kernels (one row block of at most
// 256 rows per (sequence, KV head), keys split): the unnormalised rows go to the split's
// workspace slot (slot rows = the workgroup's rows) for kv_split_prefill_merge_kernel,
// which follows on the stream. Measured and not kept: the merge in the last-arriving
// workgroup of each unit, as the split decode kernel does it (full-block step 50.3 us
// against 45.7 us: one workgroup folding 224 rows of four or five splits is a serial
// tail longer than the merge kernel and its launch); fp16 rows with a power-of-two
// scale per row folded into (m, l) (44.95 against 46.9 us, but the 7B end-to-end greedy
// agreement fell from 0.8721 / 0.8751 to 0.8700 / 0.8724 against a noise floor of 0.8739,
// s.e. 0.0013, as with bf16 rows: the extra rounding of every split moves near-tied
// greedy choices), so the rows stay fp32.
__device__ __forceinline__ void split_prefill_partial(const AttnParams& p, int64_t slot0, int split, int r, int h,
                                                      const f32x16 (&acc)[4], float m_run, float l_run) {
  constexpr int D = 128;
  if (r < p.R) {
    const int64_t slot = slot0 + split;
    const auto orsrc = __builtin_amdgcn_make_buffer_rsrc(p.ws_o + slot * 256 * D, 0, 256 * D * 4, kBufferFlags);
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        __builtin_amdgcn_raw_buffer_store_b128(
            __builtin_bit_cast(u32x4, f32x4{acc[dt][4 * i], acc[dt][4 * i + 1], acc[dt][4 * i + 2], acc[dt][4 * i + 3]}),
            orsrc, (r * D + 32 * dt + 8 * i + 4 * h) * 4, 0, 0);
    if (h == 0) {
      const auto mrsrc = __builtin_amdgcn_make_buffer_rsrc(p.ws_ml + slot * 256, 0, 256 * 8, kBufferFlags);
      __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, make_float2(m_run, l_run)), mrsrc, r * 8, 0, 0);
    }
  }
}

// ---------------------------------------------------------------------------
// Prefill attention: many query rows per KV head (block-causal prefill and
// commit forwards), head_dim 128, no key split.
//
// Workgroup = 8 waves = 256 query rows of one (sequence, KV head), rows
// r = t * G + hh in token order, 32 rows per wave (two waves per SIMD); keys in
// 64-key tiles, each read once per workgroup and used by all 256 rows.
//   * S^T = K Q^T on v_mfma_f32_32x32x16_bf16: A = 32 keys x 16 d read from LDS,
//     B = Q^T held in registers for the whole loop (lane (n, h) = row n, d
//     16 ks + 8 h .. + 8). Accumulator lane (n, h), element 4 i + j = row n,
//     key 8 i + 4 h + j of the 32-key subtile.
//   * O^T += V^T P^T on the same instruction. Its k-slot e of lane half h stands
//     for key 4 h + e (e < 4) or 8 + 4 h + (e - 4) of a 16-key step, so the P^T
//     operand is eight consecutive accumulator elements as they are, and the V^T
//     operand is two ds_read_b64_tr_b16 of four keys each.
//   * Online softmax in base 2: the row max is shared by the two lane halves of a
//     row; the reference max moves only when it would be exceeded by more than
//     8 / log2-scale, so exponentials stay below 2^8 and most tiles skip the
//     rescale of the 64 accumulators.
//   * Staging: every thread owns 2 K and 2 V 16-byte chunks of a tile, fetched two
//     tiles ahead into registers by buffer loads whose descriptor ends at the
//     last visible key (rows past it read as zero without traffic), then stored
//     to one of two padded LDS buffers; one barrier per tile.
//   * Grid (B * Hkv, row blocks), row blocks in reverse so the longest key ranges
//     start first; workgroup ids of one (sequence, KV head) differ by a multiple
//     of B * Hkv, which keeps its row blocks on one XCD (and its K/V in one L2)
//     when B * Hkv is a multiple of 8.
//   * FUSED: the call also stores the K / V rows of its query tokens (positions
//     qs + t) into the cache. Keys at or past qs are read from those rows instead of
//     the cache (so no workgroup reads a cache row this call writes), and each new row
//     is stored by exactly one workgroup before its loop: the row block holding the
//     last query row of its token (rows u G .. u G + G - 1 of token u), or the split
//     whose key range holds it (the last split for rows past the visible length). The
//     copy's loads are issued with the first tiles' and share their wait. Measured and
//     not kept: stores from the staging registers inside the loop (the address
//     arithmetic and branches sat in every step), and the copy after the loop (its
//     load latency then sat at the end of every workgroup; its stores alone there
//     were slower too).
template <bool F16, bool PAGED, bool SPLIT, bool FUSED, int NW>
__global__ __launch_bounds__(64 * NW, 2) void kv_prefill_kernel(FDLLM_LEAD_PARAMS, const AttnParams p) {
  FDLLM_LEAD_LOCAL;
  constexpr int D = 128;
  constexpr int KT = 64;
  constexpr int NT = 64 * NW;      // threads
  constexpr int ROWS = 32 * NW;    // query rows per workgroup
  constexpr int CPT = 1024 / NT;   // 16-byte chunks of a K (or V) tile per thread
  constexpr int RPS = NT / 16;     // key rows covered by one chunk index
  static_assert(NW == 8 || (NW == 4 && !SPLIT), "split mode keeps 256 rows per workgroup");
  constexpr int KS = D + 8;  // K row stride in LDS: 16-byte pad
  // V in two regions, columns 32 d + [0, 16) in the first and 32 d + [16, 32) in the
  // second (row stride 80 elements each), the second shifted by 128 bytes past the
  // first: the transposing reads of lanes 16-31 (the upper 16 columns of the rows lanes
  // 0-15 read) then fall on the other half of the banks
  constexpr int VS2 = 80;
  constexpr int VOFF = KT * VS2 + 64;
  constexpr int KBUF = KT * KS;
  constexpr int VBUF = 2 * VOFF;
  __shared__ __attribute__((aligned(16))) uint16_t sKV[2][KBUF + VBUF];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int n32 = lane & 31;
  const int h = lane >> 5;
  const int l16 = lane & 15;
  const int g16 = lane >> 4;

  int b, kvh, rb, k_lo, k_hi, n_act, split, first;
  SeqInfo si;
  if constexpr (SPLIT) {
    // one row block of at most 256 rows per (sequence, KV head); keys split as in the
    // split decode kernel, in 64-key tiles
    kvh = blockIdx.y;
    const DecodePart dp = decode_partition<PAGED, KT>(p, ld);
    if (dp.b < 0) return;  // idle slot (uniform over the workgroup)
    b = __builtin_amdgcn_readfirstlane(dp.b);
    split = __builtin_amdgcn_readfirstlane(dp.split);
    n_act = __builtin_amdgcn_readfirstlane(dp.n_act);
    first = __builtin_amdgcn_readfirstlane(dp.first);
    k_lo = __builtin_amdgcn_readfirstlane(dp.k_lo);
    k_hi = __builtin_amdgcn_readfirstlane(dp.k_hi);
    rb = 0;
    si.seqlen = dp.seqlen;
    si.qs = dp.qs;
    si.kv_end = dp.kv_end;
  } else {
    const int unit = blockIdx.x;
    b = unit / p.Hkv;
    kvh = unit - b * p.Hkv;
    rb = p.n_rb - 1 - static_cast<int>(blockIdx.y);
    si = seq_info<PAGED>(p, ld, b, rb);
    k_lo = 0;
    k_hi = si.kv_end;
    n_act = 1;
    split = first = 0;
  }
  const int row0 = rb * ROWS;
  const int ntiles = k_hi > k_lo ? (k_hi - k_lo + KT - 1) / KT : 0;

  // FUSED: new rows at key positions [w_lo, w_hi) are this workgroup's to store
  int w_lo = 0, w_hi = 0;
  if constexpr (FUSED) {
    const int qend = si.qs + p.Sq;
    if constexpr (SPLIT) {
      w_lo = max(k_lo, si.qs);
      w_hi = split == n_act - 1 ? qend : min(k_hi, qend);
    } else {
      w_lo = si.qs + (ROWS * rb) / p.G;
      w_hi = si.qs + min(p.Sq, (ROWS * (rb + 1)) / p.G);
    }
    w_lo = __builtin_amdgcn_readfirstlane(max(w_lo, 0));
    w_hi = __builtin_amdgcn_readfirstlane(min(w_hi, p.cap));
  }

  // ---- this lane's query row: Q^T fragments and key limit
  const int r = row0 + wave * 32 + n32;
  const int rc = min(r, p.R - 1);  // padding rows reuse a valid row: finite, never written
  const int t = rc / p.G;
  const int hh = rc - t * p.G;
  const int lim = row_key_limit(p, si.seqlen, si.qs, t);
  u32x4 qf[8];
  {
    const uint16_t* qrow = p.q + b * p.q_sb + t * p.q_ss + (kvh * p.G + hh) * p.q_sh;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) qf[ks] = *reinterpret_cast<const u32x4*>(qrow + 16 * ks + 8 * h);
  }
  const int lim_min =
      __builtin_amdgcn_readfirstlane(-static_cast<int>(wave_allreduce_max(-static_cast<float>(lim))));
  const int lim_max = __builtin_amdgcn_readfirstlane(static_cast<int>(wave_allreduce_max(static_cast<float>(lim))));
  const float c2 = p.scale_log2;
  const float rescale_thr = 8.f / c2;

  f32x16 acc[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[dt][e] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;

  // ---- staging: chunk c = tid + NT i of a tile is key c / 16, 16-byte column c % 16
  const int krow_bytes = static_cast<int>(p.k_ss) * 2;
  const int vrow_bytes = static_cast<int>(p.v_ss) * 2;
  int koff[CPT], voff[CPT];
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int c = tid + NT * i;
    koff[i] = (c >> 4) * krow_bytes + (c & 15) * 16;
    voff[i] = (c >> 4) * vrow_bytes + (c & 15) * 16;
  }
  const uint16_t* kbase = p.k + kvh * p.k_sh + (PAGED ? 0 : b * p.k_sp);
  const uint16_t* vbase = p.v + kvh * p.v_sh + (PAGED ? 0 : b * p.v_sp);
  const int32_t* pt_row = PAGED ? ld.page_table + static_cast<int64_t>(b) * ld.max_pages : nullptr;
  struct Stage {
    u32x4 k[CPT];
    u32x4 v[CPT];
  };
  Stage st0, st1;

  // FUSED staging: per 32-key half, from the cache (keys before qs), from the new
  // rows (keys from qs on), or, for the half that holds qs, one load per lane from its
  // own row's source (rows past k_hi repeat row k_hi - 1, whose scores are masked).
  const int hrow = tid >> 4;        // row of this thread's chunk 0 (chunk i: hrow + RPS i)
  const int hcol = (tid & 15) * 8;  // element column of the chunks
  const uint16_t* knbase = FUSED ? p.kn + b * p.n_sb + kvh * p.n_sh : nullptr;
  const uint16_t* vnbase = FUSED ? p.vn + b * p.n_sb + kvh * p.n_sh : nullptr;
  const int nrow_bytes = FUSED ? static_cast<int>(p.n_ss) * 2 : 0;
  // page of the 32-key half starting at kh (kh a multiple of 32, pages of >= 32 keys:
  // every key of the half is on it); a uniform index, so a scalar load
  auto half_page = [&](int kh) -> int {
    if constexpr (PAGED) {
      return pt_row[min(kh >> p.page_shift, p.max_pages - 1)];
    } else {
      return 0;
    }
  };
  // element offset of key's row from kbase / vbase, given the page of its half
  auto cache_off = [&](int page, int key, bool kcache) -> int64_t {
    const int64_t ss = kcache ? p.k_ss : p.v_ss;
    if constexpr (PAGED) {
      return static_cast<int64_t>(page) * (kcache ? p.k_sp : p.v_sp) + (key & (p.page_size - 1)) * ss;
    } else {
      return static_cast<int64_t>(key) * ss;
    }
  };
  // the chunks of half `half` (32 keys from kh): chunk i holds key row hrow + RPS i of the tile
  auto load_half_fused = [&](Stage& sg, int half, int kh) {
    const int valid = __builtin_amdgcn_readfirstlane(max(0, min(32, k_hi - kh)));
    const int qs = si.qs;
    const int page = half_page(kh);
    if (kh < qs && qs < kh + 32 && valid > 0) {  // wave-uniform
      // addresses of both sources, then one load per lane (same load count as below)
#pragma unroll
      for (int i = 0; i < CPT; ++i) {
        if ((RPS * i) / 32 != half) continue;  // compile-time
        const int key = min(kh + hrow + RPS * i - 32 * half, k_hi - 1);
        const uint16_t* kc = kbase + cache_off(page, key, true);
        const uint16_t* vc = vbase + cache_off(page, key, false);
        const uint16_t* kq = knbase + static_cast<int64_t>(key - qs) * p.n_ss;
        const uint16_t* vq = vnbase + static_cast<int64_t>(key - qs) * p.n_ss;
        const bool nw = key >= qs;
        sg.k[i] = *reinterpret_cast<const u32x4*>((nw ? kq : kc) + hcol);
        sg.v[i] = *reinterpret_cast<const u32x4*>((nw ? vq : vc) + hcol);
      }
      return;
    }
    const uint16_t* kp;
    const uint16_t* vp;
    int kbytes, vbytes;
    if (kh >= qs) {
      kp = knbase + static_cast<int64_t>(kh - qs) * p.n_ss;
      vp = vnbase + static_cast<int64_t>(kh - qs) * p.n_ss;
      kbytes = vbytes = nrow_bytes;
    } else {
      kp = kbase + cache_off(page, kh, true);
      vp = vbase + cache_off(page, kh, false);
      kbytes = krow_bytes;
      vbytes = vrow_bytes;
    }
    const __amdgpu_buffer_rsrc_t kr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(kp), 0, valid * kbytes, kBufferFlags);
    const __amdgpu_buffer_rsrc_t vr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(vp), 0, valid * vbytes, kBufferFlags);
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      if ((RPS * i) / 32 != half) continue;  // compile-time
      const int row = hrow + RPS * i - 32 * half;
      sg.k[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(kr, row * kbytes + hcol * 2, 0, 0));
      sg.v[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(vr, row * vbytes + hcol * 2, 0, 0));
    }
  };
  int noff[CPT];  // FUSED: byte offsets of this thread's chunks in a tile of new rows
#pragma unroll
  for (int i = 0; i < CPT; ++i) noff[i] = (hrow + RPS * i) * nrow_bytes + hcol * 2;
  auto load_tile = [&](Stage& sg, int j) {
    const int kb = k_lo + j * KT;
    if constexpr (FUSED) {
      const int qs = si.qs;
      if (kb >= qs) {  // wave-uniform: the whole tile is new rows (every tile of a plain prefill)
        const int valid = __builtin_amdgcn_readfirstlane(max(0, min(KT, k_hi - kb)));
        const int64_t noffs = static_cast<int64_t>(kb - qs) * p.n_ss;
        const __amdgpu_buffer_rsrc_t kr = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(knbase + noffs), 0,
                                                                            valid * nrow_bytes, kBufferFlags);
        const __amdgpu_buffer_rsrc_t vr = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(vnbase + noffs), 0,
                                                                            valid * nrow_bytes, kBufferFlags);
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
          sg.k[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(kr, noff[i], 0, 0));
          sg.v[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(vr, noff[i], 0, 0));
        }
        return;
      }
      if (kb + KT > qs) {  // wave-uniform: the tile that holds qs, half by half
        load_half_fused(sg, 0, kb);
        load_half_fused(sg, 1, kb + 32);
        return;
      }
      // otherwise every row of the tile is cached: the statement below
    }
    if constexpr (PAGED) {
      if (p.page_size < KT) {
        // 32-key pages: chunk i of every thread (key row tid / 16 + RPS i) lies in key
        // half (RPS i) / 32 of the tile, each half on its own page
#pragma unroll
        for (int half = 0; half < 2; ++half) {
          const int kh = kb + 32 * half;
          const int valid = __builtin_amdgcn_readfirstlane(max(0, min(32, k_hi - kh)));
          const int page = pt_row[min(kh >> p.page_shift, p.max_pages - 1)];
          const int slot0 = kh & (p.page_size - 1);
          const int64_t koffs = static_cast<int64_t>(page) * p.k_sp + slot0 * p.k_ss;
          const int64_t voffs = static_cast<int64_t>(page) * p.v_sp + slot0 * p.v_ss;
          const __amdgpu_buffer_rsrc_t kr = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(kbase + koffs), 0,
                                                                              valid * krow_bytes, kBufferFlags);
          const __amdgpu_buffer_rsrc_t vr = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(vbase + voffs), 0,
                                                                              valid * vrow_bytes, kBufferFlags);
#pragma unroll
          for (int i = 0; i < CPT; ++i) {
            if ((RPS * i) / 32 != half) continue;  // compile-time
            sg.k[i] = __builtin_bit_cast(
                u32x4, __builtin_amdgcn_raw_buffer_load_b128(kr, koff[i] - 32 * half * krow_bytes, 0, 0));
            sg.v[i] = __builtin_bit_cast(
                u32x4, __builtin_amdgcn_raw_buffer_load_b128(vr, voff[i] - 32 * half * vrow_bytes, 0, 0));
          }
        }
        return;
      }
    }
    const int valid = __builtin_amdgcn_readfirstlane(max(0, min(KT, k_hi - kb)));
    int64_t koffs, voffs;
    if constexpr (PAGED) {
      // page_size >= 64 and tiles start at multiples of 64: one page per tile
      const int page = pt_row[min(kb >> p.page_shift, p.max_pages - 1)];
      const int slot0 = kb & (p.page_size - 1);
      koffs = static_cast<int64_t>(page) * p.k_sp + slot0 * p.k_ss;
      voffs = static_cast<int64_t>(page) * p.v_sp + slot0 * p.v_ss;
    } else {
      koffs = static_cast<int64_t>(kb) * p.k_ss;
      voffs = static_cast<int64_t>(kb) * p.v_ss;
    }
    const __amdgpu_buffer_rsrc_t kr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(kbase + koffs), 0, valid * krow_bytes, kBufferFlags);
    const __amdgpu_buffer_rsrc_t vr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(vbase + voffs), 0, valid * vrow_bytes, kBufferFlags);
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      sg.k[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(kr, koff[i], 0, 0));
      sg.v[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(vr, voff[i], 0, 0));
    }
  };
  auto store_tile = [&](const Stage& sg, int buf) {
    uint16_t* sk = sKV[buf];
    uint16_t* sv = sk + KBUF;
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = tid + NT * i;
      *reinterpret_cast<u32x4*>(&sk[(c >> 4) * KS + (c & 15) * 8]) = sg.k[i];
      *reinterpret_cast<u32x4*>(&sv[((c >> 1) & 1) * VOFF + (c >> 4) * VS2 + ((c >> 2) & 3) * 16 + (c & 1) * 8]) =
          sg.v[i];
    }
  };
  auto compute_tile = [&](int buf, int kb) {
    const uint16_t* sk = sKV[buf];
    const uint16_t* sv = sk + KBUF;
    f32x16 s[2];
    {
      // the 16 K fragments are read ahead of their products: four reads first, then
      // one read per product, so each read has three products' time to land
      u32x4 kf[8][2];
#pragma unroll
      for (int ks = 0; ks < 8; ++ks)
#pragma unroll
        for (int st = 0; st < 2; ++st)
          kf[ks][st] = *reinterpret_cast<const u32x4*>(&sk[(32 * st + n32) * KS + 16 * ks + 8 * h]);
#pragma unroll
      for (int st = 0; st < 2; ++st)
#pragma unroll
        for (int e = 0; e < 16; ++e) s[st][e] = 0.f;
#pragma unroll
      for (int ks = 0; ks < 8; ++ks)
#pragma unroll
        for (int st = 0; st < 2; ++st) s[st] = mfma32x32x16<F16>(kf[ks][st], qf[ks], s[st]);
      __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);  // DS reads
#pragma unroll
      for (int i = 0; i < 12; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
    }
    if (!(kb + KT <= lim_min)) {  // wave-uniform: some row of the wave sees part of the tile
#pragma unroll
      for (int st = 0; st < 2; ++st)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (kb + 32 * st + 8 * i + 4 * h + j >= lim) s[st][4 * i + j] = -INFINITY;
    }
    float mx = -INFINITY;
#pragma unroll
    for (int st = 0; st < 2; ++st)
#pragma unroll
      for (int e = 0; e < 16; ++e) mx = fmaxf(mx, s[st][e]);
    mx = halves_max(mx);
    if (__builtin_amdgcn_ballot_w64(mx > m_run + rescale_thr) != 0) {
      const float m_new = fmaxf(m_run, mx);
      const float alpha = m_run == -INFINITY ? 0.f : fast_exp2((m_run - m_new) * c2);
      l_run *= alpha;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) acc[dt] *= alpha;
      m_run = m_new;
    }
    const float mc = m_run == -INFINITY ? 0.f : m_run * c2;
    float lsum = 0.f;
#pragma unroll
    for (int st = 0; st < 2; ++st)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const float v = fast_exp2(fmaf(s[st][e], c2, -mc));
        s[st][e] = v;
        lsum += v;
      }
    l_run += lsum;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int st = kk >> 1;
      const int e0 = 8 * (kk & 1);
      const u32x4 pf = {pack2<F16>(s[st][e0], s[st][e0 + 1]), pack2<F16>(s[st][e0 + 2], s[st][e0 + 3]),
                        pack2<F16>(s[st][e0 + 4], s[st][e0 + 5]), pack2<F16>(s[st][e0 + 6], s[st][e0 + 7])};
      const int vr = 16 * kk + 4 * (g16 >> 1) + (l16 >> 2);
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        // column 32 dt + 16 (g16 & 1) + 4 (l16 & 3) in the split layout
        const int vi = (g16 & 1) * VOFF + 16 * dt + 4 * (l16 & 3);
        const u32x2 lo = __builtin_bit_cast(u32x2, lds_read_tr16(&sv[vi + vr * VS2]));
        const u32x2 hi = __builtin_bit_cast(u32x2, lds_read_tr16(&sv[vi + (vr + 8) * VS2]));
        acc[dt] = mfma32x32x16<F16>(u32x4{lo[0], lo[1], hi[0], hi[1]}, pf, acc[dt]);
      }
    }
  };

  // Every step stores, synchronises and issues its loads whether or not its tile
  // exists (loads past the range are zero-filled without traffic), so the loads in
  // flight are the same on every path; only the math is conditional.
  auto step = [&](Stage& sg, int j) {
    store_tile(sg, j & 1);
    lds_barrier();
    if (FDLLM_TIMELINE && j == 0) FDLLM_STAMP(2, __builtin_amdgcn_s_memrealtime());  // first tiles in LDS
    load_tile(sg, j + 2);
    const int kb = k_lo + j * KT;
    if (j < ntiles && kb < lim_max) compute_tile(j & 1, kb);  // wave-uniform
  };
  // FUSED: the owned new rows go into the cache before the loop, 2 NT 16-byte chunks of
  // each tensor per round (two per thread). The first round's loads are issued with the
  // first tiles' and wait alongside them; more rounds (> NT / 8 owned rows) run after.
  const int own_n = FUSED ? max(0, w_hi - w_lo) * 16 : 0;  // chunks per tensor
  struct Own {
    u32x4 k[2], v[2];
    int page[2];
  };
  auto own_load = [&](Own& o, int base) {
    const int64_t roff = static_cast<int64_t>(w_lo - si.qs) * p.n_ss;
    const __amdgpu_buffer_rsrc_t kr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(knbase + roff), 0, own_n > 0 ? (w_hi - w_lo) * nrow_bytes : 0, kBufferFlags);
    const __amdgpu_buffer_rsrc_t vr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(vnbase + roff), 0, own_n > 0 ? (w_hi - w_lo) * nrow_bytes : 0, kBufferFlags);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int c = base + tid + NT * i;  // row c / 16 of the owned range, chunk c % 16
      const int off = (c >> 4) * nrow_bytes + (c & 15) * 16;
      o.k[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(kr, off, 0, 0));
      o.v[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(vr, off, 0, 0));
      o.page[i] = 0;
      if constexpr (PAGED) {
        const int key = max(0, min(w_lo + (c >> 4), w_hi - 1));  // in range even with nothing owned
        o.page[i] = pt_row[min(key >> p.page_shift, p.max_pages - 1)];
      }
    }
  };
  auto own_store = [&](const Own& o, int base) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int c = base + tid + NT * i;
      if (c < own_n) {
        const int key = w_lo + (c >> 4);
        const int col = (c & 15) * 8;
        *reinterpret_cast<u32x4*>(const_cast<uint16_t*>(kbase) + cache_off(o.page[i], key, true) + col) = o.k[i];
        *reinterpret_cast<u32x4*>(const_cast<uint16_t*>(vbase) + cache_off(o.page[i], key, false) + col) = o.v[i];
      }
    }
  };
  Own own;
  if constexpr (FUSED) own_load(own, 0);
  if (ntiles > 0) {
    load_tile(st0, 0);
    load_tile(st1, 1);
  }
  if constexpr (FUSED) {
    own_store(own, 0);
    for (int base = 2 * NT; base < own_n; base += 2 * NT) {
      own_load(own, base);
      own_store(own, base);
    }
  }
  if (ntiles > 0) {
    for (int j = 0; j < ntiles; j += 2) {
      step(st0, j);
      step(st1, j + 1);
    }
  }

  // ---- epilogue: rows of both lane halves are whole after the exchange of l
  l_run = halves_sum(l_run);
  if constexpr (SPLIT) {
    // the unit's (first slot, splits) for the merge kernel, rewritten on every call by
    // the workgroup of split 0: every unit has one, also a unit of a single split,
    // which the merge kernel then skips (its entry must not be left from an earlier call)
    if (split == 0 && tid == 0 && p.ws_unit != nullptr) p.ws_unit[b * p.Hkv + kvh] = make_int2(first, n_act);
    if (n_act > 1) {
      split_prefill_partial(p, first, split, r, h, acc, m_run, l_run);
      return;
    }
  }
  if (r < p.R) {
    const float inv = l_run > 0.f ? 1.f / l_run : 0.f;
    uint16_t* orow = p.out + b * p.o_sb + t * p.o_ss + (kvh * p.G + hh) * p.o_sh;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int e = 4 * i;
        *reinterpret_cast<u32x2*>(orow + 32 * dt + 8 * i + 4 * h) =
            u32x2{pack2<F16>(acc[dt][e] * inv, acc[dt][e + 1] * inv),
                  pack2<F16>(acc[dt][e + 2] * inv, acc[dt][e + 3] * inv)};
      }
  }
}

// 1: the ping-pong schedule below (two tiles in flight); 0: the plain schedule (three
// tiles in flight, every wave runs S, softmax, PV in turn). On the 4 x 4096-token
// prefill the ping-pong form measured 475-482 us against 484-488 us for the plain one.
#ifndef FDLLM_PREFILL_PIPE
#define FDLLM_PREFILL_PIPE 1
#endif
// LDS operand reads issued ahead of their MFMA in the ring kernel's ping-pong phases:
// K fragments of S = K Q^T, and the V^T fragment pairs of O^T += V^T P^T (0 leaves the
// PV order to the compiler, which kept one to two MFMAs of reads in flight). Measured on
// one box (4 x 4096 prefill with the cache write / bs16 full-block step): PV 0 465.0 /
// 45.56 us, PV 4 459.6 / 45.19 us; PV 2, 6, 8 within 0.3 % of PV 4 or slower; QK 8
// instead of 4 no faster (465.9 / 45.75 us).
#ifndef FDLLM_QK_READ_AHEAD
#define FDLLM_QK_READ_AHEAD 4
#endif
// 1: the ring kernel sums a tile's probabilities in four partial sums instead of one
// chain. Measured and not kept: 465.9 -> 464.1 us / 46.81 -> 46.58 us on one box, within
// the spread between boxes, and it changes the sums' rounding.
#ifndef FDLLM_RING_LSUM_TREE
#define FDLLM_RING_LSUM_TREE 0
#endif
#ifndef FDLLM_PV_READ_AHEAD
#define FDLLM_PV_READ_AHEAD 4
#endif
// Key halves (32 keys) whose page ids the ring prefill kernel stages in LDS: 65536 keys
// per workgroup; longer paged ranges take kv_prefill_kernel.
constexpr int kRingMaxHalves = 2048;

// ---------------------------------------------------------------------------
// Prefill attention with direct-to-LDS staging (same work split, math and results
// as kv_prefill_kernel).
//   * K / V tiles go from memory straight into a ring of four LDS slots
//     (buffer_load ... lds), three tiles in flight, one barrier per tile; no
//     staging registers and no LDS store instructions.
//   * Wave w loads key rows [8 w, 8 w + 8) of each tile, 4 rows (1 KB) per load.
//     Rows are 256 bytes without padding; bank conflicts of the MFMA operand reads
//     are avoided by an XOR swizzle of the 16-byte chunks, applied on the source
//     side: LDS chunk p of K row r holds column chunk p ^ (r & 15), of V row r
//     chunk p ^ 4 (r & 3).
template <bool F16, bool PAGED, bool SPLIT, bool FUSED>
__global__ __launch_bounds__(512, 2) void kv_prefill_ring_kernel(FDLLM_LEAD_PARAMS, const AttnParams p) {
  FDLLM_LEAD_LOCAL;
  FDLLM_STAMP(0, __builtin_amdgcn_s_memrealtime());  // start
  constexpr int D = 128;
  constexpr int KT = 64;
  constexpr int NSLOT = 4;
  constexpr int TB = KT * D * 2;       // bytes of one K (or V) tile
  constexpr int VREG = NSLOT * TB;     // V slots follow the K slots
  __shared__ __attribute__((aligned(1024))) uint8_t ring[2 * NSLOT * TB];
  // page ids of the workgroup's 32-key halves, read once: a page-table load inside the
  // loop would be a vector load the compiler waits for with vmcnt(0), which would also
  // wait for every tile in flight
  __shared__ int sPg[PAGED ? kRingMaxHalves : 1];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int n32 = lane & 31;
  const int h = lane >> 5;
  const int l16 = lane & 15;
  const int g16 = lane >> 4;

  int b, kvh, rb, k_lo, k_hi, n_act, split, first;
  SeqInfo si;
  if constexpr (SPLIT) {
    kvh = blockIdx.y;
    const DecodePart dp = decode_partition<PAGED, KT>(p, ld);
    FDLLM_STAMP(1, __builtin_amdgcn_s_memrealtime());  // partition known
    if (dp.b < 0) return;  // idle slot (uniform over the workgroup)
    b = __builtin_amdgcn_readfirstlane(dp.b);
    split = __builtin_amdgcn_readfirstlane(dp.split);
    n_act = __builtin_amdgcn_readfirstlane(dp.n_act);
    first = __builtin_amdgcn_readfirstlane(dp.first);
    k_lo = __builtin_amdgcn_readfirstlane(dp.k_lo);
    k_hi = __builtin_amdgcn_readfirstlane(dp.k_hi);
    rb = 0;
    si.seqlen = dp.seqlen;
    si.qs = dp.qs;
    si.kv_end = dp.kv_end;
  } else {
    const int unit = blockIdx.x;
    b = unit / p.Hkv;
    kvh = unit - b * p.Hkv;
    rb = p.n_rb - 1 - static_cast<int>(blockIdx.y);
    si = seq_info<PAGED>(p, ld, b, rb);
    k_lo = 0;
    k_hi = si.kv_end;
    n_act = 1;
    split = first = 0;
  }
  const int row0 = rb * 256;
  const int ntiles = k_hi > k_lo ? (k_hi - k_lo + KT - 1) / KT : 0;
  const int qs = si.qs;

  // FUSED: new rows at key positions [w_lo, w_hi) are this workgroup's to store
  int w_lo = 0, w_hi = 0;
  if constexpr (FUSED) {
    const int qend = qs + p.Sq;
    if constexpr (SPLIT) {
      w_lo = max(k_lo, qs);
      w_hi = split == n_act - 1 ? qend : min(k_hi, qend);
    } else {
      w_lo = qs + (256 * rb) / p.G;
      w_hi = qs + min(p.Sq, (256 * (rb + 1)) / p.G);
    }
    w_lo = __builtin_amdgcn_readfirstlane(max(w_lo, 0));
    w_hi = __builtin_amdgcn_readfirstlane(min(w_hi, p.cap));
  }

  // ---- this lane's query row: Q^T fragments and key limit
  const int r = row0 + wave * 32 + n32;
  const int rc = min(r, p.R - 1);  // padding rows reuse a valid row: finite, never written
  const int t = rc / p.G;
  const int hh = rc - t * p.G;
  const int lim = row_key_limit(p, si.seqlen, qs, t);
  u32x4 qf[8];  // loaded after the first tiles are issued (see the main loop)
  const int lim_min =
      __builtin_amdgcn_readfirstlane(-static_cast<int>(wave_allreduce_max(-static_cast<float>(lim))));
  // A wave whose 32 rows are all padding (past the unit's R rows: the full block's 224
  // rows fill 7 of the 8 waves) issues its share of the tile loads and passes every
  // barrier, but computes nothing: no tile is active for it (kb < INT_MIN never holds).
  const int lim_max =
      row0 + __builtin_amdgcn_readfirstlane(wave) * 32 >= p.R
          ? INT_MIN
          : __builtin_amdgcn_readfirstlane(static_cast<int>(wave_allreduce_max(static_cast<float>(lim))));
  const float c2 = p.scale_log2;
  const float rescale_thr = 8.f / c2;

  f32x16 acc[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[dt][e] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;

  const int krow_bytes = static_cast<int>(p.k_ss) * 2;
  const int vrow_bytes = static_cast<int>(p.v_ss) * 2;
  const uint16_t* kbase = p.k + kvh * p.k_sh + (PAGED ? 0 : b * p.k_sp);
  const uint16_t* vbase = p.v + kvh * p.v_sh + (PAGED ? 0 : b * p.v_sp);
  const int32_t* pt_row = PAGED ? ld.page_table + static_cast<int64_t>(b) * ld.max_pages : nullptr;
  const uint16_t* knbase = FUSED ? p.kn + b * p.n_sb + kvh * p.n_sh : nullptr;
  const uint16_t* vnbase = FUSED ? p.vn + b * p.n_sb + kvh * p.n_sh : nullptr;
  const int nrow_bytes = FUSED ? static_cast<int>(p.n_ss) * 2 : 0;

  // element offset of key's row from kbase / vbase, given the page of its 32-key half
  auto cache_off = [&](int page, int key, bool kcache) __attribute__((always_inline)) -> int64_t {
    const int64_t ss = kcache ? p.k_ss : p.v_ss;
    if constexpr (PAGED) {
      return static_cast<int64_t>(page) * (kcache ? p.k_sp : p.v_sp) + (key & (p.page_size - 1)) * ss;
    } else {
      return static_cast<int64_t>(key) * ss;
    }
  };
  // page of the 32-key half starting at kh (pages of >= 32 keys hold whole halves)
  const int n_halves = PAGED ? min(kRingMaxHalves, 2 * (ntiles + 6)) : 1;
  auto half_page = [&](int kh) __attribute__((always_inline)) -> int {
    if constexpr (PAGED) {
      return sPg[min((kh - k_lo) >> 5, n_halves - 1)];
    } else {
      return 0;
    }
  };

  // ---- DMA source offsets: load i (0, 1) of wave w covers tile rows 8 w + 4 i + lane / 16,
  // lane % 16 = the chunk's place in the LDS row; all of a wave's rows lie in half w / 4
  // (scalars, not arrays: a select between two arrays' elements would keep them in
  // scratch memory)
  const int half = __builtin_amdgcn_readfirstlane(wave >> 2);  // uniform: page lookups stay scalar loads
  const int hrow0 = 8 * (wave & 3) + (lane >> 4);  // half row of load 0; load 1: + 4
  const int hrow1 = hrow0 + 4;
  const int kc0 = (lane & 15) ^ ((hrow0 + 32 * half) & 15), kc1 = (lane & 15) ^ ((hrow1 + 32 * half) & 15);
  const int vc0 = (lane & 15) ^ ((hrow0 & 3) << 2), vc1 = (lane & 15) ^ ((hrow1 & 3) << 2);
  const int kso0 = hrow0 * krow_bytes + (kc0 << 4), kso1 = hrow1 * krow_bytes + (kc1 << 4);
  const int vso0 = hrow0 * vrow_bytes + (vc0 << 4), vso1 = hrow1 * vrow_bytes + (vc1 << 4);
  const int knso0 = hrow0 * nrow_bytes + (kc0 << 4), knso1 = hrow1 * nrow_bytes + (kc1 << 4);
  const int vnso0 = hrow0 * nrow_bytes + (vc0 << 4), vnso1 = hrow1 * nrow_bytes + (vc1 << 4);
  const uint32_t ring_lds = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(ring));
  const uint32_t kdst = ring_lds + 8 * wave * 256;
  const uint32_t vdst = ring_lds + VREG + 8 * wave * 256;

  // Tile tt into slot `slot`: 2 K and 2 V loads per wave (4 more where a 32-key half
  // holds qs: each lane then loads from its own row's source under an exec mask).
  // The SPLIT form reads each tile in one workgroup only and streams it (non-temporal:
  // 46.46 -> 45.75 us per bs16 full-block step); the prefill form's row blocks of one
  // (sequence, KV head) read the same tiles again from L2, so it keeps them cached
  // (non-temporal there: 456 -> 472 us for the 4 x 4096 attention).
  // mode (a constant at every call site, so each loop copy below folds it away):
  // 0 every key from the cache, 1 every key from the new rows, 2 either, per half / lane
  auto issue = [&](int tt, int slot, const int mode) __attribute__((always_inline)) {
    const int kh = k_lo + tt * KT + 32 * half;
    const int valid = __builtin_amdgcn_readfirstlane(max(0, min(32, k_hi - kh)));
    const uint32_t kd = kdst + slot * TB;
    const uint32_t vd = vdst + slot * TB;
    if (mode == 1) {
      const int64_t noffs = static_cast<int64_t>(kh - qs) * p.n_ss;
      const i32x4 ks = make_srd(knbase + noffs, valid * nrow_bytes);
      const i32x4 vs = make_srd(vnbase + noffs, valid * nrow_bytes);
      lds_dma16<SPLIT>(ks, knso0, kd);
      lds_dma16<SPLIT>(vs, vnso0, vd);
      lds_dma16<SPLIT>(ks, knso1, kd + 1024);
      lds_dma16<SPLIT>(vs, vnso1, vd + 1024);
      return;
    }
    const int page = half_page(kh);
    if (mode == 0) {
      const i32x4 ks = make_srd(kbase + cache_off(page, kh, true), valid * krow_bytes);
      const i32x4 vs = make_srd(vbase + cache_off(page, kh, false), valid * vrow_bytes);
      lds_dma16<SPLIT>(ks, kso0, kd);
      lds_dma16<SPLIT>(vs, vso0, vd);
      lds_dma16<SPLIT>(ks, kso1, kd + 1024);
      lds_dma16<SPLIT>(vs, vso1, vd + 1024);
      return;
    }
    if (FUSED && kh < qs && qs < kh + 32 && valid > 0) {
      const i32x4 kc = make_srd(kbase + cache_off(page, kh, true), (qs - kh) * krow_bytes);
      const i32x4 vc = make_srd(vbase + cache_off(page, kh, false), (qs - kh) * vrow_bytes);
      const i32x4 kq = make_srd(knbase, (kh + valid - qs) * nrow_bytes);
      const i32x4 vq = make_srd(vnbase, (kh + valid - qs) * nrow_bytes);
      // per lane: row key - qs of the new rows, or row key - kh of the cache rows
      const int d = (kh - qs) * nrow_bytes;  // shifts a new-row offset from half row hr to row kh + hr - qs
      if (kh + hrow0 >= qs) {
        lds_dma16<SPLIT>(kq, knso0 + d, kd);
        lds_dma16<SPLIT>(vq, vnso0 + d, vd);
      } else {
        lds_dma16<SPLIT>(kc, kso0, kd);
        lds_dma16<SPLIT>(vc, vso0, vd);
      }
      if (kh + hrow1 >= qs) {
        lds_dma16<SPLIT>(kq, knso1 + d, kd + 1024);
        lds_dma16<SPLIT>(vq, vnso1 + d, vd + 1024);
      } else {
        lds_dma16<SPLIT>(kc, kso1, kd + 1024);
        lds_dma16<SPLIT>(vc, vso1, vd + 1024);
      }
      return;
    }
    i32x4 ks, vs;
    const bool from_new = FUSED && kh >= qs;  // wave-uniform
    if (from_new) {
      const int64_t noffs = static_cast<int64_t>(kh - qs) * p.n_ss;
      ks = make_srd(knbase + noffs, valid * nrow_bytes);
      vs = make_srd(vnbase + noffs, valid * nrow_bytes);
    } else {
      ks = make_srd(kbase + cache_off(page, kh, true), valid * krow_bytes);
      vs = make_srd(vbase + cache_off(page, kh, false), valid * vrow_bytes);
    }
    // value selects (a conditional of two named ints is an lvalue: clang would select
    // their addresses and keep them in scratch memory)
    const int sel = from_new ? 1 : 0;
    lds_dma16<SPLIT>(ks, kso0 + sel * (knso0 - kso0), kd);
    lds_dma16<SPLIT>(vs, vso0 + sel * (vnso0 - vso0), vd);
    lds_dma16<SPLIT>(ks, kso1 + sel * (knso1 - kso1), kd + 1024);
    lds_dma16<SPLIT>(vs, vso1 + sel * (vnso1 - vso1), vd + 1024);
  };

  // ---- MFMA operand addresses (bytes from ring): K row 32 st + n32, chunk 2 ks + h;
  // V^T reads: rows 16 kk + 4 (g16 >> 1) + (l16 >> 2) (+ 8), columns 32 dt + 16 (g16 & 1) + 4 (l16 & 3)
  int kaddr[8], vaddr[4];
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) kaddr[ks] = n32 * 256 + (((2 * ks + h) ^ (n32 & 15)) << 4);
  {
    const int vrow = 4 * (g16 >> 1) + (l16 >> 2);
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      const int lc = 4 * dt + 2 * (g16 & 1) + ((l16 >> 1) & 1);
      vaddr[dt] = VREG + vrow * 256 + ((lc ^ ((l16 >> 2) << 2)) << 4) + ((l16 & 1) << 3);
    }
  }

  auto compute_tile = [&](int slot, int kb) __attribute__((always_inline)) {
    const uint8_t* sk = ring + slot * TB;
    const uint8_t* sv = ring + slot * TB;
    f32x16 s[2];
    {
      u32x4 kf[8][2];
#pragma unroll
      for (int ks = 0; ks < 8; ++ks)
#pragma unroll
        for (int st = 0; st < 2; ++st) kf[ks][st] = *reinterpret_cast<const u32x4*>(sk + st * 8192 + kaddr[ks]);
#pragma unroll
      for (int st = 0; st < 2; ++st)
#pragma unroll
        for (int e = 0; e < 16; ++e) s[st][e] = 0.f;
#pragma unroll
      for (int ks = 0; ks < 8; ++ks)
#pragma unroll
        for (int st = 0; st < 2; ++st) s[st] = mfma32x32x16<F16>(kf[ks][st], qf[ks], s[st]);
      __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);  // DS reads
#pragma unroll
      for (int i = 0; i < 12; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
    }
    if (!(kb + KT <= lim_min)) {  // wave-uniform: some row of the wave sees part of the tile
#pragma unroll
      for (int st = 0; st < 2; ++st)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (kb + 32 * st + 8 * i + 4 * h + j >= lim) s[st][4 * i + j] = -INFINITY;
    }
    float mx = -INFINITY;
#pragma unroll
    for (int st = 0; st < 2; ++st)
#pragma unroll
      for (int e = 0; e < 16; ++e) mx = fmaxf(mx, s[st][e]);
    mx = halves_max(mx);
    if (__builtin_amdgcn_ballot_w64(mx > m_run + rescale_thr) != 0) {
      const float m_new = fmaxf(m_run, mx);
      const float alpha = m_run == -INFINITY ? 0.f : fast_exp2((m_run - m_new) * c2);
      l_run *= alpha;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) acc[dt] *= alpha;
      m_run = m_new;
    }
    const float mc = m_run == -INFINITY ? 0.f : m_run * c2;
    float lsum = 0.f;
#pragma unroll
    for (int st = 0; st < 2; ++st)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const float v = fast_exp2(fmaf(s[st][e], c2, -mc));
        s[st][e] = v;
        lsum += v;
      }
    l_run += lsum;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int st = kk >> 1;
      const int e0 = 8 * (kk & 1);
      const u32x4 pf = {pack2<F16>(s[st][e0], s[st][e0 + 1]), pack2<F16>(s[st][e0 + 2], s[st][e0 + 3]),
                        pack2<F16>(s[st][e0 + 4], s[st][e0 + 5]), pack2<F16>(s[st][e0 + 6], s[st][e0 + 7])};
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        const u32x2 lo = __builtin_bit_cast(u32x2, lds_read_tr16(reinterpret_cast<const uint16_t*>(
                                                       sv + kk * 4096 + vaddr[dt])));
        const u32x2 hi = __builtin_bit_cast(u32x2, lds_read_tr16(reinterpret_cast<const uint16_t*>(
                                                       sv + kk * 4096 + 2048 + vaddr[dt])));
        acc[dt] = mfma32x32x16<F16>(u32x4{lo[0], lo[1], hi[0], hi[1]}, pf, acc[dt]);
      }
    }
  };

  // ---- ping-pong form (FDLLM_PREFILL_PIPE): each wave alternates an MFMA phase (PV of
  // tile j - 1, then S of tile j) and a VALU phase (softmax of tile j into packed P), and
  // the two waves of a SIMD (w and w + 4) run half a step apart: waves 0-3 pass the
  // step's barrier before their MFMA phase, waves 4-7 before their VALU phase, so on
  // every SIMD one wave's MFMAs run beside the other wave's softmax.
  auto qk = [&](int slot, f32x16 (&s)[2]) __attribute__((always_inline)) {
    const uint8_t* sk = ring + slot * TB;
    u32x4 kf[8][2];
#pragma unroll
    for (int ks = 0; ks < 8; ++ks)
#pragma unroll
      for (int st = 0; st < 2; ++st) kf[ks][st] = *reinterpret_cast<const u32x4*>(sk + st * 8192 + kaddr[ks]);
#pragma unroll
    for (int st = 0; st < 2; ++st)
#pragma unroll
      for (int e = 0; e < 16; ++e) s[st][e] = 0.f;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks)
#pragma unroll
      for (int st = 0; st < 2; ++st) s[st] = mfma32x32x16<F16>(kf[ks][st], qf[ks], s[st]);
    constexpr int RA = FDLLM_QK_READ_AHEAD;
    __builtin_amdgcn_sched_group_barrier(0x100, RA, 0);  // DS reads
#pragma unroll
    for (int i = 0; i < 16 - RA; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
    }
    __builtin_amdgcn_sched_group_barrier(0x008, RA, 0);
  };
  auto pv = [&](const u32x4 (&P)[4], int slot) __attribute__((always_inline)) {
    const uint8_t* sv = ring + slot * TB;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        const u32x2 lo = __builtin_bit_cast(u32x2, lds_read_tr16(reinterpret_cast<const uint16_t*>(
                                                       sv + kk * 4096 + vaddr[dt])));
        const u32x2 hi = __builtin_bit_cast(u32x2, lds_read_tr16(reinterpret_cast<const uint16_t*>(
                                                       sv + kk * 4096 + 2048 + vaddr[dt])));
        acc[dt] = mfma32x32x16<F16>(u32x4{lo[0], lo[1], hi[0], hi[1]}, P[kk], acc[dt]);
      }
    if constexpr (FDLLM_PV_READ_AHEAD > 0) {
      constexpr int RA = FDLLM_PV_READ_AHEAD;  // MFMAs whose two reads go ahead
      __builtin_amdgcn_sched_group_barrier(0x100, 2 * RA, 0);
#pragma unroll
      for (int i = 0; i < 16 - RA; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, RA, 0);
    }
  };
  // softmax of the scores s of the tile at keys kb: mask, running max (lazy rescale of
  // acc), exponentials, running sum; P = the probabilities packed as the PV operand
  auto softmax_p = [&](f32x16 (&s)[2], int kb, u32x4 (&P)[4]) __attribute__((always_inline)) {
    if (!(kb + KT <= lim_min)) {  // wave-uniform: some row of the wave sees part of the tile
#pragma unroll
      for (int st = 0; st < 2; ++st)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (kb + 32 * st + 8 * i + 4 * h + j >= lim) s[st][4 * i + j] = -INFINITY;
    }
    float mx = -INFINITY;
#pragma unroll
    for (int st = 0; st < 2; ++st)
#pragma unroll
      for (int e = 0; e < 16; ++e) mx = fmaxf(mx, s[st][e]);
    mx = halves_max(mx);
    if (__builtin_amdgcn_ballot_w64(mx > m_run + rescale_thr) != 0) {
      const float m_new = fmaxf(m_run, mx);
      const float alpha = m_run == -INFINITY ? 0.f : fast_exp2((m_run - m_new) * c2);
      l_run *= alpha;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) acc[dt] *= alpha;
      m_run = m_new;
    }
    const float mc = m_run == -INFINITY ? 0.f : m_run * c2;
#if FDLLM_RING_LSUM_TREE
    float ls[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int st = 0; st < 2; ++st)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const float v = fast_exp2(fmaf(s[st][e], c2, -mc));
        s[st][e] = v;
        ls[e & 3] += v;
      }
    l_run += (ls[0] + ls[1]) + (ls[2] + ls[3]);
#else
    float lsum = 0.f;
#pragma unroll
    for (int st = 0; st < 2; ++st)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const float v = fast_exp2(fmaf(s[st][e], c2, -mc));
        s[st][e] = v;
        lsum += v;
      }
    l_run += lsum;
#endif
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int st = kk >> 1;
      const int e0 = 8 * (kk & 1);
      P[kk] = u32x4{pack2<F16>(s[st][e0], s[st][e0 + 1]), pack2<F16>(s[st][e0 + 2], s[st][e0 + 3]),
                    pack2<F16>(s[st][e0 + 4], s[st][e0 + 5]), pack2<F16>(s[st][e0 + 6], s[st][e0 + 7])};
    }
  };

  // ---- FUSED: the owned new rows into the cache. The first 1024 chunks of each tensor
  // (64 rows; all of them at GQA >= 4) are loaded before the first tiles are issued and
  // stored after the common wait below, so their round trip overlaps the tiles' and
  // Q's; any further rows are copied after that, in rounds. Measured and not kept: the
  // stores after the loop (498 us against 486-492 us on the 4 x 4096 prefill).
  const int own_n = FUSED ? max(0, w_hi - w_lo) * 16 : 0;  // 16-byte chunks per tensor
  u32x4 own_k[2], own_v[2];
  int own_pg[2] = {0, 0};
  auto own_load = [&](int base) __attribute__((always_inline)) {
    const int64_t roff = static_cast<int64_t>(w_lo - qs) * p.n_ss;
    const int bytes = own_n > 0 ? (w_hi - w_lo) * nrow_bytes : 0;
    const __amdgpu_buffer_rsrc_t kr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(knbase + roff), 0, bytes, kBufferFlags);
    const __amdgpu_buffer_rsrc_t vr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(vnbase + roff), 0, bytes, kBufferFlags);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int c = base + tid + 512 * i;  // row c / 16 of the owned range, chunk c % 16
      const int off = (c >> 4) * nrow_bytes + (c & 15) * 16;
      own_k[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(kr, off, 0, 0));
      own_v[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(vr, off, 0, 0));
      if constexpr (PAGED) {
        const int key = max(0, min(w_lo + (c >> 4), w_hi - 1));  // in range even with nothing owned
        own_pg[i] = pt_row[min(key >> p.page_shift, p.max_pages - 1)];
      }
    }
  };
  auto own_store = [&](int base) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int c = base + tid + 512 * i;
      if (c < own_n) {
        const int key = w_lo + (c >> 4);
        const int col = (c & 15) * 8;
        *reinterpret_cast<u32x4*>(const_cast<uint16_t*>(kbase) + cache_off(own_pg[i], key, true) + col) = own_k[i];
        *reinterpret_cast<u32x4*>(const_cast<uint16_t*>(vbase) + cache_off(own_pg[i], key, false) + col) = own_v[i];
      }
    }
  };
  if constexpr (FUSED) own_load(0);

  // ---- main loop: tile j in slot j % 4; tiles j + 1, j + 2 in flight; tile j + 3
  // issued into the slot step j - 1 read, after the barrier that ends that step
  // The first tiles (0-2 here, 0-1 in the ping-pong form) are covered by the full wait
  // after the prologue, so their steps skip the count wait: the owned rows' stores
  // (FUSED) are issued after that wait, count in vmcnt like loads and are older than
  // every later tile, so a count wait there would wait for their acknowledgement.
  auto step = [&](int j, int slot, const int mode) __attribute__((always_inline)) {
    if (j >= 3) wait_vmcnt<8>();  // this wave's loads of tile j have landed (two younger tiles in flight)
    lds_barrier();                // ... and every wave's; every wave is done with step j - 1
    issue(j + 3, (slot + 3) & 3, mode);
    const int kb = k_lo + j * KT;
    if (j < ntiles && kb < lim_max) compute_tile(slot, kb);  // wave-uniform
  };
  if constexpr (PAGED) {
    for (int i = tid; i < n_halves; i += 512) sPg[i] = pt_row[min((k_lo + 32 * i) >> p.page_shift, p.max_pages - 1)];
    __syncthreads();
  }
  // The first tiles, then the query fragments, then one wait for all of them (or, for
  // the forms without a cache write, the query rows first, below). The compiler sees
  // that wait (a builtin, unlike the loads' asm): it knows qf has landed and puts no
  // wait of its own for qf inside the loop, where a vmcnt(0) would drain the tiles in
  // flight every step; the query-first form reads qf from LDS, which needs no such wait.
  // source of the keys: the cache only (no new rows, or all of them past k_hi), the new
  // rows only (the plain prefill: qs <= k_lo), or both
  const int src_mode = !FUSED || qs >= k_hi ? 0 : (qs <= k_lo ? 1 : 2);
  // Without the cache write (and in the ping-pong form), the query rows go first, straight
  // into the LDS of ring slots 2 and 3 (free until tile 2 is issued, after barrier instance
  // 0): each wave loads the 32 rows it computes, local row lr at the K region 2 TB + 256 lr
  // (lr < 128) or the V region VREG + 2 TB + 256 (lr - 128), its 16-byte chunks XOR-swizzled
  // by lr & 15; then tiles 0 and 1; the wait covers the rows and tile 0 only, so the first
  // step's math starts while tile 1 is in flight (the first steps then wait for tile 1).
  const int64_t q_span = (static_cast<int64_t>(p.Sq - 1) * p.q_ss + static_cast<int64_t>(p.Hq - 1) * p.q_sh + D) * 2;
  const bool early_q = !FUSED && FDLLM_PREFILL_PIPE && q_span <= 0x7fffffff;  // uniform
  if (early_q) {
    const i32x4 qsrd = make_srd(p.q + b * p.q_sb, static_cast<int>(q_span));
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int lr0 = 32 * wave + 4 * i;  // rows lr0 .. lr0 + 3 of this load
      const int lr = lr0 + (lane >> 4);
      const int rq = min(row0 + lr, p.R - 1);  // padding rows load a valid row, never used
      const int tq = rq / p.G;
      const int hq = rq - tq * p.G;
      const int off = (tq * static_cast<int>(p.q_ss) + (kvh * p.G + hq) * static_cast<int>(p.q_sh)) * 2 +
                      (((lane & 15) ^ (lr & 15)) << 4);
      const uint32_t dst = ring_lds + (lr0 < 128 ? 2 * TB + lr0 * 256 : VREG + 2 * TB + (lr0 - 128) * 256);
      lds_dma16<false>(qsrd, off, dst);
    }
  }
  // tiles 0, 1 (and 2 for the plain form, which keeps three in flight)
  if (ntiles > 0) {
    if (src_mode == 0) {
      issue(0, 0, 0);
      issue(1, 1, 0);
      if (!FDLLM_PREFILL_PIPE) issue(2, 2, 0);
    } else if (src_mode == 1) {
      issue(0, 0, 1);
      issue(1, 1, 1);
      if (!FDLLM_PREFILL_PIPE) issue(2, 2, 1);
    } else {
      issue(0, 0, 2);
      issue(1, 1, 2);
      if (!FDLLM_PREFILL_PIPE) issue(2, 2, 2);
    }
  }
  if (early_q) {
    if (ntiles > 0) wait_vmcnt<4>();  // the rows and tile 0 (tile 1's 4 loads may be in flight)
    else wait_vmcnt<0>();
    lds_barrier();  // orders the LDS reads below after the wait
    const int lr = 32 * wave + n32;
    const int rbase = lr < 128 ? 2 * TB + lr * 256 : VREG + 2 * TB + (lr - 128) * 256;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks)
      qf[ks] = *reinterpret_cast<const u32x4*>(ring + rbase + (((2 * ks + h) ^ (lr & 15)) << 4));
  } else {
    const uint16_t* qrow = p.q + b * p.q_sb + t * p.q_ss + (kvh * p.G + hh) * p.q_sh;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) qf[ks] = *reinterpret_cast<const u32x4*>(qrow + 16 * ks + 8 * h);
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0) expcnt(7) lgkmcnt(15): vector memory only
  }
  FDLLM_STAMP(2, __builtin_amdgcn_s_memrealtime());  // first tiles and Q landed (this wave)
  if constexpr (FUSED) {
    own_store(0);
    for (int base = 1024; base < own_n; base += 1024) {  // more than 64 owned rows (GQA < 4)
      own_load(base);
      own_store(base);
    }
  }
  auto run = [&](const int mode) __attribute__((always_inline)) {
    for (int j = 0; j < ntiles; j += 4) {
      step(j, 0, mode);
      step(j + 1, 1, mode);
      step(j + 2, 2, mode);
      step(j + 3, 3, mode);
    }
  };
  if (ntiles > 0 && !FDLLM_PREFILL_PIPE) {
    if (src_mode == 0) run(0);
    else if (src_mode == 1) run(1);
    else run(2);
    wait_vmcnt<0>();  // no load may land in LDS after the workgroup ends
  }
  if (ntiles > 0 && FDLLM_PREFILL_PIPE) {
    // Barrier instance i (once per step for every wave): tile i has landed in every
    // wave's view, and every wave is done with the LDS reads of steps before i - 1
    // (K of i - 1, V of i - 2), so tile i + 2 goes into slot (i + 2) % 4 right after it.
    // Waves 0-3 pass instance j just before step j's MFMA phase; waves 4-7 pass it in
    // the prologue (j = 0) or just before step j - 1's VALU phase. Both groups pass
    // ceil4(ntiles) + 1 instances.
    const int grp = __builtin_amdgcn_readfirstlane(wave >> 2);
    u32x4 P[4];
    f32x16 s[2];
    bool prev_active = false;
    auto pstep = [&](int j, int slot, const int mode) __attribute__((always_inline)) {
      if (grp == 0) {
        // this wave's loads of tile j have landed (tile j + 1 in flight); the prologue's wait
        // covered tiles 0 and 1, or tile 0 only with the query rows loaded first
        if (j >= (early_q ? 1 : 2)) wait_vmcnt<4>();
        lds_barrier();
        issue(j + 2, (slot + 2) & 3, mode);
      }
      if (prev_active) pv(P, (slot + 3) & 3);  // PV of tile j - 1
      const int kb = k_lo + j * KT;
      const bool act = j < ntiles && kb < lim_max;  // wave-uniform
      if (act) qk(slot, s);
      if (grp == 1) {
        // this wave's loads of tile j + 1 have landed (tile j + 2 in flight)
        if (j >= (early_q ? 0 : 1)) wait_vmcnt<4>();
        lds_barrier();                // instance j + 1
        issue(j + 3, (slot + 3) & 3, mode);
      }
      if (act) softmax_p(s, kb, P);
      prev_active = act;
    };
    auto prun = [&](const int mode) __attribute__((always_inline)) {
      if (grp == 1) {  // instance 0 (tile 0, and tile 1 unless the query rows went first, waited for above)
        lds_barrier();
        issue(2, 2, mode);
      }
      for (int j = 0; j < ntiles; j += 4) {
        pstep(j, 0, mode);
        pstep(j + 1, 1, mode);
        pstep(j + 2, 2, mode);
        pstep(j + 3, 3, mode);
      }
      if (grp == 0) lds_barrier();  // the last instance
    };
    if (src_mode == 0) prun(0);
    else if (src_mode == 1) prun(1);
    else prun(2);
    if (prev_active) pv(P, ((ntiles + 3) / 4 * 4 - 1) & 3);  // PV of the last step's tile
    wait_vmcnt<0>();  // no load may land in LDS after the workgroup ends
  }
  FDLLM_STAMP(3, __builtin_amdgcn_s_memrealtime());  // key loop done (this wave)
  FDLLM_STAMP(6, (static_cast<uint64_t>(b) << 48) | (static_cast<uint64_t>(split) << 32) |
                     (static_cast<uint64_t>(n_act) << 16) | static_cast<uint64_t>(ntiles));

  // ---- epilogue: rows of both lane halves are whole after the exchange of l
  l_run = halves_sum(l_run);
  if constexpr (SPLIT) {
    // the unit's (first slot, splits) for the merge kernel, rewritten on every call by
    // the workgroup of split 0: every unit has one, also a unit of a single split,
    // which the merge kernel then skips (its entry must not be left from an earlier call)
    if (split == 0 && tid == 0 && p.ws_unit != nullptr) p.ws_unit[b * p.Hkv + kvh] = make_int2(first, n_act);
    if (n_act > 1) {
      split_prefill_partial(p, first, split, r, h, acc, m_run, l_run);
      FDLLM_STAMP(4, __builtin_amdgcn_s_memrealtime());  // partial stores issued
      return;
    }
  }
  if (r < p.R) {
    const float inv = l_run > 0.f ? 1.f / l_run : 0.f;
    uint16_t* orow = p.out + b * p.o_sb + t * p.o_ss + (kvh * p.G + hh) * p.o_sh;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int e = 4 * i;
        *reinterpret_cast<u32x2*>(orow + 32 * dt + 8 * i + 4 * h) =
            u32x2{pack2<F16>(acc[dt][e] * inv, acc[dt][e + 1] * inv),
                  pack2<F16>(acc[dt][e + 2] * inv, acc[dt][e + 3] * inv)};
      }
  }
  FDLLM_STAMP(4, __builtin_amdgcn_s_memrealtime());  // output stores issued
}

// Merge of the split prefill kernel's partials: grid (row chunks of 32, units),
// 256 threads = 32 rows x 8 column groups. The unit's slots and split count come from
// the table the kernel wrote in the same call; units with one split were written by
// the kernel itself. Spreading the merge over the whole chip instead of the last
// workgroup of each unit matters here: a unit's partials are 224 rows x 520 bytes
// per split, several hundred KB, more than one compute unit reads quickly. Partial
// rows stay fp32 in both split kernels. Measured and not kept, bf16 rows: the
// full-block step went from 44.6 to 42.1 us on one box, but the 7B end-to-end greedy
// agreement fell from 0.872 / 0.875 to 0.867 / 0.869 against a noise floor of 0.874
// (s.e. 0.0013), a systematic loss; in the split decode kernel bf16 was also slower
// (27.6 -> 27.9 us).
template <bool F16>
__global__ __launch_bounds__(256) void kv_split_prefill_merge_kernel(const AttnParams p) {
  const int unit = blockIdx.y;
  const int2 e = p.ws_unit[unit];
  if (e.y <= 1) return;
  const int b = unit / p.Hkv;
  const int kvh = unit - b * p.Hkv;
  const int item0 = static_cast<int>(blockIdx.x) * 256;
  merge_splits_n<F16, 256, 0>(p, b, kvh, e.x, e.y, item0 + static_cast<int>(threadIdx.x), 256,
                              min(p.R * 8, item0 + 256));
}

// Merge the split partials of every (sequence, KV head, row block) with more than
// one active split. 8 output columns per thread, D / 8 threads per row.
template <int D, bool F16, bool PAGED, bool OUT_F32 = false>
__global__ __launch_bounds__(256) void kv_attn_combine_kernel(const AttnParams p) {
  constexpr int TPR = D / 8;
  constexpr int RPB = 256 / TPR;
  constexpr int U = 4;  // splits whose loads are in flight together
  const int unit = blockIdx.y;
  const int bh = unit / p.n_rb;
  const int rb = unit - bh * p.n_rb;
  const int b = bh / p.Hkv;
  const int kvh = bh - b * p.Hkv;
  const SeqInfo si = seq_info<PAGED>(p, b, rb);
  if (si.n_act <= 1) return;  // written directly by the attention kernel
  const int rl = blockIdx.x * RPB + threadIdx.x / TPR;
  const int r = rb * p.rows_per_wg + rl;
  if (rl >= p.rows_per_wg || r >= p.R) return;
  const int d0 = (threadIdx.x % TPR) * 8;
  const int64_t base = static_cast<int64_t>(unit) * p.n_splits * p.rows_per_wg + rl;

  // online merge: m = running reference max, l / o scaled to it; the fp32 kernel's
  // partials carry m in base-2 score units already (scale applied)
  const float ms = OUT_F32 ? 1.f : p.scale_log2;
  float m = -INFINITY, l = 0.f;
  float o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int sp0 = 0; sp0 < si.n_act; sp0 += U) {
    float2 ml[U];
    f32x4 x0[U], x1[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t sl = base + static_cast<int64_t>(min(sp0 + u, si.n_act - 1)) * p.rows_per_wg;
      ml[u] = p.ws_ml[sl];
      const f32x4* po = reinterpret_cast<const f32x4*>(p.ws_o + sl * D + d0);
      x0[u] = po[0];
      x1[u] = po[1];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (sp0 + u >= si.n_act) break;
      const float mn = fmaxf(m, ml[u].x);
      if (mn == -INFINITY) continue;  // neither side has a visible key yet
      const float a = m == -INFINITY ? 0.f : fast_exp2((m - mn) * ms);
      const float w = ml[u].x == -INFINITY ? 0.f : fast_exp2((ml[u].x - mn) * ms);
      l = l * a + w * ml[u].y;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        o[j] = o[j] * a + w * x0[u][j];
        o[4 + j] = o[4 + j] * a + w * x1[u][j];
      }
      m = mn;
    }
  }
  const float inv = l > 0.f ? 1.f / l : 0.f;
  const int t = r / p.G;
  const int hh = r - t * p.G;
  if constexpr (OUT_F32) {
    float* orow = reinterpret_cast<float*>(p.out) + b * p.o_sb + t * p.o_ss + (kvh * p.G + hh) * p.o_sh + d0;
#pragma unroll
    for (int j = 0; j < 8; ++j) orow[j] = o[j] * inv;
  } else {
    uint16_t* orow = p.out + b * p.o_sb + t * p.o_ss + (kvh * p.G + hh) * p.o_sh + d0;
    u32x4 w4;
#pragma unroll
    for (int j = 0; j < 4; ++j) w4[j] = pack2<F16>(o[2 * j] * inv, o[2 * j + 1] * inv);
    *reinterpret_cast<u32x4*>(orow) = w4;
  }
}

// ---------------------------------------------------------------------------
// KV cache write (StaticKVCache.update / write_scratch_compiled / write_sparse)
// ---------------------------------------------------------------------------
struct KVWriteArgs {
  const uint16_t* k_new;
  const uint16_t* v_new;
  int64_t n_sb, n_ss, n_sh;
  uint16_t* k_cache;
  uint16_t* v_cache;
  int64_t c_sp, c_ss, c_sh;
  const int32_t* page_table;
  int max_pages, page_size, max_seqlen;
  const int32_t* write_start;
  int write_offset;
  const int64_t* positions;
  int pos_bias;  // added to write_start[b] / write_offset (the attention call's fallback write)
  int B, T, Hkv, D;
};

// One 16-byte vector per thread; grid covers B * T * Hkv * D / 8 vectors.
__global__ __launch_bounds__(256) void kv_write_kernel(const KVWriteArgs a) {
  const int dch = a.D / 8;
  const int64_t n = static_cast<int64_t>(a.B) * a.T * a.Hkv * dch;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int dc = static_cast<int>(i % dch);
  int64_t rest = i / dch;
  const int h = static_cast<int>(rest % a.Hkv);
  rest /= a.Hkv;
  const int t = static_cast<int>(rest % a.T);
  const int b = static_cast<int>(rest / a.T);
  int64_t pos;
  if (a.positions) {
    pos = a.positions[static_cast<int64_t>(b) * a.T + t];
  } else {
    pos = static_cast<int64_t>(a.write_start ? a.write_start[b] : a.write_offset) + a.pos_bias + t;
  }
  int64_t off;
  if (a.page_table) {
    if (pos < 0 || pos >= static_cast<int64_t>(a.max_pages) * a.page_size) return;
    const int page = a.page_table[static_cast<int64_t>(b) * a.max_pages + pos / a.page_size];
    off = page * a.c_sp + (pos % a.page_size) * a.c_ss;
  } else {
    if (pos < 0 || pos >= a.max_seqlen) return;
    off = b * a.c_sp + pos * a.c_ss;
  }
  off += h * a.c_sh + dc * 8;
  const int64_t src = b * a.n_sb + t * a.n_ss + h * a.n_sh + dc * 8;
  *reinterpret_cast<u32x4*>(a.k_cache + off) = *reinterpret_cast<const u32x4*>(a.k_new + src);
  *reinterpret_cast<u32x4*>(a.v_cache + off) = *reinterpret_cast<const u32x4*>(a.v_new + src);
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
// The plan (kernel family, workspace, grids, argument checks) is host-only code in
// attn_plan.h; the launchers below take the grids it computes.

inline dim3 to_dim3(const GridDims& g) { return dim3(g.x, g.y, g.z); }

template <int D, bool F16, bool PAGED>
void launch_combine(const AttnParams& p, dim3 cgrid, hipStream_t s) {
  kv_attn_combine_kernel<D, F16, PAGED><<<cgrid, dim3(256), 0, s>>>(p);
}

// The ring kernel (direct-to-LDS staging) takes prefill shapes; the split kernel for
// full-block decode stays on register staging, which measured faster there (46.4 against
// 47.3 us per full-block step: the ring kernel's first tiles and Q wait in series).
#ifndef FDLLM_PREFILL_RING
#define FDLLM_PREFILL_RING 1
#endif
template <bool SPLIT, bool FUSED>
void launch_prefill(const AttnParams& p, bool f16, dim3 grid, hipStream_t s) {
  constexpr int NW = SPLIT ? 8 : kPrefillWaves;
  const bool paged = p.page_table != nullptr;
  const dim3 block(64 * NW);
  const int64_t max_keys = paged ? std::min<int64_t>(p.max_seqlen, static_cast<int64_t>(p.max_pages) * p.page_size)
                                 : p.max_seqlen;
  if (FDLLM_PREFILL_RING && (!SPLIT || FDLLM_PREFILL_RING_SPLIT) &&
      (!paged || max_keys + 6 * 64 <= static_cast<int64_t>(kRingMaxHalves) * 32)) {
    if (f16) {
      if (paged) kv_prefill_ring_kernel<true, true, SPLIT, FUSED><<<grid, dim3(512), 0, s>>>(FDLLM_LEAD_ARGS(p), p);
      else kv_prefill_ring_kernel<true, false, SPLIT, FUSED><<<grid, dim3(512), 0, s>>>(FDLLM_LEAD_ARGS(p), p);
    } else {
      if (paged) kv_prefill_ring_kernel<false, true, SPLIT, FUSED><<<grid, dim3(512), 0, s>>>(FDLLM_LEAD_ARGS(p), p);
      else kv_prefill_ring_kernel<false, false, SPLIT, FUSED><<<grid, dim3(512), 0, s>>>(FDLLM_LEAD_ARGS(p), p);
    }
    return;
  }
  if (f16) {
    if (paged) kv_prefill_kernel<true, true, SPLIT, FUSED, NW><<<grid, block, 0, s>>>(FDLLM_LEAD_ARGS(p), p);
    else kv_prefill_kernel<true, false, SPLIT, FUSED, NW><<<grid, block, 0, s>>>(FDLLM_LEAD_ARGS(p), p);
  } else {
    if (paged) kv_prefill_kernel<false, true, SPLIT, FUSED, NW><<<grid, block, 0, s>>>(FDLLM_LEAD_ARGS(p), p);
    else kv_prefill_kernel<false, false, SPLIT, FUSED, NW><<<grid, block, 0, s>>>(FDLLM_LEAD_ARGS(p), p);
  }
}

template <int HKV>
void launch_decode(const AttnParams& p, bool f16, const LaunchSet& ls, hipStream_t s) {
  const bool paged = p.page_table != nullptr;
  const dim3 grid = to_dim3(ls.main_grid);
  const dim3 block(128 * HKV);
  if (f16) {
    if (paged) kv_decode_kernel<HKV, true, true><<<grid, block, 0, s>>>(p);
    else kv_decode_kernel<HKV, true, false><<<grid, block, 0, s>>>(p);
  } else {
    if (paged) kv_decode_kernel<HKV, false, true><<<grid, block, 0, s>>>(p);
    else kv_decode_kernel<HKV, false, false><<<grid, block, 0, s>>>(p);
  }
  if (ls.second) {
    const dim3 cgrid = to_dim3(ls.second_grid);
    if (f16) {
      if (paged) launch_combine<128, true, true>(p, cgrid, s);
      else launch_combine<128, true, false>(p, cgrid, s);
    } else {
      if (paged) launch_combine<128, false, true>(p, cgrid, s);
      else launch_combine<128, false, false>(p, cgrid, s);
    }
  }
}

template <int D, int MT>
void launch_attn(const AttnParams& p, bool f16, const LaunchSet& ls, hipStream_t s) {
  const bool paged = p.page_table != nullptr;
  const dim3 grid = to_dim3(ls.main_grid);
  if (f16) {
    if (paged) kv_attn_kernel<D, MT, true, true><<<grid, dim3(kThreads), 0, s>>>(p);
    else kv_attn_kernel<D, MT, true, false><<<grid, dim3(kThreads), 0, s>>>(p);
  } else {
    if (paged) kv_attn_kernel<D, MT, false, true><<<grid, dim3(kThreads), 0, s>>>(p);
    else kv_attn_kernel<D, MT, false, false><<<grid, dim3(kThreads), 0, s>>>(p);
  }
  if (ls.second) {
    const dim3 cgrid = to_dim3(ls.second_grid);
    if (f16) {
      if (paged) launch_combine<D, true, true>(p, cgrid, s);
      else launch_combine<D, true, false>(p, cgrid, s);
    } else {
      if (paged) launch_combine<D, false, true>(p, cgrid, s);
      else launch_combine<D, false, false>(p, cgrid, s);
    }
  }
}

}  // namespace
}  // namespace fdllm

extern "C" int fdllm_kv_attn_workspace_size(const fdllm_kv_attn_desc* desc, size_t* bytes) {
  using namespace fdllm;
  FDLLM_CHECK_ARG(bytes != nullptr, "fdllm_kv_attn_workspace_size: null output");
  Plan pl;
  const int rc = make_plan(desc, &pl);
  if (rc != FDLLM_OK) return rc;
  *bytes = plan_workspace_bytes(desc, pl);
  return FDLLM_OK;
}

// The library's attention scratch (one copy per device; see fdllm_kv_attn_fwd_noalloc).
// In host code `scratch` names a host-side stand-in: kernels receive the device
// address that hipGetSymbolAddress returns for it, never the name itself.
static __device__ __align__(256) unsigned char scratch[FDLLM_KV_ATTN_SCRATCH_BYTES];

namespace fdllm {
namespace {

// Validates `d` against its plan and launches the kernels on `stream`, with the
// caller's workspace or the library's scratch (see fdllm_kv_attn_fwd_noalloc).
#if FDLLM_TIMELINE
uint64_t* g_timeline = nullptr;  // device buffer of the phase stamps (instrumented build only)
#endif

int kv_attn_launch(const fdllm_kv_attn_desc* d, const Plan& pl, void* workspace, size_t workspace_bytes,
                   void* stream) {
  if (d->batch == 0 || d->q_len == 0) return FDLLM_OK;
  int rc = validate_call(d, pl, workspace, workspace_bytes);
  if (rc != FDLLM_OK) return rc;
  LaunchSet ls;
  rc = plan_launches(d, pl, &ls);
  if (rc != FDLLM_OK) return rc;
  const size_t need = plan_workspace_bytes(d, pl);

  AttnParams p;
  p.q = static_cast<const uint16_t*>(d->q);
  p.q_sb = d->q_stride_b;
  p.q_ss = d->q_stride_s;
  p.q_sh = d->q_stride_h;
  p.k = static_cast<const uint16_t*>(d->k);
  p.k_sp = d->k_stride_page;
  p.k_ss = d->k_stride_slot;
  p.k_sh = d->k_stride_h;
  p.v = static_cast<const uint16_t*>(d->v);
  p.v_sp = d->v_stride_page;
  p.v_ss = d->v_stride_slot;
  p.v_sh = d->v_stride_h;
  p.out = static_cast<uint16_t*>(d->out);
  p.o_sb = d->out_stride_b;
  p.o_ss = d->out_stride_s;
  p.o_sh = d->out_stride_h;
  p.page_table = d->page_table;
  p.seqlens = d->seqlens;
  p.q_start = d->q_start;
  p.max_pages = d->max_pages;
  p.page_size = d->page_size;
  p.page_shift = 0;
  while (d->page_table && (1 << p.page_shift) < d->page_size) ++p.page_shift;
  p.max_seqlen = d->max_seqlen;
  p.B = d->batch;
  p.Sq = d->q_len;
  p.Hq = d->num_q_heads;
  p.Hkv = d->num_kv_heads;
  p.G = d->num_q_heads / d->num_kv_heads;
  p.R = pl.R;
  p.rows_per_wg = pl.rows_per_wg;
  p.n_rb = pl.n_rb;
  p.n_splits = pl.n_splits;
  p.chunk = pl.chunk;
  p.mask_mode = d->mask_mode;
  p.mask_block = d->mask_block > 0 ? d->mask_block : 1;
  p.scale_log2 = d->softmax_scale * 1.4426950408889634f;
  p.kn = static_cast<const uint16_t*>(d->k_new);
  p.vn = static_cast<const uint16_t*>(d->v_new);
  p.n_sb = d->new_stride_b;
  p.n_ss = d->new_stride_s;
  p.n_sh = d->new_stride_h;
  p.cap = d->page_table ? static_cast<int>(std::min<int64_t>(static_cast<int64_t>(d->max_pages) * d->page_size,
                                                              int64_t{1} << 30))
                        : d->max_seqlen;
#if FDLLM_TIMELINE
  p.tl = g_timeline;
#endif
  if (need > 0) {
    char* w = static_cast<char*>(workspace);
    p.ws_cnt = reinterpret_cast<int*>(w);
    w += kCounterBytes;
    p.ws_ml = reinterpret_cast<float2*>(w);
    p.ws_o = reinterpret_cast<float*>(w + align256(pl.ws_ml_bytes));
    p.ws_unit = pl.kind == kPlanSplitPrefill ? reinterpret_cast<int2*>(w + pl.ws_unit_off) : nullptr;
  } else {
    p.ws_cnt = nullptr;
    p.ws_ml = nullptr;
    p.ws_o = nullptr;
    p.ws_unit = nullptr;
  }
  const bool f16 = d->dtype == FDLLM_DTYPE_F16;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (pl.kind == kPlanF32) {
    // 4 FDLLM_F32_ROWS_PER_WAVE rows of one (sequence, KV head) per workgroup
    const dim3 grid = to_dim3(ls.main_grid);
    const bool paged = d->page_table != nullptr;
    const bool merge = plan_f32_merge_in_kernel(pl, d->batch, d->num_kv_heads);
    if (d->head_dim == 128) {
      if (merge) {
        if (paged) kv_attn_f32_kernel<2, true, true><<<grid, dim3(256), 0, s>>>(p);
        else kv_attn_f32_kernel<2, false, true><<<grid, dim3(256), 0, s>>>(p);
      } else {
        if (paged) kv_attn_f32_kernel<2, true, false><<<grid, dim3(256), 0, s>>>(p);
        else kv_attn_f32_kernel<2, false, false><<<grid, dim3(256), 0, s>>>(p);
      }
    } else {
      if (merge) {
        if (paged) kv_attn_f32_kernel<1, true, true><<<grid, dim3(256), 0, s>>>(p);
        else kv_attn_f32_kernel<1, false, true><<<grid, dim3(256), 0, s>>>(p);
      } else {
        if (paged) kv_attn_f32_kernel<1, true, false><<<grid, dim3(256), 0, s>>>(p);
        else kv_attn_f32_kernel<1, false, false><<<grid, dim3(256), 0, s>>>(p);
      }
    }
    if (ls.second) {  // key splits: fold the partials of each row block
      const dim3 cgrid = to_dim3(ls.second_grid);
      if (d->head_dim == 128) {
        if (paged) kv_attn_combine_kernel<128, false, true, true><<<cgrid, dim3(256), 0, s>>>(p);
        else kv_attn_combine_kernel<128, false, false, true><<<cgrid, dim3(256), 0, s>>>(p);
      } else {
        if (paged) kv_attn_combine_kernel<64, false, true, true><<<cgrid, dim3(256), 0, s>>>(p);
        else kv_attn_combine_kernel<64, false, false, true><<<cgrid, dim3(256), 0, s>>>(p);
      }
    }
    FDLLM_RETURN_LAUNCH_STATUS("fdllm_kv_attn_fwd");
  }
  // Cache write of the call (k_new / v_new): inside the prefill kernels, otherwise (and
  // with FDLLM_ATTN_CACHE_WRITE_KERNEL or an explicit q_start) as a kernel of its own
  // before the attention, at q_start[b] + t (seqlens[b] - q_len + t). On the 4 x 4096-token
  // prefill, timed in rotation: 473-475 us in-kernel against 479-480 us with the copy kernel.
  const bool fuse_write = plan_fuses_cache_write(d, pl);
  if (ls.write) {
    KVWriteArgs a;
    a.k_new = p.kn;
    a.v_new = p.vn;
    a.n_sb = p.n_sb;
    a.n_ss = p.n_ss;
    a.n_sh = p.n_sh;
    a.k_cache = const_cast<uint16_t*>(p.k);
    a.v_cache = const_cast<uint16_t*>(p.v);
    a.c_sp = p.k_sp;
    a.c_ss = p.k_ss;
    a.c_sh = p.k_sh;
    a.page_table = p.page_table;
    a.max_pages = p.max_pages;
    a.page_size = p.page_size;
    a.max_seqlen = p.max_seqlen;
    a.write_start = p.q_start ? p.q_start : p.seqlens;
    a.write_offset = 0;
    a.positions = nullptr;
    a.pos_bias = p.q_start ? 0 : -p.Sq;
    a.B = p.B;
    a.T = p.Sq;
    a.Hkv = p.Hkv;
    a.D = d->head_dim;
    kv_write_kernel<<<to_dim3(ls.write_grid), dim3(256), 0, s>>>(a);
  }
  if (pl.kind == kPlanBalancedDecode) {
    const bool paged = p.page_table != nullptr;
    const dim3 grid = to_dim3(ls.main_grid);
    if (f16) {
      if (paged) kv_balanced_decode_kernel<true, true><<<grid, dim3(512), 0, s>>>(FDLLM_LEAD_ARGS(p), p);
      else kv_balanced_decode_kernel<true, false><<<grid, dim3(512), 0, s>>>(FDLLM_LEAD_ARGS(p), p);
    } else {
      if (paged) kv_balanced_decode_kernel<false, true><<<grid, dim3(512), 0, s>>>(FDLLM_LEAD_ARGS(p), p);
      else kv_balanced_decode_kernel<false, false><<<grid, dim3(512), 0, s>>>(FDLLM_LEAD_ARGS(p), p);
    }
    FDLLM_RETURN_LAUNCH_STATUS("fdllm_kv_attn_fwd");
  }
  if (pl.kind == kPlanSplitDecode) {
    const bool paged = p.page_table != nullptr;
    const dim3 grid = to_dim3(ls.main_grid);
    if (f16) {
      if (paged) kv_split_decode_kernel<kDecodeStages, true, true><<<grid, dim3(256 * kDecodeTeams), 0, s>>>(FDLLM_LEAD_ARGS(p), p);
      else kv_split_decode_kernel<kDecodeStages, true, false><<<grid, dim3(256 * kDecodeTeams), 0, s>>>(FDLLM_LEAD_ARGS(p), p);
    } else {
      if (paged) kv_split_decode_kernel<kDecodeStages, false, true><<<grid, dim3(256 * kDecodeTeams), 0, s>>>(FDLLM_LEAD_ARGS(p), p);
      else kv_split_decode_kernel<kDecodeStages, false, false><<<grid, dim3(256 * kDecodeTeams), 0, s>>>(FDLLM_LEAD_ARGS(p), p);
    }
    FDLLM_RETURN_LAUNCH_STATUS("fdllm_kv_attn_fwd");
  }
  if (pl.kind == kPlanPrefill) {
    const dim3 grid = to_dim3(ls.main_grid);
    if (fuse_write) launch_prefill<false, true>(p, f16, grid, s);
    else launch_prefill<false, false>(p, f16, grid, s);
    FDLLM_RETURN_LAUNCH_STATUS("fdllm_kv_attn_fwd");
  }
  if (pl.kind == kPlanSplitPrefill) {
    const dim3 grid = to_dim3(ls.main_grid);
    if (fuse_write) launch_prefill<true, true>(p, f16, grid, s);
    else launch_prefill<true, false>(p, f16, grid, s);
    if (ls.second) {
      // one workgroup row per (sequence, KV head); 32 rows per workgroup
      const dim3 mgrid = to_dim3(ls.second_grid);
      if (f16) kv_split_prefill_merge_kernel<true><<<mgrid, dim3(256), 0, s>>>(p);
      else kv_split_prefill_merge_kernel<false><<<mgrid, dim3(256), 0, s>>>(p);
    }
    FDLLM_RETURN_LAUNCH_STATUS("fdllm_kv_attn_fwd");
  }
  if (pl.decode) {
    switch (d->num_kv_heads) {
      case 1: launch_decode<1>(p, f16, ls, s); break;
      case 2: launch_decode<2>(p, f16, ls, s); break;
      case 4: launch_decode<4>(p, f16, ls, s); break;
      default: launch_decode<8>(p, f16, ls, s); break;
    }
    FDLLM_RETURN_LAUNCH_STATUS("fdllm_kv_attn_fwd");
  }
  if (d->head_dim == 128) {
    if (pl.MT == 1) launch_attn<128, 1>(p, f16, ls, s);
    else if (pl.MT == 2) launch_attn<128, 2>(p, f16, ls, s);
    else launch_attn<128, 4>(p, f16, ls, s);
  } else {
    if (pl.MT == 1) launch_attn<64, 1>(p, f16, ls, s);
    else if (pl.MT == 2) launch_attn<64, 2>(p, f16, ls, s);
    else launch_attn<64, 4>(p, f16, ls, s);
  }
  FDLLM_RETURN_LAUNCH_STATUS("fdllm_kv_attn_fwd");
}

// ---------------------------------------------------------------------------
// Library-owned scratch for fdllm_kv_attn_fwd_noalloc: the same layout as a caller
// workspace (counters, then (m, l) pairs, then partial rows), in a file-scope device
// array, so the entry point allocates nothing. Every device that runs the library
// holds its own copy at its own address until the process ends.
// ---------------------------------------------------------------------------
constexpr size_t kScratchBytes = static_cast<size_t>(FDLLM_KV_ATTN_SCRATCH_BYTES);
static_assert(kScratchBytes > kCounterBytes, "scratch must hold the arrival counters");

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices] = {};  // device address of `scratch`, per device

// Clears the arrival counters at the head of a device's scratch (a fill kernel, not a
// memset node, so nothing but a kernel enters a stream).
__global__ __launch_bounds__(256) void zero_words_kernel(uint32_t* p, int n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = 0u;
}

// Device address of the current device's scratch. The first call on a device
// resolves it with that device current, clears the counters on `stream` and waits for
// the clear; it is refused under stream capture, where the clearing kernel would only
// run at replay.
int scratch_for_current_device(hipStream_t stream, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    set_last_error("fdllm_kv_attn_fwd_noalloc: hipGetDevice failed: %s", hipGetErrorString(e));
    return static_cast<int>(e);
  }
  FDLLM_CHECK_ARG(dev >= 0 && dev < kMaxScratchDevices, "fdllm_kv_attn_fwd_noalloc: device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    e = hipStreamIsCapturing(stream, &cs);
    if (e != hipSuccess) {
      set_last_error("fdllm_kv_attn_fwd_noalloc: hipStreamIsCapturing failed: %s", hipGetErrorString(e));
      return static_cast<int>(e);
    }
    if (cs != hipStreamCaptureStatusNone) {
      set_last_error(
          "fdllm_kv_attn_fwd_noalloc: the first call on device %d must not be under stream capture "
          "(it clears the scratch counters); make one call before capturing",
          dev);
      return FDLLM_ERR_UNSUPPORTED;
    }
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr) {
      set_last_error("fdllm_kv_attn_fwd_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                     hipGetErrorString(e));
      return e != hipSuccess ? static_cast<int>(e) : FDLLM_ERR_UNSUPPORTED;
    }
    constexpr int kWords = static_cast<int>(kCounterBytes / sizeof(uint32_t));
    zero_words_kernel<<<dim3((kWords + 255) / 256), dim3(256), 0, stream>>>(static_cast<uint32_t*>(ptr), kWords);
    e = hipGetLastError();
    // Waited for here, once per device, so that a later call from any stream or
    // thread runs after the clear, not only one that follows it on `stream`.
    if (e == hipSuccess) e = hipStreamSynchronize(stream);
    if (e != hipSuccess) {
      set_last_error("fdllm_kv_attn_fwd_noalloc: clearing the scratch failed: %s", hipGetErrorString(e));
      return static_cast<int>(e);
    }
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return FDLLM_OK;
}

}  // namespace
}  // namespace fdllm

extern "C" int fdllm_kv_attn_fwd(const fdllm_kv_attn_desc* d, void* workspace, size_t workspace_bytes,
                                 void* stream) {
  using namespace fdllm;
  Plan pl;
  const int rc = make_plan(d, &pl);
  if (rc != FDLLM_OK) return rc;
  return kv_attn_launch(d, pl, workspace, workspace_bytes, stream);
}

#if FDLLM_TIMELINE
// Instrumented build only (not part of include/fdllm_hip.h): later attention calls
// write their split decode kernel's phase stamps, 8 uint64 words per workgroup
// (linear workgroup id), into `stamps` (device memory; null detaches). The caller
// sizes it for the grid and clears it before a call.
extern "C" int fdllm_timeline_attach(void* stamps) {
  fdllm::g_timeline = static_cast<uint64_t*>(stamps);
  return FDLLM_OK;
}
#endif

extern "C" int fdllm_kv_attn_fwd_noalloc(const fdllm_kv_attn_desc* d, void* stream) {
  using namespace fdllm;
  Plan pl;
  int rc = make_plan(d, &pl);
  if (rc != FDLLM_OK) return rc;
  const size_t need = plan_workspace_bytes(d, pl);
  if (need > kScratchBytes) {
    set_last_error("fdllm_kv_attn_fwd_noalloc: this call needs %zu bytes of scratch, above the library's "
                   "maximum of %zu (FDLLM_KV_ATTN_SCRATCH_BYTES); use fdllm_kv_attn_fwd with a workspace",
                   need, kScratchBytes);
    return FDLLM_ERR_WORKSPACE;
  }
  if (d->batch == 0 || d->q_len == 0) return FDLLM_OK;
  void* ws = nullptr;
  if (need > 0) {
    rc = scratch_for_current_device(static_cast<hipStream_t>(stream), &ws);
    if (rc != FDLLM_OK) return rc;
  }
  return kv_attn_launch(d, pl, ws, need > 0 ? kScratchBytes : 0, stream);
}

extern "C" int fdllm_kv_cache_write(const void* k_new, const void* v_new,
                                    int64_t new_stride_b, int64_t new_stride_s, int64_t new_stride_h,
                                    void* k_cache, void* v_cache,
                                    int64_t cache_stride_page, int64_t cache_stride_slot, int64_t cache_stride_h,
                                    const int32_t* page_table, int32_t max_pages, int32_t page_size,
                                    int32_t max_seqlen,
                                    const int32_t* write_start, int32_t write_offset,
                                    const int64_t* positions,
                                    int batch, int num_tokens, int num_kv_heads, int head_dim,
                                    int dtype, void* stream) {
  using namespace fdllm;
  FDLLM_CHECK_ARG(dtype == FDLLM_DTYPE_BF16 || dtype == FDLLM_DTYPE_F16,
                  "fdllm_kv_cache_write: dtype %d unsupported (bf16 or fp16 only)", dtype);
  FDLLM_CHECK_ARG(batch >= 0 && num_tokens >= 0 && num_kv_heads > 0 && head_dim > 0 && head_dim % 8 == 0,
                  "fdllm_kv_cache_write: bad sizes");
  if (static_cast<int64_t>(batch) * num_tokens == 0) return FDLLM_OK;
  FDLLM_CHECK_ARG(k_new && v_new && k_cache && v_cache, "fdllm_kv_cache_write: null pointer");
  FDLLM_CHECK_ARG(page_table == nullptr || (page_size > 0 && max_pages > 0),
                  "fdllm_kv_cache_write: page table needs page_size > 0 and max_pages > 0");
  FDLLM_CHECK_ARG(aligned16(k_new) && aligned16(v_new) && aligned16(k_cache) && aligned16(v_cache),
                  "fdllm_kv_cache_write: pointers must be 16-byte aligned");
  FDLLM_CHECK_ARG(new_stride_b % 8 == 0 && new_stride_s % 8 == 0 && new_stride_h % 8 == 0 &&
                      cache_stride_page % 8 == 0 && cache_stride_slot % 8 == 0 && cache_stride_h % 8 == 0,
                  "fdllm_kv_cache_write: strides must be multiples of 8 elements");
  KVWriteArgs a;
  a.k_new = static_cast<const uint16_t*>(k_new);
  a.v_new = static_cast<const uint16_t*>(v_new);
  a.n_sb = new_stride_b;
  a.n_ss = new_stride_s;
  a.n_sh = new_stride_h;
  a.k_cache = static_cast<uint16_t*>(k_cache);
  a.v_cache = static_cast<uint16_t*>(v_cache);
  a.c_sp = cache_stride_page;
  a.c_ss = cache_stride_slot;
  a.c_sh = cache_stride_h;
  a.page_table = page_table;
  a.max_pages = max_pages;
  a.page_size = page_size;
  a.max_seqlen = max_seqlen;
  a.write_start = write_start;
  a.write_offset = write_offset;
  a.positions = positions;
  a.pos_bias = 0;
  a.B = batch;
  a.T = num_tokens;
  a.Hkv = num_kv_heads;
  a.D = head_dim;
  const int64_t n = static_cast<int64_t>(batch) * num_tokens * num_kv_heads * (head_dim / 8);
  kv_write_kernel<<<dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, static_cast<hipStream_t>(stream)>>>(a);
  FDLLM_RETURN_LAUNCH_STATUS("fdllm_kv_cache_write");
}
