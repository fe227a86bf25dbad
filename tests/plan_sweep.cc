// Host-only sweep of the attention planner (fast_v2_amd/csrc/attn_plan.h), built by
// tests/test_plan_sanitizers.py with AddressSanitizer and UndefinedBehaviorSanitizer
// (-fno-sanitize-recover: any report aborts the run). Every descriptor field is swept out
// to its limits; for every descriptor the planner accepts, the sweep checks that
//   - the workspace sizes equal an exact 128-bit recomputation (no size_t wrap),
//   - every grid lies within the launch limits and covers the work (rows, keys, vectors),
//   - each kernel family's stated preconditions hold (slots per sequence, keys per split,
//     page-table entries staged in LDS, row counts),
//   - validate_call accepts a well-formed call and refuses a short workspace, a misaligned
//     pointer and a stride off the 8-element grid with an error code and a message.
// Prints one summary line: descriptors tried, accepted, and accepted per plan kind.
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <climits>
#include <vector>

#include "attn_plan.h"

namespace fdllm {
static char g_msg[512];
void set_last_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_msg, sizeof(g_msg), fmt, ap);
  va_end(ap);
}
int dtype_size(int dtype) { return dtype == FDLLM_DTYPE_F32 ? 4 : (dtype == FDLLM_DTYPE_BF16 || dtype == FDLLM_DTYPE_F16) ? 2 : 0; }
}  // namespace fdllm

using namespace fdllm;
typedef __int128 i128;

static long long g_fail = 0;
#define CHECK(cond, ...)                                                          \
  do {                                                                            \
    if (!(cond)) {                                                                \
      if (g_fail < 20) {                                                          \
        fprintf(stderr, "FAIL %s:%d: %s | ", __FILE__, __LINE__, #cond);         \
        fprintf(stderr, __VA_ARGS__);                                             \
        fprintf(stderr, "\n");                                                    \
      }                                                                           \
      ++g_fail;                                                                   \
    }                                                                             \
  } while (0)

static int64_t sat_mul(int64_t a, int64_t b) {
  const i128 r = static_cast<i128>(a) * b;
  return r > INT64_MAX / 2 ? (INT64_MAX / 2) & ~int64_t{7} : static_cast<int64_t>(r);
}
static i128 cdiv(i128 a, i128 b) { return (a + b - 1) / b; }

static const char* describe(const fdllm_kv_attn_desc& d) {
  static char buf[400];
  snprintf(buf, sizeof(buf),
           "dtype=%d D=%d B=%d Sq=%d Hq=%d Hkv=%d maxS=%d paged=%d ps=%d mp=%d split=%d flags=%d mask=%d/%d "
           "kss=%lld new=%d qs=%d",
           d.dtype, d.head_dim, d.batch, d.q_len, d.num_q_heads, d.num_kv_heads, d.max_seqlen, d.page_table != nullptr,
           d.page_size, d.max_pages, d.kv_split, d.flags, d.mask_mode, d.mask_block,
           static_cast<long long>(d.k_stride_slot), d.k_new != nullptr, d.q_start != nullptr);
  return buf;
}

static void check_plan(const fdllm_kv_attn_desc& d, const Plan& pl) {
  const i128 B = d.batch, Bm = d.batch > 0 ? d.batch : 1, hkv = d.num_kv_heads, D = d.head_dim;
  const i128 R = static_cast<i128>(d.q_len) * (d.num_q_heads / d.num_kv_heads);
  CHECK(pl.R == R, "R %d vs %lld: %s", pl.R, static_cast<long long>(R), describe(d));
  const i128 max_keys = d.page_table ? std::min<i128>(d.max_seqlen, static_cast<i128>(d.max_pages) * d.page_size)
                                     : d.max_seqlen;
  const i128 len = max_keys > 1 ? max_keys : 1;
  i128 o = 0, ml = 0;  // exact partial sizes
  switch (pl.kind) {
    case kPlanF32: {
      const i128 chunks = cdiv(len, 64);
      CHECK(static_cast<i128>(pl.n_rb) * pl.rows_per_wg >= R && pl.rows_per_wg == 4 * FDLLM_F32_ROWS_PER_WAVE,
            "f32 rows: %s", describe(d));
      CHECK(pl.chunk % 64 == 0 && pl.chunk >= 64 && pl.n_splits >= 1 && pl.n_splits <= kF32MaxSplits &&
                static_cast<i128>(pl.n_splits) * pl.chunk >= chunks * 64 &&
                static_cast<i128>(pl.n_splits - 1) * pl.chunk < chunks * 64,
            "f32 splits %d x %d: %s", pl.n_splits, pl.chunk, describe(d));
      if (pl.n_splits > 1) {
        const i128 units = B * hkv * pl.n_rb;
        o = units * pl.n_splits * pl.rows_per_wg * D * 4;
        ml = units * pl.n_splits * pl.rows_per_wg * 8;
      }
      break;
    }
    case kPlanBalancedDecode: {
      CHECK(Bm <= kBalancedMaxBatch && d.head_dim == 128 && R <= 64, "balanced shape: %s", describe(d));
      CHECK(d.page_table == nullptr || Bm * d.max_pages <= kBalMaxPages, "balanced pages: %s", describe(d));
      CHECK(pl.n_splits % 8 == 0 && pl.n_splits >= 8, "balanced slots %d: %s", pl.n_splits, describe(d));
      o = (pl.n_splits + Bm) * hkv * 64 * D * 4;
      ml = (pl.n_splits + Bm) * hkv * 64 * 8;
      break;
    }
    case kPlanSplitDecode: {
      const i128 max_t = cdiv(len, 32);
      CHECK(d.head_dim == 128 && R <= 64 && max_t <= i128{kDecodeMaxTiles} * kMaxDecodeSplits,
            "split decode shape: %s", describe(d));
      CHECK(d.k_stride_slot < (1 << 24) && d.v_stride_slot < (1 << 24), "slot stride: %s", describe(d));
      CHECK(B * hkv <= static_cast<i128>(kCounterBytes / 4), "counters: %s", describe(d));
      i128 slots;
      if (pl.chunk == 0) {
        CHECK(Bm <= kBalancedMaxBatch, "per-sequence partition batch: %s", describe(d));
        CHECK(pl.n_splits >= Bm * cdiv(max_t, kDecodeMaxTiles) && pl.n_splits >= cdiv(kDecodeSlotsTarget, hkv),
              "slots %d: %s", pl.n_splits, describe(d));
        slots = pl.n_splits;
      } else {
        CHECK(pl.chunk % 32 == 0 && pl.chunk <= kSplitMaxChunk && pl.chunk >= 32, "chunk %d: %s", pl.chunk,
              describe(d));
        CHECK(static_cast<i128>(pl.n_splits) * pl.chunk >= max_t * 32 && pl.n_splits <= kMaxDecodeSplits,
              "splits %d x %d: %s", pl.n_splits, pl.chunk, describe(d));
        slots = Bm * pl.n_splits;
      }
      const bool split = pl.chunk == 0 ? slots > Bm : pl.n_splits > 1;
      o = split ? slots * hkv * 64 * D * 4 : 0;
      ml = split ? slots * hkv * 64 * 8 : 0;
      break;
    }
    case kPlanAllHeads: {
      const i128 max_t32 = cdiv(len, 32);
      CHECK(hkv == 1 || hkv == 2 || hkv == 4 || hkv == 8, "all-heads hkv: %s", describe(d));
      CHECK(R <= 64 && d.head_dim == 128 && d.k_stride_h == 128 && d.v_stride_h == 128, "all-heads shape: %s",
            describe(d));
      CHECK(pl.chunk % 32 == 0 && pl.chunk >= 32 && static_cast<i128>(pl.n_splits) * pl.chunk >= max_t32 * 32,
            "all-heads splits %d x %d: %s", pl.n_splits, pl.chunk, describe(d));
      if (pl.n_splits > 1) {
        o = B * hkv * pl.n_splits * 64 * D * 4;
        ml = B * hkv * pl.n_splits * 64 * 8;
      }
      break;
    }
    case kPlanSplitPrefill: {
      const i128 max_t = cdiv(len, 64);
      CHECK(R > 64 && R <= 256 && d.head_dim == 128 && max_t <= i128{kDecodeMaxTiles} * kMaxDecodeSplits,
            "split prefill shape: %s", describe(d));
      CHECK(B * hkv <= static_cast<i128>(kCounterBytes / 4), "counters: %s", describe(d));
      i128 slots;
      if (pl.chunk == 0) {
        CHECK(Bm <= kBalancedMaxBatch && pl.n_splits >= Bm * cdiv(max_t, kDecodeMaxTiles), "slots %d: %s",
              pl.n_splits, describe(d));
        slots = pl.n_splits;
      } else {
        CHECK(pl.chunk % 64 == 0 && pl.chunk <= kDecodeMaxTiles * 64, "chunk %d: %s", pl.chunk, describe(d));
        CHECK(static_cast<i128>(pl.n_splits) * pl.chunk >= max_t * 64 && pl.n_splits <= kMaxDecodeSplits,
              "splits %d x %d: %s", pl.n_splits, pl.chunk, describe(d));
        slots = Bm * pl.n_splits;
      }
      const bool split = pl.chunk == 0 ? slots > Bm : pl.n_splits > 1;
      if (split) {
        o = slots * hkv * 256 * D * 4;
        ml = slots * hkv * 256 * 8 + Bm * hkv * 8;
        CHECK(static_cast<i128>(pl.ws_unit_off) == slots * hkv * 256 * 8, "unit table offset: %s", describe(d));
      }
      break;
    }
    case kPlanPrefill:
      CHECK(R >= 2048 && static_cast<i128>(pl.n_rb) * pl.rows_per_wg >= R && pl.rows_per_wg == 256 &&
                pl.n_rb <= 65535,
            "prefill rows: %s", describe(d));
      break;
    default: {  // general
      const i128 max_tiles = cdiv(len, kKT);
      CHECK(static_cast<i128>(pl.n_rb) * pl.rows_per_wg >= R && pl.rows_per_wg == 64 * pl.MT &&
                (pl.MT == 1 || pl.MT == 2 || pl.MT == 4),
            "general rows: %s", describe(d));
      CHECK(pl.chunk % kKT == 0 && pl.chunk >= kKT && static_cast<i128>(pl.n_splits) * pl.chunk >= max_tiles * kKT,
            "general splits %d x %d: %s", pl.n_splits, pl.chunk, describe(d));
      if (pl.n_splits > 1) {
        const i128 units = B * hkv * pl.n_rb;
        o = units * pl.n_splits * pl.rows_per_wg * D * 4;
        ml = units * pl.n_splits * pl.rows_per_wg * 8;
      }
      break;
    }
  }
  CHECK(o <= static_cast<i128>(SIZE_MAX / 4) && ml <= static_cast<i128>(SIZE_MAX / 4), "sizes overflow: %s",
        describe(d));
  CHECK(static_cast<i128>(pl.ws_o_bytes) == o && static_cast<i128>(pl.ws_ml_bytes) == ml,
        "workspace o %zu / %lld, ml %zu / %lld: %s", pl.ws_o_bytes, static_cast<long long>(o), pl.ws_ml_bytes,
        static_cast<long long>(ml), describe(d));
  const size_t need = plan_workspace_bytes(&d, pl);
  CHECK(need == (o > 0 ? kCounterBytes + align256(pl.ws_ml_bytes) + pl.ws_o_bytes : 0), "need: %s", describe(d));
}

static void check_launches(const fdllm_kv_attn_desc& d, const Plan& pl) {
  LaunchSet ls;
  g_msg[0] = 0;
  const int rc = plan_launches(&d, pl, &ls);
  if (rc != FDLLM_OK) {
    CHECK(rc == FDLLM_ERR_INVALID_ARGUMENT && g_msg[0] != 0, "launch refusal without message: %s", describe(d));
    return;
  }
  const auto in_range = [](const GridDims& g) {
    return g.x >= 1 && g.y >= 1 && g.z >= 1 && g.x <= 0x7fffffffu && g.y <= 65535u && g.z <= 65535u;
  };
  CHECK(in_range(ls.main_grid), "main grid: %s", describe(d));
  CHECK(ls.main_block >= 64 && ls.main_block <= 1024 && ls.main_block % 64 == 0, "block %u: %s", ls.main_block,
        describe(d));
  const i128 B = d.batch, hkv = d.num_kv_heads;
  const GridDims& g = ls.main_grid;
  const i128 total = static_cast<i128>(g.x) * g.y * g.z;
  switch (pl.kind) {
    case kPlanF32:
      CHECK(static_cast<i128>(g.x) == static_cast<i128>(pl.n_rb) * pl.n_splits && g.y == hkv && g.z == B &&
                ls.second == (pl.n_splits > 1 && !plan_f32_merge_in_kernel(pl, d.batch, d.num_kv_heads)),
            "f32 grid: %s", describe(d));
      // the in-kernel merge counts arrivals per row block unit in the counter region
      if (plan_f32_merge_in_kernel(pl, d.batch, d.num_kv_heads))
        CHECK(B * hkv * pl.n_rb <= static_cast<i128>(kCounterBytes / sizeof(int)) && pl.ws_o_bytes > 0,
              "f32 merge counters: %s", describe(d));
      break;
    case kPlanBalancedDecode:
      CHECK(g.x == static_cast<uint32_t>(pl.n_splits) && g.y == hkv && g.z == 1, "balanced grid: %s", describe(d));
      break;
    case kPlanSplitDecode:
    case kPlanSplitPrefill:
      CHECK(g.x == static_cast<uint32_t>(pl.n_splits) && g.y == hkv && g.z == (pl.chunk > 0 ? B : 1),
            "split grid: %s", describe(d));
      break;
    case kPlanPrefill:
      CHECK(g.x == B * hkv && g.y == static_cast<uint32_t>(pl.n_rb), "prefill grid: %s", describe(d));
      break;
    case kPlanAllHeads:
      CHECK(g.x == static_cast<uint32_t>(pl.n_splits) && g.y == B && ls.main_block == 128 * hkv,
            "all-heads grid: %s", describe(d));
      break;
    default:
      CHECK(g.x == static_cast<uint32_t>(pl.n_splits) && g.y == static_cast<uint32_t>(pl.n_rb) && g.z == B * hkv,
            "general grid: %s", describe(d));
  }
  CHECK(total >= 1, "empty grid: %s", describe(d));
  if (ls.second) {
    CHECK(in_range(ls.second_grid), "second grid: %s", describe(d));
    if (pl.kind == kPlanSplitPrefill) {
      CHECK(static_cast<i128>(ls.second_grid.x) * 32 >= pl.R && ls.second_grid.y == B * hkv, "merge grid: %s",
            describe(d));
    } else {
      const int rpb = 256 / (d.head_dim / 8);
      const i128 units = pl.kind == kPlanAllHeads ? B * hkv : B * hkv * pl.n_rb;
      CHECK(static_cast<i128>(ls.second_grid.x) * rpb >= pl.rows_per_wg && ls.second_grid.y == units,
            "combine grid: %s", describe(d));
    }
  }
  CHECK(ls.write == (d.k_new != nullptr && !plan_fuses_cache_write(&d, pl)), "write choice: %s", describe(d));
  if (ls.write) {
    CHECK(in_range(ls.write_grid), "write grid: %s", describe(d));
    const i128 vecs = B * d.q_len * hkv * (d.head_dim / 8);
    CHECK(static_cast<i128>(ls.write_grid.x) * 256 >= vecs, "write grid covers %lld vectors: %s",
          static_cast<long long>(vecs), describe(d));
  }
}

static void check_validation(fdllm_kv_attn_desc d, const Plan& pl) {
  alignas(16) static unsigned char ws_dummy[16];
  const size_t need = plan_workspace_bytes(&d, pl);
  // a well-formed call (the workspace pointer is only checked, never dereferenced)
  void* ws = need > 0 ? static_cast<void*>(ws_dummy) : nullptr;
  int rc = validate_call(&d, pl, ws, need);
  CHECK(rc == FDLLM_OK, "well-formed call refused (%d: %s): %s", rc, g_msg, describe(d));
  if (need > 0) {
    g_msg[0] = 0;
    rc = validate_call(&d, pl, ws, need - 1);
    CHECK(rc == FDLLM_ERR_WORKSPACE && g_msg[0], "short workspace accepted: %s", describe(d));
  }
  fdllm_kv_attn_desc bad = d;
  bad.q = static_cast<const char*>(d.q) + 2;
  g_msg[0] = 0;
  CHECK(validate_call(&bad, pl, ws, need) == FDLLM_ERR_INVALID_ARGUMENT && g_msg[0], "misaligned q accepted: %s",
        describe(d));
  bad = d;
  bad.out_stride_s += 4;
  g_msg[0] = 0;
  CHECK(validate_call(&bad, pl, ws, need) == FDLLM_ERR_INVALID_ARGUMENT && g_msg[0], "odd stride accepted: %s",
        describe(d));
}

int main() {
  alignas(16) static unsigned char dev[256];  // stand-in device pointers: checked, never read
  static const int32_t table_dummy[1] = {0};
  const int dtypes[] = {FDLLM_DTYPE_BF16, FDLLM_DTYPE_F16, FDLLM_DTYPE_F32, 7};
  const int head_dims[] = {128, 64, 96};
  const int batches[] = {0, 1, 2, 16, 64, 65, 4096, 65535, 65536, INT_MAX};
  const int q_lens[] = {0, 1, 8, 32, 64, 4096, 1 << 20, 1 << 30, INT_MAX};
  const int heads[][2] = {{28, 4}, {32, 8}, {8, 8}, {7, 1}, {64, 2}, {130, 65}, {65535 * 2, 65535}, {INT_MAX, 1}};
  const int max_seqlens[] = {0, 1, 32, 544, 4096, 1 << 16, 81920, 1 << 20, 1 << 30, (1 << 30) + 1, INT_MAX};
  const int pagings[][2] = {{0, 0}, {16, 4}, {32, 128}, {32, 1 << 20}, {64, INT_MAX}, {1 << 20, 1 << 11}, {48, 10}};
  const int splits[] = {0, 64, 96, 4096, 1 << 30};
  const int flag_sets[] = {0, FDLLM_ATTN_NO_DECODE_KERNEL, FDLLM_ATTN_ALL_HEADS_DECODE, FDLLM_ATTN_BALANCED_SPLITS,
                           FDLLM_ATTN_CACHE_WRITE_KERNEL};
  long long tried = 0, accepted = 0, kinds[7] = {0};
  unsigned rot = 0;
  for (int dt : dtypes)
    for (int hd : head_dims)
      for (int b : batches)
        for (int sq : q_lens)
          for (const auto& h : heads)
            for (int ms : max_seqlens)
              for (const auto& pg : pagings)
                for (int ks : splits) {
                  ++rot;
                  // the fields not swept in the nested loops vary with a hash of the loop
                  // count, so that each of their values meets every combination above
                  const uint32_t hsh = (rot * 2654435761u) ^ (rot >> 13);
                  fdllm_kv_attn_desc d;
                  memset(&d, 0, sizeof(d));
                  d.dtype = dt;
                  d.head_dim = hd;
                  d.batch = b;
                  d.q_len = sq;
                  d.num_q_heads = h[0];
                  d.num_kv_heads = h[1];
                  d.max_seqlen = ms;
                  d.kv_split = ks;
                  d.flags = flag_sets[(hsh >> 3) % 5];
                  d.mask_mode = static_cast<int>((hsh >> 7) % 3);
                  d.mask_block = d.mask_mode == FDLLM_MASK_BLOCK_CAUSAL ? ((hsh >> 10) % 4 == 0 ? 0 : 32) : 0;
                  d.softmax_scale = 0.088f;
                  d.q = d.k = d.v = dev;
                  d.out = dev;
                  d.seqlens = table_dummy;
                  if (pg[0] > 0) {
                    d.page_table = table_dummy;
                    d.page_size = pg[0];
                    d.max_pages = pg[1];
                  }
                  const int64_t Dl = hd, Hq = h[0], Hk = h[1];
                  d.q_stride_h = d.out_stride_h = Dl;
                  d.q_stride_s = d.out_stride_s = sat_mul(Hq, Dl);
                  d.q_stride_b = d.out_stride_b = sat_mul(sat_mul(sq, Hq), Dl);
                  // K/V: head-major pages, token-major pages, or a slot stride past 2^24
                  const int layout = static_cast<int>((hsh >> 13) % 3);
                  const int64_t rows = pg[0] > 0 ? pg[0] : std::max(ms, 1);
                  if (layout == 0) {
                    d.k_stride_h = d.v_stride_h = Dl;
                    d.k_stride_slot = d.v_stride_slot = sat_mul(Hk, Dl);
                  } else if (layout == 1) {
                    d.k_stride_slot = d.v_stride_slot = Dl;
                    d.k_stride_h = d.v_stride_h = sat_mul(rows, Dl);
                  } else {
                    d.k_stride_h = d.v_stride_h = Dl;
                    d.k_stride_slot = d.v_stride_slot = int64_t{1} << 24;
                  }
                  d.k_stride_page = d.v_stride_page = sat_mul(rows, sat_mul(Hk, Dl));
                  if ((hsh >> 17) % 4 == 1) {
                    d.k_new = d.v_new = dev;
                    d.new_stride_h = Dl;
                    d.new_stride_s = sat_mul(Hk, Dl) < (1 << 24) ? sat_mul(Hk, Dl) : 8;
                    d.new_stride_b = sat_mul(sq, d.new_stride_s);
                  }
                  if ((hsh >> 21) % 3 == 1) d.q_start = table_dummy;
                  ++tried;
                  Plan pl;
                  memset(&pl, 0xA5, sizeof(pl));
                  g_msg[0] = 0;
                  const int rc = make_plan(&d, &pl);
                  if (rc != FDLLM_OK) {
                    CHECK(rc == FDLLM_ERR_INVALID_ARGUMENT && g_msg[0] != 0, "refusal without message: %s",
                          describe(d));
                    continue;
                  }
                  ++accepted;
                  CHECK(pl.kind >= 0 && pl.kind <= 6, "kind %d: %s", pl.kind, describe(d));
                  if (pl.kind < 0 || pl.kind > 6) continue;
                  ++kinds[pl.kind];
                  check_plan(d, pl);
                  if (d.batch > 0 && d.q_len > 0) {
                    check_launches(d, pl);
                    check_validation(d, pl);
                  }
                }
  printf("tried %lld accepted %lld kinds", tried, accepted);
  for (long long k : kinds) printf(" %lld", k);
  printf(" failures %lld\n", g_fail);
  return g_fail == 0 ? 0 : 1;
}
