// RoPE of the new queries and keys fused with the static / block KV cache write
// (fdllm_rope_kv_write): the step between the q/k/v projections and attention.
//
// One workgroup per token (grid (seq_len, batch)), 256 threads. A rope work item
// is one head and eight dimension pairs (i, i + D/2): two 16-byte loads of the
// row, two of cos and two of sin, eight pairs computed, two 16-byte stores per
// destination. V rows are copied in 16-byte vectors. The arithmetic rounds to the
// 16-bit type after each product and after the sum, exactly as the eager
// expression q * cos + rotate_half(q) * sin (utils/attention_backends.py:777-788).
#include "fdllm_common.h"

namespace fdllm {
namespace {

struct RopeArgs {
  fdllm_rope_kv_desc d;
  int npair;  // head_dim / 16: 8-pair work items per head
};

template <typename T>
__device__ __forceinline__ void unpack8(const u32x4& w, float* f) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = Elt<T>::lo(w[i]);
    f[2 * i + 1] = Elt<T>::hi(w[i]);
  }
}

template <typename T>
__device__ __forceinline__ u32x4 pack8(const float* f) {
  u32x4 w;
#pragma unroll
  for (int i = 0; i < 4; ++i) w[i] = Elt<T>::pack(f[2 * i], f[2 * i + 1]);
  return w;
}

template <typename T>
__device__ __forceinline__ float rnd(float x) {
  return Elt<T>::round(x);
}

// RoPE of dimensions [c, c + 8) and their partners [c + half, c + half + 8) of one
// head row: xa / xb the two 8-element blocks, cs / sn the token's cos / sin rows.
// rotate_half gives (-x1, x0); negation is exact and rounding symmetric, so
// x0 * cos + (-x1) * sin rounds as x0 * cos - x1 * sin.
template <typename T>
__device__ __forceinline__ void rope8(const u32x4& xa, const u32x4& xb, const uint16_t* cs, const uint16_t* sn, int c,
                                      int half, u32x4& wa, u32x4& wb) {
  // Each product and the sum are rounded on their own: no fused multiply-add, which
  // hipcc would otherwise form from the 16-bit operations it recognises in them.
#pragma clang fp contract(off)
  float x0[8], x1[8], c0[8], c1[8], s0[8], s1[8];
  unpack8<T>(xa, x0);
  unpack8<T>(xb, x1);
  unpack8<T>(*reinterpret_cast<const u32x4*>(cs + c), c0);
  unpack8<T>(*reinterpret_cast<const u32x4*>(cs + half + c), c1);
  unpack8<T>(*reinterpret_cast<const u32x4*>(sn + c), s0);
  unpack8<T>(*reinterpret_cast<const u32x4*>(sn + half + c), s1);
  float y0[8], y1[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    y0[j] = rnd<T>(rnd<T>(x0[j] * c0[j]) - rnd<T>(x1[j] * s0[j]));
    y1[j] = rnd<T>(rnd<T>(x1[j] * c1[j]) + rnd<T>(x0[j] * s1[j]));
  }
  wa = pack8<T>(y0);
  wb = pack8<T>(y1);
}

// the two 8-element blocks of one head row at element offset `off` of `base`
__device__ __forceinline__ void put_pair(void* base, int64_t off, int c, int half, const u32x4& wa, const u32x4& wb) {
  uint16_t* o = static_cast<uint16_t*>(base) + off;
  *reinterpret_cast<u32x4*>(o + c) = wa;
  *reinterpret_cast<u32x4*>(o + half + c) = wb;
}

template <typename T>
__global__ __launch_bounds__(256) void rope_kv_kernel(const RopeArgs a) {
  const fdllm_rope_kv_desc& d = a.d;
  const int t = blockIdx.x;
  const int b = blockIdx.y;
  const int D = d.head_dim;
  const int half = D / 2;
  const uint16_t* cs = static_cast<const uint16_t*>(d.cos) + b * d.cs_stride_b + t * d.cs_stride_s;
  const uint16_t* sn = static_cast<const uint16_t*>(d.sin) + b * d.cs_stride_b + t * d.cs_stride_s;
  const int pos1 = (d.write_start ? d.write_start[b] : 0) + d.write_offset + t;
  const int pos2 = d.block_offset + t;
  const bool to_cache = d.k_cache != nullptr && pos1 >= 0 && pos1 < d.cache_len;
  const bool to_block = d.k_block != nullptr && pos2 >= 0 && pos2 < d.block_len;

  const int n_rope = (d.num_q_heads + d.num_kv_heads) * a.npair;
  for (int item = threadIdx.x; item < n_rope; item += blockDim.x) {
    const int head = item / a.npair;
    const int c = (item - head * a.npair) * 8;  // first dimension of the pair block
    const bool is_q = head < d.num_q_heads;
    const int g = head - d.num_q_heads;
    const uint16_t* src = is_q ? static_cast<const uint16_t*>(d.q) + b * d.q_stride_b + t * d.q_stride_s +
                                     head * d.q_stride_h
                               : static_cast<const uint16_t*>(d.k) + b * d.k_stride_b + t * d.k_stride_s +
                                     g * d.k_stride_h;
    u32x4 w0, w1;
    rope8<T>(*reinterpret_cast<const u32x4*>(src + c), *reinterpret_cast<const u32x4*>(src + half + c), cs, sn, c,
             half, w0, w1);
    if (is_q) {
      put_pair(d.q_out, b * d.qo_stride_b + t * d.qo_stride_s + head * d.qo_stride_h, c, half, w0, w1);
    } else {
      if (d.k_out) put_pair(d.k_out, b * d.ko_stride_b + t * d.ko_stride_s + g * d.ko_stride_h, c, half, w0, w1);
      if (to_cache) put_pair(d.k_cache, b * d.c_stride_b + pos1 * d.c_stride_s + g * d.c_stride_h, c, half, w0, w1);
      if (to_block) put_pair(d.k_block, b * d.bc_stride_b + pos2 * d.bc_stride_s + g * d.bc_stride_h, c, half, w0, w1);
    }
  }
  // V rows: plain 16-byte copies to every destination
  const int vch = D / 8;
  const int n_v = d.num_kv_heads * vch;
  for (int item = threadIdx.x; item < n_v; item += blockDim.x) {
    const int g = item / vch;
    const int c = (item - g * vch) * 8;
    const u32x4 w = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(d.v) + b * d.v_stride_b +
                                                     t * d.v_stride_s + g * d.v_stride_h + c);
    if (d.v_out)
      *reinterpret_cast<u32x4*>(static_cast<uint16_t*>(d.v_out) + b * d.ko_stride_b + t * d.ko_stride_s +
                                g * d.ko_stride_h + c) = w;
    if (to_cache)
      *reinterpret_cast<u32x4*>(static_cast<uint16_t*>(d.v_cache) + b * d.c_stride_b + pos1 * d.c_stride_s +
                                g * d.c_stride_h + c) = w;
    if (to_block)
      *reinterpret_cast<u32x4*>(static_cast<uint16_t*>(d.v_block) + b * d.bc_stride_b + pos2 * d.bc_stride_s +
                                g * d.bc_stride_h + c) = w;
  }
}

// ---------------------------------------------------------------------------
// q / k / v projections with RoPE and the cache writes as their epilogue
// (fdllm_qkv_rope_kv_write).
//
// Workgroup = one tile of 128 tokens x one head's 128 columns (or, with few tiles, half
// of them: 32 columns and their RoPE partners 64 further on), so the RoPE partners i and
// i + 64 are in the tile; 4 waves as 2 x 2; the weight rows and the 128 token rows stream
// through a ring of LDS slots of 64-deep K steps (direct-to-LDS loads, all but two slots'
// steps in flight, one barrier per step);
// v_mfma_f32_32x32x16 with both operands read from LDS (XOR-swizzled 16-byte chunks,
// chunk p of row r at p ^ ((r >> 1) & 7), so the 16 lanes of a read phase hit 16
// distinct bank groups). A wave's two column tiles are columns j and j + 64 of the
// head (j = 32 wn + lane % 32), which keeps the rotation pairs in one lane's view of
// the accumulators; the epilogue goes through LDS anyway so that its loads and stores
// are 16-byte vectors: y = to_dtype(acc + bias) into a 128 x 136 tile, then each
// thread rotates and stores 8-dimension pairs exactly as rope_kv_kernel does.
// Tiles are numbered head-major and dealt XCD-major (tile = (wg % 8) * per + wg / 8),
// so the token tiles of one head share an XCD's L2 for its weight rows.
struct QkvArgs {
  fdllm_qkv_rope_desc d;
  int T;        // token rows: batch * seq_len
  int n_mt;     // 128-row token tiles
  int n_tiles;  // n_mt * (num_q_heads + 2 num_kv_heads) * workgroups per (head, token tile)
  int per_xcd;  // ceil(n_tiles / 8)
};

// LDS operand reads issued ahead of the MFMAs in each K step (0: the compiler's order),
// and the K depth of a ring slot. Measured on the 7B layout at 512 / 128 / 2048 rows (whole-
// head tiles): reads 8 ahead 40.5 / 41.1 / 117.1 us, 0, 4 or 16 ahead within 1 us of that;
// 32-deep slots (eight of them) 48.2 / 49.7 / 144.6 us: the per-step barrier and waits
// cost more than the deeper ring gains.
#ifndef FDLLM_QKV_SCHED
#define FDLLM_QKV_SCHED 8
#endif
#ifndef FDLLM_QKV_KT
#define FDLLM_QKV_KT 64
#endif

constexpr int kQkvBM = 128;  // token rows per tile (and head_dim: columns per tile)
constexpr int kQkvKT = FDLLM_QKV_KT;  // K step per LDS slot (64 or 32)
constexpr int kQkvYS = 136;  // epilogue tile row stride (elements; 272 bytes)

// BN: columns of one head per workgroup (128: the whole head; 64: two workgroups per
// head, each with 32 columns and their RoPE partners 64 further on); NS: LDS ring slots.
template <typename T, bool F16, int BN, int NS>
__global__ __launch_bounds__(256) void qkv_rope_kernel(const QkvArgs a) {
  constexpr int KT = kQkvKT;
  constexpr int kQkvParts = 128 / BN;      // workgroups per (head, token tile)
  constexpr int NT = BN / 64;              // 32-column MFMA tiles per wave
  constexpr int ROWB = KT * 2;             // bytes of one row of an operand tile
  constexpr int CH = ROWB / 16;            // 16-byte chunks per row
  constexpr int RPD = 1024 / ROWB;         // rows one direct-to-LDS load (1 KB per wave) covers
  constexpr int NDX = kQkvBM / RPD / 4;    // loads per wave of the token tile
  constexpr int NDW = BN / RPD / 4;        // loads per wave of the weight tile
  constexpr int TB = kQkvBM * ROWB;        // bytes of the token tile
  constexpr int SLOT = TB + BN * ROWB;     // token rows, then weight rows
  constexpr int KK = KT / 16;              // MFMA k-steps per slot
  static_assert(NS >= 3 && CH >= 4 && NDW >= 1 && NS * SLOT <= 131072, "ring shape");
  __shared__ __attribute__((aligned(1024))) uint8_t lds[NS * SLOT];
  static_assert(kQkvBM * kQkvYS * 2 <= NS * SLOT, "epilogue tile fits the ring");
  const fdllm_qkv_rope_desc& d = a.d;
  const fdllm_rope_kv_desc& r = d.rope;

  const int tile = static_cast<int>(blockIdx.x & 7) * a.per_xcd + static_cast<int>(blockIdx.x >> 3);
  if (tile >= a.n_tiles) return;  // uniform over the workgroup
  const int head = tile / (a.n_mt * kQkvParts);  // q heads, then k heads, then v heads
  const int part = (tile - head * a.n_mt * kQkvParts) / a.n_mt;
  const int mt = tile - (head * kQkvParts + part) * a.n_mt;
  const int c0 = part * (BN / 2);  // first column of each half this workgroup computes
  // head column of weight-tile row rw: the first BN / 2 rows are columns c0.., the rest
  // their RoPE partners 64 further on (the identity for a whole head)
  auto hcol = [c0](int rw) __attribute__((always_inline)) { return rw < BN / 2 ? c0 + rw : 64 + c0 + rw - BN / 2; };
  const int Hq = r.num_q_heads, Hkv = r.num_kv_heads;
  const int kind = head < Hq ? 0 : (head < Hq + Hkv ? 1 : 2);
  const int hh = kind == 0 ? head : (kind == 1 ? head - Hq : head - Hq - Hkv);
  const int K = d.hidden;
  const uint16_t* w = static_cast<const uint16_t*>(kind == 0 ? d.wq : (kind == 1 ? d.wk : d.wv)) +
                      static_cast<int64_t>(hh) * kQkvBM * K;
  const uint16_t* bias = static_cast<const uint16_t*>(kind == 0 ? d.bq : (kind == 1 ? d.bk : d.bv));
  const int row0 = mt * kQkvBM;
  const int rows = min(kQkvBM, a.T - row0);
  const int nk = K / KT;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int xs_row = static_cast<int>(d.x_stride_row);
  const uint16_t* xbase = static_cast<const uint16_t*>(d.x) + static_cast<int64_t>(row0) * xs_row;
  const i32x4 xsrd = make_srd(xbase, rows * xs_row * 2);  // token rows past the end read as zero
  const i32x4 wsrd = make_srd(w, kQkvBM * K * 2);
  const i32x4 zsrd = make_srd(xbase, 0);  // steps past the end: zeros, no memory traffic

  // LDS chunk p of tile row r holds source chunk p ^ swz(r): the rows that share a
  // 256-byte bank line are spread over distinct 16-byte bank groups
  auto swz = [](int row) __attribute__((always_inline)) { return (row / (256 / ROWB)) & (CH - 1); };
  // load i of wave w fills rows RPD (NDMA w + i) .. + RPD of both tiles: lane -> row
  // + lane / CH, LDS chunk lane % CH
  int xoff[NDX], woff[NDW];
#pragma unroll
  for (int i = 0; i < NDX; ++i) {
    const int row = RPD * (NDX * wave + i) + lane / CH;
    xoff[i] = row * xs_row * 2 + (((lane % CH) ^ swz(row)) * 16);
  }
#pragma unroll
  for (int i = 0; i < NDW; ++i) {
    const int row = RPD * (NDW * wave + i) + lane / CH;
    woff[i] = hcol(row) * K * 2 + (((lane % CH) ^ swz(row)) * 16);
  }
  const uint32_t lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds));
  auto issue = [&](int st, int slot) __attribute__((always_inline)) {
    const bool live = st < nk;  // uniform
    const int kb = st * ROWB;
    const uint32_t dst = lds0 + slot * SLOT;
#pragma unroll
    for (int i = 0; i < NDX; ++i) lds_dma16(live ? xsrd : zsrd, xoff[i] + kb, dst + (NDX * wave + i) * 1024);
#pragma unroll
    for (int i = 0; i < NDW; ++i) lds_dma16(live ? wsrd : zsrd, woff[i] + kb, dst + TB + (NDW * wave + i) * 1024);
  };

  // operand reads: wave (wm, wn) takes token rows 64 wm + 32 m2 + lane % 32 and weight-
  // tile rows 64 n2 + 32 wn + lane % 32; lane / 32 picks the upper 8 of each 16-deep step
  const int wm = wave & 1, wn = wave >> 1;
  const int l32 = lane & 31, kh = lane >> 5;
  int arow[2], brow[NT];
#pragma unroll
  for (int i = 0; i < 2; ++i) arow[i] = 64 * wm + 32 * i + l32;
#pragma unroll
  for (int j = 0; j < NT; ++j) brow[j] = 64 * j + 32 * wn + l32;
  f32x16 acc[2][NT];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  auto compute = [&](int slot) __attribute__((always_inline)) {
    const uint8_t* sx = lds + slot * SLOT;
    const uint8_t* sw = sx + TB;
    u32x4 av[KK][2], bv[KK][NT];
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      const int chunk = 2 * kk + kh;
#pragma unroll
      for (int i = 0; i < 2; ++i)
        av[kk][i] = *reinterpret_cast<const u32x4*>(sx + arow[i] * ROWB + ((chunk ^ swz(arow[i])) << 4));
#pragma unroll
      for (int j = 0; j < NT; ++j)
        bv[kk][j] = *reinterpret_cast<const u32x4*>(sw + brow[j] * ROWB + ((chunk ^ swz(brow[j])) << 4));
    }
#pragma unroll
    for (int kk = 0; kk < KK; ++kk)
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[i][j] = mfma32x32x16<F16>(av[kk][i], bv[kk][j], acc[i][j]);
#if FDLLM_QKV_SCHED
    if constexpr (NT == 2) {
      // the step's operand reads go out QA ahead of the MFMAs that use them
      constexpr int QA = FDLLM_QKV_SCHED < 4 * KK ? FDLLM_QKV_SCHED : 4 * KK;
      __builtin_amdgcn_sched_group_barrier(0x100, QA, 0);  // DS reads
#pragma unroll
      for (int i = 0; i < 4 * KK - QA; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
      }
      __builtin_amdgcn_sched_group_barrier(0x008, QA, 0);
    }
#endif
  };

  // main loop: step j in slot j % NS, the next NS - 2 steps in flight; step j + NS - 1
  // is issued into the slot step j - 1 read, after the barrier that ends that step.
  // Every step issues its loads (zero-size past the end), so each count wait is exact.
#pragma unroll
  for (int st = 0; st < NS - 1; ++st) issue(st, st);
  for (int j = 0; j < nk; ++j) {
    wait_vmcnt<(NS - 2) * (NDX + NDW)>();  // this thread's loads of step j have landed
    lds_barrier();                        // ... and every thread's; every wave is done with step j - 1
    issue(j + NS - 1, (j + NS - 1) % NS);
    compute(j % NS);
  }
  wait_vmcnt<0>();  // no load may land in LDS after this point
  lds_barrier();

  // ---- epilogue: y = to_dtype(acc + bias) into the tile Y[row][col]
  uint16_t* Y = reinterpret_cast<uint16_t*>(lds);
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    const int col = hcol(brow[j]);
    const float bcol = bias != nullptr ? Elt<T>::lo(static_cast<uint32_t>(bias[hh * kQkvBM + col])) : 0.f;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int row = 64 * wm + 32 * i + 8 * (e >> 2) + 4 * kh + (e & 3);
        Y[row * kQkvYS + col] = static_cast<uint16_t>(Elt<T>::pack(acc[i][j][e] + bcol, 0.f) & 0xffffu);
      }
  }
  lds_barrier();

  // ---- rotation and stores: item = (token row, 8-dimension block c in the first half)
  const int S = r.seq_len;
  constexpr int half = kQkvBM / 2;
  constexpr int NB = BN / 16;  // 8-dimension blocks per row in each half of this workgroup
  for (int it = tid; it < kQkvBM * NB; it += 256) {
    const int rr = it / NB;
    const int c = c0 + (it % NB) * 8;
    if (rr >= rows) break;  // items are row-major: every later item is past the end too
    const int tok = row0 + rr;
    const int b = tok / S;
    const int t = tok - b * S;
    const u32x4 ya = *reinterpret_cast<const u32x4*>(Y + rr * kQkvYS + c);
    const u32x4 yb = *reinterpret_cast<const u32x4*>(Y + rr * kQkvYS + half + c);
    const int pos1 = (r.write_start ? r.write_start[b] : 0) + r.write_offset + t;
    const int pos2 = r.block_offset + t;
    const bool to_cache = r.k_cache != nullptr && pos1 >= 0 && pos1 < r.cache_len;
    const bool to_block = r.k_block != nullptr && pos2 >= 0 && pos2 < r.block_len;
    if (kind == 2) {
      if (r.v_out) put_pair(r.v_out, b * r.ko_stride_b + t * r.ko_stride_s + hh * r.ko_stride_h, c, half, ya, yb);
      if (to_cache) put_pair(r.v_cache, b * r.c_stride_b + pos1 * r.c_stride_s + hh * r.c_stride_h, c, half, ya, yb);
      if (to_block) put_pair(r.v_block, b * r.bc_stride_b + pos2 * r.bc_stride_s + hh * r.bc_stride_h, c, half, ya, yb);
      continue;
    }
    const uint16_t* cs = static_cast<const uint16_t*>(r.cos) + b * r.cs_stride_b + t * r.cs_stride_s;
    const uint16_t* sn = static_cast<const uint16_t*>(r.sin) + b * r.cs_stride_b + t * r.cs_stride_s;
    u32x4 w0, w1;
    rope8<T>(ya, yb, cs, sn, c, half, w0, w1);
    if (kind == 0) {
      put_pair(r.q_out, b * r.qo_stride_b + t * r.qo_stride_s + hh * r.qo_stride_h, c, half, w0, w1);
    } else {
      if (r.k_out) put_pair(r.k_out, b * r.ko_stride_b + t * r.ko_stride_s + hh * r.ko_stride_h, c, half, w0, w1);
      if (to_cache) put_pair(r.k_cache, b * r.c_stride_b + pos1 * r.c_stride_s + hh * r.c_stride_h, c, half, w0, w1);
      if (to_block) put_pair(r.k_block, b * r.bc_stride_b + pos2 * r.bc_stride_s + hh * r.bc_stride_h, c, half, w0, w1);
    }
  }
}

inline bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace fdllm

extern "C" int fdllm_rope_kv_write(const fdllm_rope_kv_desc* d, void* stream) {
  using namespace fdllm;
  FDLLM_CHECK_ARG(d != nullptr, "fdllm_rope_kv_write: null descriptor");
  FDLLM_CHECK_ARG(d->dtype == FDLLM_DTYPE_BF16 || d->dtype == FDLLM_DTYPE_F16,
                  "fdllm_rope_kv_write: dtype %d unsupported (bf16 or fp16)", d->dtype);
  FDLLM_CHECK_ARG(d->batch >= 0 && d->seq_len >= 0 && d->num_q_heads >= 0 && d->num_kv_heads >= 0,
                  "fdllm_rope_kv_write: bad sizes");
  FDLLM_CHECK_ARG(d->head_dim > 0 && d->head_dim % 16 == 0 && d->head_dim <= 512,
                  "fdllm_rope_kv_write: head_dim %d must be a multiple of 16 (<= 512)", d->head_dim);
  if (d->batch == 0 || d->seq_len == 0) return FDLLM_OK;
  FDLLM_CHECK_ARG(d->batch < 65536, "fdllm_rope_kv_write: batch too large");
  FDLLM_CHECK_ARG(d->q && d->k && d->v && d->cos && d->sin && d->q_out, "fdllm_rope_kv_write: null pointer");
  FDLLM_CHECK_ARG((d->k_out == nullptr) == (d->v_out == nullptr) &&
                      (d->k_cache == nullptr) == (d->v_cache == nullptr) &&
                      (d->k_block == nullptr) == (d->v_block == nullptr),
                  "fdllm_rope_kv_write: k and v destinations must be given together");
  const void* ptrs[] = {d->q, d->k, d->v, d->cos, d->sin, d->q_out, d->k_out, d->v_out,
                        d->k_cache, d->v_cache, d->k_block, d->v_block};
  for (const void* ptr : ptrs) FDLLM_CHECK_ARG(ptr == nullptr || al16(ptr), "fdllm_rope_kv_write: pointers must be 16-byte aligned");
  const int64_t strides[] = {d->q_stride_b, d->q_stride_s, d->q_stride_h, d->k_stride_b, d->k_stride_s, d->k_stride_h,
                             d->v_stride_b, d->v_stride_s, d->v_stride_h, d->cs_stride_b, d->cs_stride_s,
                             d->qo_stride_b, d->qo_stride_s, d->qo_stride_h, d->ko_stride_b, d->ko_stride_s,
                             d->ko_stride_h, d->c_stride_b, d->c_stride_s, d->c_stride_h, d->bc_stride_b,
                             d->bc_stride_s, d->bc_stride_h};
  for (int64_t s : strides) FDLLM_CHECK_ARG(s % 8 == 0, "fdllm_rope_kv_write: strides must be multiples of 8 elements");
  RopeArgs a;
  a.d = *d;
  a.npair = d->head_dim / 16;
  const dim3 grid(d->seq_len, d->batch);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (d->dtype == FDLLM_DTYPE_BF16) rope_kv_kernel<bf16_t><<<grid, dim3(256), 0, s>>>(a);
  else rope_kv_kernel<f16_t><<<grid, dim3(256), 0, s>>>(a);
  FDLLM_RETURN_LAUNCH_STATUS("fdllm_rope_kv_write");
}

extern "C" int fdllm_qkv_rope_kv_write(const fdllm_qkv_rope_desc* d, void* stream) {
  using namespace fdllm;
  FDLLM_CHECK_ARG(d != nullptr, "fdllm_qkv_rope_kv_write: null descriptor");
  const fdllm_rope_kv_desc& r = d->rope;
  FDLLM_CHECK_ARG(r.dtype == FDLLM_DTYPE_BF16 || r.dtype == FDLLM_DTYPE_F16,
                  "fdllm_qkv_rope_kv_write: dtype %d unsupported (bf16 or fp16)", r.dtype);
  FDLLM_CHECK_ARG(r.batch >= 0 && r.seq_len >= 0 && r.num_q_heads >= 0 && r.num_kv_heads >= 0,
                  "fdllm_qkv_rope_kv_write: bad sizes");
  FDLLM_CHECK_ARG(r.head_dim == kQkvBM, "fdllm_qkv_rope_kv_write: head_dim %d unsupported (128)", r.head_dim);
  FDLLM_CHECK_ARG(d->hidden >= 64 && d->hidden % 64 == 0 && d->hidden <= 65536,
                  "fdllm_qkv_rope_kv_write: hidden %d must be a multiple of 64 (at most 65536)", d->hidden);
  FDLLM_CHECK_ARG(d->x_stride_row >= d->hidden && d->x_stride_row % 8 == 0 && d->x_stride_row <= (1 << 22),
                  "fdllm_qkv_rope_kv_write: x_stride_row %lld must be a multiple of 8, at least hidden",
                  static_cast<long long>(d->x_stride_row));
  if (r.batch == 0 || r.seq_len == 0 || r.num_q_heads + r.num_kv_heads == 0) return FDLLM_OK;
  const int64_t T = static_cast<int64_t>(r.batch) * r.seq_len;
  FDLLM_CHECK_ARG(T < (int64_t{1} << 30), "fdllm_qkv_rope_kv_write: too many tokens");
  FDLLM_CHECK_ARG(d->x && d->wq && d->wk && d->wv && r.cos && r.sin && r.q_out, "fdllm_qkv_rope_kv_write: null pointer");
  FDLLM_CHECK_ARG((r.k_out == nullptr) == (r.v_out == nullptr) && (r.k_cache == nullptr) == (r.v_cache == nullptr) &&
                      (r.k_block == nullptr) == (r.v_block == nullptr),
                  "fdllm_qkv_rope_kv_write: k and v destinations must be given together");
  const void* ptrs[] = {d->x, d->wq, d->wk, d->wv, r.cos, r.sin, r.q_out, r.k_out, r.v_out,
                        r.k_cache, r.v_cache, r.k_block, r.v_block};
  for (const void* ptr : ptrs)
    FDLLM_CHECK_ARG(ptr == nullptr || al16(ptr), "fdllm_qkv_rope_kv_write: pointers must be 16-byte aligned");
  const int64_t strides[] = {r.cs_stride_b, r.cs_stride_s, r.qo_stride_b, r.qo_stride_s, r.qo_stride_h,
                             r.ko_stride_b, r.ko_stride_s, r.ko_stride_h, r.c_stride_b, r.c_stride_s,
                             r.c_stride_h, r.bc_stride_b, r.bc_stride_s, r.bc_stride_h};
  for (int64_t st : strides)
    FDLLM_CHECK_ARG(st % 8 == 0, "fdllm_qkv_rope_kv_write: strides must be multiples of 8 elements");
  QkvArgs a;
  a.d = *d;
  a.T = static_cast<int>(T);
  a.n_mt = static_cast<int>((T + kQkvBM - 1) / kQkvBM);
  const int heads = r.num_q_heads + 2 * r.num_kv_heads;
  FDLLM_CHECK_ARG(static_cast<int64_t>(a.n_mt) * heads * 2 < (int64_t{1} << 30), "fdllm_qkv_rope_kv_write: too many tiles");
  // Whole-head tiles while they give the compute units more than half a workgroup each;
  // with fewer (the 128-row sub-block forward: 36 tiles), half-head tiles, twice as many
  // workgroups each streaming 3/4 of the bytes: 29 against 41 us on the 7B layout (at 512
  // rows the half-head form, 288 workgroups for 256 compute units, took 55 against 40 us).
  const bool half_head = a.n_mt * heads <= 128;
  a.n_tiles = a.n_mt * heads * (half_head ? 2 : 1);
  a.per_xcd = (a.n_tiles + 7) / 8;
  const dim3 grid(static_cast<unsigned>(8 * a.per_xcd));
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (r.dtype == FDLLM_DTYPE_BF16) {
    if (half_head) qkv_rope_kernel<bf16_t, false, 64, 5><<<grid, dim3(256), 0, s>>>(a);
    else qkv_rope_kernel<bf16_t, false, 128, 4><<<grid, dim3(256), 0, s>>>(a);
  } else {
    if (half_head) qkv_rope_kernel<f16_t, true, 64, 5><<<grid, dim3(256), 0, s>>>(a);
    else qkv_rope_kernel<f16_t, true, 128, 4><<<grid, dim3(256), 0, s>>>(a);
  }
  FDLLM_RETURN_LAUNCH_STATUS("fdllm_qkv_rope_kv_write");
}
