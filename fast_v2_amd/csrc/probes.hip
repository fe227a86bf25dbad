// Measurement probes for gfx950 (libfdllm_probes.so; bench.py only, not part of the
// operator library): the practical floor of the two HBM-bound calls, as plain data
// movement in the same access pattern and launch shape.
//
//   fdllm_probe_read_kv    reads every visible K and V row of every KV head of a paged
//                          (or contiguous) cache once, in the split decode kernel's
//                          pattern: one KV head per workgroup, 32-key tiles of one page,
//                          two teams of 256 threads taking alternate tiles,
//                          FDLLM_PROBE_STAGES (default two) tiles in flight per team
//                          (2 / 4 / 6 measured 16.9 / 17.1 / 17.6 us on the bs16 step:
//                          a deeper pipeline does not lower the floor), the keys of all
//                          sequences dealt evenly over
//                          the workgroups. No math: the data is folded with XOR and a
//                          word is written only if the fold hits a constant (it never
//                          does in practice), so nothing is skipped by the compiler.
//   fdllm_probe_copy_rows  copies dst[t] = src[idx[t]] for rows of a multiple of 16 bytes
//                          (at most 16 KB), one wave per row (one row per workgroup),
//                          every load issued before the first store.
//   fdllm_probe_mfma       the sustained rate of v_mfma_f32_32x32x16_bf16, the instruction
//                          of the prefill / full-block kernels: one wave per SIMD, four
//                          independent accumulator chains per wave (one chain is bound by
//                          the 48-cycle dependent latency, two or more issue every 32
//                          cycles), operands in registers, no memory traffic in the loop.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/fdllm_probes.h"

#ifndef FDLLM_PROBE_STAGES
#define FDLLM_PROBE_STAGES 2
#endif

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr int kBufferFlags = 0x00020000;
constexpr int kProbeMaxPages = 4096;

__device__ __forceinline__ int probe_scan_i32(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false);  // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);  // row_bcast:15
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);  // row_bcast:31
  return v;
}

struct ReadArgs {
  const uint16_t* k;
  const uint16_t* v;
  int64_t k_sp, k_ss, k_sh, v_sp, v_ss, v_sh;  // element strides
  const int32_t* page_table;                   // [batch, max_pages] or null (contiguous: page = sequence)
  const int32_t* seqlens;
  int max_pages, page_shift, batch;
  uint32_t* sink;
};

// grid (S, Hkv), 512 threads; S a multiple of 8 (slot order XCD-major as in the decode kernel)
__global__ __launch_bounds__(512) void probe_read_kv_kernel(const ReadArgs a) {
  __shared__ int sPages[kProbeMaxPages];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int team = __builtin_amdgcn_readfirstlane(tid >> 8);
  const int ttid = tid & 255;
  const int kvh = blockIdx.y;
  const int n_pt = a.page_table ? a.batch * a.max_pages : 0;
  for (int i = tid; i < n_pt; i += 512) sPages[i] = a.page_table[i];
  // tiles of 32 keys per sequence (lane b), dealt evenly over the S slots of the head
  const bool has = lane < a.batch;
  const int len = has ? max(0, a.seqlens[lane]) : 0;
  const int tiles = (len + 31) >> 5;
  const int incl = probe_scan_i32(tiles);
  const int T = __builtin_amdgcn_readlane(incl, 63);
  const int S = gridDim.x;
  const int x = blockIdx.x;
  const int slot = (S & 7) == 0 ? (x & 7) * (S >> 3) + (x >> 3) : x;
  const int lo = static_cast<int>(static_cast<int64_t>(slot) * T / S);
  const int hi = static_cast<int>(static_cast<int64_t>(slot + 1) * T / S);
  __syncthreads();
  if (hi <= lo) return;  // uniform
  // cursor over the sequences of the run (moves forward only)
  int b = static_cast<int>(__builtin_ctzll(__builtin_amdgcn_ballot_w64(has && incl - tiles <= lo && lo < incl)));
  int b_off = __builtin_amdgcn_readlane(incl - tiles, b);
  int b_end = __builtin_amdgcn_readlane(incl, b);
  int b_len = __builtin_amdgcn_readlane(len, b);
  const int krow = static_cast<int>(a.k_ss) * 2, vrow = static_cast<int>(a.v_ss) * 2;
  int koff[2], voff[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int c = ttid + 256 * i;
    koff[i] = (c >> 4) * krow + (c & 15) * 16;
    voff[i] = (c >> 4) * vrow + (c & 15) * 16;
  }
  constexpr int NS = FDLLM_PROBE_STAGES;
  struct Stage {
    u32x4 k[2], v[2];
  } st[NS];
  const int n = hi - lo;  // tiles of this workgroup; team tm takes tiles 2 j + tm
  auto load = [&](Stage& sg, int j) {
    const int t = 2 * j + team;
    const int g = lo + min(t, n - 1);
    while (g >= b_end) {  // uniform, forward only
      ++b;
      b_off = b_end;
      b_end = __builtin_amdgcn_readlane(incl, b);
      b_len = __builtin_amdgcn_readlane(len, b);
    }
    const int kb = (g - b_off) * 32;
    const int valid = t < n ? min(32, b_len - kb) : 0;
    int64_t ko, vo;
    if (a.page_table) {
      const int page = sPages[b * a.max_pages + min(kb >> a.page_shift, a.max_pages - 1)];
      const int s0 = kb & ((1 << a.page_shift) - 1);
      ko = page * a.k_sp + s0 * a.k_ss;
      vo = page * a.v_sp + s0 * a.v_ss;
    } else {
      ko = b * a.k_sp + static_cast<int64_t>(kb) * a.k_ss;
      vo = b * a.v_sp + static_cast<int64_t>(kb) * a.v_ss;
    }
    const auto kr = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.k + kvh * a.k_sh + ko), 0,
                                                      __builtin_amdgcn_readfirstlane(valid * krow), kBufferFlags);
    const auto vr = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.v + kvh * a.v_sh + vo), 0,
                                                      __builtin_amdgcn_readfirstlane(valid * vrow), kBufferFlags);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      sg.k[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(kr, koff[i], 0, 2));
      sg.v[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(vr, voff[i], 0, 2));
    }
  };
  u32x4 acc = {0u, 0u, 0u, 0u};
  const int nsteps = (n + 1) >> 1;
#pragma unroll
  for (int s = 0; s < NS; ++s) load(st[s], s);
  for (int j = 0; j < nsteps; j += NS) {
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      acc ^= st[s].k[0] ^ st[s].k[1] ^ st[s].v[0] ^ st[s].v[1];
      load(st[s], j + NS + s);  // steps past the last read nothing (empty descriptor)
    }
  }
  if ((acc[0] ^ acc[1] ^ acc[2] ^ acc[3]) == 0x9e3779b9u) a.sink[0] = acc[0];
}

// one wave per row: rows[t] = src[idx[t]], nvec 16-byte vectors per row (<= 64 * VPL)
template <int VPL>
__global__ __launch_bounds__(64) void probe_copy_rows_kernel(const u32x4* src, int64_t src_row_vec, const int64_t* idx,
                                                             int src_rows, u32x4* dst, int rows, int nvec) {
  const int t = blockIdx.x;
  const int lane = threadIdx.x;
  const int64_t r = idx[t];
  if (static_cast<uint64_t>(r) >= static_cast<uint64_t>(src_rows)) return;  // uniform
  const u32x4* s = src + r * src_row_vec;
  u32x4* d = dst + static_cast<int64_t>(t) * nvec;
  u32x4 x[VPL];
#pragma unroll
  for (int v = 0; v < VPL; ++v) {
    const int c = lane + 64 * v;
    x[v] = c < nvec ? __builtin_nontemporal_load(s + c) : u32x4{0u, 0u, 0u, 0u};
  }
#pragma unroll
  for (int v = 0; v < VPL; ++v) {
    const int c = lane + 64 * v;
    if (c < nvec) __builtin_nontemporal_store(x[v], d + c);
  }
}

// rounds x 4 MFMAs per wave on register operands; 256 threads = one wave per SIMD
__global__ __launch_bounds__(256) void probe_mfma_kernel(float* sink, int rounds, float seed) {
  typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
  typedef float f32x16 __attribute__((ext_vector_type(16)));
  bf16x8 a, b;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    a[i] = static_cast<__bf16>(seed * static_cast<float>((threadIdx.x + i) & 15));
    b[i] = static_cast<__bf16>(seed * static_cast<float>((threadIdx.x * 3 + i) & 15));
  }
  f32x16 c[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) c[k] = f32x16{};
#pragma unroll 4
  for (int n = 0; n < rounds; ++n) {
#pragma unroll
    for (int k = 0; k < 4; ++k) c[k] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c[k], 0, 0, 0);
  }
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < 4; ++k)
#pragma unroll
    for (int e = 0; e < 16; ++e) s += c[k][e];
  if (s == 1234.5f) sink[blockIdx.x * 256 + threadIdx.x] = s;  // keeps the chains live
}

}  // namespace

extern "C" int fdllm_probe_read_kv(const void* k, const void* v, int64_t k_stride_page, int64_t k_stride_slot,
                                   int64_t k_stride_h, int64_t v_stride_page, int64_t v_stride_slot,
                                   int64_t v_stride_h, const int32_t* page_table, int32_t max_pages,
                                   int32_t page_size, const int32_t* seqlens, int batch, int num_kv_heads,
                                   int slots, void* sink, void* stream) {
  if (!k || !v || !seqlens || !sink || batch < 1 || batch > 64 || num_kv_heads < 1 || num_kv_heads > 65535 ||
      slots < 8 || slots % 8 != 0 || slots > 65535)
    return FDLLM_PROBE_ERR_ARGS;
  if (k_stride_slot < 8 || v_stride_slot < 8 || k_stride_slot >= (1 << 24) || v_stride_slot >= (1 << 24))
    return FDLLM_PROBE_ERR_ARGS;
  int shift = 0;
  if (page_table) {
    if (page_size < 32 || (page_size & (page_size - 1)) != 0 || max_pages < 1 ||
        static_cast<int64_t>(batch) * max_pages > kProbeMaxPages)
      return FDLLM_PROBE_ERR_ARGS;
    while ((1 << shift) < page_size) ++shift;
  }
  ReadArgs a;
  a.k = static_cast<const uint16_t*>(k);
  a.v = static_cast<const uint16_t*>(v);
  a.k_sp = k_stride_page;
  a.k_ss = k_stride_slot;
  a.k_sh = k_stride_h;
  a.v_sp = v_stride_page;
  a.v_ss = v_stride_slot;
  a.v_sh = v_stride_h;
  a.page_table = page_table;
  a.seqlens = seqlens;
  a.max_pages = max_pages;
  a.page_shift = shift;
  a.batch = batch;
  a.sink = static_cast<uint32_t*>(sink);
  probe_read_kv_kernel<<<dim3(slots, num_kv_heads), dim3(512), 0, static_cast<hipStream_t>(stream)>>>(a);
  return hipGetLastError() == hipSuccess ? 0 : FDLLM_PROBE_ERR_LAUNCH;
}

extern "C" int fdllm_probe_copy_rows(const void* src, int64_t src_row_bytes, int src_rows, const int64_t* idx,
                                     void* dst, int rows, int row_bytes, void* stream) {
  if (!src || !idx || !dst || rows < 0 || src_rows < 0 || row_bytes <= 0 || row_bytes % 16 != 0 ||
      row_bytes > 16 * 1024 || src_row_bytes % 16 != 0 || src_row_bytes < row_bytes ||
      (reinterpret_cast<uintptr_t>(src) & 15) || (reinterpret_cast<uintptr_t>(dst) & 15))
    return FDLLM_PROBE_ERR_ARGS;
  if (rows == 0) return 0;
  const int nvec = row_bytes / 16;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const u32x4* sp = static_cast<const u32x4*>(src);
  u32x4* dp = static_cast<u32x4*>(dst);
  const int64_t srv = src_row_bytes / 16;
  if (nvec <= 64 * 4) probe_copy_rows_kernel<4><<<dim3(rows), dim3(64), 0, s>>>(sp, srv, idx, src_rows, dp, rows, nvec);
  else if (nvec <= 64 * 8) probe_copy_rows_kernel<8><<<dim3(rows), dim3(64), 0, s>>>(sp, srv, idx, src_rows, dp, rows, nvec);
  else probe_copy_rows_kernel<16><<<dim3(rows), dim3(64), 0, s>>>(sp, srv, idx, src_rows, dp, rows, nvec);
  return hipGetLastError() == hipSuccess ? 0 : FDLLM_PROBE_ERR_LAUNCH;
}

extern "C" int fdllm_probe_mfma(int workgroups, int rounds, float* sink, void* stream) {
  if (!sink || workgroups < 1 || workgroups > 65535 || rounds < 1 || rounds > (1 << 24)) return FDLLM_PROBE_ERR_ARGS;
  probe_mfma_kernel<<<dim3(workgroups), dim3(256), 0, static_cast<hipStream_t>(stream)>>>(sink, rounds, 1.f / 64.f);
  return hipGetLastError() == hipSuccess ? 0 : FDLLM_PROBE_ERR_LAUNCH;
}
