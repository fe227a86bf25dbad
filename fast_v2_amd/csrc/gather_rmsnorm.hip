// Row gather + RMSNorm and row scatter for gfx950.
//
// Semantics follow cuda_bench/fused_gather_norm.cu (select_gather_rmsnorm_kernel
// :123-175, gather_rmsnorm_kernel :21-58, scatter_and_return_kernel :79-99) and
// the RMSNorm rounding order of Fast_dLLM_QwenRMSNorm.forward (modeling.py:427-432).
//
// Design (HBM-bound, one pass over each selected row):
//   - one 64-lane wavefront per output row; the row is pulled into registers
//     with 16-byte loads (VPL loads per lane, all issued before any use),
//   - sum of squares in fp32, reduced across the wave with DPP row moves plus
//     two cross-row swizzles; no LDS, no atomics, deterministic order,
//   - the gathered copy and the normalised row are written from the same
//     registers, so each input byte is read exactly once.
#include <stdarg.h>
#include <stdio.h>

#include <type_traits>

#include "fdllm_common.h"

namespace fdllm {

namespace {

// 16 bytes of T unpacked to fp32 and back.
template <typename T>
struct Vec16;
template <>
struct Vec16<bf16_t> {
  static constexpr int N = 8;
  __device__ __forceinline__ static void unpack(const u32x4& v, float* f) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = Elt<bf16_t>::lo(v[i]);
      f[2 * i + 1] = Elt<bf16_t>::hi(v[i]);
    }
  }
  __device__ __forceinline__ static u32x4 pack(const float* f) {
    u32x4 v;
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = Elt<bf16_t>::pack(f[2 * i], f[2 * i + 1]);
    return v;
  }
  __device__ __forceinline__ static float round(float x) { return Elt<bf16_t>::round(x); }
};
template <>
struct Vec16<f16_t> {
  static constexpr int N = 8;
  __device__ __forceinline__ static void unpack(const u32x4& v, float* f) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = Elt<f16_t>::lo(v[i]);
      f[2 * i + 1] = Elt<f16_t>::hi(v[i]);
    }
  }
  __device__ __forceinline__ static u32x4 pack(const float* f) {
    u32x4 v;
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = Elt<f16_t>::pack(f[2 * i], f[2 * i + 1]);
    return v;
  }
  __device__ __forceinline__ static float round(float x) { return Elt<f16_t>::round(x); }
};
template <>
struct Vec16<float> {
  static constexpr int N = 4;
  __device__ __forceinline__ static void unpack(const u32x4& v, float* f) {
#pragma unroll
    for (int i = 0; i < 4; ++i) f[i] = __uint_as_float(v[i]);
  }
  __device__ __forceinline__ static u32x4 pack(const float* f) {
    u32x4 v;
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = __float_as_uint(f[i]);
    return v;
  }
  __device__ __forceinline__ static float round(float x) { return x; }
};

// Weight kinds of the vector path: none, the 16-bit type of the rows (T), fp32.
constexpr int kWNone = 0;
constexpr int kW16 = 1;
constexpr int kW32 = 2;

// Load elements [e0, e0 + N) of the weight vector as fp32 (unconditional loads).
template <typename T, int WK, int N>
__device__ __forceinline__ void load_weight(const void* w, int e0, float* out) {
  if constexpr (WK == kW32) {
    const u32x4* p = reinterpret_cast<const u32x4*>(static_cast<const float*>(w) + e0);
#pragma unroll
    for (int i = 0; i < N / 4; ++i) {
      const u32x4 v = p[i];
#pragma unroll
      for (int j = 0; j < 4; ++j) out[4 * i + j] = __uint_as_float(v[j]);
    }
  } else if constexpr (WK == kW16) {
    const uint16_t* base = static_cast<const uint16_t*>(w) + e0;
    uint32_t words[N / 2];
    if constexpr (N == 8) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(base);
#pragma unroll
      for (int j = 0; j < 4; ++j) words[j] = v[j];
    } else {
      const u32x2 v = *reinterpret_cast<const u32x2*>(base);
      words[0] = v[0];
      words[1] = v[1];
    }
#pragma unroll
    for (int j = 0; j < N / 2; ++j) {
      out[2 * j] = Elt<T>::lo(words[j]);
      out[2 * j + 1] = Elt<T>::hi(words[j]);
    }
  } else {
#pragma unroll
    for (int i = 0; i < N; ++i) out[i] = 1.f;
  }
}

__device__ __forceinline__ float load_weight_scalar(const void* w, int wdtype, int e) {
  if (wdtype == FDLLM_DTYPE_F32) return static_cast<const float*>(w)[e];
  const uint16_t bits = static_cast<const uint16_t*>(w)[e];
  return wdtype == FDLLM_DTYPE_BF16 ? bf16_bits_to_f32(bits) : f16_bits_to_f32(bits);
}

template <typename T>
__device__ __forceinline__ float apply_norm(float x, float inv, float w, int mode) {
  if (mode == FDLLM_NORM_PLAIN) return x * inv;
  if (mode == FDLLM_NORM_WEIGHT_FP32) return (x * inv) * w;
  // FDLLM_NORM_WEIGHT_AFTER_CAST: weight * normalized.to(dtype), product rounded once more
  return w * Vec16<T>::round(x * inv);
}

// Compile-time form of apply_norm for the vector path. NORM_PLAIN is the fp32 form with
// a weight of 1 (x * inv * 1 == x * inv exactly).
template <typename T, bool CAST>
__device__ __forceinline__ float apply_norm_ct(float x, float inv, float w) {
  if constexpr (CAST) return w * Vec16<T>::round(x * inv);
  return (x * inv) * w;
}

struct GatherArgs {
  const void* hidden;
  int64_t hs_b, hs_s;
  const int64_t* idx;
  int64_t is_b;
  const void* weight;
  int wdtype;
  void* normed;
  void* gathered;
  int B, S, T, H;
  float eps;
  int mode;
};

// Vector path: H * sizeof(T) is a multiple of 16 and every row is 16-byte aligned.
// VPL = 16-byte vectors per lane (the whole row stays in registers). The norm form is a
// template parameter, so the per-element code is straight-line. Outputs are written once
// and not read again by this kernel: non-temporal (streaming) stores.
//
// The arguments the index load and the row address need come first, as scalars: with
// kernel-argument preloading they arrive in SGPRs at wave launch, so the index load
// is the first memory access (the rest of the arguments load beside it).
// Rows (waves) per workgroup of the vector path.
#ifndef FDLLM_GATHER_ROWS_PER_WG
#define FDLLM_GATHER_ROWS_PER_WG 4
#endif
constexpr int kGatherRows = FDLLM_GATHER_ROWS_PER_WG;

template <typename T, int WK, bool CAST, bool GATHERED, int VPL>
__global__ __launch_bounds__(64 * kGatherRows) void gather_rmsnorm_vec_kernel(const int64_t* idx, int64_t is_b,
                                                                 const void* hidden, int64_t hs_b, int64_t hs_s,
                                                                 int T_rows, int S_rows, const GatherArgs a) {
  constexpr int N = Vec16<T>::N;
  const int lane = threadIdx.x & (kWave - 1);
  // grid (ceil(T / kGatherRows), B): kGatherRows rows of one sequence per workgroup, no
  // division; the row is wave-uniform, so its index, bounds check and addresses live in
  // scalar registers
  const int b = blockIdx.y;
  const int t = static_cast<int>(blockIdx.x) * kGatherRows + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (t >= T_rows) return;
  const int64_t src = idx[b * is_b + t];
  const int nvec = a.H / N;
  const int64_t row = static_cast<int64_t>(b) * T_rows + t;
  const T* hbase = static_cast<const T*>(hidden) + b * hs_b;
  u32x4* nrow = reinterpret_cast<u32x4*>(static_cast<T*>(a.normed) + row * a.H);
  u32x4* grow = GATHERED ? reinterpret_cast<u32x4*>(static_cast<T*>(a.gathered) + row * a.H) : nullptr;
  // an index outside [0, S) gives zero rows (a wave-uniform exit before any row load)
  if (__builtin_expect(static_cast<uint64_t>(src) >= static_cast<uint64_t>(S_rows), 0)) {
    const u32x4 z = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int v = 0; v < VPL; ++v) {
      const int c = lane + kWave * v;
      if (c < nvec) {
        __builtin_nontemporal_store(z, nrow + c);
        if constexpr (GATHERED) __builtin_nontemporal_store(z, grow + c);
      }
    }
    return;
  }

  const u32x4* hrow = reinterpret_cast<const u32x4*>(hbase + src * hs_s);
  // All loads are issued unconditionally and back to back, so the whole row is in flight
  // at once; they are non-temporal (each row is read once: 4.42 -> 4.08 us per call at
  // 1024 rows x 3584 bf16, against 3.79 us for a plain gathered copy of the rows). nvec lies in (64 (VPL - 1), 64 VPL], so only the last vector can run past the
  // row end: its index is clamped and its lanes past the end are zeroed afterwards.
  const int clast = lane + kWave * (VPL - 1);
  const bool last_in = clast < nvec;
  u32x4 x[VPL];
#pragma unroll
  for (int v = 0; v < VPL - 1; ++v) x[v] = __builtin_nontemporal_load(hrow + lane + kWave * v);
  x[VPL - 1] = __builtin_nontemporal_load(hrow + (last_in ? clast : nvec - 1));
  float w[VPL][N];
#pragma unroll
  for (int v = 0; v < VPL - 1; ++v) load_weight<T, WK, N>(a.weight, (lane + kWave * v) * N, w[v]);
  load_weight<T, WK, N>(a.weight, (last_in ? clast : nvec - 1) * N, w[VPL - 1]);
  if (!last_in) x[VPL - 1] = u32x4{0u, 0u, 0u, 0u};

  float ss = 0.f;
#pragma unroll
  for (int v = 0; v < VPL; ++v) {
    float f[N];
    Vec16<T>::unpack(x[v], f);
#pragma unroll
    for (int i = 0; i < N; ++i) ss += f[i] * f[i];
  }
  ss = wave_allreduce_sum(ss);
  const float inv = 1.0f / sqrtf(ss / static_cast<float>(a.H) + a.eps);

#pragma unroll
  for (int v = 0; v < VPL; ++v) {
    float f[N];
    Vec16<T>::unpack(x[v], f);
    if constexpr (CAST && std::is_same<T, bf16_t>::value) {
      // weight * bf16(x * inv): two elements rounded by one v_cvt_pk_bf16_f32 (round to
      // nearest even on each, as two single conversions), then widened and weighted
#pragma unroll
      for (int i = 0; i < N; i += 2) {
        const uint32_t r = Elt<T>::pack(f[i] * inv, f[i + 1] * inv);
        f[i] = w[v][i] * Elt<T>::lo(r);
        f[i + 1] = w[v][i + 1] * Elt<T>::hi(r);
      }
    } else {
#pragma unroll
      for (int i = 0; i < N; ++i) f[i] = apply_norm_ct<T, CAST>(f[i], inv, w[v][i]);
    }
    const u32x4 o = Vec16<T>::pack(f);
    if (v < VPL - 1 || last_in) {
      const int c = lane + kWave * v;
      if constexpr (GATHERED) __builtin_nontemporal_store(x[v], grow + c);
      __builtin_nontemporal_store(o, nrow + c);
    }
  }
}

// Generic path: any H, any alignment. One wave per row, two passes over the row.
template <typename T>
__device__ __forceinline__ float load_elem(const T* p);
template <>
__device__ __forceinline__ float load_elem<float>(const float* p) { return *p; }
template <>
__device__ __forceinline__ float load_elem<bf16_t>(const bf16_t* p) { return bf16_bits_to_f32(p->bits); }
template <>
__device__ __forceinline__ float load_elem<f16_t>(const f16_t* p) { return f16_bits_to_f32(p->bits); }

template <typename T>
__device__ __forceinline__ void store_elem(T* p, float v);
template <>
__device__ __forceinline__ void store_elem<float>(float* p, float v) { *p = v; }
template <>
__device__ __forceinline__ void store_elem<bf16_t>(bf16_t* p, float v) { p->bits = static_cast<uint16_t>(f32_to_bf16_bits(v)); }
template <>
__device__ __forceinline__ void store_elem<f16_t>(f16_t* p, float v) { p->bits = static_cast<uint16_t>(f32_to_f16_bits(v)); }

template <typename T>
__global__ __launch_bounds__(256) void gather_rmsnorm_generic_kernel(const GatherArgs a) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= static_cast<int64_t>(a.B) * a.T) return;
  const int b = static_cast<int>(row / a.T);
  const int t = static_cast<int>(row - static_cast<int64_t>(b) * a.T);
  const int64_t src = a.idx[b * a.is_b + t];
  T* nrow = static_cast<T*>(a.normed) + row * a.H;
  T* grow = a.gathered ? static_cast<T*>(a.gathered) + row * a.H : nullptr;
  if (src < 0 || src >= a.S) {
    for (int e = lane; e < a.H; e += kWave) {
      store_elem<T>(nrow + e, 0.f);
      if (grow) store_elem<T>(grow + e, 0.f);
    }
    return;
  }
  const T* hrow = static_cast<const T*>(a.hidden) + b * a.hs_b + src * a.hs_s;
  float ss = 0.f;
  for (int e = lane; e < a.H; e += kWave) {
    const float x = load_elem<T>(hrow + e);
    ss += x * x;
  }
  ss = wave_allreduce_sum(ss);
  const float inv = 1.0f / sqrtf(ss / static_cast<float>(a.H) + a.eps);
  for (int e = lane; e < a.H; e += kWave) {
    if (grow) grow[e] = hrow[e];
    const float x = load_elem<T>(hrow + e);
    const float w = a.mode != FDLLM_NORM_PLAIN ? load_weight_scalar(a.weight, a.wdtype, e) : 1.f;
    store_elem<T>(nrow + e, apply_norm<T>(x, inv, w, a.mode));
  }
}


// Row scatter to two destinations (scatter_and_return_kernel, fused_gather_norm.cu:79-99):
// one wave per source row, 16-byte vectors when rows are aligned, else 2/4-byte elements.
struct ScatterArgs {
  const void* values;
  const int64_t* idx;
  int64_t is_b;
  void* cache;
  int64_t cs_b, cs_s;
  void* cur;
  int64_t us_b, us_s;
  int B, S, T, H;  // H in elements
  int esize;       // bytes per element
  int vec16;       // rows are 16-byte aligned and H * esize % 16 == 0
};

__global__ __launch_bounds__(256) void scatter_rows_kernel(const ScatterArgs a) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= static_cast<int64_t>(a.B) * a.T) return;
  const int b = static_cast<int>(row / a.T);
  const int t = static_cast<int>(row - static_cast<int64_t>(b) * a.T);
  const int64_t dst = a.idx[b * a.is_b + t];
  if (dst < 0 || dst >= a.S) return;
  const char* src = static_cast<const char*>(a.values) + row * a.H * a.esize;
  char* c = static_cast<char*>(a.cache) + (b * a.cs_b + dst * a.cs_s) * a.esize;
  // the second destination is optional (single-destination row scatter)
  char* u = a.cur ? static_cast<char*>(a.cur) + (b * a.us_b + dst * a.us_s) * a.esize : nullptr;
  if (a.vec16) {
    const int nvec = a.H * a.esize / 16;
    for (int i = lane; i < nvec; i += kWave) {
      const u32x4 v = reinterpret_cast<const u32x4*>(src)[i];
      reinterpret_cast<u32x4*>(c)[i] = v;
      if (u) reinterpret_cast<u32x4*>(u)[i] = v;
    }
  } else if (a.esize == 4) {
    for (int i = lane; i < a.H; i += kWave) {
      const uint32_t v = reinterpret_cast<const uint32_t*>(src)[i];
      reinterpret_cast<uint32_t*>(c)[i] = v;
      if (u) reinterpret_cast<uint32_t*>(u)[i] = v;
    }
  } else {
    for (int i = lane; i < a.H; i += kWave) {
      const uint16_t v = reinterpret_cast<const uint16_t*>(src)[i];
      reinterpret_cast<uint16_t*>(c)[i] = v;
      if (u) reinterpret_cast<uint16_t*>(u)[i] = v;
    }
  }
}

// The 16-byte-aligned form: one wave per source row, the row's VPL vectors per lane all
// loaded before any store (the element loop above waits for each load in turn, since the
// destinations may alias the values as far as the compiler knows). grid (B * T). Loads and
// stores are non-temporal (streaming): at 1024 rows x 3584 bf16 into two destinations
// this took the call from 6.90 to 4.77 us (plain loads with streaming stores: 5.0 us).
template <int VPL>
__global__ __launch_bounds__(64) void scatter_rows_vec_kernel(const ScatterArgs a) {
  const int lane = threadIdx.x;
  const int64_t row = blockIdx.x;
  const int b = static_cast<int>(row / a.T);
  const int t = static_cast<int>(row - static_cast<int64_t>(b) * a.T);
  const int64_t dst = a.idx[b * a.is_b + t];
  if (dst < 0 || dst >= a.S) return;  // uniform: one row per wave
  const int nvec = a.H * a.esize / 16;
  const u32x4* src = reinterpret_cast<const u32x4*>(static_cast<const char*>(a.values) + row * a.H * a.esize);
  u32x4* c = reinterpret_cast<u32x4*>(static_cast<char*>(a.cache) + (b * a.cs_b + dst * a.cs_s) * a.esize);
  u32x4 x[VPL];
#pragma unroll
  for (int v = 0; v < VPL; ++v) {
    const int i = lane + kWave * v;
    x[v] = i < nvec ? __builtin_nontemporal_load(src + i) : u32x4{0u, 0u, 0u, 0u};
  }
#pragma unroll
  for (int v = 0; v < VPL; ++v) {
    const int i = lane + kWave * v;
    if (i < nvec) __builtin_nontemporal_store(x[v], c + i);
  }
  if (a.cur) {
    u32x4* u = reinterpret_cast<u32x4*>(static_cast<char*>(a.cur) + (b * a.us_b + dst * a.us_s) * a.esize);
#pragma unroll
    for (int v = 0; v < VPL; ++v) {
      const int i = lane + kWave * v;
      if (i < nvec) __builtin_nontemporal_store(x[v], u + i);
    }
  }
}

template <typename T, int WK, bool CAST, bool GATHERED>
bool launch_gather_vec(const GatherArgs& a, dim3 grid, hipStream_t stream) {
  const int nvec = a.H / Vec16<T>::N;
  const int vpl = (nvec + kWave - 1) / kWave;
  switch (vpl) {
#define FDLLM_VPL_CASE(n)                                                                  \
  case n:                                                                                  \
    gather_rmsnorm_vec_kernel<T, WK, CAST, GATHERED, n><<<grid, dim3(64 * kGatherRows), 0, stream>>>(  \
        a.idx, a.is_b, a.hidden, a.hs_b, a.hs_s, a.T, a.S, a);                              \
    return true;
    FDLLM_VPL_CASE(1)
    FDLLM_VPL_CASE(2)
    FDLLM_VPL_CASE(3)
    FDLLM_VPL_CASE(4)
    FDLLM_VPL_CASE(5)
    FDLLM_VPL_CASE(6)
    FDLLM_VPL_CASE(7)
    FDLLM_VPL_CASE(8)
    FDLLM_VPL_CASE(10)
    FDLLM_VPL_CASE(12)
    FDLLM_VPL_CASE(14)
    FDLLM_VPL_CASE(16)
#undef FDLLM_VPL_CASE
    default:
      return false;  // uneven or very wide rows: generic path
  }
}

template <typename T, int WK, bool CAST>
bool launch_gather_vec_out(const GatherArgs& a, dim3 grid, hipStream_t stream) {
  return a.gathered ? launch_gather_vec<T, WK, CAST, true>(a, grid, stream)
                    : launch_gather_vec<T, WK, CAST, false>(a, grid, stream);
}

template <typename T, int WK>
bool launch_gather_vec_mode(const GatherArgs& a, dim3 grid, hipStream_t stream) {
  return a.mode == FDLLM_NORM_WEIGHT_AFTER_CAST ? launch_gather_vec_out<T, WK, true>(a, grid, stream)
                                                : launch_gather_vec_out<T, WK, false>(a, grid, stream);
}

template <typename T>
int launch_gather(const GatherArgs& a, bool vec, hipStream_t stream) {
  const int64_t rows = static_cast<int64_t>(a.B) * a.T;
  const dim3 grid(static_cast<unsigned>((rows + 3) / 4));
  if (vec && a.B <= 65535) {
    const dim3 vgrid(static_cast<unsigned>((a.T + kGatherRows - 1) / kGatherRows), static_cast<unsigned>(a.B));
    bool done;
    if (a.mode == FDLLM_NORM_PLAIN) {
      done = launch_gather_vec_out<T, kWNone, false>(a, vgrid, stream);
    } else if (a.wdtype == FDLLM_DTYPE_F32) {
      done = launch_gather_vec_mode<T, kW32>(a, vgrid, stream);
    } else if constexpr (!std::is_same<T, float>::value) {
      // 16-bit weights in the rows' own format; other combinations take the generic path
      const bool same = (a.wdtype == FDLLM_DTYPE_BF16) == std::is_same<T, bf16_t>::value;
      done = same && launch_gather_vec_mode<T, kW16>(a, vgrid, stream);
    } else {
      done = false;
    }
    if (done) return 0;
  }
  gather_rmsnorm_generic_kernel<T><<<grid, dim3(256), 0, stream>>>(a);
  return 0;
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// ---------------------------------------------------------------------------
// Residual add + RMSNorm of contiguous rows: the decoder layer's
//   hidden_states = residual + hidden_states; normed = norm(hidden_states)
// (modeling.py:465-488 with the norm of :427-432). sum = x + r rounded to the rows' type
// (as the 16-bit add rounds), written to `sum`; the norm reads that rounded sum. One wave
// per row, the row in registers (VPL 16-byte vectors per lane), as the gather kernel.
struct AddNormArgs {
  const void* x;
  const void* r;
  const void* weight;
  void* sum;
  void* normed;
  int rows, H;
  float eps;
};

template <typename T, int WK, bool CAST, int VPL>
__global__ __launch_bounds__(256) void add_rmsnorm_kernel(const AddNormArgs a) {
  constexpr int N = Vec16<T>::N;
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (row >= a.rows) return;
  const int nvec = a.H / N;
  const u32x4* xr = reinterpret_cast<const u32x4*>(static_cast<const T*>(a.x) + row * a.H);
  const u32x4* rr = reinterpret_cast<const u32x4*>(static_cast<const T*>(a.r) + row * a.H);
  u32x4* sr = reinterpret_cast<u32x4*>(static_cast<T*>(a.sum) + row * a.H);
  u32x4* nr = reinterpret_cast<u32x4*>(static_cast<T*>(a.normed) + row * a.H);
  // only the last vector can run past the row end (nvec in (64 (VPL - 1), 64 VPL])
  const int clast = lane + kWave * (VPL - 1);
  const bool last_in = clast < nvec;
  u32x4 xv[VPL], rv[VPL];
#pragma unroll
  for (int v = 0; v < VPL; ++v) {
    const int c = v < VPL - 1 ? lane + kWave * v : (last_in ? clast : nvec - 1);
    xv[v] = xr[c];
    rv[v] = rr[c];
  }
  float w[VPL][N];
#pragma unroll
  for (int v = 0; v < VPL; ++v)
    load_weight<T, WK, N>(a.weight, (v < VPL - 1 ? lane + kWave * v : (last_in ? clast : nvec - 1)) * N, w[v]);
  float f[VPL][N];
  float ss = 0.f;
#pragma unroll
  for (int v = 0; v < VPL; ++v) {
    float fx[N], fr[N];
    Vec16<T>::unpack(xv[v], fx);
    Vec16<T>::unpack(rv[v], fr);
    const bool in = v < VPL - 1 || last_in;
#pragma unroll
    for (int i = 0; i < N; ++i) {
      f[v][i] = in ? Vec16<T>::round(fx[i] + fr[i]) : 0.f;
      ss += f[v][i] * f[v][i];
    }
  }
  ss = wave_allreduce_sum(ss);
  const float inv = 1.0f / sqrtf(ss / static_cast<float>(a.H) + a.eps);
#pragma unroll
  for (int v = 0; v < VPL; ++v) {
    if (v < VPL - 1 || last_in) {
      const int c = lane + kWave * v;
      float o[N];
#pragma unroll
      for (int i = 0; i < N; ++i) o[i] = apply_norm_ct<T, CAST>(f[v][i], inv, w[v][i]);
      __builtin_nontemporal_store(Vec16<T>::pack(f[v]), sr + c);
      __builtin_nontemporal_store(Vec16<T>::pack(o), nr + c);
    }
  }
}

template <typename T, int WK, bool CAST>
bool launch_add_rmsnorm(const AddNormArgs& a, hipStream_t stream) {
  const int vpl = (a.H / Vec16<T>::N + kWave - 1) / kWave;
  const dim3 grid(static_cast<unsigned>((a.rows + 3) / 4));
  switch (vpl) {
#define FDLLM_ADD_VPL_CASE(n)                                                          \
  case n:                                                                              \
    add_rmsnorm_kernel<T, WK, CAST, n><<<grid, dim3(256), 0, stream>>>(a);             \
    return true;
    FDLLM_ADD_VPL_CASE(1)
    FDLLM_ADD_VPL_CASE(2)
    FDLLM_ADD_VPL_CASE(3)
    FDLLM_ADD_VPL_CASE(4)
    FDLLM_ADD_VPL_CASE(5)
    FDLLM_ADD_VPL_CASE(6)
    FDLLM_ADD_VPL_CASE(7)
    FDLLM_ADD_VPL_CASE(8)
#undef FDLLM_ADD_VPL_CASE
    default:
      return false;
  }
}

// ---------------------------------------------------------------------------
// SiLU-gated product of the MLP, act_fn(gate_proj(x)) * up_proj(x) (modeling.py:164):
// out = round(round(silu(g)) * u) in the 16-bit type, silu(g) = g / (1 + exp(-g)) in
// fp32 (the 16-bit SiLU rounds its result, then the product rounds again). Eight
// elements per thread, 16-byte loads and stores.
template <typename T>
__global__ __launch_bounds__(256) void silu_mul_kernel(const u32x4* g, const u32x4* u, u32x4* out, int64_t nvec) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= nvec) return;
  float fg[8], fu[8], o[8];
  Vec16<T>::unpack(g[i], fg);
  Vec16<T>::unpack(u[i], fu);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float sg = Vec16<T>::round(fg[j] / (1.0f + expf(-fg[j])));
    o[j] = sg * fu[j];
  }
  __builtin_nontemporal_store(Vec16<T>::pack(o), out + i);
}

}  // namespace

static thread_local char g_last_error[512];

void set_last_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

int dtype_size(int dtype) {
  switch (dtype) {
    case FDLLM_DTYPE_F32:
      return 4;
    case FDLLM_DTYPE_BF16:
    case FDLLM_DTYPE_F16:
      return 2;
    default:
      return 0;
  }
}

}  // namespace fdllm

extern "C" int fdllm_abi_version(void) { return FDLLM_ABI_VERSION; }

extern "C" const char* fdllm_last_error(void) { return fdllm::g_last_error; }

extern "C" int fdllm_gather_rmsnorm(const void* hidden, int64_t hidden_batch_stride, int64_t hidden_row_stride,
                                    const int64_t* indices, int64_t indices_batch_stride,
                                    const void* weight, int weight_dtype,
                                    void* normed, void* gathered,
                                    int batch, int seq_len, int num_tokens, int hidden_size,
                                    float eps, int dtype, int norm_mode, void* stream) {
  using namespace fdllm;
  const int es = dtype_size(dtype);
  FDLLM_CHECK_ARG(es != 0, "fdllm_gather_rmsnorm: unsupported dtype %d", dtype);
  FDLLM_CHECK_ARG(norm_mode >= FDLLM_NORM_PLAIN && norm_mode <= FDLLM_NORM_WEIGHT_AFTER_CAST,
                  "fdllm_gather_rmsnorm: unknown norm_mode %d", norm_mode);
  FDLLM_CHECK_ARG(batch >= 0 && seq_len >= 0 && num_tokens >= 0 && hidden_size > 0,
                  "fdllm_gather_rmsnorm: bad sizes B=%d S=%d T=%d H=%d", batch, seq_len, num_tokens, hidden_size);
  if (static_cast<int64_t>(batch) * num_tokens == 0) return FDLLM_OK;
  FDLLM_CHECK_ARG(static_cast<int64_t>(batch) * num_tokens <= INT32_MAX - 3,
                  "fdllm_gather_rmsnorm: B * T = %lld rows exceeds 2^31 - 4", static_cast<long long>(batch) * num_tokens);
  FDLLM_CHECK_ARG(hidden && indices && normed, "fdllm_gather_rmsnorm: null pointer");
  FDLLM_CHECK_ARG(norm_mode == FDLLM_NORM_PLAIN || weight != nullptr,
                  "fdllm_gather_rmsnorm: norm_mode %d needs a weight", norm_mode);
  FDLLM_CHECK_ARG(norm_mode == FDLLM_NORM_PLAIN || dtype_size(weight_dtype) != 0,
                  "fdllm_gather_rmsnorm: unsupported weight dtype %d", weight_dtype);
  FDLLM_CHECK_ARG(!(eps < 0.f), "fdllm_gather_rmsnorm: eps must be >= 0");

  GatherArgs a;
  a.hidden = hidden;
  a.hs_b = hidden_batch_stride;
  a.hs_s = hidden_row_stride;
  a.idx = indices;
  a.is_b = indices_batch_stride;
  a.weight = weight;
  a.wdtype = weight_dtype;
  a.normed = normed;
  a.gathered = gathered;
  a.B = batch;
  a.S = seq_len;
  a.T = num_tokens;
  a.H = hidden_size;
  a.eps = eps;
  a.mode = norm_mode;

  const int N = 16 / es;
  const int wsz = norm_mode == FDLLM_NORM_PLAIN ? 0 : dtype_size(weight_dtype);
  const bool vec = (hidden_size % N == 0) && aligned16(hidden) && aligned16(normed) &&
                   (gathered == nullptr || aligned16(gathered)) &&
                   ((hidden_batch_stride * es) % 16 == 0) && ((hidden_row_stride * es) % 16 == 0) &&
                   (wsz == 0 || (reinterpret_cast<uintptr_t>(weight) % (wsz * N < 16 ? wsz * N : 16)) == 0);
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case FDLLM_DTYPE_BF16:
      launch_gather<bf16_t>(a, vec, s);
      break;
    case FDLLM_DTYPE_F16:
      launch_gather<f16_t>(a, vec, s);
      break;
    default:
      launch_gather<float>(a, vec, s);
      break;
  }
  FDLLM_RETURN_LAUNCH_STATUS("fdllm_gather_rmsnorm");
}

extern "C" int fdllm_scatter_rows(const void* values, const int64_t* indices, int64_t indices_batch_stride,
                                  void* cache, int64_t cache_batch_stride, int64_t cache_row_stride,
                                  void* current, int64_t current_batch_stride, int64_t current_row_stride,
                                  int batch, int seq_len, int num_tokens, int hidden_size,
                                  int dtype, void* stream) {
  using namespace fdllm;
  const int es = dtype_size(dtype);
  FDLLM_CHECK_ARG(es != 0, "fdllm_scatter_rows: unsupported dtype %d", dtype);
  FDLLM_CHECK_ARG(batch >= 0 && seq_len >= 0 && num_tokens >= 0 && hidden_size > 0,
                  "fdllm_scatter_rows: bad sizes B=%d S=%d T=%d H=%d", batch, seq_len, num_tokens, hidden_size);
  if (static_cast<int64_t>(batch) * num_tokens == 0) return FDLLM_OK;
  FDLLM_CHECK_ARG(values && indices && cache, "fdllm_scatter_rows: null pointer");
  ScatterArgs a;
  a.values = values;
  a.idx = indices;
  a.is_b = indices_batch_stride;
  a.cache = cache;
  a.cs_b = cache_batch_stride;
  a.cs_s = cache_row_stride;
  a.cur = current;
  a.us_b = current_batch_stride;
  a.us_s = current_row_stride;
  a.B = batch;
  a.S = seq_len;
  a.T = num_tokens;
  a.H = hidden_size;
  a.esize = es;
  a.vec16 = ((static_cast<int64_t>(hidden_size) * es) % 16 == 0) && aligned16(values) && aligned16(cache) &&
            (current == nullptr || aligned16(current)) && (cache_batch_stride * es) % 16 == 0 && (cache_row_stride * es) % 16 == 0 &&
            (current_batch_stride * es) % 16 == 0 && (current_row_stride * es) % 16 == 0;
  const int64_t rows = static_cast<int64_t>(batch) * num_tokens;
  FDLLM_CHECK_ARG(rows <= INT32_MAX, "fdllm_scatter_rows: %lld rows exceed the grid", static_cast<long long>(rows));
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t nvec = a.vec16 ? static_cast<int64_t>(hidden_size) * es / 16 : 0;
  if (a.vec16 && nvec <= kWave * 8) {
    const dim3 grid(static_cast<unsigned>(rows));
    if (nvec <= kWave * 2) scatter_rows_vec_kernel<2><<<grid, dim3(kWave), 0, s>>>(a);
    else if (nvec <= kWave * 4) scatter_rows_vec_kernel<4><<<grid, dim3(kWave), 0, s>>>(a);
    else if (nvec <= kWave * 6) scatter_rows_vec_kernel<6><<<grid, dim3(kWave), 0, s>>>(a);
    else scatter_rows_vec_kernel<8><<<grid, dim3(kWave), 0, s>>>(a);
  } else {
    scatter_rows_kernel<<<dim3(static_cast<unsigned>((rows + 3) / 4)), dim3(256), 0, s>>>(a);
  }
  FDLLM_RETURN_LAUNCH_STATUS("fdllm_scatter_rows");
}

extern "C" int fdllm_add_rmsnorm(const void* x, const void* residual, const void* weight, int weight_dtype,
                                 void* sum_out, void* normed, int rows, int hidden_size, float eps, int dtype,
                                 int norm_mode, void* stream) {
  using namespace fdllm;
  FDLLM_CHECK_ARG(dtype == FDLLM_DTYPE_BF16 || dtype == FDLLM_DTYPE_F16,
                  "fdllm_add_rmsnorm: dtype %d unsupported (bf16 or fp16)", dtype);
  FDLLM_CHECK_ARG(norm_mode >= FDLLM_NORM_PLAIN && norm_mode <= FDLLM_NORM_WEIGHT_AFTER_CAST,
                  "fdllm_add_rmsnorm: unknown norm_mode %d", norm_mode);
  FDLLM_CHECK_ARG(rows >= 0 && hidden_size > 0 && hidden_size % 8 == 0 && hidden_size <= 8 * 64 * 8,
                  "fdllm_add_rmsnorm: bad sizes rows=%d H=%d (H a multiple of 8, at most 4096)", rows, hidden_size);
  if (rows == 0) return FDLLM_OK;
  FDLLM_CHECK_ARG(x && residual && sum_out && normed, "fdllm_add_rmsnorm: null pointer");
  FDLLM_CHECK_ARG(aligned16(x) && aligned16(residual) && aligned16(sum_out) && aligned16(normed),
                  "fdllm_add_rmsnorm: rows must be 16-byte aligned");
  FDLLM_CHECK_ARG(norm_mode == FDLLM_NORM_PLAIN || weight != nullptr, "fdllm_add_rmsnorm: norm_mode %d needs a weight",
                  norm_mode);
  FDLLM_CHECK_ARG(norm_mode == FDLLM_NORM_PLAIN || weight_dtype == FDLLM_DTYPE_F32 || weight_dtype == dtype,
                  "fdllm_add_rmsnorm: weight dtype %d must be fp32 or the rows' type", weight_dtype);
  FDLLM_CHECK_ARG(norm_mode == FDLLM_NORM_PLAIN || aligned16(weight), "fdllm_add_rmsnorm: weight must be 16-byte aligned");
  FDLLM_CHECK_ARG(!(eps < 0.f), "fdllm_add_rmsnorm: eps must be >= 0");
  AddNormArgs a;
  a.x = x;
  a.r = residual;
  a.weight = weight;
  a.sum = sum_out;
  a.normed = normed;
  a.rows = rows;
  a.H = hidden_size;
  a.eps = eps;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool cast = norm_mode == FDLLM_NORM_WEIGHT_AFTER_CAST;
  bool done;
  if (dtype == FDLLM_DTYPE_BF16) {
    if (norm_mode == FDLLM_NORM_PLAIN) done = launch_add_rmsnorm<bf16_t, kWNone, false>(a, s);
    else if (weight_dtype == FDLLM_DTYPE_F32)
      done = cast ? launch_add_rmsnorm<bf16_t, kW32, true>(a, s) : launch_add_rmsnorm<bf16_t, kW32, false>(a, s);
    else done = cast ? launch_add_rmsnorm<bf16_t, kW16, true>(a, s) : launch_add_rmsnorm<bf16_t, kW16, false>(a, s);
  } else {
    if (norm_mode == FDLLM_NORM_PLAIN) done = launch_add_rmsnorm<f16_t, kWNone, false>(a, s);
    else if (weight_dtype == FDLLM_DTYPE_F32)
      done = cast ? launch_add_rmsnorm<f16_t, kW32, true>(a, s) : launch_add_rmsnorm<f16_t, kW32, false>(a, s);
    else done = cast ? launch_add_rmsnorm<f16_t, kW16, true>(a, s) : launch_add_rmsnorm<f16_t, kW16, false>(a, s);
  }
  FDLLM_CHECK_ARG(done, "fdllm_add_rmsnorm: hidden_size %d unsupported", hidden_size);
  FDLLM_RETURN_LAUNCH_STATUS("fdllm_add_rmsnorm");
}

extern "C" int fdllm_silu_mul(const void* gate, const void* up, void* out, int64_t n, int dtype, void* stream) {
  using namespace fdllm;
  FDLLM_CHECK_ARG(dtype == FDLLM_DTYPE_BF16 || dtype == FDLLM_DTYPE_F16,
                  "fdllm_silu_mul: dtype %d unsupported (bf16 or fp16)", dtype);
  FDLLM_CHECK_ARG(n >= 0 && n % 8 == 0, "fdllm_silu_mul: n = %lld must be a multiple of 8", static_cast<long long>(n));
  if (n == 0) return FDLLM_OK;
  FDLLM_CHECK_ARG(gate && up && out, "fdllm_silu_mul: null pointer");
  FDLLM_CHECK_ARG(aligned16(gate) && aligned16(up) && aligned16(out), "fdllm_silu_mul: tensors must be 16-byte aligned");
  const int64_t nvec = n / 8;
  FDLLM_CHECK_ARG(nvec / 256 < (int64_t{1} << 31), "fdllm_silu_mul: n too large");
  const dim3 grid(static_cast<unsigned>((nvec + 255) / 256));
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == FDLLM_DTYPE_BF16)
    silu_mul_kernel<bf16_t><<<grid, dim3(256), 0, s>>>(static_cast<const u32x4*>(gate), static_cast<const u32x4*>(up),
                                                       static_cast<u32x4*>(out), nvec);
  else
    silu_mul_kernel<f16_t><<<grid, dim3(256), 0, s>>>(static_cast<const u32x4*>(gate), static_cast<const u32x4*>(up),
                                                      static_cast<u32x4*>(out), nvec);
  FDLLM_RETURN_LAUNCH_STATUS("fdllm_silu_mul");
}
