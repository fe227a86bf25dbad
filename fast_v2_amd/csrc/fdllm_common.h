// Shared device/host helpers for the gfx950 kernels of libfdllm_hip.so.
//
// Everything here is CDNA4-specific: 64-lane wavefronts, DPP row operations,
// bf16 conversions that lower to v_cvt_pk_bf16_f32 on gfx950.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/fdllm_hip.h"

namespace fdllm {

constexpr int kWave = 64;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------
// 16-bit float <-> fp32 (round-to-nearest-even on the way down).
// ---------------------------------------------------------------------------
struct bf16_t {
  uint16_t bits;
};
struct f16_t {
  uint16_t bits;
};

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) {
  return __uint_as_float(b << 16);
}
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  __bf16 h = static_cast<__bf16>(f);  // RNE, NaN-preserving
  return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, h));
}
__device__ __forceinline__ float f16_bits_to_f32(uint32_t b) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(b)));
}
__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
  return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(f)));
}

// Element traits: load/store one element through fp32.
template <typename T>
struct Elt;
template <>
struct Elt<bf16_t> {
  static constexpr int kBytes = 2;
  __device__ __forceinline__ static float lo(uint32_t w) { return __uint_as_float(w << 16); }
  __device__ __forceinline__ static float hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
  // one v_cvt_pk_bf16_f32 (RNE), the same rounding as two single conversions
  __device__ __forceinline__ static uint32_t pack(float a, float b) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
  }
  __device__ __forceinline__ static float round(float a) {
    return bf16_bits_to_f32(f32_to_bf16_bits(a));
  }
};
template <>
struct Elt<f16_t> {
  static constexpr int kBytes = 2;
  __device__ __forceinline__ static float lo(uint32_t w) { return f16_bits_to_f32(w & 0xffffu); }
  __device__ __forceinline__ static float hi(uint32_t w) { return f16_bits_to_f32(w >> 16); }
  __device__ __forceinline__ static uint32_t pack(float a, float b) {
    typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, f16x2));
  }
  __device__ __forceinline__ static float round(float a) {
    return f16_bits_to_f32(f32_to_f16_bits(a));
  }
};

// ---------------------------------------------------------------------------
// Wavefront all-reduce (sum / max) over 64 lanes.
// Lanes 0..15 of each DPP row are combined with quad_perm / mirror DPP moves,
// the four rows with two cross-row swizzles.
// ---------------------------------------------------------------------------
template <int kCtrl>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), kCtrl, 0xf, 0xf, false));
}

__device__ __forceinline__ float wave_allreduce_sum(float v) {
  v += dpp_f32<0xB1>(v);   // quad_perm [1,0,3,2]  (xor 1)
  v += dpp_f32<0x4E>(v);   // quad_perm [2,3,0,1]  (xor 2)
  v += dpp_f32<0x141>(v);  // row_half_mirror      (8-lane groups)
  v += dpp_f32<0x140>(v);  // row_mirror           (16-lane rows)
  v += __shfl_xor(v, 16, kWave);
  v += __shfl_xor(v, 32, kWave);
  return v;
}

__device__ __forceinline__ float wave_allreduce_max(float v) {
  v = fmaxf(v, dpp_f32<0xB1>(v));
  v = fmaxf(v, dpp_f32<0x4E>(v));
  v = fmaxf(v, dpp_f32<0x141>(v));
  v = fmaxf(v, dpp_f32<0x140>(v));
  v = fmaxf(v, __shfl_xor(v, 16, kWave));
  v = fmaxf(v, __shfl_xor(v, 32, kWave));
  return v;
}

// Reduce across the four 16-lane groups only (lanes i, i^16, i^32, i^48).
__device__ __forceinline__ float group4_allreduce_max(float v) {
  v = fmaxf(v, __shfl_xor(v, 16, kWave));
  v = fmaxf(v, __shfl_xor(v, 32, kWave));
  return v;
}
__device__ __forceinline__ float group4_allreduce_sum(float v) {
  v += __shfl_xor(v, 16, kWave);
  v += __shfl_xor(v, 32, kWave);
  return v;
}

// ---------------------------------------------------------------------------
// MFMA, buffer descriptors and direct-to-LDS staging shared by the attention and
// projection kernels.
// ---------------------------------------------------------------------------
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

constexpr int kBufferFlags = 0x00020000;  // raw buffer descriptor word 3 (gfx9: 32-bit data format)

template <bool F16>
__device__ __forceinline__ f32x16 mfma32x32x16(const u32x4& a, const u32x4& b, const f32x16& c) {
  if constexpr (F16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0,
                                                  0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                   0, 0);
  }
}

// Raw buffer descriptor in scalar registers: base address, size in bytes, 32-bit format.
__device__ __forceinline__ i32x4 make_srd(const void* base, int bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  i32x4 r;
  r[0] = __builtin_amdgcn_readfirstlane(static_cast<int>(a & 0xffffffffu));
  r[1] = __builtin_amdgcn_readfirstlane(static_cast<int>(a >> 32));
  r[2] = __builtin_amdgcn_readfirstlane(bytes);
  r[3] = kBufferFlags;
  return r;
}

// Direct-to-LDS load: 16 bytes per lane from buffer offset voff to LDS byte address
// lds + 16 * lane (one 1 KB block per wave; lanes past the descriptor's size write
// zeros without memory traffic). The compiler does not see the LDS write, so readers
// wait with wait_vmcnt and a barrier; M0 is restored after the load. NT: the
// non-temporal (streaming) policy, for data read once; without it the lines stay in L2
// for other workgroups that read them again.
template <bool NT = false>
__device__ __forceinline__ void lds_dma16(i32x4 srd_in, int voff, uint32_t lds_in) {
  // both are wave-uniform by construction; readfirstlane puts them in scalar registers
  i32x4 srd;
#pragma unroll
  for (int i = 0; i < 4; ++i) srd[i] = __builtin_amdgcn_readfirstlane(srd_in[i]);
  const uint32_t lds = __builtin_amdgcn_readfirstlane(lds_in);
  int saved;
  if constexpr (NT) {
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %3\n\t"
        "buffer_load_dwordx4 %1, %2, 0 offen nt lds\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(voff), "s"(srd), "s"(lds));
  } else {
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %3\n\t"
        "buffer_load_dwordx4 %1, %2, 0 offen lds\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(voff), "s"(srd), "s"(lds));
  }
}

// Wait until at most N vector memory operations of this wave are outstanding.
// Neither asm declares a memory clobber: such a clobber would keep every local whose
// address a lambda captured in scratch memory. Their order against the LDS reads comes
// from the workgroup barrier between them (volatile asm is not moved across the
// barrier and its fences).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N));
}

// Workgroup barrier that orders LDS only: waits for this wave's LDS operations,
// then s_barrier. Outstanding global loads stay in flight across it.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}


}  // namespace fdllm

// ---------------------------------------------------------------------------
// Host-side error plumbing shared by the C-ABI entry points.
// ---------------------------------------------------------------------------
#include "host_errors.h"

#define FDLLM_RETURN_LAUNCH_STATUS(what)                                            \
  do {                                                                              \
    hipError_t _e = hipGetLastError();                                              \
    if (_e != hipSuccess) {                                                         \
      ::fdllm::set_last_error("%s: launch failed: %s", what, hipGetErrorString(_e)); \
      return static_cast<int>(_e);                                                  \
    }                                                                               \
    return FDLLM_OK;                                                                \
  } while (0)
