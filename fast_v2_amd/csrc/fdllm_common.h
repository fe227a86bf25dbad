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

}  // namespace fdllm

// ---------------------------------------------------------------------------
// Host-side error plumbing shared by the C-ABI entry points.
// ---------------------------------------------------------------------------
namespace fdllm {
void set_last_error(const char* fmt, ...);
int dtype_size(int dtype);  // bytes per element of an FDLLM_DTYPE_*, 0 if unknown
}

#define FDLLM_CHECK_ARG(cond, ...)          \
  do {                                      \
    if (!(cond)) {                          \
      ::fdllm::set_last_error(__VA_ARGS__); \
      return FDLLM_ERR_INVALID_ARGUMENT;    \
    }                                       \
  } while (0)

#define FDLLM_RETURN_LAUNCH_STATUS(what)                                            \
  do {                                                                              \
    hipError_t _e = hipGetLastError();                                              \
    if (_e != hipSuccess) {                                                         \
      ::fdllm::set_last_error("%s: launch failed: %s", what, hipGetErrorString(_e)); \
      return static_cast<int>(_e);                                                  \
    }                                                                               \
    return FDLLM_OK;                                                                \
  } while (0)
