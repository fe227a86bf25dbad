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

template <typename T>
__global__ __launch_bounds__(256) void rope_kv_kernel(const RopeArgs a) {
  // Each product and the sum are rounded on their own: no fused multiply-add, which
  // hipcc would otherwise form from the 16-bit operations it recognises in them.
#pragma clang fp contract(off)
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
    float x0[8], x1[8], c0[8], c1[8], s0[8], s1[8];
    unpack8<T>(*reinterpret_cast<const u32x4*>(src + c), x0);
    unpack8<T>(*reinterpret_cast<const u32x4*>(src + half + c), x1);
    unpack8<T>(*reinterpret_cast<const u32x4*>(cs + c), c0);
    unpack8<T>(*reinterpret_cast<const u32x4*>(cs + half + c), c1);
    unpack8<T>(*reinterpret_cast<const u32x4*>(sn + c), s0);
    unpack8<T>(*reinterpret_cast<const u32x4*>(sn + half + c), s1);
    float y0[8], y1[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      // rotate_half: (-x1, x0); negation is exact and rounding symmetric, so
      // q * cos + (-x1) * sin rounds as q * cos - x1 * sin
      y0[j] = rnd<T>(rnd<T>(x0[j] * c0[j]) - rnd<T>(x1[j] * s0[j]));
      y1[j] = rnd<T>(rnd<T>(x1[j] * c1[j]) + rnd<T>(x0[j] * s1[j]));
    }
    const u32x4 w0 = pack8<T>(y0);
    const u32x4 w1 = pack8<T>(y1);
    if (is_q) {
      uint16_t* o = static_cast<uint16_t*>(d.q_out) + b * d.qo_stride_b + t * d.qo_stride_s + head * d.qo_stride_h;
      *reinterpret_cast<u32x4*>(o + c) = w0;
      *reinterpret_cast<u32x4*>(o + half + c) = w1;
    } else {
      if (d.k_out) {
        uint16_t* o = static_cast<uint16_t*>(d.k_out) + b * d.ko_stride_b + t * d.ko_stride_s + g * d.ko_stride_h;
        *reinterpret_cast<u32x4*>(o + c) = w0;
        *reinterpret_cast<u32x4*>(o + half + c) = w1;
      }
      if (to_cache) {
        uint16_t* o = static_cast<uint16_t*>(d.k_cache) + b * d.c_stride_b + pos1 * d.c_stride_s + g * d.c_stride_h;
        *reinterpret_cast<u32x4*>(o + c) = w0;
        *reinterpret_cast<u32x4*>(o + half + c) = w1;
      }
      if (to_block) {
        uint16_t* o = static_cast<uint16_t*>(d.k_block) + b * d.bc_stride_b + pos2 * d.bc_stride_s + g * d.bc_stride_h;
        *reinterpret_cast<u32x4*>(o + c) = w0;
        *reinterpret_cast<u32x4*>(o + half + c) = w1;
      }
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
