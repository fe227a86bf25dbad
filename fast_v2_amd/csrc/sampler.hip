// Greedy sampling + threshold unmasking of one diffusion step (fdllm_unmask_step):
// softmax / argmax / confidence over the vocabulary (modeling.py:2263-2270 at
// temperature 0) and the unmask rule of generation_functions.py:784-807, on the GPU,
// so the step leaves its decisions in device memory and the host reads four counters.
//
// Kernel 1 (one workgroup per sub-block position and sequence) reads one logits row
// twice: pass 1 keeps the running maximum, its first index and the sum of
// exp(l - max) (online, per 16-byte vector); pass 2 finds the first index whose
// probability, rounded to the logits' type, equals the rounded maximum probability
// (torch.argmax over the rounded softmax returns the first of equal values; only
// logits within 2^-8 of the maximum can tie, so pass 2 computes probabilities for
// those alone). Kernel 2 (one wave per sequence) applies the rule to the positions.
#include <math.h>

#include "fdllm_common.h"

namespace fdllm {
namespace {

struct UnmaskArgs {
  const uint16_t* logits;
  int64_t lg_sb, lg_sr;
  int V, row_offset, shift;
  int64_t* tokens;
  int64_t tok_sb;
  uint8_t* finished;
  int64_t mask_id, stop_token;
  float threshold;
  int64_t* row_tok;
  float* row_conf;
  int32_t* counts;
  int B, L;
};

constexpr int kThreads = 512;

template <typename T>
__device__ __forceinline__ float rnd16(float x) {
  return Elt<T>::round(x);
}

// (max, first index, sum of exp(x - max)) of two partial states
__device__ __forceinline__ void combine(float& m, int& idx, float& s, float m2, int idx2, float s2) {
  if (m2 > m || (m2 == m && idx2 < idx)) {
    const float sc = m == -INFINITY ? 0.f : expf(m - m2);
    s = s * sc + s2;
    m = m2;
    idx = idx2;
  } else {
    const float sc = m2 == -INFINITY ? 0.f : expf(m2 - m);
    s += s2 * sc;
  }
}

template <typename T>
__global__ __launch_bounds__(kThreads) void unmask_rows_kernel(const UnmaskArgs a) {
  __shared__ float sm[kThreads / 64], ss[kThreads / 64];
  __shared__ int si[kThreads / 64];
  __shared__ float s_fin[2];
  __shared__ int s_fin_idx;
  const int i = blockIdx.x;
  const int b = blockIdx.y;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  if (i == 0 && b == 0 && tid < 4) a.counts[tid] = 0;  // kernel 2 accumulates into these
  const int r = max(a.row_offset + i - a.shift, 0);
  const uint16_t* row = a.logits + b * a.lg_sb + static_cast<int64_t>(r) * a.lg_sr;
  const bool vec = (a.V % 8 == 0) && ((reinterpret_cast<uintptr_t>(row) & 15u) == 0);

  // ---- pass 1: max, its first index, sum of exp(x - max)
  float m = -INFINITY, s = 0.f;
  int idx = 0x7fffffff;
  if (vec) {
    const int nv = a.V / 8;
    for (int v = tid; v < nv; v += kThreads) {
      const u32x4 w = *reinterpret_cast<const u32x4*>(row + 8 * v);
      float x[8];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        x[2 * j] = Elt<T>::lo(w[j]);
        x[2 * j + 1] = Elt<T>::hi(w[j]);
      }
      float mv = x[0];
      int iv = 0;
#pragma unroll
      for (int j = 1; j < 8; ++j)
        if (x[j] > mv) {
          mv = x[j];
          iv = j;
        }
      if (mv > m) {  // a strictly larger value: indices grow, so the first one is kept
        s = m == -INFINITY ? 0.f : s * expf(m - mv);
        m = mv;
        idx = 8 * v + iv;
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) s += expf(x[j] - m);
    }
  } else {
    for (int v = tid; v < a.V; v += kThreads) {
      const float x = Elt<T>::lo(row[v]);
      if (x > m) {
        s = m == -INFINITY ? 0.f : s * expf(m - x);
        m = x;
        idx = v;
      }
      s += expf(x - m);
    }
  }
  // wave then workgroup reduction
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float m2 = __shfl_xor(m, o, kWave);
    const int i2 = __shfl_xor(idx, o, kWave);
    const float s2 = __shfl_xor(s, o, kWave);
    combine(m, idx, s, m2, i2, s2);
  }
  if (lane == 0) {
    sm[wave] = m;
    si[wave] = idx;
    ss[wave] = s;
  }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < kThreads / 64; ++w) combine(m, idx, s, sm[w], si[w], ss[w]);
    s_fin[0] = m;
    s_fin[1] = s;
    s_fin_idx = idx;
  }
  __syncthreads();
  m = s_fin[0];
  s = s_fin[1];
  // ---- pass 2: first index whose rounded probability equals the rounded maximum
  const float pmax = rnd16<T>(1.f / s);
  const float lo_cut = m - 0.0078125f;  // exp(x - m) < 1 - 2^-8 below it: no tie possible
  int cand = s_fin_idx;
  if (vec) {
    const int nv = a.V / 8;
    for (int v = tid; v < nv; v += kThreads) {
      const u32x4 w = *reinterpret_cast<const u32x4*>(row + 8 * v);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float x = (j & 1) ? Elt<T>::hi(w[j >> 1]) : Elt<T>::lo(w[j >> 1]);
        if (x >= lo_cut && 8 * v + j < cand && rnd16<T>(expf(x - m) / s) == pmax) cand = 8 * v + j;
      }
    }
  } else {
    for (int v = tid; v < a.V; v += kThreads) {
      const float x = Elt<T>::lo(row[v]);
      if (x >= lo_cut && v < cand && rnd16<T>(expf(x - m) / s) == pmax) cand = v;
    }
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) cand = min(cand, __shfl_xor(cand, o, kWave));
  __syncthreads();
  if (lane == 0) si[wave] = cand;
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < kThreads / 64; ++w) cand = min(cand, si[w]);
    a.row_tok[b * a.L + i] = cand;
    a.row_conf[b * a.L + i] = pmax;
  }
}

// One wave per sequence; lane i < L is position i of the sub-block.
__global__ __launch_bounds__(64) void unmask_select_kernel(const UnmaskArgs a) {
  const int b = blockIdx.x;
  const int i = threadIdx.x;
  const bool live = i < a.L;
  const bool fin = a.finished != nullptr && a.finished[b] != 0;
  int64_t* tp = a.tokens + b * a.tok_sb + i;
  const int64_t t = live ? *tp : 0;
  const bool masked = live && t == a.mask_id && !fin;
  const float c = masked ? a.row_conf[b * a.L + i] : -INFINITY;
  const int64_t tok = live ? a.row_tok[b * a.L + i] : 0;
  bool unmask = c > a.threshold;
  // most confident masked position, first on ties (torch.argmax over the row)
  float cm = live ? c : -INFINITY;
  int im = live ? i : 0x7fffffff;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float c2 = __shfl_xor(cm, o, kWave);
    const int i2 = __shfl_xor(im, o, kWave);
    if (c2 > cm || (c2 == cm && i2 < im)) {
      cm = c2;
      im = i2;
    }
  }
  if (i == im) unmask = true;
  unmask = unmask && masked;
  if (unmask) *tp = tok;
  const bool stop_hit = unmask && a.stop_token >= 0 && tok == a.stop_token;
  const uint64_t stops = __builtin_amdgcn_ballot_w64(stop_hit);
  const bool fin_after = fin || stops != 0;
  const uint64_t n_unmask = __builtin_amdgcn_ballot_w64(unmask);
  const uint64_t n_left = __builtin_amdgcn_ballot_w64(masked && !unmask && !fin_after);
  const bool first_masked = live && i == 0 && !unmask && t == a.mask_id;
  if (i == 0) {
    if (a.finished != nullptr && stops != 0) a.finished[b] = 1;
    atomicAdd(&a.counts[0], static_cast<int>(__builtin_popcountll(n_unmask)));
    atomicAdd(&a.counts[1], static_cast<int>(__builtin_popcountll(n_left)));
    atomicAdd(&a.counts[2], first_masked ? 1 : 0);
    atomicAdd(&a.counts[3], fin_after ? 1 : 0);
  }
}

}  // namespace
}  // namespace fdllm

extern "C" int fdllm_unmask_step(const void* logits, int64_t logits_stride_b, int64_t logits_stride_row,
                                 int vocab, int row_offset, int shift, int64_t* tokens, int64_t tokens_stride_b,
                                 uint8_t* finished, int64_t mask_id, float threshold, int64_t stop_token,
                                 int64_t* row_tok, float* row_conf, int32_t* counts, int batch, int num_positions,
                                 int dtype, void* stream) {
  using namespace fdllm;
  FDLLM_CHECK_ARG(dtype == FDLLM_DTYPE_BF16 || dtype == FDLLM_DTYPE_F16,
                  "fdllm_unmask_step: dtype %d unsupported (bf16 or fp16 logits)", dtype);
  FDLLM_CHECK_ARG(batch >= 0 && num_positions >= 0 && num_positions <= 64 && vocab > 0,
                  "fdllm_unmask_step: need 0 <= num_positions <= 64 and vocab > 0");
  FDLLM_CHECK_ARG(shift == 0 || shift == 1, "fdllm_unmask_step: shift must be 0 or 1");
  if (batch == 0 || num_positions == 0) return FDLLM_OK;
  FDLLM_CHECK_ARG(batch < 65536, "fdllm_unmask_step: batch too large");
  FDLLM_CHECK_ARG(logits && tokens && row_tok && row_conf && counts, "fdllm_unmask_step: null pointer");
  UnmaskArgs a;
  a.logits = static_cast<const uint16_t*>(logits);
  a.lg_sb = logits_stride_b;
  a.lg_sr = logits_stride_row;
  a.V = vocab;
  a.row_offset = row_offset;
  a.shift = shift;
  a.tokens = tokens;
  a.tok_sb = tokens_stride_b;
  a.finished = finished;
  a.mask_id = mask_id;
  a.stop_token = stop_token;
  a.threshold = threshold;
  a.row_tok = row_tok;
  a.row_conf = row_conf;
  a.counts = counts;
  a.B = batch;
  a.L = num_positions;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 g1(num_positions, batch);
  if (dtype == FDLLM_DTYPE_BF16) unmask_rows_kernel<bf16_t><<<g1, dim3(kThreads), 0, s>>>(a);
  else unmask_rows_kernel<f16_t><<<g1, dim3(kThreads), 0, s>>>(a);
  unmask_select_kernel<<<dim3(batch), dim3(64), 0, s>>>(a);
  FDLLM_RETURN_LAUNCH_STATUS("fdllm_unmask_step");
}
