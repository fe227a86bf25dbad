/*
 * libfdllm_probes.so — measurement probes for bench.py (not part of the operator
 * library; no counterpart in the reference): plain data movement in the access pattern
 * and launch shape of the two HBM-bound hot-path calls, the practical floor each call
 * is measured against, and the sustained MFMA rate the MFMA-bound calls are measured
 * against.
 *
 * Return value: 0, FDLLM_PROBE_ERR_ARGS (nothing launched) or FDLLM_PROBE_ERR_LAUNCH.
 */
#ifndef FDLLM_PROBES_H_
#define FDLLM_PROBES_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FDLLM_PROBE_ERR_ARGS (-1)
#define FDLLM_PROBE_ERR_LAUNCH (-2)

/* Reads every visible K and V row (seqlens[b] keys of sequence b, every KV head) once,
 * with the split decode kernel's pattern: grid (slots, num_kv_heads) of 512 threads, one
 * KV head per workgroup, 32-key tiles of one page (page_size a power of two >= 32, at
 * most 4096 page-table entries; page_table NULL: contiguous [batch, max_S, Hkv, D] with
 * the sequence as the page), the keys of all sequences dealt evenly over the slots
 * (slots a multiple of 8), two tiles in flight per team of 256 threads. head_dim 128,
 * 16-bit elements; strides in elements. batch <= 64. sink: 4 writable bytes (written
 * only if the data folds to a fixed constant). */
int fdllm_probe_read_kv(const void* k, const void* v, int64_t k_stride_page, int64_t k_stride_slot,
                        int64_t k_stride_h, int64_t v_stride_page, int64_t v_stride_slot, int64_t v_stride_h,
                        const int32_t* page_table, int32_t max_pages, int32_t page_size, const int32_t* seqlens,
                        int batch, int num_kv_heads, int slots, void* sink, void* stream);

/* dst[t, :] = src[idx[t], :] for t < rows: row_bytes (a multiple of 16, at most 16 KB)
 * per row, source rows src_row_bytes apart; rows whose index is outside [0, src_rows)
 * are left unwritten. One wave (workgroup) per row; all loads before the stores. */
int fdllm_probe_copy_rows(const void* src, int64_t src_row_bytes, int src_rows, const int64_t* idx, void* dst,
                          int rows, int row_bytes, void* stream);

/* Sustained bf16 MFMA rate: `workgroups` workgroups of 256 threads (one wave per SIMD;
 * one workgroup per compute unit fills the chip), each wave `rounds` rounds of four
 * independent v_mfma_f32_32x32x16_bf16 chains on register operands (32768 flop each), no
 * memory traffic. Flops = workgroups * 4 * rounds * 4 * 32768. sink: workgroups * 256
 * writable floats (written only if the sums hit a fixed constant). */
int fdllm_probe_mfma(int workgroups, int rounds, float* sink, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FDLLM_PROBES_H_ */
