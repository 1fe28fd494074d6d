/*
 * neptune_oracle.h — CPU oracle for the HTile hot path.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the
 * checker (or the timed CPU baseline). The product library
 * (libneptune_hip.so) never links, loads or calls it.
 *
 * Functions take the descriptor types of the product ABI (include/
 * neptune_hip.h) so a test can hand the same request to both sides.
 *
 * What pins each function (none is "parity unpinned"):
 *   codecs          exhaustive / random comparison with numpy float16,
 *                   torch bfloat16 and torch float8_e4m3fn
 *   attn_fwd        attn_exact (fp64 closed form), brute-force numpy softmax,
 *                   Q=0 -> mean(V) / prefix mean, causal row 0 = V[0],
 *                   shift and key-permutation invariance, bf16 vs fp32 gap
 *   attn_exact      numpy float64 softmax on tiny inputs (written in the test
 *                   from the textbook definition, not from this file)
 *   decode_splitk   attn_exact with seq_q = 1; splits=1 == splits=k; GQA ==
 *                   MHA with repeated KV heads; fp8 == bf16 run on the
 *                   dequantised values
 *   decode_paged    == decode_splitk bit for bit over a shuffled pool (both
 *                   page layouts) at full lengths; ragged lengths against
 *                   attn_exact on each sequence's own tokens; empty sequence
 *                   and out-of-pool table entries
 *   decode_paged_fp8 == decode_splitk (fp8, scale block = page size) bit for
 *                   bit over a shuffled pool of the same codes and scales;
 *                   ragged lengths against decode_splitk on each sequence's
 *                   prefix
 *   kv_quantize     codes decode to within half an E4M3 ulp of x/scale,
 *                   scale = amax/448, block amax maps to code 0x7e
 *   selective_scan  brute-force numpy recurrence on tiny inputs; delta -> 0,
 *                   B = 0 and C = 0 closed forms; L = 1 closed form;
 *                   linearity in u at fixed delta
 */
#ifndef NEPTUNE_ORACLE_H
#define NEPTUNE_ORACLE_H

#include "../include/neptune_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* scalar codecs (round to nearest even) */
uint16_t neptune_cpu_f32_to_bf16(float f);
float neptune_cpu_bf16_to_f32(uint16_t h);
uint16_t neptune_cpu_f32_to_f16(float f);
float neptune_cpu_f16_to_f32(uint16_t h);
uint8_t neptune_cpu_f32_to_e4m3(float f); /* saturates to +-448 */
float neptune_cpu_e4m3_to_f32(uint8_t c);

/* array forms of the codecs (for tests) */
void neptune_cpu_convert_f32(const float *src, void *dst, int64_t n,
                             int32_t dst_dtype);
void neptune_cpu_to_f32(const void *src, float *dst, int64_t n,
                        int32_t src_dtype);

int32_t neptune_cpu_num_threads(void);

/* HTile-policy attention (see neptune_attn_desc). Returns a status code. */
int32_t neptune_cpu_attn_fwd(const neptune_attn_desc *d, const void *q,
                             const void *k, const void *v, void *o, float *lse);

/* fp64 closed form: two-pass softmax, no rounding of P. o and lse are
 * contiguous fp64 [batch, heads_q, seq_q, head_dim] / [.., seq_q]. */
int32_t neptune_cpu_attn_exact(const neptune_attn_desc *d, const void *q,
                               const void *k, const void *v, double *o,
                               double *lse);

/* split-K decode with the combine; partials (nullable) receives
 * [batch, heads_q, splits, head_dim + 2] = (o~..., m, l). */
int32_t neptune_cpu_decode_splitk(const neptune_decode_desc *d, const void *q,
                                  const void *k, const void *v,
                                  const float *k_scale, const float *v_scale,
                                  void *o, float *lse, float *partials);

/* split-K decode over a paged KV pool (neptune_decode_paged's twin) */
int32_t neptune_cpu_decode_paged(const neptune_decode_desc *d,
                                 const neptune_paged_kv_desc *pk, const void *q,
                                 const void *k_pages, const void *v_pages,
                                 const int32_t *block_table,
                                 const int32_t *seq_lens, void *o, float *lse);

/* the same over fp8 E4M3 pools with one scale per (page, kv head)
 * (neptune_decode_paged_fp8's twin) */
int32_t neptune_cpu_decode_paged_fp8(const neptune_decode_desc *d,
                                     const neptune_paged_kv_desc *pk, const void *q,
                                     const uint8_t *k_pages, const uint8_t *v_pages,
                                     const float *k_scales, const float *v_scales,
                                     const int32_t *block_table, const int32_t *seq_lens,
                                     void *o, float *lse);

/* number of splits and tokens per split the decode path uses */
int32_t neptune_cpu_decode_layout(const neptune_decode_desc *d,
                                  int64_t *splits, int64_t *chunk);

int32_t neptune_cpu_kv_quantize_fp8(int64_t batch, int64_t heads_kv,
                                    int64_t seq_kv, int64_t head_dim,
                                    int64_t scale_block, const void *src,
                                    uint8_t *codes, float *scales);

/* fp64 sequential scan; y (io dtype, nullable) and y64 (fp64, nullable). */
int32_t neptune_cpu_selective_scan_fwd(const neptune_scan_desc *d,
                                       const void *u, const void *delta_raw,
                                       const float *A, const void *B,
                                       const void *C, const float *D,
                                       const void *z, const float *delta_bias,
                                       void *y, double *y64);

#ifdef __cplusplus
}
#endif

#endif
