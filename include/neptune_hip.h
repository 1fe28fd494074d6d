/*
 * neptune_hip.h — C-ABI of the MI355X (gfx950) backend for Neptune's HTile
 * attention tile program, split-K decode and the Mamba-1 selective scan.
 *
 * This header is the drop-in boundary. Everything crossing it is a plain
 * pointer, an integer or a float; no HIP or torch types appear. Device
 * buffers are owned by the caller, work is enqueued on the caller's stream
 * (`stream` is a hipStream_t; NULL = the null stream) and the call returns
 * without synchronising. No entry point allocates device memory.
 *
 * Reference interfaces this header replaces (paths relative to the
 * Evan-Zhao/mlir-toy checkout):
 *   - plugin discovery: `mlirGetDialectPluginInfo` / `mlirGetPassPluginInfo`
 *     (lib/HTile/HTileDialect.cpp:27-37, lib/HTile/HTilePasses.cpp:159-163)
 *     -> neptune_hip_get_backend_info
 *   - the kernel produced from tests/data/flash_attention_htile.mlir and
 *     launched as `flash_attention_htile[(32,32,1)](q, k, v, out)`
 *     (tests/golden/flash_attention_triton.py:4-5,
 *      tests/test_translators.py:184-194) -> neptune_attn_fwd
 *   - error conventions (RuntimeError / NotImplementedError,
 *     src/neptune_mlir/translators/common.py:187-197,217-224)
 *     -> neptune_status + neptune_last_error
 * Split-K decode, fp8 KV and the selective scan have no counterpart in the
 * reference; their contracts are stated next to each declaration.
 */
#ifndef NEPTUNE_HIP_H
#define NEPTUNE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NEPTUNE_HIP_ABI_VERSION 1u

#if defined(__GNUC__)
#define NEPTUNE_API __attribute__((visibility("default")))
#else
#define NEPTUNE_API
#endif

typedef enum neptune_status {
  NEPTUNE_OK = 0,
  NEPTUNE_ERR_INVALID_ARGUMENT = 1, /* null pointer, bad shape, bad stride   */
  NEPTUNE_ERR_UNSUPPORTED = 2,      /* valid request the kernels do not cover */
  NEPTUNE_ERR_HIP = 3,              /* a HIP runtime call or launch failed    */
  NEPTUNE_ERR_NO_DEVICE = 4,        /* no HIP device visible                  */
  NEPTUNE_ERR_WORKSPACE_TOO_SMALL = 5
} neptune_status;

typedef enum neptune_dtype {
  NEPTUNE_DTYPE_F32 = 0,
  NEPTUNE_DTYPE_F16 = 1,
  NEPTUNE_DTYPE_BF16 = 2,
  NEPTUNE_DTYPE_FP8_E4M3 = 3 /* OCP E4M3FN: bias 7, max 448, no infinities */
} neptune_dtype;

/* Versioned info record, the same discovery pattern as MLIR's
 * DialectPluginLibraryInfo {api version, plugin name, build version, hook}
 * (lib/HTile/HTileDialect.cpp:27-37). */
typedef struct neptune_backend_info {
  uint32_t abi_version;        /* NEPTUNE_HIP_ABI_VERSION               */
  const char *name;            /* "NeptuneHTileHIP"                     */
  const char *gcn_arch;        /* code-object target: "gfx950"          */
  int32_t hip_runtime_version; /* hipRuntimeGetVersion, or -1 (no HIP)  */
} neptune_backend_info;

/* Attention forward: O = softmax(Q K^T / sqrt(D)) V per (batch, head).
 * Layout: Q, O [batch, heads_q, seq_q, head_dim]; K, V [batch, heads_kv,
 * seq_kv, head_dim]; the head_dim axis is contiguous. Strides are in
 * elements for the (batch, head, seq) axes; a zero stride array means
 * contiguous. With k_dim_order = 1, K is [batch, heads_kv, head_dim,
 * seq_kv] instead (seq contiguous; k_stride gives the batch, head and
 * head_dim-row strides): the order a dimension_order = [1, 0] tile load
 * reads (lib/HTile/HTilePasses.cpp:122-140). pipeline_stages is the number
 * of K and V tiles the kernel keeps in LDS per operand, i.e. how far its
 * loads run ahead (the htile.pipeline_stages loop attribute, HTile:128);
 * neither knob changes the result. Both apply to the head_dim-128 16-bit
 * kernel (0 = default elsewhere); k_dim_order = 1 needs seq_kv % 8 == 0. Query head h reads KV head h / (heads_q / heads_kv).
 * Numerics follow tests/data/flash_attention_htile.mlir:23-143: scores are
 * scaled by scale_log2 (= log2(e)/sqrt(D) when 0, HTile:24) into the exp2
 * domain, the running max starts at -FLT_MAX, keys stream in blocks of 64,
 * the row sum accumulates fp32 probabilities, probabilities are rounded to
 * the input type before P·V (HTile:93-94) and the output is divided then
 * rounded (HTile:137-140). causal != 0 masks key j > i + (seq_kv - seq_q).
 * lse (nullable) receives ln(sum_j exp(s_ij)) per row, [batch, heads_q,
 * seq_q] fp32 contiguous. */
typedef struct neptune_attn_desc {
  int64_t batch, heads_q, heads_kv, seq_q, seq_kv, head_dim;
  int64_t q_stride[3], k_stride[3], v_stride[3], o_stride[3];
  int32_t dtype;  /* F32, F16 or BF16 for q, k, v and o */
  int32_t causal;
  float scale_log2;
  int16_t pipeline_stages; /* 0 = default (2), or 1, 2, 3               */
  int16_t k_dim_order;     /* 0: K [.., seq, head_dim]; 1: [.., head_dim, seq] */
} neptune_attn_desc;

/* Split-K decode with grouped KV heads (one query token per sequence).
 * Q, O [batch, heads_q, head_dim]; K, V [batch, heads_kv, seq_kv, head_dim]
 * contiguous. kv_dtype BF16, or FP8_E4M3 with per-(batch, kv head,
 * scale_block-token block) fp32 scales k_scale/v_scale [batch, heads_kv,
 * ceil(seq_kv/scale_block)]; the dequantised value is code * scale.
 * The keys are cut into num_splits chunks; each chunk yields (m, l, o~)
 * in the exp2 domain and a combine pass forms M = max m_s,
 * L = sum 2^(m_s-M) l_s, O = sum 2^(m_s-M) o~_s / L and
 * lse = (M + log2 L) ln 2. */
typedef struct neptune_decode_desc {
  int64_t batch, heads_q, heads_kv, seq_kv, head_dim;
  int64_t num_splits;   /* 0 => chosen by the library                */
  int64_t scale_block;  /* tokens per fp8 scale; 0 => 64             */
  int32_t q_dtype;      /* BF16 (query and output)                   */
  int32_t kv_dtype;     /* BF16 or FP8_E4M3                           */
  float scale_log2;     /* 0 => log2(e)/sqrt(head_dim)               */
  int32_t reserved;
} neptune_decode_desc;

/* Paged KV for split-K decode: K and V live in pools of fixed-size pages and
 * sequence b's token t is in page block_table[b * max_pages + t / page_size]
 * at position t % page_size. Element (page, kv head, position, d) of the K
 * pool is at page * k_stride[0] + head * k_stride[1] + position * k_stride[2]
 * + d (head_dim contiguous; the same for V), so both [pages, heads_kv,
 * page_size, head_dim] and [pages, page_size, heads_kv, head_dim] pools are
 * described. Sequence b has seq_lens[b] tokens (0 .. desc->seq_kv, the
 * longest); an empty sequence yields O = 0 and lse = -inf. Block-table
 * entries outside [0, num_pages) are clamped into range by the kernel (the
 * results are then meaningless, but no memory outside the pools is read). */
typedef struct neptune_paged_kv_desc {
  int64_t num_pages;   /* pages in each pool                              */
  int64_t page_size;   /* tokens per page, a multiple of 32               */
  int64_t max_pages;   /* block-table row length, >= ceil(seq_kv/page)    */
  int64_t k_stride[3]; /* elements: page, kv head, position               */
  int64_t v_stride[3];
} neptune_paged_kv_desc;

/* Mamba-1 selective scan (Gu & Dao 2023, selective_scan_fn semantics):
 *   delta = softplus(delta_raw + delta_bias[d])   (if delta_softplus)
 *   x_n  <- exp(delta * A[d,n]) x_n + delta * B[b,n,l] * u[b,d,l]
 *   y     = (sum_n C[b,n,l] x_n + D[d] u) * silu(z)      (z nullable)
 * u, delta_raw, z, y [batch, dim, seq_len]; B, C [batch, d_state, seq_len]
 * in io_dtype (BF16); A [dim, d_state], D and delta_bias [dim] fp32 (D,
 * z and delta_bias may be NULL: no skip term, no gate, no bias). The state
 * is carried in fp32 from x = 0. y must not overlap any input: the call
 * writes y while it still reads later steps, and for few channels over a
 * long sequence it keeps per-chunk state in y before the outputs overwrite
 * it (no workspace); a y that shares a byte with an input is
 * NEPTUNE_ERR_INVALID_ARGUMENT. Supported: d_state 16 and seq_len below 2^26
 * (NEPTUNE_ERR_UNSUPPORTED otherwise). */
typedef struct neptune_scan_desc {
  int64_t batch, dim, seq_len, d_state;
  int32_t io_dtype;        /* BF16 */
  int32_t delta_softplus;  /* 1: apply softplus (threshold 20) */
} neptune_scan_desc;

/* ---- discovery and errors ------------------------------------------- */

NEPTUNE_API neptune_status neptune_hip_get_backend_info(neptune_backend_info *info);

/* Text of the last failure on the calling thread ("" if none). */
NEPTUNE_API const char *neptune_last_error(void);

/* Number of visible HIP devices (0 when none or when HIP is unusable). */
NEPTUNE_API int32_t neptune_device_count(void);

/* ---- attention prefill (the HTile tile program) ---------------------- */

NEPTUNE_API neptune_status neptune_attn_fwd(const neptune_attn_desc *desc, const void *q,
                                const void *k, const void *v, void *o,
                                float *lse, void *stream);

/* ---- split-K decode ---------------------------------------------------- */

NEPTUNE_API neptune_status neptune_decode_workspace_bytes(const neptune_decode_desc *desc,
                                              size_t *bytes);

NEPTUNE_API neptune_status neptune_decode_splitk(const neptune_decode_desc *desc,
                                     const void *q, const void *k,
                                     const void *v, const float *k_scale,
                                     const float *v_scale, void *o, float *lse,
                                     void *workspace, size_t workspace_bytes,
                                     void *stream);

/* neptune_decode_splitk without a workspace argument; it allocates nothing.
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops). The
 * split partials go to a static device scratch of 16 MiB that each GPU
 * holds until the process ends (520 bytes per batch x heads_q x split row:
 * config 3's 16 x 32 x 16 rows use 4.3 MB); a request that needs more
 * returns NEPTUNE_ERR_WORKSPACE_TOO_SMALL. The kernels use the scratch of the
 * device that owns `stream` (the current device for the null stream). Every
 * call on one GPU shares that scratch: calls that overlap on one GPU (concurrent streams, or threads
 * enqueueing at once) race on it and must be ordered by the caller. The
 * results equal neptune_decode_splitk's bit for bit. */
NEPTUNE_API neptune_status neptune_decode_splitk_noalloc(const neptune_decode_desc *desc,
                                             const void *q, const void *k,
                                             const void *v, const float *k_scale,
                                             const float *v_scale, void *o, float *lse,
                                             void *stream);

/* Quantise a BF16 KV tensor [batch, heads_kv, seq_kv, head_dim] to E4M3FN
 * codes with one fp32 scale per (batch, kv head, scale_block tokens):
 * scale = amax/448, code = RNE-saturate(x * (448/amax)); amax == 0 gives
 * scale 0 and all-zero codes. */
NEPTUNE_API neptune_status neptune_kv_quantize_fp8(int64_t batch, int64_t heads_kv,
                                       int64_t seq_kv, int64_t head_dim,
                                       int64_t scale_block, const void *src,
                                       uint8_t *codes, float *scales,
                                       void *stream);

/* Split-K decode over a paged KV cache (neptune_paged_kv_desc). No
 * counterpart in the reference: the block-table layout of serving caches,
 * consumed by the same split-K kernel. desc->kv_dtype must be BF16;
 * desc->seq_kv is the longest sequence and sets the split layout (the
 * workspace is sized by neptune_decode_workspace_bytes(desc)). block_table
 * [batch, max_pages] and seq_lens [batch] are int32 device arrays. */
NEPTUNE_API neptune_status neptune_decode_paged(const neptune_decode_desc *desc,
                                    const neptune_paged_kv_desc *pages,
                                    const void *q, const void *k_pages,
                                    const void *v_pages,
                                    const int32_t *block_table,
                                    const int32_t *seq_lens, void *o, float *lse,
                                    void *workspace, size_t workspace_bytes,
                                    void *stream);

/* Split-K decode over paged pools of E4M3FN codes. No counterpart in the
 * reference: neptune_decode_paged with the fp8 KV of neptune_decode_splitk.
 * desc->kv_dtype must be FP8_E4M3. Each page holds one fp32 scale per kv
 * head for K and for V: k_scales, v_scales [num_pages, heads_kv]
 * contiguous (desc->scale_block must be 0 or page_size); the dequantised
 * value of a code in page p, kv head h is code * scale[p * heads_kv + h].
 * Pool strides are in elements (bytes) and must be multiples of 16; the
 * rest is as in neptune_decode_paged. */
NEPTUNE_API neptune_status neptune_decode_paged_fp8(const neptune_decode_desc *desc,
                                        const neptune_paged_kv_desc *pages,
                                        const void *q, const uint8_t *k_pages,
                                        const uint8_t *v_pages,
                                        const float *k_scales,
                                        const float *v_scales,
                                        const int32_t *block_table,
                                        const int32_t *seq_lens, void *o,
                                        float *lse, void *workspace,
                                        size_t workspace_bytes, void *stream);

/* ---- selective scan ---------------------------------------------------- */

NEPTUNE_API neptune_status neptune_selective_scan_fwd(
    const neptune_scan_desc *desc, const void *u, const void *delta_raw,
    const float *A, const void *B, const void *C, const float *D,
    const void *z, const float *delta_bias, void *y, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* NEPTUNE_HIP_H */
