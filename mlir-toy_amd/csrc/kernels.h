// kernels.h — host-side launch interface between the C-ABI layer (abi.cpp)
// and the HIP kernels. Arguments are already validated and resolved.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace neptune {

struct AttnLaunch {
  const void *q, *k, *v;
  void *o;
  float *lse;  // nullable
  int64_t batch, heads_q, heads_kv, seq_q, seq_kv, head_dim;
  int64_t qs[3], ks[3], vs[3], os[3];  // (batch, head, seq) strides, elements
  int32_t dtype;
  int32_t causal;
  float scale_log2;
  int32_t stages;       // LDS slots per K/V operand (1, 2, 3)
  int32_t k_dim_order;  // 1: K is [batch, head, head_dim, seq]; ks[2] = head_dim-row stride
};

struct DecodeLaunch {
  const void *q, *k, *v;
  const float *k_scale, *v_scale;  // fp8 only
  void *o;
  float *lse;        // nullable
  float *part_o;     // [batch, heads_q, splits, head_dim]
  float *part_ml;    // [batch, heads_q, splits, 2]
  int64_t batch, heads_q, heads_kv, seq_kv, head_dim;
  int64_t splits, chunk, scale_block, n_scale_blocks;
  int32_t kv_dtype;
  float scale_log2;
  // paged KV (block_table != nullptr): k/v are page pools; seq_kv is the
  // longest sequence, seq_lens[b] each sequence's length
  const int32_t *block_table = nullptr, *seq_lens = nullptr;
  int64_t page_size = 0, max_pages = 0, num_pages = 0;
  int64_t k_pstride[3] = {0, 0, 0}, v_pstride[3] = {0, 0, 0};  // page, head, token (elements)
};

struct QuantLaunch {
  const void *src;
  uint8_t *codes;
  float *scales;
  int64_t batch, heads_kv, seq_kv, head_dim, scale_block, n_scale_blocks;
};

struct ScanLaunch {
  const void *u, *delta_raw, *B, *C, *z;
  const float *A, *D, *delta_bias;
  void *y;
  int64_t batch, dim, seq_len, d_state;
  int32_t delta_softplus;
};

// Bytes of the static device scratch behind neptune_decode_splitk_noalloc
// (the split partials of one call: 520 bytes per (batch, query head, split)).
constexpr size_t kDecodeScratchBytes = size_t(16) << 20;

// Device address of that scratch on the device that owns stream s (the
// current device for the null stream), resolved once per device by
// hipGetSymbolAddress and kept; hipSuccess or the HIP error.
hipError_t decode_scratch(hipStream_t s, void **ptr);

// Each returns hipSuccess or the launch error. Shapes the kernels do not
// cover are rejected by the ABI layer before these are called.
hipError_t launch_attn_fwd(const AttnLaunch &a, hipStream_t s);
hipError_t launch_decode(const DecodeLaunch &a, hipStream_t s);
hipError_t launch_kv_quantize(const QuantLaunch &a, hipStream_t s);
hipError_t launch_selective_scan(const ScanLaunch &a, hipStream_t s);

// Coverage predicates used by the ABI layer for NEPTUNE_ERR_UNSUPPORTED.
bool attn_supported(const AttnLaunch &a, const char **why);
bool decode_supported(const DecodeLaunch &a, const char **why);
bool scan_supported(const ScanLaunch &a, const char **why);

}  // namespace neptune
