// abi.cpp — the extern "C" entry points of libneptune_hip.so
// (declared in include/neptune_hip.h).
//
// Every request is validated on the host before any HIP call, so argument
// errors are reported identically with or without a GPU. Failures return a
// status code and leave a message for neptune_last_error() on the calling
// thread; no C++ exception crosses the boundary. The reference reports the
// same classes of failure as RuntimeError (toolchain/runtime failure,
// src/neptune_mlir/translators/common.py:217-224) and NotImplementedError
// (valid input outside what the backend covers, common.py:187-197).
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <string>

#include "../../include/neptune_hip.h"
#include "kernels.h"

using namespace neptune;

namespace {

thread_local std::string g_last_error;

neptune_status fail(neptune_status st, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return st;
}

neptune_status ok() {
  g_last_error.clear();
  return NEPTUNE_OK;
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Resolve (batch, head, seq) strides; all-zero means contiguous.
bool resolve_strides(const int64_t in[3], int64_t heads, int64_t seq, int64_t dim,
                     int64_t out[3]) {
  if (in[0] == 0 && in[1] == 0 && in[2] == 0) {
    out[2] = dim;
    out[1] = seq * dim;
    out[0] = heads * seq * dim;
    return true;
  }
  for (int i = 0; i < 3; ++i) {
    if (in[i] <= 0) return false;
    out[i] = in[i];
  }
  return true;
}

neptune_status device_ready() {
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n <= 0)
    return fail(NEPTUNE_ERR_NO_DEVICE, "no HIP device available (%s)",
                e == hipSuccess ? "device count is 0" : hipGetErrorString(e));
  return NEPTUNE_OK;
}

neptune_status hip_result(hipError_t e, const char *what) {
  if (e != hipSuccess)
    return fail(NEPTUNE_ERR_HIP, "%s: HIP error %d (%s)", what, (int)e, hipGetErrorString(e));
  return ok();
}

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Split layout; identical rule in the CPU oracle (neptune_cpu_decode_layout).
void decode_layout(const neptune_decode_desc *d, int64_t *splits, int64_t *chunk) {
  int64_t want = d->num_splits;
  if (want <= 0) {
    int64_t groups = d->batch * d->heads_kv;
    want = cdiv(2048, groups);
    int64_t cap = cdiv(d->seq_kv, 256);
    if (want > cap) want = cap;
    if (want < 1) want = 1;
  }
  int64_t c = cdiv(cdiv(d->seq_kv, want), 64) * 64;
  *chunk = c;
  *splits = cdiv(d->seq_kv, c);
}

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

// whether the byte ranges [a, a + na) and [b, b + nb) share a byte
bool overlaps(const void *a, size_t na, const void *b, size_t nb) {
  const uintptr_t x = (uintptr_t)a, y = (uintptr_t)b;
  return na && nb && x < y + nb && y < x + na;
}

neptune_status decode_check(const neptune_decode_desc *d) {
  if (!d) return fail(NEPTUNE_ERR_INVALID_ARGUMENT, "decode: desc is NULL");
  if (d->batch <= 0 || d->heads_q <= 0 || d->heads_kv <= 0 || d->seq_kv <= 0 ||
      d->head_dim <= 0 || d->num_splits < 0 || d->scale_block < 0)
    return fail(NEPTUNE_ERR_INVALID_ARGUMENT,
                "decode: sizes must be positive (batch=%lld heads_q=%lld heads_kv=%lld "
                "seq_kv=%lld head_dim=%lld num_splits=%lld)",
                (long long)d->batch, (long long)d->heads_q, (long long)d->heads_kv,
                (long long)d->seq_kv, (long long)d->head_dim, (long long)d->num_splits);
  if (d->heads_q % d->heads_kv)
    return fail(NEPTUNE_ERR_INVALID_ARGUMENT, "decode: heads_q (%lld) %% heads_kv (%lld) != 0",
                (long long)d->heads_q, (long long)d->heads_kv);
  if (d->q_dtype != NEPTUNE_DTYPE_BF16)
    return fail(NEPTUNE_ERR_UNSUPPORTED, "decode: q_dtype must be BF16");
  if (d->kv_dtype != NEPTUNE_DTYPE_BF16 && d->kv_dtype != NEPTUNE_DTYPE_FP8_E4M3)
    return fail(NEPTUNE_ERR_UNSUPPORTED, "decode: kv_dtype must be BF16 or FP8_E4M3");
  if (!(d->scale_log2 >= 0.0f) || !std::isfinite(d->scale_log2))
    return fail(NEPTUNE_ERR_INVALID_ARGUMENT, "decode: scale_log2 must be finite and >= 0");
  return NEPTUNE_OK;
}

size_t decode_ws_bytes(const neptune_decode_desc *d, int64_t splits) {
  size_t rows = (size_t)d->batch * d->heads_q * splits;
  return align256(rows * d->head_dim * 4) + align256(rows * 2 * 4);
}

}  // namespace

extern "C" {

neptune_status neptune_hip_get_backend_info(neptune_backend_info *info) {
  if (!info) return fail(NEPTUNE_ERR_INVALID_ARGUMENT, "info is NULL");
  info->abi_version = NEPTUNE_HIP_ABI_VERSION;
  info->name = "NeptuneHTileHIP";
  info->gcn_arch = "gfx950";
  int v = -1;
  if (hipRuntimeGetVersion(&v) != hipSuccess) v = -1;
  info->hip_runtime_version = v;
  return ok();
}

const char *neptune_last_error(void) { return g_last_error.c_str(); }

int32_t neptune_device_count(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) return 0;
  return n;
}

neptune_status neptune_attn_fwd(const neptune_attn_desc *d, const void *q, const void *k,
                                const void *v, void *o, float *lse, void *stream) {
  if (!d) return fail(NEPTUNE_ERR_INVALID_ARGUMENT, "attn_fwd: desc is NULL");
  if (!q || !k || !v || !o)
    return fail(NEPTUNE_ERR_INVALID_ARGUMENT, "attn_fwd: q, k, v and o must be non-NULL");
  if (d->batch <= 0 || d->heads_q <= 0 || d->heads_kv <= 0 || d->seq_q <= 0 ||
      d->seq_kv <= 0 || d->head_dim <= 0)
    return fail(NEPTUNE_ERR_INVALID_ARGUMENT,
                "attn_fwd: sizes must be positive (batch=%lld heads_q=%lld heads_kv=%lld "
                "seq_q=%lld seq_kv=%lld head_dim=%lld)",
                (long long)d->batch, (long long)d->heads_q, (long long)d->heads_kv,
                (long long)d->seq_q, (long long)d->seq_kv, (long long)d->head_dim);
  if (d->heads_q % d->heads_kv)
    return fail(NEPTUNE_ERR_INVALID_ARGUMENT, "attn_fwd: heads_q (%lld) %% heads_kv (%lld) != 0",
                (long long)d->heads_q, (long long)d->heads_kv);
  if (d->dtype != NEPTUNE_DTYPE_F32 && d->dtype != NEPTUNE_DTYPE_F16 &&
      d->dtype != NEPTUNE_DTYPE_BF16)
    return fail(NEPTUNE_ERR_UNSUPPORTED, "attn_fwd: dtype %d (need F32, F16 or BF16)",
                (int)d->dtype);
  if (!(d->scale_log2 >= 0.0f) || !std::isfinite(d->scale_log2))
    return fail(NEPTUNE_ERR_INVALID_ARGUMENT, "attn_fwd: scale_log2 must be finite and >= 0");
  if (d->pipeline_stages < 0 || d->pipeline_stages > 3)
    return fail(NEPTUNE_ERR_INVALID_ARGUMENT, "attn_fwd: pipeline_stages %d (need 0..3)",
                (int)d->pipeline_stages);
  if (d->k_dim_order != 0 && d->k_dim_order != 1)
    return fail(NEPTUNE_ERR_INVALID_ARGUMENT, "attn_fwd: k_dim_order %d (need 0 or 1)",
                (int)d->k_dim_order);
  AttnLaunch L;
  L.q = q; L.k = k; L.v = v; L.o = o; L.lse = lse;
  L.batch = d->batch; L.heads_q = d->heads_q; L.heads_kv = d->heads_kv;
  L.seq_q = d->seq_q; L.seq_kv = d->seq_kv; L.head_dim = d->head_dim;
  if (!resolve_strides(d->q_stride, d->heads_q, d->seq_q, d->head_dim, L.qs) ||
      !(d->k_dim_order ? resolve_strides(d->k_stride, d->heads_kv, d->head_dim, d->seq_kv, L.ks)
                       : resolve_strides(d->k_stride, d->heads_kv, d->seq_kv, d->head_dim, L.ks)) ||
      !resolve_strides(d->v_stride, d->heads_kv, d->seq_kv, d->head_dim, L.vs) ||
      !resolve_strides(d->o_stride, d->heads_q, d->seq_q, d->head_dim, L.os))
    return fail(NEPTUNE_ERR_INVALID_ARGUMENT,
                "attn_fwd: strides must be all zero (contiguous) or all positive");
  L.dtype = d->dtype;
  L.causal = d->causal ? 1 : 0;
  L.stages = d->pipeline_stages ? d->pipeline_stages : 2;
  L.k_dim_order = d->k_dim_order;
  L.scale_log2 = d->scale_log2 != 0.0f
                     ? d->scale_log2
                     : (float)(1.4426950408889634 / std::sqrt((double)d->head_dim));
  if (d->dtype != NEPTUNE_DTYPE_F32) {
    bool strides8 = true;
    for (int i = 0; i < 3; ++i)
      strides8 = strides8 && L.qs[i] % 8 == 0 && L.ks[i] % 8 == 0 && L.vs[i] % 8 == 0 &&
                 L.os[i] % 8 == 0;
    if (!strides8 || !aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o))
      return fail(NEPTUNE_ERR_UNSUPPORTED,
                  "attn_fwd: 16-bit tensors need 16-byte aligned base pointers and strides "
                  "that are multiples of 8 elements");
  }
  const char *why = "";
  if (!attn_supported(L, &why)) return fail(NEPTUNE_ERR_UNSUPPORTED, "attn_fwd: %s", why);
  neptune_status st = device_ready();
  if (st != NEPTUNE_OK) return st;
  return hip_result(launch_attn_fwd(L, (hipStream_t)stream), "attn_fwd launch");
}

neptune_status neptune_decode_workspace_bytes(const neptune_decode_desc *d, size_t *bytes) {
  if (!bytes) return fail(NEPTUNE_ERR_INVALID_ARGUMENT, "decode_workspace_bytes: bytes is NULL");
  neptune_status st = decode_check(d);
  if (st != NEPTUNE_OK) return st;
  int64_t splits, chunk;
  decode_layout(d, &splits, &chunk);
  *bytes = decode_ws_bytes(d, splits);
  return ok();
}

namespace {
// shared tail of the decode entry points (pk != nullptr: paged KV;
// scratch: the partials go to the library's static device scratch, and
// workspace / workspace_bytes are not used)
neptune_status decode_run(const neptune_decode_desc *d, const neptune_paged_kv_desc *pk,
                          const void *q, const void *k, const void *v, const float *k_scale,
                          const float *v_scale, const int32_t *block_table,
                          const int32_t *seq_lens, void *o, float *lse, bool scratch,
                          void *workspace, size_t workspace_bytes, void *stream) {
  if (!scratch && !workspace)
    return fail(NEPTUNE_ERR_INVALID_ARGUMENT, "decode: workspace is NULL");
  int64_t splits, chunk;
  decode_layout(d, &splits, &chunk);
  const size_t need = decode_ws_bytes(d, splits);
  if (scratch && need > kDecodeScratchBytes)
    return fail(NEPTUNE_ERR_WORKSPACE_TOO_SMALL,
                "decode_noalloc: %lld splits x %lld rows need %zu bytes of partials, the static "
                "scratch holds %zu (use neptune_decode_splitk with a workspace)",
                (long long)splits, (long long)(d->batch * d->heads_q), need,
                kDecodeScratchBytes);
  if (!scratch && workspace_bytes < need)
    return fail(NEPTUNE_ERR_WORKSPACE_TOO_SMALL, "decode: workspace %zu bytes, need %zu",
                workspace_bytes, need);
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || (!scratch && !aligned16(workspace)))
    return fail(NEPTUNE_ERR_UNSUPPORTED, "decode: q, k, v and workspace must be 16-byte aligned");
  DecodeLaunch L;
  L.q = q; L.k = k; L.v = v; L.k_scale = k_scale; L.v_scale = v_scale;
  L.o = o; L.lse = lse;
  L.batch = d->batch; L.heads_q = d->heads_q; L.heads_kv = d->heads_kv;
  L.seq_kv = d->seq_kv; L.head_dim = d->head_dim;
  L.splits = splits; L.chunk = chunk;
  L.scale_block = d->scale_block > 0 ? d->scale_block : 64;
  L.n_scale_blocks = cdiv(d->seq_kv, L.scale_block);
  L.kv_dtype = d->kv_dtype;
  L.scale_log2 = d->scale_log2 != 0.0f
                     ? d->scale_log2
                     : (float)(1.4426950408889634 / std::sqrt((double)d->head_dim));
  if (pk) {
    L.block_table = block_table;
    L.seq_lens = seq_lens;
    L.page_size = pk->page_size;
    L.max_pages = pk->max_pages;
    L.num_pages = pk->num_pages;
    for (int i = 0; i < 3; ++i) {
      L.k_pstride[i] = pk->k_stride[i];
      L.v_pstride[i] = pk->v_stride[i];
    }
  }
  const char *why = "";
  if (!decode_supported(L, &why)) return fail(NEPTUNE_ERR_UNSUPPORTED, "decode: %s", why);
  neptune_status st = device_ready();
  if (st != NEPTUNE_OK) return st;
  if (scratch) {
    st = hip_result(decode_scratch((hipStream_t)stream, &workspace), "decode_noalloc: scratch address");
    if (st != NEPTUNE_OK) return st;
  }
  const size_t rows = (size_t)d->batch * d->heads_q * splits;
  L.part_o = (float *)workspace;
  L.part_ml = (float *)((char *)workspace + align256(rows * d->head_dim * 4));
  return hip_result(launch_decode(L, (hipStream_t)stream), "decode launch");
}
}  // namespace

neptune_status neptune_decode_splitk(const neptune_decode_desc *d, const void *q,
                                     const void *k, const void *v, const float *k_scale,
                                     const float *v_scale, void *o, float *lse,
                                     void *workspace, size_t workspace_bytes, void *stream) {
  neptune_status st = decode_check(d);
  if (st != NEPTUNE_OK) return st;
  if (!q || !k || !v || !o)
    return fail(NEPTUNE_ERR_INVALID_ARGUMENT, "decode: q, k, v and o must be non-NULL");
  const bool fp8 = d->kv_dtype == NEPTUNE_DTYPE_FP8_E4M3;
  if (fp8 && (!k_scale || !v_scale))
    return fail(NEPTUNE_ERR_INVALID_ARGUMENT, "decode: fp8 KV needs k_scale and v_scale");
  return decode_run(d, nullptr, q, k, v, k_scale, v_scale, nullptr, nullptr, o, lse, false,
                    workspace, workspace_bytes, stream);
}

neptune_status neptune_decode_splitk_noalloc(const neptune_decode_desc *d, const void *q,
                                             const void *k, const void *v,
                                             const float *k_scale, const float *v_scale,
                                             void *o, float *lse, void *stream) {
  neptune_status st = decode_check(d);
  if (st != NEPTUNE_OK) return st;
  if (!q || !k || !v || !o)
    return fail(NEPTUNE_ERR_INVALID_ARGUMENT, "decode_noalloc: q, k, v and o must be non-NULL");
  if (d->kv_dtype == NEPTUNE_DTYPE_FP8_E4M3 && (!k_scale || !v_scale))
    return fail(NEPTUNE_ERR_INVALID_ARGUMENT, "decode_noalloc: fp8 KV needs k_scale and v_scale");
  return decode_run(d, nullptr, q, k, v, k_scale, v_scale, nullptr, nullptr, o, lse, true,
                    nullptr, 0, stream);
}

namespace {
// checks shared by the two paged entry points; esize: bytes per pool element
neptune_status paged_check(const char *fn, const neptune_decode_desc *d,
                           const neptune_paged_kv_desc *pk, const void *q, const void *k_pages,
                           const void *v_pages, const int32_t *block_table,
                           const int32_t *seq_lens, const void *o, int64_t esize) {
  neptune_status st = decode_check(d);
  if (st != NEPTUNE_OK) return st;
  if (!pk) return fail(NEPTUNE_ERR_INVALID_ARGUMENT, "%s: pages desc is NULL", fn);
  if (!q || !k_pages || !v_pages || !block_table || !seq_lens || !o)
    return fail(NEPTUNE_ERR_INVALID_ARGUMENT,
                "%s: q, pools, block_table, seq_lens and o must be non-NULL", fn);
  if (pk->num_pages <= 0 || pk->page_size <= 0 || pk->max_pages <= 0)
    return fail(NEPTUNE_ERR_INVALID_ARGUMENT,
                "%s: num_pages, page_size and max_pages must be positive", fn);
  if (pk->max_pages * pk->page_size < d->seq_kv)
    return fail(NEPTUNE_ERR_INVALID_ARGUMENT,
                "%s: max_pages (%lld) * page_size (%lld) < seq_kv (%lld)", fn,
                (long long)pk->max_pages, (long long)pk->page_size, (long long)d->seq_kv);
  // 16-byte copy units: strides in whole units
  const int64_t unit = 16 / esize;
  for (int i = 0; i < 3; ++i)
    if (pk->k_stride[i] <= 0 || pk->v_stride[i] <= 0 || pk->k_stride[i] % unit ||
        pk->v_stride[i] % unit)
      return fail(NEPTUNE_ERR_UNSUPPORTED,
                  "%s: pool strides must be positive multiples of %lld elements", fn,
                  (long long)unit);
  return NEPTUNE_OK;
}
}  // namespace

neptune_status neptune_decode_paged(const neptune_decode_desc *d, const neptune_paged_kv_desc *pk,
                                    const void *q, const void *k_pages, const void *v_pages,
                                    const int32_t *block_table, const int32_t *seq_lens, void *o,
                                    float *lse, void *workspace, size_t workspace_bytes,
                                    void *stream) {
  neptune_status st =
      paged_check("decode_paged", d, pk, q, k_pages, v_pages, block_table, seq_lens, o, 2);
  if (st != NEPTUNE_OK) return st;
  if (d->kv_dtype != NEPTUNE_DTYPE_BF16)
    return fail(NEPTUNE_ERR_UNSUPPORTED,
                "decode_paged: kv_dtype must be BF16 (fp8 pools: neptune_decode_paged_fp8)");
  return decode_run(d, pk, q, k_pages, v_pages, nullptr, nullptr, block_table, seq_lens, o, lse,
                    false, workspace, workspace_bytes, stream);
}

neptune_status neptune_decode_paged_fp8(const neptune_decode_desc *d,
                                        const neptune_paged_kv_desc *pk, const void *q,
                                        const uint8_t *k_pages, const uint8_t *v_pages,
                                        const float *k_scales, const float *v_scales,
                                        const int32_t *block_table, const int32_t *seq_lens,
                                        void *o, float *lse, void *workspace,
                                        size_t workspace_bytes, void *stream) {
  neptune_status st =
      paged_check("decode_paged_fp8", d, pk, q, k_pages, v_pages, block_table, seq_lens, o, 1);
  if (st != NEPTUNE_OK) return st;
  if (d->kv_dtype != NEPTUNE_DTYPE_FP8_E4M3)
    return fail(NEPTUNE_ERR_INVALID_ARGUMENT, "decode_paged_fp8: kv_dtype must be FP8_E4M3");
  if (!k_scales || !v_scales)
    return fail(NEPTUNE_ERR_INVALID_ARGUMENT,
                "decode_paged_fp8: k_scales and v_scales must be non-NULL");
  if (d->scale_block != 0 && d->scale_block != pk->page_size)
    return fail(NEPTUNE_ERR_UNSUPPORTED,
                "decode_paged_fp8: one scale per page: scale_block must be 0 or page_size "
                "(%lld), not %lld",
                (long long)pk->page_size, (long long)d->scale_block);
  neptune_decode_desc dd = *d;
  dd.scale_block = pk->page_size;
  return decode_run(&dd, pk, q, k_pages, v_pages, k_scales, v_scales, block_table, seq_lens, o,
                    lse, false, workspace, workspace_bytes, stream);
}

neptune_status neptune_kv_quantize_fp8(int64_t batch, int64_t heads_kv, int64_t seq_kv,
                                       int64_t head_dim, int64_t scale_block, const void *src,
                                       uint8_t *codes, float *scales, void *stream) {
  if (!src || !codes || !scales)
    return fail(NEPTUNE_ERR_INVALID_ARGUMENT, "kv_quantize: src, codes and scales must be non-NULL");
  if (batch <= 0 || heads_kv <= 0 || seq_kv <= 0 || head_dim <= 0 || scale_block < 0)
    return fail(NEPTUNE_ERR_INVALID_ARGUMENT, "kv_quantize: sizes must be positive");
  if (batch * heads_kv * cdiv(seq_kv, scale_block > 0 ? scale_block : 64) > ((int64_t)1 << 31) - 1 ||
      seq_kv * head_dim > ((int64_t)1 << 31) - 1)
    return fail(NEPTUNE_ERR_UNSUPPORTED, "kv_quantize: shape too large for one launch");
  QuantLaunch L;
  L.src = src; L.codes = codes; L.scales = scales;
  L.batch = batch; L.heads_kv = heads_kv; L.seq_kv = seq_kv; L.head_dim = head_dim;
  L.scale_block = scale_block > 0 ? scale_block : 64;
  L.n_scale_blocks = cdiv(seq_kv, L.scale_block);
  neptune_status st = device_ready();
  if (st != NEPTUNE_OK) return st;
  return hip_result(launch_kv_quantize(L, (hipStream_t)stream), "kv_quantize launch");
}

neptune_status neptune_selective_scan_fwd(const neptune_scan_desc *d, const void *u,
                                          const void *delta_raw, const float *A, const void *B,
                                          const void *C, const float *D, const void *z,
                                          const float *delta_bias, void *y, void *stream) {
  if (!d) return fail(NEPTUNE_ERR_INVALID_ARGUMENT, "selective_scan: desc is NULL");
  if (!u || !delta_raw || !A || !B || !C || !y)
    return fail(NEPTUNE_ERR_INVALID_ARGUMENT,
                "selective_scan: u, delta, A, B, C and y must be non-NULL");
  if (d->batch <= 0 || d->dim <= 0 || d->seq_len <= 0 || d->d_state <= 0)
    return fail(NEPTUNE_ERR_INVALID_ARGUMENT, "selective_scan: sizes must be positive");
  if (d->io_dtype != NEPTUNE_DTYPE_BF16)
    return fail(NEPTUNE_ERR_UNSUPPORTED, "selective_scan: io_dtype must be BF16");
  ScanLaunch L;
  L.u = u; L.delta_raw = delta_raw; L.B = B; L.C = C; L.z = z;
  L.A = A; L.D = D; L.delta_bias = delta_bias; L.y = y;
  L.batch = d->batch; L.dim = d->dim; L.seq_len = d->seq_len; L.d_state = d->d_state;
  L.delta_softplus = d->delta_softplus ? 1 : 0;
  const char *why = "";
  if (!scan_supported(L, &why)) return fail(NEPTUNE_ERR_UNSUPPORTED, "selective_scan: %s", why);
  // y is written while later steps of the inputs are still being read, and
  // holds per-chunk state before the outputs: it may share no input byte
  // (sizes are below 2^63 once scan_supported has passed)
  const size_t rows = (size_t)d->batch * (size_t)d->seq_len * 2;
  const size_t act = rows * (size_t)d->dim, bc = rows * (size_t)d->d_state;
  const struct { const void *p; size_t n; const char *name; } in[] = {
      {u, act, "u"},
      {delta_raw, act, "delta"},
      {z, z ? act : 0, "z"},
      {B, bc, "B"},
      {C, bc, "C"},
      {A, (size_t)d->dim * (size_t)d->d_state * 4, "A"},
      {D, D ? (size_t)d->dim * 4 : 0, "D"},
      {delta_bias, delta_bias ? (size_t)d->dim * 4 : 0, "delta_bias"}};
  for (const auto &t : in)
    if (overlaps(y, act, t.p, t.n))
      return fail(NEPTUNE_ERR_INVALID_ARGUMENT, "selective_scan: y overlaps %s", t.name);
  neptune_status st = device_ready();
  if (st != NEPTUNE_OK) return st;
  return hip_result(launch_selective_scan(L, (hipStream_t)stream), "selective_scan launch");
}

}  // extern "C"
