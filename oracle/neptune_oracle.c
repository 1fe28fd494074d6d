/*
 * neptune_oracle.c — CPU restatement of the HTile hot path (test
 * infrastructure only; see neptune_oracle.h for who may load it and what
 * pins each function).
 *
 * Attention follows tests/data/flash_attention_htile.mlir op by op:
 *   HTile:23        running max starts at -3.40282347e38 (-FLT_MAX)
 *   HTile:24,56-59  scores scaled by log2(e)/sqrt(D) into the exp2 domain
 *   HTile:40,47     keys stream in blocks of 64
 *   HTile:61-64     block row max, m_new = max(m_old, rowmax)
 *   HTile:76-82     p = exp2(s - m_new), row sum of fp32 p
 *   HTile:84-91     l = l * exp2(m_old - m_new) + rowsum
 *   HTile:93-94     p truncated (RNE) to the 16-bit input type before P.V
 *   HTile:98-121    acc = acc * exp2(m_old - m_new) + P.V  (fp32)
 *   HTile:137-143   O = acc / l, then rounded to the input type
 * The unscheduled math it must agree with is tests/data/attention_l0.mlir:
 * 10-85 and the torch reference tests/test_translators.py:122-135.
 * Causal masking, LSE, grouped KV heads, split-K decode, fp8 KV and the
 * selective scan are absent from the reference; they are restated from
 * their textbook definitions (cited per function).
 */
#include "neptune_oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define LOG2E 1.4426950408889634
#define LN2 0.6931471805599453
#define HTILE_BLOCK_N 64

/* ---------------------------------------------------------------- codecs */

static inline float f_from_u(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}
static inline uint32_t u_from_f(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

uint16_t neptune_cpu_f32_to_bf16(float f) {
  uint32_t u = u_from_f(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

float neptune_cpu_bf16_to_f32(uint16_t h) { return f_from_u((uint32_t)h << 16); }

uint16_t neptune_cpu_f32_to_f16(float f) {
  uint32_t u = u_from_f(f);
  uint32_t sign = (u >> 16) & 0x8000u;
  uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);
  if (a >= 0x38800000u) { /* |f| >= 2^-14: normal half (or overflow) */
    if (a >= 0x47800000u) return (uint16_t)(sign | 0x7c00u);
    uint32_t r = a - 0x38000000u; /* rebias 127 -> 15 */
    r += 0xfffu + ((r >> 13) & 1u);
    r >>= 13;
    if (r > 0x7c00u) r = 0x7c00u;
    return (uint16_t)(sign | r);
  }
  /* subnormal half: units of 2^-24, round half to even */
  double scaled = (double)f_from_u(a) * 16777216.0;
  double fl = floor(scaled);
  double rem = scaled - fl;
  uint32_t m = (uint32_t)fl;
  if (rem > 0.5 || (rem == 0.5 && (m & 1u))) m++;
  return (uint16_t)(sign | m);
}

float neptune_cpu_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  float v;
  if (e == 0)
    v = (float)m * 5.9604644775390625e-08f; /* 2^-24 */
  else if (e == 31)
    v = m ? NAN : INFINITY;
  else
    v = f_from_u(((e + 112u) << 23) | (m << 13));
  return f_from_u(u_from_f(v) | sign);
}

/* OCP 8-bit floating point spec v1.0, E4M3: bias 7, no infinities, S.1111.111
 * is NaN, largest finite 448 = 1.75 * 2^8, subnormals m * 2^-9. Conversion
 * is round-to-nearest-even with saturation to +-448 (the "satfinite" mode). */
uint8_t neptune_cpu_f32_to_e4m3(float f) {
  uint32_t u = u_from_f(f);
  uint8_t sign = (uint8_t)((u >> 24) & 0x80u);
  uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return (uint8_t)(sign | 0x7fu);
  float af = f_from_u(a);
  if (af >= 448.0f) return (uint8_t)(sign | 0x7eu);
  if (af < 0.015625f) { /* below 2^-6: subnormal codes, units of 2^-9 */
    double scaled = (double)af * 512.0;
    double fl = floor(scaled);
    double rem = scaled - fl;
    uint32_t m = (uint32_t)fl;
    if (rem > 0.5 || (rem == 0.5 && (m & 1u))) m++;
    return (uint8_t)(sign | m); /* m == 8 is the smallest normal, 0x08 */
  }
  int32_t e = (int32_t)(a >> 23) - 127; /* -6 .. 8 */
  uint32_t mant = a & 0x7fffffu;
  uint32_t r = ((uint32_t)(e + 7) << 3) | (mant >> 20);
  uint32_t rem = mant & 0xfffffu;
  if (rem > 0x80000u || (rem == 0x80000u && (r & 1u))) r++;
  if (r > 0x7eu) r = 0x7eu;
  return (uint8_t)(sign | r);
}

float neptune_cpu_e4m3_to_f32(uint8_t c) {
  uint32_t e = (c >> 3) & 0xfu, m = c & 7u;
  float v;
  if (e == 15 && m == 7)
    v = NAN;
  else if (e == 0)
    v = (float)m * 0.001953125f; /* 2^-9 */
  else
    v = ldexpf(1.0f + (float)m / 8.0f, (int)e - 7);
  return (c & 0x80u) ? -v : v;
}

static inline float load_elem(const void *p, int64_t i, int32_t dt) {
  switch (dt) {
  case NEPTUNE_DTYPE_F32:
    return ((const float *)p)[i];
  case NEPTUNE_DTYPE_F16:
    return neptune_cpu_f16_to_f32(((const uint16_t *)p)[i]);
  case NEPTUNE_DTYPE_BF16:
    return neptune_cpu_bf16_to_f32(((const uint16_t *)p)[i]);
  default:
    return neptune_cpu_e4m3_to_f32(((const uint8_t *)p)[i]);
  }
}

static inline void store_elem(void *p, int64_t i, int32_t dt, float v) {
  switch (dt) {
  case NEPTUNE_DTYPE_F32:
    ((float *)p)[i] = v;
    break;
  case NEPTUNE_DTYPE_F16:
    ((uint16_t *)p)[i] = neptune_cpu_f32_to_f16(v);
    break;
  case NEPTUNE_DTYPE_BF16:
    ((uint16_t *)p)[i] = neptune_cpu_f32_to_bf16(v);
    break;
  default:
    ((uint8_t *)p)[i] = neptune_cpu_f32_to_e4m3(v);
    break;
  }
}

/* value after a store/load round trip through dtype (HTile's truncf) */
static inline float round_to(float v, int32_t dt) {
  switch (dt) {
  case NEPTUNE_DTYPE_F16:
    return neptune_cpu_f16_to_f32(neptune_cpu_f32_to_f16(v));
  case NEPTUNE_DTYPE_BF16:
    return neptune_cpu_bf16_to_f32(neptune_cpu_f32_to_bf16(v));
  default:
    return v;
  }
}

void neptune_cpu_convert_f32(const float *src, void *dst, int64_t n,
                             int32_t dst_dtype) {
  for (int64_t i = 0; i < n; ++i) store_elem(dst, i, dst_dtype, src[i]);
}

void neptune_cpu_to_f32(const void *src, float *dst, int64_t n,
                        int32_t src_dtype) {
  for (int64_t i = 0; i < n; ++i) dst[i] = load_elem(src, i, src_dtype);
}

int32_t neptune_cpu_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* ------------------------------------------------------------ attention */

static int attn_check(const neptune_attn_desc *d, const void *q, const void *k,
                      const void *v) {
  if (!d || !q || !k || !v) return NEPTUNE_ERR_INVALID_ARGUMENT;
  if (d->batch <= 0 || d->heads_q <= 0 || d->heads_kv <= 0 || d->seq_q <= 0 ||
      d->seq_kv <= 0 || d->head_dim <= 0 || d->head_dim > 1024)
    return NEPTUNE_ERR_INVALID_ARGUMENT;
  if (d->heads_q % d->heads_kv) return NEPTUNE_ERR_INVALID_ARGUMENT;
  if (d->dtype != NEPTUNE_DTYPE_F32 && d->dtype != NEPTUNE_DTYPE_F16 &&
      d->dtype != NEPTUNE_DTYPE_BF16)
    return NEPTUNE_ERR_INVALID_ARGUMENT;
  if (d->pipeline_stages < 0 || d->pipeline_stages > 3 ||
      (d->k_dim_order != 0 && d->k_dim_order != 1))
    return NEPTUNE_ERR_INVALID_ARGUMENT;
  return NEPTUNE_OK;
}

static void strides_or_contig(const int64_t in[3], int64_t heads, int64_t seq,
                              int64_t dim, int64_t out[3]) {
  if (in[0] == 0 && in[1] == 0 && in[2] == 0) {
    out[2] = dim;
    out[1] = seq * dim;
    out[0] = heads * seq * dim;
  } else {
    out[0] = in[0];
    out[1] = in[1];
    out[2] = in[2];
  }
}

/* K's (batch, head) base strides plus its token and head_dim strides:
 * k_dim_order 0 stores K [B, Hk, S, D], 1 stores it [B, Hk, D, S]. */
static void k_layout(const neptune_attn_desc *d, int64_t ks[3], int64_t *tok,
                     int64_t *dim) {
  if (d->k_dim_order) {
    strides_or_contig(d->k_stride, d->heads_kv, d->head_dim, d->seq_kv, ks);
    *tok = 1;
    *dim = ks[2];
  } else {
    strides_or_contig(d->k_stride, d->heads_kv, d->seq_kv, d->head_dim, ks);
    *tok = ks[2];
    *dim = 1;
  }
}

static float default_scale_log2(float given, int64_t dim) {
  return given != 0.0f ? given : (float)(LOG2E / sqrt((double)dim));
}

/* One query row through the HTile recurrence over keys [k0, k1), given
 * fp32 copies of the query row and a key/value accessor. Writes the
 * unnormalised accumulator acc[D] and returns (m, l). */
typedef struct {
  const void *k, *v;
  int32_t dt;          /* storage type of k and v */
  int64_t kbase, vbase, kstride, vstride; /* element offsets; strides per token */
  int64_t kdstride;    /* K's head_dim stride: 1, or the row stride of [.., D, S] */
  const float *kscale, *vscale; /* per token block (fp8), or NULL */
  int64_t scale_block;
  int32_t p_dtype;     /* type P is rounded to before P.V */
  /* paged KV (btab != NULL): token t lives in page btab[t / page_size]
   * (clamped to [0, num_pages)), at that page's base (page strides kpage /
   * vpage) plus kbase / vbase, row t % page_size */
  const int32_t *btab;
  int64_t page_size, num_pages, kpage, vpage;
  /* paged fp8: kscale / vscale hold one scale per page at this stride (the
   * pool's [pages, heads_kv] rows, already offset to the KV head) */
  int64_t scale_page_stride;
} kv_view;

static inline float kv_load(const kv_view *kv, int which, int64_t t,
                            int64_t dd) {
  const void *base = which ? kv->v : kv->k;
  int64_t row = t, page_off = 0, pg = 0;
  if (kv->btab) {
    pg = kv->btab[t / kv->page_size];
    pg = pg < 0 ? 0 : (pg >= kv->num_pages ? kv->num_pages - 1 : pg);
    page_off = pg * (which ? kv->vpage : kv->kpage);
    row = t % kv->page_size;
  }
  int64_t off = which ? page_off + kv->vbase + row * kv->vstride + dd
                      : page_off + kv->kbase + row * kv->kstride + dd * kv->kdstride;
  float x = load_elem(base, off, kv->dt);
  const float *sc = which ? kv->vscale : kv->kscale;
  if (sc) x *= kv->btab ? sc[pg * kv->scale_page_stride] : sc[t / kv->scale_block];
  return x;
}

static void htile_row(const float *qrow, int64_t D, const kv_view *kv,
                      int64_t k0, int64_t k1, int64_t visible_end,
                      float scale2, float *acc, float *m_out, float *l_out) {
  float m = -FLT_MAX, l = 0.0f;
  float s[HTILE_BLOCK_N], p[HTILE_BLOCK_N];
  double *rf = (double *)malloc(sizeof(double) * (size_t)D);
  for (int64_t dd = 0; dd < D; ++dd) acc[dd] = 0.0f;
  for (int64_t j0 = k0; j0 < k1; j0 += HTILE_BLOCK_N) {
    if (j0 >= visible_end) break; /* fully masked block: exact no-op */
    int64_t jn = k1 - j0 < HTILE_BLOCK_N ? k1 - j0 : HTILE_BLOCK_N;
    float rowmax = -INFINITY;
    for (int64_t jj = 0; jj < jn; ++jj) {
      int64_t t = j0 + jj;
      if (t >= visible_end) {
        s[jj] = -INFINITY;
        continue;
      }
      double dot = 0.0;
      for (int64_t dd = 0; dd < D; ++dd)
        dot += (double)qrow[dd] * (double)kv_load(kv, 0, t, dd);
      s[jj] = (float)dot * scale2;
      if (s[jj] > rowmax) rowmax = s[jj];
    }
    float m_new = m > rowmax ? m : rowmax;
    double rowsum = 0.0;
    for (int64_t jj = 0; jj < jn; ++jj) {
      p[jj] = exp2f(s[jj] - m_new);
      rowsum += p[jj];
    }
    float alpha = exp2f(m - m_new);
    l = l * alpha + (float)rowsum;
    for (int64_t dd = 0; dd < D; ++dd) rf[dd] = 0.0;
    for (int64_t jj = 0; jj < jn; ++jj) {
      float pr = round_to(p[jj], kv->p_dtype);
      if (pr == 0.0f) continue;
      for (int64_t dd = 0; dd < D; ++dd)
        rf[dd] += (double)pr * (double)kv_load(kv, 1, j0 + jj, dd);
    }
    for (int64_t dd = 0; dd < D; ++dd) acc[dd] = acc[dd] * alpha + (float)rf[dd];
    m = m_new;
  }
  free(rf);
  *m_out = m;
  *l_out = l;
}

int32_t neptune_cpu_attn_fwd(const neptune_attn_desc *d, const void *q,
                             const void *k, const void *v, void *o,
                             float *lse) {
  int st = attn_check(d, q, k, v);
  if (st) return st;
  if (!o) return NEPTUNE_ERR_INVALID_ARGUMENT;
  const int64_t B = d->batch, Hq = d->heads_q, Hk = d->heads_kv, Sq = d->seq_q,
                Sk = d->seq_kv, D = d->head_dim, group = Hq / Hk;
  int64_t qs[3], ks[3], vs[3], os[3], ktok, kdim;
  strides_or_contig(d->q_stride, Hq, Sq, D, qs);
  k_layout(d, ks, &ktok, &kdim);
  strides_or_contig(d->v_stride, Hk, Sk, D, vs);
  strides_or_contig(d->o_stride, Hq, Sq, D, os);
  const float scale2 = default_scale_log2(d->scale_log2, D);
  const int32_t dt = d->dtype;

#pragma omp parallel for collapse(3) schedule(dynamic, 4)
  for (int64_t b = 0; b < B; ++b)
    for (int64_t h = 0; h < Hq; ++h)
      for (int64_t i = 0; i < Sq; ++i) {
        int64_t hk = h / group;
        float *qrow = (float *)malloc(sizeof(float) * (size_t)D * 2);
        float *acc = qrow + D;
        for (int64_t dd = 0; dd < D; ++dd)
          qrow[dd] = load_elem(q, b * qs[0] + h * qs[1] + i * qs[2] + dd, dt);
        kv_view kv = {.k = k, .v = v, .dt = dt, .kbase = b * ks[0] + hk * ks[1],
                      .vbase = b * vs[0] + hk * vs[1], .kstride = ktok, .vstride = vs[2],
                      .kdstride = kdim, .kscale = NULL, .vscale = NULL, .scale_block = 1,
                      .p_dtype = dt};
        int64_t visible = Sk;
        if (d->causal) {
          int64_t last = i + (Sk - Sq);
          visible = last < 0 ? 0 : (last + 1 < Sk ? last + 1 : Sk);
        }
        float m, l;
        htile_row(qrow, D, &kv, 0, Sk, visible, scale2, acc, &m, &l);
        int64_t obase = b * os[0] + h * os[1] + i * os[2];
        for (int64_t dd = 0; dd < D; ++dd)
          store_elem(o, obase + dd, dt, l > 0.0f ? acc[dd] / l : 0.0f);
        if (lse)
          lse[(b * Hq + h) * Sq + i] =
              l > 0.0f ? (m + log2f(l)) * (float)LN2 : -INFINITY;
        free(qrow);
      }
  return NEPTUNE_OK;
}

/* Closed form of tests/data/attention_l0.mlir:10-13 (and the torch
 * reference tests/test_translators.py:122-135) in fp64, with the causal
 * mask added: S = scale * Q K^T, P = softmax(S), O = P V. */
int32_t neptune_cpu_attn_exact(const neptune_attn_desc *d, const void *q,
                               const void *k, const void *v, double *o,
                               double *lse) {
  int st = attn_check(d, q, k, v);
  if (st) return st;
  if (!o) return NEPTUNE_ERR_INVALID_ARGUMENT;
  const int64_t B = d->batch, Hq = d->heads_q, Hk = d->heads_kv, Sq = d->seq_q,
                Sk = d->seq_kv, D = d->head_dim, group = Hq / Hk;
  int64_t qs[3], ks[3], vs[3], os_unused[3], ktok, kdim;
  strides_or_contig(d->q_stride, Hq, Sq, D, qs);
  k_layout(d, ks, &ktok, &kdim);
  strides_or_contig(d->v_stride, Hk, Sk, D, vs);
  (void)os_unused;
  const double scale = (double)default_scale_log2(d->scale_log2, D) * LN2;
  const int32_t dt = d->dtype;

#pragma omp parallel for collapse(3) schedule(dynamic, 4)
  for (int64_t b = 0; b < B; ++b)
    for (int64_t h = 0; h < Hq; ++h)
      for (int64_t i = 0; i < Sq; ++i) {
        int64_t hk = h / group;
        double *s = (double *)malloc(sizeof(double) * (size_t)Sk);
        int64_t visible = Sk;
        if (d->causal) {
          int64_t last = i + (Sk - Sq);
          visible = last < 0 ? 0 : (last + 1 < Sk ? last + 1 : Sk);
        }
        double mx = -INFINITY;
        for (int64_t j = 0; j < visible; ++j) {
          double dot = 0.0;
          for (int64_t dd = 0; dd < D; ++dd)
            dot += (double)load_elem(q, b * qs[0] + h * qs[1] + i * qs[2] + dd,
                                     dt) *
                   (double)load_elem(k, b * ks[0] + hk * ks[1] + j * ktok + dd * kdim,
                                     dt);
          s[j] = dot * scale;
          if (s[j] > mx) mx = s[j];
        }
        double sum = 0.0;
        for (int64_t j = 0; j < visible; ++j) {
          s[j] = exp(s[j] - mx);
          sum += s[j];
        }
        double *orow = o + ((b * Hq + h) * Sq + i) * D;
        for (int64_t dd = 0; dd < D; ++dd) {
          double acc = 0.0;
          for (int64_t j = 0; j < visible; ++j)
            acc += s[j] *
                   (double)load_elem(v, b * vs[0] + hk * vs[1] + j * vs[2] + dd,
                                     dt);
          orow[dd] = visible ? acc / sum : 0.0;
        }
        if (lse) lse[(b * Hq + h) * Sq + i] = visible ? mx + log(sum) : -INFINITY;
        free(s);
      }
  return NEPTUNE_OK;
}

/* --------------------------------------------------------------- decode */

static int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

/* Split layout shared by the library: chunks are whole 64-token blocks so
 * that fp8 scale blocks and the online-softmax blocks never straddle two
 * splits. With num_splits == 0 the library targets >= 2048 work-groups
 * (8 per CU on 256 CUs) and >= 256 tokens per split. */
int32_t neptune_cpu_decode_layout(const neptune_decode_desc *d,
                                  int64_t *splits, int64_t *chunk) {
  if (!d || d->seq_kv <= 0 || d->batch <= 0 || d->heads_kv <= 0)
    return NEPTUNE_ERR_INVALID_ARGUMENT;
  int64_t want = d->num_splits;
  if (want <= 0) {
    int64_t groups = d->batch * d->heads_kv;
    want = cdiv(2048, groups);
    int64_t cap = cdiv(d->seq_kv, 256);
    if (want > cap) want = cap;
    if (want < 1) want = 1;
  }
  int64_t c = cdiv(cdiv(d->seq_kv, want), HTILE_BLOCK_N) * HTILE_BLOCK_N;
  *chunk = c;
  *splits = cdiv(d->seq_kv, c);
  return NEPTUNE_OK;
}

int32_t neptune_cpu_decode_splitk(const neptune_decode_desc *d, const void *q,
                                  const void *k, const void *v,
                                  const float *k_scale, const float *v_scale,
                                  void *o, float *lse, float *partials) {
  if (!d || !q || !k || !v || !o) return NEPTUNE_ERR_INVALID_ARGUMENT;
  if (d->heads_q <= 0 || d->heads_kv <= 0 || d->heads_q % d->heads_kv ||
      d->head_dim <= 0)
    return NEPTUNE_ERR_INVALID_ARGUMENT;
  const int fp8 = d->kv_dtype == NEPTUNE_DTYPE_FP8_E4M3;
  if (fp8 && (!k_scale || !v_scale)) return NEPTUNE_ERR_INVALID_ARGUMENT;
  int64_t S, chunk;
  int st = neptune_cpu_decode_layout(d, &S, &chunk);
  if (st) return st;
  const int64_t B = d->batch, Hq = d->heads_q, Hk = d->heads_kv,
                L = d->seq_kv, D = d->head_dim, group = Hq / Hk;
  const int64_t sb = d->scale_block > 0 ? d->scale_block : 64;
  const int64_t nsb = cdiv(L, sb);
  const float scale2 = default_scale_log2(d->scale_log2, D);

#pragma omp parallel for collapse(2) schedule(dynamic, 1)
  for (int64_t b = 0; b < B; ++b)
    for (int64_t h = 0; h < Hq; ++h) {
      int64_t hk = h / group;
      float *buf = (float *)malloc(sizeof(float) * (size_t)(D * (S + 1) + 2 * S));
      float *qrow = buf, *ot = buf + D, *ms = ot + S * D, *ls = ms + S;
      for (int64_t dd = 0; dd < D; ++dd)
        qrow[dd] = load_elem(q, (b * Hq + h) * D + dd, d->q_dtype);
      kv_view kv = {.k = k, .v = v, .dt = d->kv_dtype, .kbase = (b * Hk + hk) * L * D,
                    .vbase = (b * Hk + hk) * L * D, .kstride = D, .vstride = D,
                    .kdstride = 1, .kscale = fp8 ? k_scale + (b * Hk + hk) * nsb : NULL,
                    .vscale = fp8 ? v_scale + (b * Hk + hk) * nsb : NULL, .scale_block = sb,
                    .p_dtype = d->q_dtype};
      for (int64_t s = 0; s < S; ++s) {
        int64_t k0 = s * chunk, k1 = k0 + chunk < L ? k0 + chunk : L;
        htile_row(qrow, D, &kv, k0, k1, k1, scale2, ot + s * D, &ms[s], &ls[s]);
        if (partials) {
          float *pp = partials + ((b * Hq + h) * S + s) * (D + 2);
          memcpy(pp, ot + s * D, sizeof(float) * (size_t)D);
          pp[D] = ms[s];
          pp[D + 1] = ls[s];
        }
      }
      float M = -FLT_MAX;
      for (int64_t s = 0; s < S; ++s) M = ms[s] > M ? ms[s] : M;
      float Lsum = 0.0f;
      for (int64_t s = 0; s < S; ++s) Lsum += exp2f(ms[s] - M) * ls[s];
      for (int64_t dd = 0; dd < D; ++dd) {
        float acc = 0.0f;
        for (int64_t s = 0; s < S; ++s) acc += exp2f(ms[s] - M) * ot[s * D + dd];
        store_elem(o, (b * Hq + h) * D + dd, d->q_dtype, acc / Lsum);
      }
      if (lse) lse[b * Hq + h] = (M + log2f(Lsum)) * (float)LN2;
      free(buf);
    }
  return NEPTUNE_OK;
}

/* Split-K decode over a paged KV pool: the same split layout (from
 * seq_kv, the longest sequence) and the same per-split recurrence and
 * combine as neptune_cpu_decode_splitk, with sequence b's tokens read
 * through its block-table row and only its first seq_lens[b] tokens (clamped
 * to [0, seq_kv]) visible. An empty sequence gives O = 0 and lse = -inf.
 * fp8 pools carry one scale per (page, kv head), k_scales / v_scales
 * [num_pages, heads_kv], and then need scale_block 0 or page_size. */
static int32_t decode_paged(const neptune_decode_desc *d, const neptune_paged_kv_desc *pk,
                            const void *q, const void *k_pages, const void *v_pages,
                            const float *k_scales, const float *v_scales,
                            const int32_t *block_table, const int32_t *seq_lens, void *o,
                            float *lse) {
  if (!d || !pk || !q || !k_pages || !v_pages || !block_table || !seq_lens || !o)
    return NEPTUNE_ERR_INVALID_ARGUMENT;
  const int fp8 = d->kv_dtype == NEPTUNE_DTYPE_FP8_E4M3;
  if (d->heads_q <= 0 || d->heads_kv <= 0 || d->heads_q % d->heads_kv ||
      d->head_dim <= 0 || (!fp8 && d->kv_dtype != NEPTUNE_DTYPE_BF16))
    return NEPTUNE_ERR_INVALID_ARGUMENT;
  if (pk->num_pages <= 0 || pk->page_size <= 0 || pk->max_pages <= 0 ||
      pk->max_pages * pk->page_size < d->seq_kv)
    return NEPTUNE_ERR_INVALID_ARGUMENT;
  if (fp8 && (!k_scales || !v_scales ||
              (d->scale_block != 0 && d->scale_block != pk->page_size)))
    return NEPTUNE_ERR_INVALID_ARGUMENT;
  int64_t S, chunk;
  int st = neptune_cpu_decode_layout(d, &S, &chunk);
  if (st) return st;
  const int64_t B = d->batch, Hq = d->heads_q, Hk = d->heads_kv,
                L = d->seq_kv, D = d->head_dim, group = Hq / Hk;
  const float scale2 = default_scale_log2(d->scale_log2, D);

#pragma omp parallel for collapse(2) schedule(dynamic, 1)
  for (int64_t b = 0; b < B; ++b)
    for (int64_t h = 0; h < Hq; ++h) {
      int64_t hk = h / group;
      int64_t len = seq_lens[b] < 0 ? 0 : (seq_lens[b] > L ? L : seq_lens[b]);
      float *buf = (float *)malloc(sizeof(float) * (size_t)(D * (S + 1) + 2 * S));
      float *qrow = buf, *ot = buf + D, *ms = ot + S * D, *ls = ms + S;
      for (int64_t dd = 0; dd < D; ++dd)
        qrow[dd] = load_elem(q, (b * Hq + h) * D + dd, d->q_dtype);
      kv_view kv = {.k = k_pages, .v = v_pages, .dt = d->kv_dtype,
                    .kbase = hk * pk->k_stride[1], .vbase = hk * pk->v_stride[1],
                    .kstride = pk->k_stride[2], .vstride = pk->v_stride[2], .kdstride = 1,
                    .kscale = fp8 ? k_scales + hk : NULL, .vscale = fp8 ? v_scales + hk : NULL,
                    .scale_block = 1, .p_dtype = d->q_dtype,
                    .btab = block_table + b * pk->max_pages, .page_size = pk->page_size,
                    .num_pages = pk->num_pages, .kpage = pk->k_stride[0],
                    .vpage = pk->v_stride[0], .scale_page_stride = Hk};
      for (int64_t s = 0; s < S; ++s) {
        int64_t k0 = s * chunk, k1 = k0 + chunk < len ? k0 + chunk : len;
        htile_row(qrow, D, &kv, k0, k1, k1, scale2, ot + s * D, &ms[s], &ls[s]);
      }
      float M = -FLT_MAX;
      for (int64_t s = 0; s < S; ++s) M = ms[s] > M ? ms[s] : M;
      float Lsum = 0.0f;
      for (int64_t s = 0; s < S; ++s) Lsum += exp2f(ms[s] - M) * ls[s];
      for (int64_t dd = 0; dd < D; ++dd) {
        float acc = 0.0f;
        for (int64_t s = 0; s < S; ++s) acc += exp2f(ms[s] - M) * ot[s * D + dd];
        store_elem(o, (b * Hq + h) * D + dd, d->q_dtype, Lsum > 0.0f ? acc / Lsum : 0.0f);
      }
      if (lse) lse[b * Hq + h] = Lsum > 0.0f ? (M + log2f(Lsum)) * (float)LN2 : -INFINITY;
      free(buf);
    }
  return NEPTUNE_OK;
}

int32_t neptune_cpu_decode_paged(const neptune_decode_desc *d,
                                 const neptune_paged_kv_desc *pk, const void *q,
                                 const void *k_pages, const void *v_pages,
                                 const int32_t *block_table,
                                 const int32_t *seq_lens, void *o, float *lse) {
  if (d && d->kv_dtype != NEPTUNE_DTYPE_BF16) return NEPTUNE_ERR_INVALID_ARGUMENT;
  return decode_paged(d, pk, q, k_pages, v_pages, NULL, NULL, block_table, seq_lens, o, lse);
}

int32_t neptune_cpu_decode_paged_fp8(const neptune_decode_desc *d,
                                     const neptune_paged_kv_desc *pk, const void *q,
                                     const uint8_t *k_pages, const uint8_t *v_pages,
                                     const float *k_scales, const float *v_scales,
                                     const int32_t *block_table, const int32_t *seq_lens,
                                     void *o, float *lse) {
  if (d && d->kv_dtype != NEPTUNE_DTYPE_FP8_E4M3) return NEPTUNE_ERR_INVALID_ARGUMENT;
  return decode_paged(d, pk, q, k_pages, v_pages, k_scales, v_scales, block_table, seq_lens,
                      o, lse);
}

int32_t neptune_cpu_kv_quantize_fp8(int64_t batch, int64_t heads_kv,
                                    int64_t seq_kv, int64_t head_dim,
                                    int64_t scale_block, const void *src,
                                    uint8_t *codes, float *scales) {
  if (!src || !codes || !scales || batch <= 0 || heads_kv <= 0 ||
      seq_kv <= 0 || head_dim <= 0)
    return NEPTUNE_ERR_INVALID_ARGUMENT;
  const int64_t sb = scale_block > 0 ? scale_block : 64;
  const int64_t nsb = cdiv(seq_kv, sb);
#pragma omp parallel for collapse(3)
  for (int64_t b = 0; b < batch; ++b)
    for (int64_t h = 0; h < heads_kv; ++h)
      for (int64_t blk = 0; blk < nsb; ++blk) {
        int64_t t0 = blk * sb, t1 = t0 + sb < seq_kv ? t0 + sb : seq_kv;
        int64_t base = (b * heads_kv + h) * seq_kv * head_dim;
        float amax = 0.0f;
        for (int64_t i = t0 * head_dim; i < t1 * head_dim; ++i) {
          float a = fabsf(load_elem(src, base + i, NEPTUNE_DTYPE_BF16));
          if (a > amax) amax = a;
        }
        float inv = amax > 0.0f ? 448.0f / amax : 0.0f;
        scales[(b * heads_kv + h) * nsb + blk] = amax > 0.0f ? amax / 448.0f : 0.0f;
        for (int64_t i = t0 * head_dim; i < t1 * head_dim; ++i)
          codes[base + i] =
              amax > 0.0f
                  ? neptune_cpu_f32_to_e4m3(
                        load_elem(src, base + i, NEPTUNE_DTYPE_BF16) * inv)
                  : 0;
      }
  return NEPTUNE_OK;
}

/* ----------------------------------------------------------------- scan */

/* Mamba-1 selective scan, sequential fp64 (Gu & Dao 2023, Alg. 2 with the
 * zero-order-hold simplification B_bar = delta * B used by mamba_ssm's
 * selective_scan_ref): x <- exp(delta A) x + delta B u, y = C.x + D u,
 * y *= silu(z). softplus uses torch's threshold 20. */
int32_t neptune_cpu_selective_scan_fwd(const neptune_scan_desc *d,
                                       const void *u, const void *delta_raw,
                                       const float *A, const void *Bm,
                                       const void *Cm, const float *Dv,
                                       const void *z, const float *delta_bias,
                                       void *y, double *y64) {
  if (!d || !u || !delta_raw || !A || !Bm || !Cm || (!y && !y64))
    return NEPTUNE_ERR_INVALID_ARGUMENT;
  if (d->batch <= 0 || d->dim <= 0 || d->seq_len <= 0 || d->d_state <= 0 ||
      d->d_state > 256)
    return NEPTUNE_ERR_INVALID_ARGUMENT;
  const int64_t Bn = d->batch, Dn = d->dim, L = d->seq_len, N = d->d_state;
  const int32_t dt = d->io_dtype;
#pragma omp parallel for collapse(2) schedule(static)
  for (int64_t b = 0; b < Bn; ++b)
    for (int64_t c = 0; c < Dn; ++c) {
      double x[256];
      for (int64_t n = 0; n < N; ++n) x[n] = 0.0;
      const int64_t row = (b * Dn + c) * L;
      for (int64_t l = 0; l < L; ++l) {
        double dr = (double)load_elem(delta_raw, row + l, dt) +
                    (delta_bias ? (double)delta_bias[c] : 0.0);
        double dl = d->delta_softplus ? (dr > 20.0 ? dr : log1p(exp(dr))) : dr;
        double uu = (double)load_elem(u, row + l, dt);
        double acc = 0.0;
        for (int64_t n = 0; n < N; ++n) {
          double bb = (double)load_elem(Bm, (b * N + n) * L + l, dt);
          double cc = (double)load_elem(Cm, (b * N + n) * L + l, dt);
          x[n] = exp(dl * (double)A[c * N + n]) * x[n] + dl * bb * uu;
          acc += cc * x[n];
        }
        if (Dv) acc += (double)Dv[c] * uu;
        if (z) {
          double zz = (double)load_elem(z, row + l, dt);
          acc *= zz / (1.0 + exp(-zz));
        }
        if (y64) y64[row + l] = acc;
        if (y) store_elem(y, row + l, dt, (float)acc);
      }
    }
  return NEPTUNE_OK;
}
