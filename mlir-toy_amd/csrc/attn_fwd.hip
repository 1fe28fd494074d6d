// attn_fwd.hip — the HTile flash-attention tile program on gfx950.
//
// Semantics: tests/data/flash_attention_htile.mlir:26-143 (one program per
// (128-row query block, head, batch); K/V streamed in 64-key blocks; fp32
// online softmax in the exp2 domain; P rounded to the 16-bit input type
// before P.V; O = acc / l rounded on store). Additions the reference lacks:
// causal masking (bottom-right aligned), per-row logsumexp, grouped KV heads,
// strided tensors and ragged sequence lengths.
//
// MFMA formulation (16-bit inputs, v_mfma_f32_32x32x16_{bf16,f16}): each of
// the 4 waves owns 32 query rows and computes the transposed products
//   S^T = K · Q^T      A = K tile rows from LDS, B = Q^T held in VGPRs
//   O^T = V^T · P^T    A = V^T from LDS,        B = P^T straight from S^T
// so every lane holds one query row (lane % 32) in both accumulators: the
// row max/sum are in-lane reductions plus one exchange with lane ^ 32, and
// the rescale of O uses one per-lane factor. The K^T read order of the
// HTile pass (dimension_order = [1,0], lib/HTile/HTilePasses.cpp:122-140)
// is realised by the A-operand read pattern; no transpose is materialised.
// V is transposed while it is written to LDS, with keys permuted within each
// 16-key chunk so that the 8 keys a lane feeds to P.V (which come from the
// 32x32 accumulator layout of S^T) are contiguous: key 8a+4g+b of a chunk is
// stored at position 8g+4a+b.
// K/V tiles are double-buffered in LDS (the htile.pipeline_stages = 2 hint,
// HTile:128): the next tile's global loads are in flight while the current
// tile is consumed, and one barrier per key block separates the phases.
#include "device_common.h"
#include "kernels.h"
#include "attn_args.h"

namespace neptune {
namespace {

constexpr int BM = 128;  // query rows per work-group (HTile %c128)
constexpr int BN = 64;   // keys per block (HTile %c64)
constexpr int NTHR = 256;


__device__ inline uint32_t perm_b32(uint32_t hi, uint32_t lo, uint32_t sel) {
  return __builtin_amdgcn_perm(hi, lo, sel);
}

template <class E, int D, bool CAUSAL>
__global__ __launch_bounds__(NTHR, 2) void attn_fwd_mfma(AttnArgs a) {
  constexpr int KP = D + 8;          // K row pitch in LDS (elements)
  constexpr int VP = BN + 8;         // V^T row pitch in LDS (elements)
  constexpr int KTILE = BN * KP;
  constexpr int VTILE = D * VP;
  constexpr int NQS = D / 16;        // MFMA k-steps over head_dim
  constexpr int NDB = D / 32;        // 32-wide head_dim blocks of O^T
  constexpr int CPR = D / 8;         // 16-byte chunks per row
  constexpr int NKL = BN * CPR / NTHR;
  constexpr int VUN = (BN / 4) * CPR;  // (4 keys x 8 dims) V units per tile
  constexpr int NVL = (VUN + NTHR - 1) / NTHR;
  typedef typename E::vec8 V8;

  __shared__ __attribute__((aligned(16))) uint16_t smem[2 * (KTILE + VTILE)];

  const int tid = threadIdx.x;
  const int w = tid >> 6, l = tid & 63, lq = l & 31, g = l >> 5;
  const int id = blockIdx.x;
  // Heaviest causal query blocks first; blocks of one (batch, head) share a
  // residue mod 8 and hence an XCD (and its L2) whenever BH % 8 == 0.
  const int qb = CAUSAL ? a.nqb - 1 - id / a.BH : id / a.BH;
  const int bh = id % a.BH;
  const int b = bh / a.Hq, h = bh % a.Hq, hk = h / a.group;
  const uint16_t *qp = (const uint16_t *)a.q + b * a.qs0 + h * a.qs1;
  const uint16_t *kp = (const uint16_t *)a.k + b * a.ks0 + hk * a.ks1;
  const uint16_t *vp = (const uint16_t *)a.v + b * a.vs0 + hk * a.vs1;

  const int row0 = qb * BM + w * 32;
  const int row = row0 + lq;

  u32x4 qf[NQS];
#pragma unroll
  for (int s = 0; s < NQS; ++s)
    qf[s] = row < a.Sq ? *(const u32x4 *)(qp + row * a.qs2 + 16 * s + 8 * g)
                       : u32x4{0, 0, 0, 0};

  int nkb = (a.Sk + BN - 1) / BN;
  if (CAUSAL) {
    int last = qb * BM + BM - 1 + a.off;
    int lim = last < 0 ? 0 : last / BN + 1;
    nkb = nkb < lim ? nkb : lim;
  }

  u32x4 kreg[NKL];
  u32x4 vreg[NVL][4];

  auto load_tile = [&](int jb) {
    const int key0 = jb * BN;
#pragma unroll
    for (int i = 0; i < NKL; ++i) {
      int c = tid + i * NTHR, r = c / CPR, c8 = c % CPR, key = key0 + r;
      kreg[i] = key < a.Sk ? *(const u32x4 *)(kp + key * a.ks2 + 8 * c8)
                           : u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int i = 0; i < NVL; ++i) {
      int u = tid + i * NTHR;
      if (u < VUN) {
        int kq = u / CPR, dc = u % CPR;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          int key = key0 + 4 * kq + t;
          vreg[i][t] = key < a.Sk ? *(const u32x4 *)(vp + key * a.vs2 + 8 * dc)
                                  : u32x4{0, 0, 0, 0};
        }
      }
    }
  };

  auto store_tile = [&](int buf) {
    uint16_t *Ks = smem + buf * (KTILE + VTILE);
    uint16_t *Vt = Ks + KTILE;
#pragma unroll
    for (int i = 0; i < NKL; ++i) {
      int c = tid + i * NTHR, r = c / CPR, c8 = c % CPR;
      *(u32x4 *)(Ks + r * KP + 8 * c8) = kreg[i];
    }
#pragma unroll
    for (int i = 0; i < NVL; ++i) {
      int u = tid + i * NTHR;
      if (u < VUN) {
        int kq = u / CPR, dc = u % CPR;
        int pos = 16 * (kq >> 2) + 8 * (kq & 1) + 4 * ((kq >> 1) & 1);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;
          u32x2 val = {perm_b32(vreg[i][1][e >> 1], vreg[i][0][e >> 1], sel),
                       perm_b32(vreg[i][3][e >> 1], vreg[i][2][e >> 1], sel)};
          *(u32x2 *)(Vt + (8 * dc + e) * VP + pos) = val;
        }
      }
    }
  };

  f32x16 oacc[NDB];
#pragma unroll
  for (int nb = 0; nb < NDB; ++nb)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[nb][r] = 0.0f;
  float m = kNegFltMax, lsum = 0.0f;
  const float sc = a.scale2;

  if (nkb > 0) {
    load_tile(0);
    store_tile(0);
  }
  __syncthreads();

  for (int jb = 0; jb < nkb; ++jb) {
    const int buf = jb & 1;
    if (jb + 1 < nkb) load_tile(jb + 1);
    const uint16_t *Ks = smem + buf * (KTILE + VTILE);
    const uint16_t *Vt = Ks + KTILE;
    const int key0 = jb * BN;
    const bool active = !CAUSAL || key0 <= row0 + 31 + a.off;
    if (active) {
      f32x16 s[2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) s[kb][r] = 0.0f;
#pragma unroll
        for (int st = 0; st < NQS; ++st) {
          u32x4 A = *(const u32x4 *)(Ks + (32 * kb + lq) * KP + 16 * st + 8 * g);
          s[kb] = E::mfma32(as_vec8<V8>(A), as_vec8<V8>(qf[st]), s[kb]);
        }
      }
      const bool need_mask =
          (key0 + BN > a.Sk) || (CAUSAL && key0 + BN - 1 > row0 + a.off);
      if (need_mask) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            int key = key0 + 32 * kb + 8 * (r >> 2) + 4 * g + (r & 3);
            if (key >= a.Sk || (CAUSAL && key > row + a.off)) s[kb][r] = -INFINITY;
          }
      }
      float mx = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[kb][r]);
      mx = fmaxf(mx, swap_halves(mx));
      const float m_new = fmaxf(m, mx * sc);
      const float alpha = fast_exp2(m - m_new);
      const float nm = -m_new;
      float rs = 0.0f;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float p = fast_exp2(fmaf(s[kb][r], sc, nm));
          s[kb][r] = p;
          rs += p;
        }
      lsum = lsum * alpha + rs;
      m = m_new;
      if (__any(alpha != 1.0f)) {
#pragma unroll
        for (int nb = 0; nb < NDB; ++nb)
#pragma unroll
          for (int r = 0; r < 16; ++r) oacc[nb][r] *= alpha;
      }
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int kb = c >> 1, hh = c & 1;
        u32x4 pf;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          pf[i] = E::pack2(s[kb][8 * hh + 2 * i], s[kb][8 * hh + 2 * i + 1]);
#pragma unroll
        for (int nb = 0; nb < NDB; ++nb) {
          u32x4 A = *(const u32x4 *)(Vt + (32 * nb + lq) * VP + 16 * c + 8 * g);
          oacc[nb] = E::mfma32(as_vec8<V8>(A), as_vec8<V8>(pf), oacc[nb]);
        }
      }
    }
    if (jb + 1 < nkb) store_tile(buf ^ 1);
    __syncthreads();
  }

  const float ltot = lsum + swap_halves(lsum);
  if (row < a.Sq) {
    uint16_t *op = (uint16_t *)a.o + b * a.os0 + h * a.os1 + row * a.os2;
#pragma unroll
    for (int nb = 0; nb < NDB; ++nb)
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        float v4[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
          v4[i] = ltot > 0.0f ? oacc[nb][4 * rq + i] / ltot : 0.0f;
        u32x2 pk = {E::pack2(v4[0], v4[1]), E::pack2(v4[2], v4[3])};
        *(u32x2 *)(op + 32 * nb + 8 * rq + 4 * g) = pk;
      }
    if (g == 0 && a.lse)
      a.lse[((int64_t)b * a.Hq + h) * a.Sq + row] =
          ltot > 0.0f ? (m + log2f(ltot)) * kLn2 : -INFINITY;
  }
}

// sum / max over the 16 lanes of a row (DPP row rotations, no LDS): every
// lane of the row gets the result
template <int R>
__device__ inline float row_ror(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x120 + R, 0xf, 0xf, false));
}
__device__ inline float row_sum16(float v) {
  v += row_ror<8>(v);
  v += row_ror<4>(v);
  v += row_ror<2>(v);
  return v + row_ror<1>(v);
}
__device__ inline float row_max16(float v) {
  v = fmaxf(v, row_ror<8>(v));
  v = fmaxf(v, row_ror<4>(v));
  v = fmaxf(v, row_ror<2>(v));
  return fmaxf(v, row_ror<1>(v));
}

// fp32 path (config 1 and any F32 request): a 256-thread work-group per 16
// query rows, 16 lanes per row. K/V blocks of 64 keys are staged in LDS;
// lane k of a row takes keys k, k + 16, k + 32, k + 48 of each block and
// keeps its own online-softmax state (m, l, acc) over them, the HTile
// recurrence with no rounding of P (the input type is fp32). The 16 states
// of a row are merged at the end in the exp2 domain, M = max m_k,
// l = sum 2^(m_k - M) l_k, acc = sum 2^(m_k - M) acc_k (the flash-decoding
// combine), so a short sequence still spreads over many waves.
constexpr int F32_BM = 16;   // query rows per work-group
constexpr int F32_KS = 16;   // lanes per row, each taking every 16th key
constexpr int F32_NT = F32_BM * F32_KS;

template <int D, bool CAUSAL>
__global__ __launch_bounds__(F32_NT) void attn_fwd_f32(AttnArgs a) {
  // rows padded by 4 floats: the 16 lanes of a row read 16 different keys
  // at one head_dim offset, spread over the banks
  constexpr int DP = D + 4;
  __shared__ __attribute__((aligned(16))) float Ks[BN][DP];
  __shared__ __attribute__((aligned(16))) float Vs[BN][DP];
  const int t = threadIdx.x;
  const int rl = t / F32_KS, kl = t % F32_KS;
  const int id = blockIdx.x;
  const int qb = id / a.BH, bh = id % a.BH;
  const int b = bh / a.Hq, h = bh % a.Hq, hk = h / a.group;
  const float *qp = (const float *)a.q + b * a.qs0 + h * a.qs1;
  const float *kp = (const float *)a.k + b * a.ks0 + hk * a.ks1;
  const float *vp = (const float *)a.v + b * a.vs0 + hk * a.vs1;
  const int row = qb * F32_BM + rl;

  // rows past the end read the last row (never stored), so no load is
  // guarded and all of them issue before the first is waited for
  const int rowc = min(row, a.Sq - 1);
  float q[D], acc[D];
#pragma unroll
  for (int d = 0; d < D; ++d) {
    q[d] = qp[rowc * a.qs2 + d];
    acc[d] = 0.0f;
  }
  float m = kNegFltMax, lsum = 0.0f;
  int nkb = (a.Sk + BN - 1) / BN;
  if (CAUSAL) {
    int last = qb * F32_BM + F32_BM - 1 + a.off;
    int lim = last < 0 ? 0 : last / BN + 1;
    nkb = nkb < lim ? nkb : lim;
  }
  constexpr int KPL = BN / F32_KS;  // keys per lane and block
  for (int jb = 0; jb < nkb; ++jb) {
    const int key0 = jb * BN;
    __syncthreads();
    // a fixed trip count, unrolled, so every element's load issues before
    // the first one is waited for
    static_assert(BN * D % F32_NT == 0, "whole staging rounds");
    float kv[BN * D / F32_NT], vv[BN * D / F32_NT];
#pragma unroll
    for (int i = 0; i < BN * D / F32_NT; ++i) {
      const int e = t + i * F32_NT;
      // keys past the end read the last key: their scores are masked to
      // -inf, so their p is 0
      const int r = e / D, c = e % D, key = min(key0 + r, a.Sk - 1);
      kv[i] = kp[key * a.ks2 + c];
      vv[i] = vp[key * a.vs2 + c];
    }
#pragma unroll
    for (int i = 0; i < BN * D / F32_NT; ++i) {
      const int e = t + i * F32_NT;
      Ks[e / D][e % D] = kv[i];
      Vs[e / D][e % D] = vv[i];
    }
    __syncthreads();
    float s[KPL];
    float mx = -INFINITY;
#pragma unroll
    for (int jj = 0; jj < KPL; ++jj) {
      const int j = F32_KS * jj + kl;
      float dot = 0.0f;
#pragma unroll
      for (int d = 0; d < D; ++d) dot = fmaf(q[d], Ks[j][d], dot);
      const int key = key0 + j;
      float sv = dot * a.scale2;
      if (key >= a.Sk || (CAUSAL && key > row + a.off)) sv = -INFINITY;
      s[jj] = sv;
      mx = fmaxf(mx, sv);
    }
    const float m_new = fmaxf(m, mx);
    const float alpha = fast_exp2(m - m_new);
    float rs = 0.0f;
#pragma unroll
    for (int jj = 0; jj < KPL; ++jj) {
      s[jj] = fast_exp2(s[jj] - m_new);
      rs += s[jj];
    }
    lsum = lsum * alpha + rs;
    m = m_new;
#pragma unroll
    for (int d = 0; d < D; ++d) acc[d] *= alpha;
#pragma unroll
    for (int jj = 0; jj < KPL; ++jj) {
      const float pj = s[jj];
      const int j = F32_KS * jj + kl;
#pragma unroll
      for (int d = 0; d < D; ++d) acc[d] = fmaf(pj, Vs[j][d], acc[d]);
    }
  }
  // merge the 16 lane states of the row (lanes rl * 16 .. rl * 16 + 15 of
  // one wave): a lane that saw no visible key has m = -FLT_MAX and l = 0
  const float M = row_max16(m);
  const float wgt = fast_exp2(m - M);
  const float ltot = row_sum16(lsum * wgt);
#pragma unroll
  for (int d = 0; d < D; ++d) acc[d] = row_sum16(acc[d] * wgt);
  if (row < a.Sq && kl == 0) {
    // the correctly rounded quotient acc / l (HTile:130-143): q = acc * (1/l)
    // with the correctly rounded reciprocal, then one residual step
    // q + fma(-q, l, acc) * (1/l) (Markstein's correction)
    const float inv = ltot > 0.0f ? 1.0f / ltot : 0.0f;
    float *op = (float *)a.o + b * a.os0 + h * a.os1 + row * a.os2;
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const float q0 = acc[d] * inv;
      op[d] = __builtin_fmaf(__builtin_fmaf(-q0, ltot, acc[d]), inv, q0);
    }
    if (a.lse)
      a.lse[((int64_t)b * a.Hq + h) * a.Sq + row] =
          ltot > 0.0f ? (M + log2f(ltot)) * kLn2 : -INFINITY;
  }
}

template <class E, int D>
void launch_mfma(const AttnArgs &args, bool causal, int grid, hipStream_t s) {
  if (causal)
    hipLaunchKernelGGL((attn_fwd_mfma<E, D, true>), dim3(grid), dim3(NTHR), 0, s, args);
  else
    hipLaunchKernelGGL((attn_fwd_mfma<E, D, false>), dim3(grid), dim3(NTHR), 0, s, args);
}

template <int D>
void launch_f32(const AttnArgs &args, bool causal, int grid, hipStream_t s) {
  if (causal)
    hipLaunchKernelGGL((attn_fwd_f32<D, true>), dim3(grid), dim3(F32_NT), 0, s, args);
  else
    hipLaunchKernelGGL((attn_fwd_f32<D, false>), dim3(grid), dim3(F32_NT), 0, s, args);
}

}  // namespace

bool attn_supported(const AttnLaunch &a, const char **why) {
  if (a.dtype == 0) {  // F32
    if (a.head_dim != 32 && a.head_dim != 64 && a.head_dim != 128) {
      *why = "fp32 attention supports head_dim 32, 64 or 128";
      return false;
    }
  } else if (a.head_dim != 64 && a.head_dim != 128) {
    *why = "16-bit attention supports head_dim 64 or 128";
    return false;
  }
  const bool d128 = a.dtype != 0 && a.head_dim == 128;
  if (a.stages != 2 && !d128) {
    *why = "pipeline_stages other than 2 applies to the head_dim-128 16-bit kernel";
    return false;
  }
  if (a.k_dim_order != 0) {
    if (!d128) {
      *why = "k_dim_order 1 applies to the head_dim-128 16-bit kernel";
      return false;
    }
    if (a.seq_kv % 8) {
      *why = "k_dim_order 1 needs seq_kv to be a multiple of 8";
      return false;
    }
  }
  if (a.seq_q > (int64_t)1 << 30 || a.seq_kv > (int64_t)1 << 30 ||
      a.batch * a.heads_q > (int64_t)1 << 24) {
    *why = "sequence or batch*heads too large for one launch";
    return false;
  }
  // The head_dim-128 kernel addresses a full K or V tile from a per-block
  // base plus per-lane 32-bit byte offsets: up to row 63 of a 64-key tile
  // (row 127 of a 128-row head_dim-major K tile) and 256 bytes into it.
  if (d128) {
    const int64_t klast = a.k_dim_order ? 127 : 63;
    if (klast * a.ks[2] * 2 + 256 > (int64_t)0xffffffff || 63 * a.vs[2] * 2 + 256 > (int64_t)0xffffffff) {
      *why = "K or V row stride too large: a 64-key tile must span less than 4 GiB";
      return false;
    }
  }
  // a dispatch covers at most 2^32 - 1 work-items: one 256-thread work-group
  // per 128 query rows and (batch, head) (the most any 16-bit path launches),
  // one 256-thread work-group per 16 rows for fp32
  const int64_t rows = a.dtype == 0 ? F32_BM : BM, thr = a.dtype == 0 ? F32_NT : NTHR;
  if ((a.seq_q + rows - 1) / rows * (a.batch * a.heads_q) * thr > (int64_t)0xffffffff) {
    *why = "batch*heads*seq_q too large for one launch";
    return false;
  }
  return true;
}

hipError_t launch_attn_fwd(const AttnLaunch &L, hipStream_t s) {
  AttnArgs a;
  a.q = L.q;
  a.k = L.k;
  a.v = L.v;
  a.o = L.o;
  a.lse = L.lse;
  a.qs0 = L.qs[0]; a.qs1 = L.qs[1]; a.qs2 = L.qs[2];
  a.ks0 = L.ks[0]; a.ks1 = L.ks[1]; a.ks2 = L.ks[2];
  a.vs0 = L.vs[0]; a.vs1 = L.vs[1]; a.vs2 = L.vs[2];
  a.os0 = L.os[0]; a.os1 = L.os[1]; a.os2 = L.os[2];
  a.Hq = (int32_t)L.heads_q;
  a.group = (int32_t)(L.heads_q / L.heads_kv);
  a.Sq = (int32_t)L.seq_q;
  a.Sk = (int32_t)L.seq_kv;
  a.BH = (int32_t)(L.batch * L.heads_q);
  a.off = (int32_t)(L.seq_kv - L.seq_q);
  a.scale2 = L.scale_log2;
  const bool causal = L.causal != 0;
  if (L.dtype == 0) {
    a.nqb = (int32_t)((L.seq_q + F32_BM - 1) / F32_BM);
    int grid = a.nqb * a.BH;
    switch (L.head_dim) {
      case 32: launch_f32<32>(a, causal, grid, s); break;
      case 64: launch_f32<64>(a, causal, grid, s); break;
      default: launch_f32<128>(a, causal, grid, s); break;
    }
  } else {
    a.nqb = (int32_t)((L.seq_q + BM - 1) / BM);
    int grid = a.nqb * a.BH;
    const bool bf16 = L.dtype == 2;
    if (L.head_dim == 64) {
      if (bf16) launch_mfma<Bf16Tag, 64>(a, causal, grid, s);
      else launch_mfma<F16Tag, 64>(a, causal, grid, s);
    } else {
      return launch_attn_d128(a, L.dtype, causal, L.stages, L.k_dim_order != 0, s);
    }
  }
  return hipGetLastError();
}

}  // namespace neptune
