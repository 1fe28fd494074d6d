// attn_fwd_pp.hip — head_dim-128, 16-bit HTile attention forward for gfx950,
// two wave groups in ping-pong.
//
// Semantics are those of attn_fwd.hip (the HTile tile program,
// tests/data/flash_attention_htile.mlir:26-143, plus causal mask, LSE, GQA,
// strides and ragged lengths); the MFMA formulation and the LDS tile layout
// are those of attn_fwd_d128.hip:
//   S^T = K . Q^T   (A = K rows from LDS, B = Q^T in VGPRs)
//   O^T = V^T . P^T (A = V^T via ds_read_b64_tr_b16, B = P^T)
// with v_mfma_f32_32x32x16, one query row per lane.
//
// Work-group: 512 threads = 8 waves on the CU's 4 SIMDs, 256 query rows.
// Waves 0-3 (group A, rows 0-127) and waves 4-7 (group B, rows 128-255)
// share each SIMD. Every key block is split into two phases separated by a
// work-group barrier; in each phase one group runs its MFMA work (QK^T of
// this block, PV of the previous one) while the other runs its softmax
// (VALU and transcendental work), so the SIMD's matrix core and its vector
// ALU are busy at the same time:
//   phase 1:  A: QK(j), PV(j-1)      B: softmax(j-1)
//   phase 2:  A: softmax(j)          B: QK(j), PV(j-1)
// K and V tiles (64 keys) are shared by all 8 waves and stream HBM -> LDS
// with global_load_lds_dwordx4 through NS slots each, NS-1 blocks ahead.
#include "attn_args.h"
#include "device_common.h"
#include "kernels.h"

namespace neptune {
namespace {

constexpr int BM = 256;             // query rows per work-group
constexpr int BN = 64;              // keys per block
constexpr int NT = 512;             // threads per work-group
constexpr int TILE = BN * 128 * 2;  // bytes per K or V tile (16 KiB)
constexpr float kSlack = 8.0f;      // lazy-rescale threshold (log2 units)

typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) v4i16 lds_v4i16;

__device__ inline lds_void *as_lds(const uint8_t *p) { return (lds_void *)(p); }

// Wave w (0..7) copies rows [8w, 8w+8) of a 64 x 128 tile (two 1 KiB chunks)
// into LDS; unit u of row r lands at u ^ (r & 15) for K, u ^ 4(r & 3) for V.
template <bool IS_V>
__device__ inline void tile_to_lds(const uint16_t *src, int64_t stride, int key0, int Sk,
                                   const uint8_t *tile, int w, int lane) {
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const int q = 2 * w + c;
    const int r = 4 * q + (lane >> 4);
    const int sw = IS_V ? ((r & 3) << 2) : (r & 15);
    const int unit = (lane & 15) ^ sw;
    const int key = min(key0 + r, Sk - 1);
    __builtin_amdgcn_global_load_lds(src + (int64_t)key * stride + unit * 8,
                                     as_lds(tile + q * 1024), 16, 0, 0);
  }
}

__device__ inline float pair_max(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ inline float pair_sum(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Phase boundary: no memory ordering is needed (tiles are stable within a
// key block), only alignment of the two groups; nothing moves across it.
__device__ inline void phase_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
}

__device__ inline void map_block(const AttnArgs &a, int id, bool causal, int *qb, int *bh) {
  if ((a.BH & 7) == 0) {
    // id % 8 is the XCD the work-group is dispatched to: each XCD walks its
    // own heads one at a time, query blocks heaviest first.
    const int x = id & 7, k = id >> 3;
    const int t = k / a.nqb, r = k - t * a.nqb;
    *bh = x + 8 * t;
    *qb = causal ? a.nqb - 1 - r : r;
  } else {
    *bh = id % a.BH;
    *qb = causal ? a.nqb - 1 - id / a.BH : id / a.BH;
  }
}

template <class E, bool CAUSAL, int NS>
__global__ __launch_bounds__(NT, 1) void attn_fwd_pp(AttnArgs a) {
  typedef typename E::vec8 V8;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];  // K[NS] V[NS]
  const uint8_t *const kt0 = smem;
  const uint8_t *const vt0 = smem + NS * TILE;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = w >> 2;
  const int lq = lane & 31, g = lane >> 5;

  int qb, bh;
  map_block(a, blockIdx.x, CAUSAL, &qb, &bh);
  const int b = bh / a.Hq, h = bh - b * a.Hq, hk = h / a.group;
  const uint16_t *qp = (const uint16_t *)a.q + b * a.qs0 + h * a.qs1;
  const uint16_t *kp = (const uint16_t *)a.k + b * a.ks0 + hk * a.ks1;
  const uint16_t *vp = (const uint16_t *)a.v + b * a.vs0 + hk * a.vs1;

  const int row0 = qb * BM + 128 * grp + 32 * (w & 3);
  const int row = row0 + lq;

  int nkb = (a.Sk + BN - 1) / BN;  // key blocks of the work-group
  int nkw = nkb;                    // key blocks this wave computes
  if (CAUSAL) {
    const int last_wg = qb * BM + BM - 1 + a.off;
    nkb = min(nkb, last_wg < 0 ? 0 : last_wg / BN + 1);
    const int last_w = row0 + 31 + a.off;
    nkw = min(nkb, last_w < 0 ? 0 : last_w / BN + 1);
  }

  auto issue_k = [&](int t) {
    if (t < nkb) tile_to_lds<false>(kp, a.ks2, t * BN, a.Sk, kt0 + (t % NS) * TILE, w, lane);
  };
  auto issue_v = [&](int t) {
    if (t < nkb) tile_to_lds<true>(vp, a.vs2, t * BN, a.Sk, vt0 + (t % NS) * TILE, w, lane);
  };
#pragma unroll
  for (int t = 0; t < NS - 1; ++t) issue_k(t);
#pragma unroll
  for (int t = 0; t < NS - 2; ++t) issue_v(t);

  u32x4 qf[8];
#pragma unroll
  for (int st = 0; st < 8; ++st)
    qf[st] = row < a.Sq ? *(const u32x4 *)(qp + row * a.qs2 + 16 * st + 8 * g)
                        : u32x4{0, 0, 0, 0};

  int ka[8];  // K A-operand: row lq (+32 kb), logical unit 2 st + g
#pragma unroll
  for (int st = 0; st < 8; ++st) ka[st] = lq * 256 + (((2 * st + g) ^ (lq & 15)) << 4);
  int va[4];  // V^T transpose reads: rows 4 g + i (+16 c + 8 t), columns 32 nb + 16 dh + 4 q
  {
    const int s16 = lane & 15, i = s16 >> 2, q = s16 & 3, dh = (lane >> 4) & 1;
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) va[nb] = (4 * g + i) * 256 + 64 * (nb ^ i) + 32 * dh + 8 * q;
  }

  f32x16 o[4];
#pragma unroll
  for (int nb = 0; nb < 4; ++nb)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[nb][r] = 0.0f;
  f32x16 s[2];
  u32x4 pf[4];
  float m = kNegFltMax, lsum = 0.0f;
  const float sc = a.scale2;
  const f32x16 zero16 = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};

  // QK^T of block j, then PV of block j-1 (MFMA phase)
  auto mfma_phase = [&](int j) {
    if (j < nkw) {
      const uint8_t *kt = kt0 + (j % NS) * TILE;
#pragma unroll
      for (int st = 0; st < 8; ++st)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
          const u32x4 A = *(const u32x4 *)(kt + kb * 8192 + ka[st]);
          s[kb] = E::mfma32(as_vec8<V8>(A), as_vec8<V8>(qf[st]), st == 0 ? zero16 : s[kb]);
        }
      // operand reads run two MFMAs ahead (bounds the live registers)
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
#pragma unroll
      for (int i = 0; i < 14; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
    }
    if (j >= 1 && j - 1 < nkw) {
      const uint8_t *vt = vt0 + ((j - 1) % NS) * TILE;
#pragma unroll
      for (int step = 0; step < 16; ++step) {
        const int c = step >> 2, nb = step & 3;
        const v4i16 t0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (lds_v4i16 *)as_lds(vt + (16 * c) * 256 + va[nb]));
        const v4i16 t1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (lds_v4i16 *)as_lds(vt + (16 * c + 8) * 256 + va[nb]));
        const u32x2 a0 = __builtin_bit_cast(u32x2, t0), a1 = __builtin_bit_cast(u32x2, t1);
        const u32x4 A = {a0[0], a0[1], a1[0], a1[1]};
        o[nb] = E::mfma32(as_vec8<V8>(A), as_vec8<V8>(pf[c]), o[nb]);
      }
      __builtin_amdgcn_sched_group_barrier(0x100, 4, 1);
#pragma unroll
      for (int i = 0; i < 14; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 1);
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 1);
    }
  };

  // mask, running max, exp2, row sum and 16-bit P of block j (VALU phase)
  auto softmax_phase = [&](int j) {
    if (j < 0 || j >= nkw) return;
    const int key0 = j * BN;
    const bool need_mask = (key0 + BN > a.Sk) || (CAUSAL && key0 + BN - 1 > row0 + a.off);
    if (need_mask) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = key0 + 32 * kb + 8 * (r >> 2) + 4 * g + (r & 3);
          if (key >= a.Sk || (CAUSAL && key > row + a.off)) s[kb][r] = -INFINITY;
        }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[kb][r]);
    mx = pair_max(mx);
    // Lazy rescaling: m only moves when a row's block max exceeds it by more
    // than kSlack; in between p = 2^(s - m) <= 2^kSlack, which fp32 sums hold
    // exactly as well and whose 16-bit rounding is relative, so results
    // differ from a rescale at every block by rounding only.
    const float m_blk = mx * sc;
    if (__any(m_blk > m + kSlack)) {
      const float m_new = fmaxf(m, m_blk);
      const float alpha = fast_exp2(m - m_new);
      lsum *= alpha;
#pragma unroll
      for (int nb = 0; nb < 4; ++nb)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[nb][r] *= alpha;
      m = m_new;
    }
    const float nm = -m;
    float rs = 0.0f;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int kb = c >> 1, hh = c & 1;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float p0 = fast_exp2(fmaf(s[kb][8 * hh + 2 * i], sc, nm));
        const float p1 = fast_exp2(fmaf(s[kb][8 * hh + 2 * i + 1], sc, nm));
        rs += p0;
        rs += p1;
        pf[c][i] = E::pack2(p0, p1);
      }
    }
    lsum += rs;
  };

  __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
  __syncthreads();

  // end of key block j: K_{j+1} and V_j (issued one block earlier) must have
  // landed; the loads issued for this block may stay in flight
  auto end_block = [&](int j) {
    if (j - 1 + NS < nkb)
      __builtin_amdgcn_s_waitcnt(0x0f74);  // vmcnt(4): K and V of this block
    else if (j - 2 + NS < nkb)
      __builtin_amdgcn_s_waitcnt(0x0f72);  // vmcnt(2): V of this block
    else
      __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
    __syncthreads();
  };
  // Each group runs its own loop (straight-line bodies keep the register
  // assignment of the accumulators fixed); both pass the same barriers.
  // Slots freed by block j-1 take blocks j-1+NS (K) and j-2+NS (V).
  if (grp == 0) {
    for (int j = 0; j <= nkb; ++j) {
      issue_k(j - 1 + NS);
      issue_v(j - 2 + NS);
      mfma_phase(j);
      phase_barrier();
      softmax_phase(j);
      end_block(j);
    }
  } else {
    for (int j = 0; j <= nkb; ++j) {
      issue_k(j - 1 + NS);
      issue_v(j - 2 + NS);
      softmax_phase(j - 1);
      phase_barrier();
      mfma_phase(j);
      end_block(j);
    }
  }

  const float ltot = pair_sum(lsum);
  if (row < a.Sq) {
    const float inv = ltot > 0.0f ? 1.0f / ltot : 0.0f;
    uint16_t *op = (uint16_t *)a.o + b * a.os0 + h * a.os1 + row * a.os2;
#pragma unroll
    for (int nb = 0; nb < 4; ++nb)
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        const u32x2 pk = {E::pack2(o[nb][4 * rq] * inv, o[nb][4 * rq + 1] * inv),
                          E::pack2(o[nb][4 * rq + 2] * inv, o[nb][4 * rq + 3] * inv)};
        *(u32x2 *)(op + 32 * nb + 8 * rq + 4 * g) = pk;
      }
    if (g == 0 && a.lse)
      a.lse[((int64_t)b * a.Hq + h) * a.Sq + row] =
          ltot > 0.0f ? (m + log2f(ltot)) * kLn2 : -INFINITY;
  }
}

template <class E, bool CAUSAL, int NS>
hipError_t launch_t(AttnArgs a, hipStream_t s) {
  const size_t lds = 2 * NS * TILE;
  static bool attr_set = false;  // benign race: the attribute is idempotent
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute((const void *)attn_fwd_pp<E, CAUSAL, NS>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  a.nqb = (a.Sq + BM - 1) / BM;
  hipLaunchKernelGGL((attn_fwd_pp<E, CAUSAL, NS>), dim3((unsigned)(a.nqb * a.BH)), dim3(NT), lds,
                     s, a);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_attn_pp(const AttnArgs &a, int32_t dtype, bool causal, hipStream_t s) {
  constexpr int NS = 3;
  if (dtype == 2)
    return causal ? launch_t<Bf16Tag, true, NS>(a, s) : launch_t<Bf16Tag, false, NS>(a, s);
  return causal ? launch_t<F16Tag, true, NS>(a, s) : launch_t<F16Tag, false, NS>(a, s);
}

}  // namespace neptune
