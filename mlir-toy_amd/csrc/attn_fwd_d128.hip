// attn_fwd_d128.hip — head_dim-128, 16-bit HTile attention forward for gfx950.
//
// Semantics are those of the generic kernel in attn_fwd.hip (the HTile tile
// program, tests/data/flash_attention_htile.mlir:26-143, plus causal mask,
// LSE, GQA, strides and ragged lengths); this file is its fast path for
// head_dim 128 in bf16 or f16.
//
// Work-group: 256 threads = 4 waves, 128 query rows (32 per wave), 64-key
// blocks; two work-groups per CU. Each wave forms the transposed products
//   S^T = K . Q^T   (A = K rows from LDS, B = Q^T in VGPRs)
//   O^T = V^T . P^T (A = V^T from LDS via ds_read_b64_tr_b16, B = P^T)
// with v_mfma_f32_32x32x16, so a lane owns one query row in both
// accumulators (row max/sum are in-lane plus one v_permlane32_swap).
//
// Data movement: K and V tiles go HBM -> LDS with global_load_lds_dwordx4
// (no VGPR staging), double-buffered per operand. Key block j+1's QK^T is
// issued in the same MFMA stream as block j's PV, so the next scores are
// ready when the softmax of the next iteration starts, and the loads for
// blocks j+2 (K) and j+1 (V) are in flight during iteration j.
//
// LDS tiles are 64 rows x 256 B of 16-byte units, XOR-swizzled per row so
// that both the DMA writes (16 lanes = one row) and the MFMA operand reads
// are bank-conflict free:
//   K: unit u of row r at u ^ (r & 15)   (reads: 32 rows, one unit each)
//   V: unit u of row r at u ^ 4(r & 3)   (transpose reads: 4 rows x 64 B)
//
// Work-group order: with batch*heads a multiple of 8, work-group id % 8 is
// the XCD it is dispatched to; each XCD walks its own heads one at a time,
// causal query blocks heaviest first, so the K/V of the heads in flight on
// an XCD stay in that XCD's L2.
#include "attn_args.h"
#include "device_common.h"
#include "kernels.h"

namespace neptune {
namespace {

constexpr int BM = 128;
constexpr int BN = 64;
constexpr int HD = 128;
constexpr int NT = 256;
constexpr int TILE = BN * HD * 2;  // bytes per K or V tile (16 KiB)
constexpr float kSlack = 8.0f;     // lazy-rescale threshold (log2 units)

typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) v4i16 lds_v4i16;

__device__ inline lds_void *as_lds(const uint8_t *p) { return (lds_void *)(p); }

// Wave w copies rows [16w, 16w+16) of a 64 x 128 tile (four 1 KiB chunks of
// four rows) straight into LDS. Rows past the end of the sequence re-read
// the last row: their scores are masked, so their P is exactly 0.
template <bool IS_V>
__device__ inline void tile_to_lds(const uint16_t *src, int64_t stride, int key0, int Sk,
                                   const uint8_t *tile, int w, int lane) {
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int q = 4 * w + c;
    const int r = 4 * q + (lane >> 4);
    const int sw = IS_V ? ((r & 3) << 2) : (r & 15);
    const int unit = (lane & 15) ^ sw;
    const int key = min(key0 + r, Sk - 1);
    __builtin_amdgcn_global_load_lds(src + (int64_t)key * stride + unit * 8,
                                     as_lds(tile + q * 1024), 16, 0, 0);
  }
}

__device__ inline void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0f70); }  // vmcnt(0)

// (lane, lane ^ 32) pair reductions through v_permlane32_swap
__device__ inline float pair_max(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ inline float pair_sum(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ inline void map_block(const AttnArgs &a, int id, bool causal, int *qb, int *bh) {
  if ((a.BH & 7) == 0) {
    const int x = id & 7, k = id >> 3;
    const int t = k / a.nqb, r = k - t * a.nqb;
    *bh = x + 8 * t;
    *qb = causal ? a.nqb - 1 - r : r;
  } else {
    *bh = id % a.BH;
    *qb = causal ? a.nqb - 1 - id / a.BH : id / a.BH;
  }
}

template <class E, bool CAUSAL>
__global__ __launch_bounds__(NT, 2) void attn_fwd_d128(AttnArgs a) {
  typedef typename E::vec8 V8;
  __shared__ __attribute__((aligned(16))) uint8_t smem[4 * TILE];  // K0 K1 V0 V1
  const uint8_t *const kt0 = smem;
  const uint8_t *const vt0 = smem + 2 * TILE;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lq = lane & 31, g = lane >> 5;

  int qb, bh;
  map_block(a, blockIdx.x, CAUSAL, &qb, &bh);
  const int b = bh / a.Hq, h = bh - b * a.Hq, hk = h / a.group;
  const uint16_t *qp = (const uint16_t *)a.q + b * a.qs0 + h * a.qs1;
  const uint16_t *kp = (const uint16_t *)a.k + b * a.ks0 + hk * a.ks1;
  const uint16_t *vp = (const uint16_t *)a.v + b * a.vs0 + hk * a.vs1;

  const int row0 = qb * BM + w * 32;
  const int row = row0 + lq;

  int nkb = (a.Sk + BN - 1) / BN;  // key blocks of the work-group
  int nkw = nkb;                    // key blocks this wave computes
  if (CAUSAL) {
    const int last_wg = qb * BM + BM - 1 + a.off;
    nkb = min(nkb, last_wg < 0 ? 0 : last_wg / BN + 1);
    const int last_w = row0 + 31 + a.off;
    nkw = min(nkb, last_w < 0 ? 0 : last_w / BN + 1);
  }

  if (nkb > 0) {
    tile_to_lds<false>(kp, a.ks2, 0, a.Sk, kt0, w, lane);
    tile_to_lds<true>(vp, a.vs2, 0, a.Sk, vt0, w, lane);
    if (nkb > 1) tile_to_lds<false>(kp, a.ks2, BN, a.Sk, kt0 + TILE, w, lane);
  }

  // Q^T operand: k-step st covers head_dim 16 st + 8 g .. +7 of this row
  u32x4 qf[8];
#pragma unroll
  for (int st = 0; st < 8; ++st)
    qf[st] = row < a.Sq ? *(const u32x4 *)(qp + row * a.qs2 + 16 * st + 8 * g)
                        : u32x4{0, 0, 0, 0};

  // per-lane LDS byte offsets of the operand reads
  int ka[8];  // K: row lq (+32 kb), logical unit 2 st + g
#pragma unroll
  for (int st = 0; st < 8; ++st) ka[st] = lq * 256 + (((2 * st + g) ^ (lq & 15)) << 4);
  int va[4];  // V^T: transpose read, rows 4 g + i (+16 c + 8 t), columns 32 nb + 16 dh + 4 q
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
  float m = kNegFltMax, lsum = 0.0f;
  const float sc = a.scale2;
  const f32x16 zero16 = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};

  wait_vmem();
  __syncthreads();
  if (nkw > 0) {
#pragma unroll
    for (int st = 0; st < 8; ++st)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const u32x4 A = *(const u32x4 *)(kt0 + kb * 8192 + ka[st]);
        s[kb] = E::mfma32(as_vec8<V8>(A), as_vec8<V8>(qf[st]), st == 0 ? zero16 : s[kb]);
      }
  }
  __syncthreads();  // every wave is done with K slot 0 before it is refilled

  for (int jb = 0; jb < nkb; ++jb) {
    if (jb + 2 < nkb) tile_to_lds<false>(kp, a.ks2, (jb + 2) * BN, a.Sk, kt0 + (jb & 1) * TILE, w, lane);
    if (jb + 1 < nkb) tile_to_lds<true>(vp, a.vs2, (jb + 1) * BN, a.Sk, vt0 + ((jb + 1) & 1) * TILE, w, lane);
    if (jb < nkw) {
      const int key0 = jb * BN;
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
      // Lazy rescaling: the running max m only moves when a row's block max
      // exceeds it by more than kSlack (a factor 2^kSlack); in between,
      // p = 2^(s - m) <= 2^kSlack, which the fp32 sums hold exactly as well
      // and whose 16-bit rounding is relative, so results differ from a
      // rescale at every block by rounding only.
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
      u32x4 pf[4];
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

      // O^T += V^T P^T for this block (A operand by transpose reads)
      const uint8_t *vt = vt0 + (jb & 1) * TILE;
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
      // reads run two MFMAs ahead
      __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
      for (int i = 0; i < 14; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);

      // S^T of the next block (its K tile arrived during the previous iteration)
      if (jb + 1 < nkw) {
        const uint8_t *kt = kt0 + ((jb + 1) & 1) * TILE;
#pragma unroll
        for (int st = 0; st < 8; ++st)
#pragma unroll
          for (int kb = 0; kb < 2; ++kb) {
            const u32x4 A = *(const u32x4 *)(kt + kb * 8192 + ka[st]);
            s[kb] = E::mfma32(as_vec8<V8>(A), as_vec8<V8>(qf[st]), st == 0 ? zero16 : s[kb]);
          }
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 1);
#pragma unroll
        for (int i = 0; i < 14; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 1);
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 2, 1);
      }
    }
    wait_vmem();
    __syncthreads();
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

template <class E>
void launch_t(const AttnArgs &a, bool causal, hipStream_t s) {
  const dim3 grid((unsigned)(a.nqb * a.BH));
  if (causal)
    hipLaunchKernelGGL((attn_fwd_d128<E, true>), grid, dim3(NT), 0, s, a);
  else
    hipLaunchKernelGGL((attn_fwd_d128<E, false>), grid, dim3(NT), 0, s, a);
}

}  // namespace

hipError_t launch_attn_d128(const AttnArgs &a, int32_t dtype, bool causal, hipStream_t s) {
  if (dtype == 2)
    launch_t<Bf16Tag>(a, causal, s);
  else
    launch_t<F16Tag>(a, causal, s);
  return hipGetLastError();
}

}  // namespace neptune
