// attn_fwd_d128.hip — head_dim-128, 16-bit HTile attention forward for gfx950.
//
// Semantics are those of the generic kernel in attn_fwd.hip (the HTile tile
// program, tests/data/flash_attention_htile.mlir:26-143, plus causal mask,
// LSE, GQA, strides and ragged lengths); this file is its fast path for
// head_dim 128 in bf16 or f16.
//
// Work-group: 256 threads = 4 waves, 128 query rows (32 per wave), 64-key
// blocks; two work-groups per CU (one with 3 stages). Each wave forms the
// transposed products
//   S^T = K . Q^T   (A = K rows from LDS, B = Q^T in VGPRs)
//   O^T = V^T . P^T (A = V^T from LDS via ds_read_b64_tr_b16, B = P^T)
// with v_mfma_f32_32x32x16, so a lane owns one query row in both
// accumulators (row max/sum are in-lane plus one v_permlane32_swap).
//
// Data movement: K and V tiles go HBM -> LDS with global_load_lds_dwordx4
// (no VGPR staging) into STAGES slots per operand (default 2). Key block
// j+1's QK^T is issued in the same MFMA stream as block j's PV, so the next
// scores are ready when the softmax of the next iteration starts; with two
// stages the loads for blocks j+2 (K) and j+1 (V) are in flight during
// iteration j.
//
// LDS tiles (K stored [.., seq, head_dim], and V) are 64 rows x 256 B of
// 16-byte units, XOR-swizzled per row so that both the DMA writes (16 lanes
// = one row) and the MFMA operand reads are bank-conflict free:
//   K: unit u of row r at u ^ (r & 15)   (reads: 32 rows, one unit each)
//   V: unit u of row r at u ^ 4(r & 3)   (transpose reads: 4 rows x 64 B)
//
// Knobs (template parameters, chosen per launch):
//   STAGES (pipeline_stages, HTile:128): K and V tiles each have STAGES LDS
//     slots and the loads run that many key blocks ahead of their use. 2 is
//     the default; 3 takes 96 KiB of LDS (one work-group per CU); 1 loads
//     each tile only once the previous one has been consumed.
//   KT (the K load order): false reads K stored [.., seq, head_dim] as key
//     rows (the A operand of S^T = K.Q^T directly); true reads K stored
//     [.., head_dim, seq] -- the layout a dimension_order = [1, 0] load
//     produces (HTilePasses.cpp:122-140) -- as head_dim rows of 64 keys, and
//     forms the A operand with ds_read_b64_tr_b16 as V^T is formed.
//
// Work-groups: without the causal mask each runs two query blocks of one
// head, q0 = nqb-1-p and q1 = p, back to back; the K/V stream simply
// continues from q0's last key block into q1's first, so q1's tiles load
// while q0 drains, and a launch has half as many prologues. Under the causal
// mask each runs one query block, and the grid dispatches the heaviest
// blocks first, so the end of the launch is filled by the lightest ones.
#include "attn_args.h"
#include "device_common.h"
#include "kernels.h"
#include "lds_dma.h"

namespace neptune {
namespace {

constexpr int BM = 128;
constexpr int BN = 64;
constexpr int HD = 128;
constexpr int NT = 256;
constexpr int TILE = BN * HD * 2;  // bytes per K or V tile (16 KiB)
constexpr float kSlack = 8.0f;     // lazy-rescale threshold (log2 units)
constexpr float kSumCap = 256.0f;  // 2^kSlack: a lane's block sum at most this skips the max

// Wave w copies rows [16w, 16w+16) of a 64 x 128 tile (four 1 KiB chunks of
// four rows) straight into LDS. Full blocks take a wave-uniform base pointer
// plus per-lane 32-bit offsets fixed for the whole kernel, so issuing a
// chunk costs no vector ALU work; a block that runs past the end of the
// sequence re-reads the last row instead (its scores are masked, so its P
// is exactly 0).
struct TileLoader {
  const char *base;   // element (0, 0) of this (batch, head)
  int64_t row_bytes;  // key stride in bytes
  uint32_t off[4];    // per-lane byte offset of chunk c within a full block
  int lane_row;       // 16 w + lane / 16: row of chunk 0 for this lane
  int sw_base;        // lane & 15
};

template <bool IS_V>
__device__ inline TileLoader make_loader(const uint16_t *src, int64_t stride, int w, int lane) {
  TileLoader t;
  t.base = (const char *)src;
  t.row_bytes = stride * 2;
  t.lane_row = 16 * w + (lane >> 4);
  t.sw_base = lane & 15;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int r = t.lane_row + 4 * c;
    const int unit = (lane & 15) ^ (IS_V ? ((r & 3) << 2) : (r & 15));
    t.off[c] = (uint32_t)((int64_t)r * t.row_bytes + unit * 16);
  }
  return t;
}

template <bool IS_V>
__device__ inline void tile_to_lds(const TileLoader &t, int key0, int Sk, const uint8_t *tile,
                                   int w) {
  if (key0 + BN <= Sk) {
    const char *blk = t.base + (int64_t)key0 * t.row_bytes;
#pragma unroll
    for (int c = 0; c < 4; ++c) dma16_sbase(blk, t.off[c], lds_offset(tile + (4 * w + c) * 1024));
  } else {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int r = t.lane_row + 4 * c;
      const int unit = t.sw_base ^ (IS_V ? ((r & 3) << 2) : (r & 15));
      const int key = min(key0 + r, Sk - 1);
      dma16(t.base + (int64_t)key * t.row_bytes + unit * 16, lds_offset(tile + (4 * w + c) * 1024));
    }
  }
}

// K stored [.., head_dim, seq]: a tile is 128 head_dim rows x 64 keys
// (128 B). Wave w copies rows [32w, 32w+32) as four 1 KiB chunks of eight
// rows; 16-byte unit u (keys 8u .. 8u+7) of row r sits at unit
// u ^ 4((r >> 1) & 1), which keeps the transpose reads (four rows x 64 B
// per 16 lanes) on distinct banks. Needs seq % 8 == 0: a unit past the end
// of the keys re-reads the last unit (its scores are masked).
struct KtLoader {
  const char *base;   // element (0, 0) of this (batch, head)
  int64_t row_bytes;  // head_dim-row stride in bytes
  uint32_t off[4];    // per-lane byte offset of chunk c within a full block
  int unit[4];        // source unit (keys 8 unit ..) of chunk c
};

__device__ inline KtLoader make_kt_loader(const uint16_t *src, int64_t stride, int w, int lane) {
  KtLoader t;
  t.base = (const char *)src;
  t.row_bytes = stride * 2;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int r = 32 * w + 8 * c + (lane >> 3);
    t.unit[c] = (lane & 7) ^ (((r >> 1) & 1) << 2);
    t.off[c] = (uint32_t)((int64_t)r * t.row_bytes + t.unit[c] * 16);
  }
  return t;
}

__device__ inline void kt_tile_to_lds(const KtLoader &t, int key0, int Sk, const uint8_t *tile,
                                      int w, int lane) {
  if (key0 + BN <= Sk) {
    const char *blk = t.base + (int64_t)key0 * 2;
#pragma unroll
    for (int c = 0; c < 4; ++c) dma16_sbase(blk, t.off[c], lds_offset(tile + (4 * w + c) * 1024));
  } else {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int r = 32 * w + 8 * c + (lane >> 3);
      const int k8 = min(key0 + 8 * t.unit[c], Sk - 8);
      dma16(t.base + (int64_t)r * t.row_bytes + (int64_t)k8 * 2,
            lds_offset(tile + (4 * w + c) * 1024));
    }
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

// Work-group -> (batch*head, query blocks q0, q1; q1 == q0 for one block).
// With batch*heads a multiple of 8, work-group id % 8 is the XCD it is
// dispatched to, and each XCD walks its own heads, so the K/V of the heads in
// flight on an XCD stay in that XCD's L2.
// - No mask: pair p of a head runs q0 = nqb-1-p and q1 = p; each XCD walks
//   its heads in order, all pairs of one head together.
// - Causal: one block per work-group. Each XCD takes its heads four at a
//   time (a window) and runs a window's blocks from the heaviest (the last
//   query block, which sees every key block) to the lightest, the four heads
//   interleaved. Work-groups are dispatched in id order as slots free up, so
//   the last ones a slot takes are the shortest, and the launch's end is
//   not held up by one long work-group per slot (the longest-first rule).
template <bool CAUSAL>
__device__ inline void map_block(const AttnArgs &a, int npair, int id, int *q0, int *q1,
                                 int *bh) {
  if constexpr (CAUSAL) {
    int q;
    if ((a.BH & 7) == 0) {
      const int x = id & 7, k = id >> 3, hx = a.BH >> 3;
      const int G = hx < 4 ? hx : 4;
      const int win = k / (G * a.nqb);
      const int gh = min(G, hx - win * G);  // heads in this (possibly last) window
      const int r = k - win * G * a.nqb;
      q = a.nqb - 1 - r / gh;
      *bh = x + 8 * (win * G + r % gh);
    } else {
      *bh = id % a.BH;
      q = a.nqb - 1 - id / a.BH;
    }
    *q0 = *q1 = q;
  } else {
    int pair;
    if ((a.BH & 7) == 0) {
      const int x = id & 7, k = id >> 3;
      const int t = k / npair;
      *bh = x + 8 * t;
      pair = k - t * npair;
    } else {
      *bh = id % a.BH;
      pair = id / a.BH;
    }
    *q0 = a.nqb - 1 - pair;
    *q1 = pair;
  }
}

template <class E, bool CAUSAL, int STAGES, bool KT>
__global__ __launch_bounds__(NT, STAGES == 3 ? 1 : 2) void attn_fwd_d128(AttnArgs a, int npair) {
  typedef typename E::vec8 V8;
  // K slots 0 .. STAGES-1, then V slots 0 .. STAGES-1; block t uses slot t % STAGES
  __shared__ __attribute__((aligned(16))) uint8_t smem[2 * STAGES * TILE];
  const uint8_t *const kt0 = smem;
  const uint8_t *const vt0 = smem + STAGES * TILE;
  auto kslot = [&](int t) { return kt0 + (t % STAGES) * TILE; };
  auto vslot = [&](int t) { return vt0 + (t % STAGES) * TILE; };

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lq = lane & 31, g = lane >> 5;

  int q0, q1, bh;
  map_block<CAUSAL>(a, npair, blockIdx.x, &q0, &q1, &bh);
  const int b = bh / a.Hq, h = bh - b * a.Hq, hk = h / a.group;
  const uint16_t *qp = (const uint16_t *)a.q + b * a.qs0 + h * a.qs1;
  const uint16_t *kp = (const uint16_t *)a.k + b * a.ks0 + hk * a.ks1;
  const uint16_t *vp = (const uint16_t *)a.v + b * a.vs0 + hk * a.vs1;

  // the query blocks (the heavier first); one block (causal, or the middle
  // block of an odd count) has n1 = 0
  const int qbs[2] = {q0, q1};
  const bool two = qbs[1] != qbs[0];
  int nkb[2], nkw[2];  // key blocks per query block: work-group, this wave
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    int n = (a.Sk + BN - 1) / BN, nw = n;
    if (CAUSAL) {
      const int last_wg = qbs[it] * BM + BM - 1 + a.off;
      n = min(n, last_wg < 0 ? 0 : last_wg / BN + 1);
      const int last_w = qbs[it] * BM + w * 32 + 31 + a.off;
      nw = min(n, last_w < 0 ? 0 : last_w / BN + 1);
    }
    nkb[it] = (it == 1 && !two) ? 0 : n;
    nkw[it] = (it == 1 && !two) ? 0 : nw;
  }
  const int n0 = nkb[0];
  const int nv = n0 + nkb[1];  // virtual key blocks: n0 for q0, then q1's

  const TileLoader kl = make_loader<false>(kp, a.ks2, w, lane);
  const KtLoader ktl = make_kt_loader(kp, a.ks2, w, lane);
  const TileLoader vl = make_loader<true>(vp, a.vs2, w, lane);
  // virtual block t -> key block of its query block
  auto vkey0 = [&](int t) { return (t < n0 ? t : t - n0) * BN; };
  auto load_k = [&](int t) {
    if constexpr (KT)
      kt_tile_to_lds(ktl, vkey0(t), a.Sk, kslot(t), w, lane);
    else
      tile_to_lds<false>(kl, vkey0(t), a.Sk, kslot(t), w);
  };
  auto load_v = [&](int t) { tile_to_lds<true>(vl, vkey0(t), a.Sk, vslot(t), w); };
  // K of blocks 0 .. STAGES-1 and V of blocks 0 .. STAGES-2 (0 when STAGES = 1)
#pragma unroll
  for (int t = 0; t < STAGES; ++t)
    if (t < nv) load_k(t);
#pragma unroll
  for (int t = 0; t < (STAGES > 1 ? STAGES - 1 : 1); ++t)
    if (t < nv) load_v(t);

  // Q^T operand: k-step st covers head_dim 16 st + 8 g .. +7 of the row
  // (KT: 16 st + 4 g .. +3 and 16 st + 8 + 4 g .. +3, the order in which the
  // K^T transpose reads deliver head_dim)
  u32x4 qf[8];
  auto load_q = [&](int qb) {
    const int row = qb * BM + w * 32 + lq;
    const uint16_t *qr = qp + row * a.qs2;
#pragma unroll
    for (int st = 0; st < 8; ++st) {
      if constexpr (KT) {
        const u32x2 lo = row < a.Sq ? *(const u32x2 *)(qr + 16 * st + 4 * g) : u32x2{0, 0};
        const u32x2 hi = row < a.Sq ? *(const u32x2 *)(qr + 16 * st + 8 + 4 * g) : u32x2{0, 0};
        qf[st] = u32x4{lo[0], lo[1], hi[0], hi[1]};
      } else {
        qf[st] = row < a.Sq ? *(const u32x4 *)(qr + 16 * st + 8 * g) : u32x4{0, 0, 0, 0};
      }
    }
  };
  load_q(qbs[0]);

  // per-lane LDS byte offsets of the operand reads
  int ka[8];  // K: row lq (+32 kb), logical unit 2 st + g
#pragma unroll
  for (int st = 0; st < 8; ++st) ka[st] = lq * 256 + (((2 * st + g) ^ (lq & 15)) << 4);
  int kta[2];  // K^T: transpose read, rows 4 g + i (+16 st + 8 t), keys 32 kb + 16 h + 4 q
  int va[4];   // V^T: transpose read, rows 4 g + i (+16 c + 8 t), columns 32 nb + 16 dh + 4 q
  {
    const int s16 = lane & 15, i = s16 >> 2, q = s16 & 3, dh = (lane >> 4) & 1;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
      kta[kb] = (4 * g + i) * 128 + 64 * (kb ^ (i >> 1)) + 32 * dh + 8 * q;
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) va[nb] = (4 * g + i) * 256 + 64 * (nb ^ i) + 32 * dh + 8 * q;
  }

  f32x16 o[4];
  f32x16 s[2];
  float m, lsum;
  auto reset = [&]() {
#pragma unroll
    for (int nb = 0; nb < 4; ++nb)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[nb][r] = 0.0f;
    m = kNegFltMax;
    lsum = 0.0f;
  };
  reset();
  const float sc = a.scale2;
  const f32x16 zero16 = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};

  // The A operand of MFMA i = 2 st + kb of S^T = K.Q^T (32 keys x 16 head_dim)
  auto k_operand = [&](const uint8_t *kt, int i) {
    const int st = i >> 1, kb = i & 1;
    if constexpr (KT) {
      const v4i16 t0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (lds_v4i16 *)as_lds(kt + (16 * st) * 128 + kta[kb]));
      const v4i16 t1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (lds_v4i16 *)as_lds(kt + (16 * st + 8) * 128 + kta[kb]));
      const u32x2 a0 = __builtin_bit_cast(u32x2, t0), a1 = __builtin_bit_cast(u32x2, t1);
      return u32x4{a0[0], a0[1], a1[0], a1[1]};
    } else {
      return *(const u32x4 *)(kt + kb * 8192 + ka[st]);
    }
  };
  // S^T of one key block, its first two A operands already read (k0, k1):
  // the caller issues those reads early, so the MFMA stream does not start
  // with an LDS round trip
  auto qk_from = [&](const uint8_t *kt, const u32x4 &k0, const u32x4 &k1) {
#pragma unroll
    for (int st = 0; st < 8; ++st)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const int i = 2 * st + kb;
        const u32x4 A = i == 0 ? k0 : i == 1 ? k1 : k_operand(kt, i);
        s[kb] = E::mfma32(as_vec8<V8>(A), as_vec8<V8>(qf[st]), st == 0 ? zero16 : s[kb]);
      }
    // the remaining operand reads run two MFMAs ahead
    constexpr int R = KT ? 2 : 1;  // LDS reads per operand
    __builtin_amdgcn_sched_group_barrier(0x100, 2 * R, 1);
#pragma unroll
    for (int i = 0; i < 12; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
      __builtin_amdgcn_sched_group_barrier(0x100, R, 1);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 4, 1);
  };
  auto qk = [&](const uint8_t *kt) { qk_from(kt, k_operand(kt, 0), k_operand(kt, 1)); };
  // The A operand of P.V step st (V^T: head_dim rows 32 nb .., keys 16 c ..)
  auto v_operand = [&](const uint8_t *vt, int st) {
    const int c = st >> 2, nb = st & 3;
    const v4i16 t0 =
        __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16 *)as_lds(vt + (16 * c) * 256 + va[nb]));
    const v4i16 t1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_v4i16 *)as_lds(vt + (16 * c + 8) * 256 + va[nb]));
    const u32x2 a0 = __builtin_bit_cast(u32x2, t0), a1 = __builtin_bit_cast(u32x2, t1);
    return u32x4{a0[0], a0[1], a1[0], a1[1]};
  };

  // O = acc / l rounded to the input type (HTile:130-143) and the LSE. The
  // quotient is the correctly rounded fp32 acc / l: q = acc * (1/l) with
  // the correctly rounded reciprocal, then one residual step
  // q + fma(-q, l, acc) * (1/l) (Markstein's correction), three VALU
  // operations per element instead of a full division each.
  auto finalize = [&](int qb) {
    const float ltot = pair_sum(lsum);
    const int row = qb * BM + w * 32 + lq;
    if (row < a.Sq) {
      const float inv = ltot > 0.0f ? 1.0f / ltot : 0.0f;
      auto quot = [&](float x) {
        const float q0 = x * inv;
        return __builtin_fmaf(__builtin_fmaf(-q0, ltot, x), inv, q0);
      };
      uint16_t *op = (uint16_t *)a.o + b * a.os0 + h * a.os1 + row * a.os2;
#pragma unroll
      for (int nb = 0; nb < 4; ++nb)
#pragma unroll
        for (int rq = 0; rq < 4; ++rq) {
          const u32x2 pk = {E::pack2(quot(o[nb][4 * rq]), quot(o[nb][4 * rq + 1])),
                            E::pack2(quot(o[nb][4 * rq + 2]), quot(o[nb][4 * rq + 3]))};
          *(u32x2 *)(op + 32 * nb + 8 * rq + 4 * g) = pk;
        }
      if (g == 0 && a.lse)
        a.lse[((int64_t)b * a.Hq + h) * a.Sq + row] =
            ltot > 0.0f ? (m + log2f(ltot)) * kLn2 : -INFINITY;
    }
  };

  wait_vmem();
  __syncthreads();
  if (nkw[0] > 0) qk(kslot(0));
  __syncthreads();  // every wave is done with K slot 0 before it is refilled

  for (int vb = 0; vb < nv; ++vb) {
    const int item = vb >= n0 ? 1 : 0;
    const int jb = vb - item * n0;  // key block within the query block
    // K of block vb + STAGES goes to the slot block vb's K has left, V of
    // block vb + STAGES - 1 to the slot of block vb - 1's V (STAGES = 1:
    // only K here, V once this block's P.V is done)
    int issued = 0;
    if constexpr (STAGES > 1) {
      if (vb + STAGES < nv) {
        load_k(vb + STAGES);
        ++issued;
      }
      if (vb + STAGES - 1 < nv) {
        load_v(vb + STAGES - 1);
        ++issued;
      }
    } else {
      if (vb + 1 < nv) load_k(vb + 1);
    }
    const int qrow0 = qbs[item] * BM + w * 32;
    if (jb < nkw[item]) {
      // the first two V^T operands of this block's P.V, read before the
      // softmax (the V tile landed in the previous iteration)
      const uint8_t *vt = vslot(vb);
      const u32x4 vp0 = v_operand(vt, 0), vp1 = v_operand(vt, 1);
      u32x4 kn0, kn1;
      const int key0 = jb * BN;
      const bool need_mask = (key0 + BN > a.Sk) || (CAUSAL && key0 + BN - 1 > qrow0 + a.off);
      if (need_mask) {
        // element (kb, r) holds key key0 + 4 g + c with c = 32 kb + 8 (r >> 2)
        // + (r & 3), a constant: it is masked when c passes the lane's last
        // visible key (the sequence end or, causally, the lane's own row)
        int lim = a.Sk - 1 - key0 - 4 * g;
        if (CAUSAL) lim = min(lim, qrow0 + lq + a.off - key0 - 4 * g);
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            if (32 * kb + 8 * (r >> 2) + (r & 3) > lim) s[kb][r] = -INFINITY;
      }
      // p = 2^(s sc - m) for the block, packed for P.V, and the lane's sum
      float rs;
      u32x4 pf[4];
      auto expo = [&]() {
        const float nm = -m;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const int kb = c >> 1, hh = c & 1;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float p0 = fast_exp2(fmaf(s[kb][8 * hh + 2 * i], sc, nm));
            const float p1 = fast_exp2(fmaf(s[kb][8 * hh + 2 * i + 1], sc, nm));
            rs = c + i == 0 ? p0 : rs + p0;  // the sum from 0.0 without its first add
            rs += p1;
            pf[c][i] = E::pack2(p0, p1);
          }
        }
      };
      // Lazy rescaling: the running max m only moves when a row's block max
      // exceeds it by more than kSlack (a factor 2^kSlack); in between,
      // p = 2^(s - m) <= 2^kSlack, which the fp32 sums hold exactly as well
      // and whose 16-bit rounding is relative, so results differ from a
      // rescale at every block by rounding only.
      // The block max is only formed when it can matter. Past a query block's
      // first key block, p is first taken against m as it stands: when every
      // lane's sum of its p stays within 2^kSlack, so does every p, and m
      // keeps. Otherwise (a p above 2^kSlack, an overflow to inf, a NaN, or
      // only a large sum) the max is formed, m moves if it must, and p is
      // taken again. The first key block always forms it (m starts at -FLT_MAX).
      bool full = jb == 0;
      if (!full) {
        expo();
        full = __any(!(rs <= kSumCap));
      }
      if (full) {
        float mx = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[kb][r]);
        mx = pair_max(mx);
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
        expo();
      }
      lsum += rs;

      // O^T += V^T P^T for this block (A operand by transpose reads; the
      // first two were read before the softmax). The wave raises its issue
      // priority for its MFMA stretch so the matrix core is fed first while
      // the other wave on the SIMD runs its softmax.
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int step = 0; step < 16; ++step) {
        const int c = step >> 2, nb = step & 3;
        const u32x4 A = step == 0 ? vp0 : step == 1 ? vp1 : v_operand(vt, step);
        o[nb] = E::mfma32(as_vec8<V8>(A), as_vec8<V8>(pf[c]), o[nb]);
      }
      // the next block's first two K operands (its K tile arrived during
      // the previous iteration; a block with no next one reads a stale
      // slot and drops the values), so its S^T starts without a round trip
      if constexpr (STAGES > 1) {
        kn0 = k_operand(kslot(vb + 1), 0);
        kn1 = k_operand(kslot(vb + 1), 1);
      }
      // reads run two MFMAs ahead
      __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
      for (int i = 0; i < 12; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, KT ? 4 : 2, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);

      // S^T of the next block of this query block
      if constexpr (STAGES > 1)
        if (jb + 1 < nkw[item]) qk_from(kslot(vb + 1), kn0, kn1);
      __builtin_amdgcn_s_setprio(0);
    }
    if constexpr (STAGES == 1) {
      wait_vmem();
      __syncthreads();  // K of block vb + 1 has landed; every wave is done with V
      if (vb + 1 < nv) load_v(vb + 1);
      if (jb + 1 < nkw[item]) qk(kslot(vb + 1));
      wait_vmem();
    } else if constexpr (STAGES == 3) {
      // the tiles issued in this iteration may stay in flight (four copies
      // per tile per wave); those issued before it are needed next
      if (issued == 2)
        __builtin_amdgcn_s_waitcnt(waitcnt_vm(8));
      else if (issued == 1)
        __builtin_amdgcn_s_waitcnt(waitcnt_vm(4));
      else
        wait_vmem();
    } else {
      wait_vmem();
    }
    __syncthreads();
    if (vb == n0 - 1) {
      // switch to q1 (its first K tile has landed): load its Q^T here, not
      // earlier, so no load into the Q^T registers is ever pending inside
      // the steady-state loop (that would make every QK^T drain the K/V
      // prefetch along with it)
      finalize(qbs[0]);
      reset();
      if (nkb[1] > 0) {
        load_q(qbs[1]);
        wait_vmem();
      }
      if (nkw[1] > 0) qk(kslot(vb + 1));
      __syncthreads();  // that K slot is refilled by the next iteration
    }
  }
  if (n0 == 0) finalize(qbs[0]);  // no visible keys: O = 0, LSE = -inf
  if (two) finalize(qbs[1]);
}

template <class E, int STAGES, bool KT>
void launch_t(const AttnArgs &a, bool causal, hipStream_t s) {
  const int npair = (a.nqb + 1) / 2;
  if (causal)
    hipLaunchKernelGGL((attn_fwd_d128<E, true, STAGES, KT>), dim3((unsigned)(a.nqb * a.BH)),
                       dim3(NT), 0, s, a, npair);
  else
    hipLaunchKernelGGL((attn_fwd_d128<E, false, STAGES, KT>), dim3((unsigned)(npair * a.BH)),
                       dim3(NT), 0, s, a, npair);
}

template <class E, bool KT>
void launch_stages(const AttnArgs &a, bool causal, int stages, hipStream_t s) {
  if (stages == 1)
    launch_t<E, 1, KT>(a, causal, s);
  else if (stages == 3)
    launch_t<E, 3, KT>(a, causal, s);
  else
    launch_t<E, 2, KT>(a, causal, s);
}

template <class E>
void launch_e(const AttnArgs &a, bool causal, int stages, bool kt, hipStream_t s) {
  if (kt)
    launch_stages<E, true>(a, causal, stages, s);
  else
    launch_stages<E, false>(a, causal, stages, s);
}

}  // namespace

hipError_t launch_attn_d128(const AttnArgs &a, int32_t dtype, bool causal, int stages, bool kt,
                            hipStream_t s) {
  if (dtype == 2)
    launch_e<Bf16Tag>(a, causal, stages, kt, s);
  else
    launch_e<F16Tag>(a, causal, stages, kt, s);
  return hipGetLastError();
}

}  // namespace neptune
