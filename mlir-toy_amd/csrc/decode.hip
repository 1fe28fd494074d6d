// decode.hip — split-K flash-decoding with grouped KV heads, bf16 or
// fp8-E4M3 KV, plus the partial-softmax combine and the fp8 KV quantiser.
//
// Not in the reference (Evan-Zhao/mlir-toy has only the prefill tile
// program); the per-split recurrence is the HTile one
// (tests/data/flash_attention_htile.mlir:40-128) with one query row per
// head, and the combine is the textbook flash-decoding reduction in the
// exp2 domain:  M = max m_s, w_s = 2^(m_s - M), L = sum w_s l_s,
// O = sum w_s o~_s / L, lse = (M + log2 L) ln 2.
//
// Work decomposition: one single-wave work-group per (batch, kv head,
// split); the wave streams its split in 32-token steps through a private
// LDS ring filled by global_load_lds_dwordx4 (no K/V byte passes through
// VGPRs on its way to LDS). All query heads of the group
// (heads_q / heads_kv <= 16) ride in one MFMA tile, so every K/V byte is
// read from HBM exactly once. One wave per work-group lets the LDS budget,
// not the work-group shape, set occupancy (measured fastest).
//
// Per 32-token step (v_mfma_f32_16x16x32_bf16, one lane column per head):
//   S^T[16 keys x 16 heads]  = K[16 keys x 32 d] . Q^T   (A = K rows, LDS)
//   O^T[16 d x 16 heads]    += V^T[16 d x 32 keys] . P^T (A = V^T by LDS
//                              transpose reads, B = P^T from S^T)
// K/V loads are non-temporal: each byte is used once, and the nt hint
// measured ~10% more HBM bandwidth for this stream.
#include <mutex>
#include <type_traits>
#include <utility>

#include "device_common.h"
#include "kernels.h"
#include "lds_dma.h"

namespace neptune {
namespace {

constexpr int STEP = 32;    // tokens per wave step
// Lazy-rescale margin (log2 units): the running max only moves when a step's
// max exceeds it by more than this; in between p = 2^(s - m) <= 2^kSlack,
// which fp32 sums hold exactly as well and whose bf16 rounding is relative,
// so results differ from a rescale at every step by rounding only.
constexpr float kSlack = 8.0f;

// One step's p = 2^(s - m) and the lane's sum rs, with the lazy rescale: the
// running max m moves only when a row's step max passes it by more than
// kSlack, rescaling O and l. Past the first step p is first taken against m
// as it stands; when every lane's sum stays within 2^kSlack, so does every
// p, and the step max is not needed. Otherwise (a p above 2^kSlack, an
// overflow, a NaN, or only a large sum) the max is formed, m moves if it
// must, and p is taken again. The first step always forms it (m starts at
// -FLT_MAX). A row's four lanes (lane ^ 16, ^ 32) decide together.
__device__ inline void softmax_step(const f32x4 (&s)[2], bool first, float &m, float &lsum,
                                    f32x4 (&oacc)[8], float (&p)[8], float &rs) {
  auto expo = [&]() {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      p[j] = fast_exp2(s[j >> 2][j & 3] - m);
      rs = j == 0 ? p[j] : rs + p[j];
    }
  };
  bool full = first;
  if (!full) {
    expo();
    full = __any(!(rs <= 256.0f));  // 2^kSlack
  }
  if (full) {
    float mx = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 4; ++r) mx = fmaxf(mx, s[kb][r]);
    mx = max_xor32(max_xor16(mx));
    if (__any(mx > m + kSlack)) {
      const float m_new = fmaxf(m, mx);
      const float alpha = fast_exp2(m - m_new);
      m = m_new;
      lsum *= alpha;
#pragma unroll
      for (int mb = 0; mb < 8; ++mb)
#pragma unroll
        for (int r = 0; r < 4; ++r) oacc[mb][r] *= alpha;
    }
    expo();
  }
}
constexpr int DH = 128;     // head_dim covered by the decode kernels
constexpr int64_t kMaxSplits = 16384;  // combine: one fp32 weight per split in 64 KiB of LDS

struct DecArgs {
  const uint16_t *q;
  const void *k, *v;
  // fp8 scales: [B, Hk, nsb] per sb-token block; paged, [npages, Hk]
  const float *ksc, *vsc;
  float *part_o, *part_ml;
  int32_t Hq, Hk, group, L, chunk, splits, nsb, sb;
  float scale2;
  // paged KV (decode_partial_ring<true>, decode_partial_ring8<true>): token t
  // of sequence b lives in page btab[b * maxp + t / ps], at element offset
  // page * k_ps[0] + head * k_ps[1] + (t % ps) * tok (the same for V with
  // v_ps); seqlens[b] tokens
  const int32_t *btab, *seqlens;
  int32_t ps, maxp, npages, tok;
  int64_t k_ps[2], v_ps[2];
};

// Work-group -> (batch, kv head, split). Contiguous KV: split fastest, so
// neighbouring work-groups stream neighbouring ranges of one head. Paged KV:
// kv head fastest, so the work-groups reading the heads of the same tokens
// run together; in a token-major pool ([pages, page, Hkv, D]) those heads
// share every token's row, and fp8 decode over such a pool measured 7%
// faster (bf16 1%) with this order, while contiguous fp8 decode measured 1%
// slower with it.
template <bool PAGED>
__device__ inline void grid_item(const DecArgs &a, int id, int *b, int *hk, int *split) {
  if (PAGED) {
    *hk = id % a.Hk;
    const int rest = id / a.Hk;
    *split = rest % a.splits;
    *b = rest / a.splits;
  } else {
    *split = id % a.splits;
    const int bk = id / a.splits;
    *b = bk / a.Hk;
    *hk = bk % a.Hk;
  }
}

// bf16 bits of 4 E4M3 codes packed in one dword -> two dwords of bf16 pairs
// (v_cvt_scalef32_pk_bf16_fp8 with scale 1: every E4M3 value is a bf16 value,
// so the widening is exact)
__device__ inline u32x2 e4m3x4_to_bf16(uint32_t c) {
  const bf16x2 lo = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(c, 1.0f, false);
  const bf16x2 hi = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(c, 1.0f, true);
  return u32x2{__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi)};
}

// bf16 KV through LDS: each wave streams its token range in 32-token steps
// through a private two-slot ring (K and V tiles of 32 x 128 bf16, 8 KiB
// each) filled by global_load_lds_dwordx4, one step ahead of use. The K tile
// feeds S^T = K.Q^T (v_mfma_f32_16x16x32_bf16, A = K rows by ds_read_b128),
// the V tile feeds O^T += V^T.P^T with A read by ds_read_b64_tr_b16. No
// data passes through VGPRs on its way to LDS and no vector ALU work is
// spent on transposing V.
//   K tile: unit u of token row r at u ^ (r & 15)      (16 rows per read)
//   V tile: unit u of token row r at u ^ 2 (r & 7)     (transpose reads of
//           rows 0-15 or 16-31, 32 bytes each)
constexpr int RSTEP = 32;                   // tokens per step
constexpr int RTILE = RSTEP * DH * 2;       // bytes of one K or V tile
constexpr int RSLOT = 2 * RTILE;            // K + V
constexpr int RWAVE = 2 * RSLOT;            // two slots per wave
constexpr int RW = 1;                       // waves per work-group (LDS-bound occupancy)
constexpr int RT = 64 * RW;                 // threads per work-group
constexpr int RLDS = RW * RWAVE;

template <bool PAGED>
__global__ __launch_bounds__(RT) void decode_partial_ring(DecArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 15, G = lane >> 4;  // MFMA column (query head) / lane group
  const int id = blockIdx.x;
  int split, b, hk;
  grid_item<PAGED>(a, id, &b, &hk, &split);
  const int bk = b * a.Hk + hk;  // batch * Hk + kv head
  const int Gq = a.group;
  // this sequence's length (paged: its own; out-of-range values clamped)
  const int Lb = PAGED ? min(max(a.seqlens[b], 0), a.L) : a.L;

  const int c0 = split * a.chunk;
  const int c1 = min(c0 + a.chunk, Lb);
  const int wlen = ((a.chunk + RW * RSTEP - 1) / (RW * RSTEP)) * RSTEP;
  const int t0 = c0 + w * wlen;
  const int t1 = min(t0 + wlen, c1);
  const int nsteps = t1 > t0 ? (t1 - t0 + RSTEP - 1) / RSTEP : 0;

  const uint8_t *ring = smem + w * RWAVE;
  // token-row stride in bytes; contiguous KV: row t of (b, kv head) at
  // (bk * L + t) * DH elements
  const int64_t tokb = PAGED ? (int64_t)a.tok * 2 : DH * 2;
  const char *kbase = (const char *)a.k + (PAGED ? (int64_t)hk * a.k_ps[1] * 2
                                                 : (int64_t)bk * a.L * DH * 2);
  const char *vbase = (const char *)a.v + (PAGED ? (int64_t)hk * a.v_ps[1] * 2
                                                 : (int64_t)bk * a.L * DH * 2);
  // paged: 64 block-table entries of this wave's range held in a register,
  // lane j holding entry tab0 + j, so a step takes its page with one
  // v_readlane instead of a dependent memory load; reloaded every 64 pages
  int tab0 = 0, tabv = 0;
  auto load_tab = [&](int first) {
    tab0 = first;
    const int j = first + lane;
    tabv = j < a.maxp ? a.btab[(int64_t)b * a.maxp + j] : 0;
  };
  // bytes from kbase / vbase to the first row of the 32-token step at tb: a
  // step never straddles a page (the page size is a multiple of 32 and steps
  // start on multiples of 32); a block-table entry outside [0, npages) is
  // clamped so that a bad table cannot address memory outside the pages
  auto step_base = [&](int tb, int64_t *kb, int64_t *vb) {
    if (PAGED) {
      const int pi = tb / a.ps;
      if (pi - tab0 >= 64) {
        load_tab(pi);
        settle(tabv);
      }
      int pg = __builtin_amdgcn_readlane(tabv, pi - tab0);
      pg = min(max(pg, 0), a.npages - 1);
      const int64_t in_page = (int64_t)(tb % a.ps) * tokb;
      *kb = (int64_t)pg * a.k_ps[0] * 2 + in_page;
      *vb = (int64_t)pg * a.v_ps[0] * 2 + in_page;
    } else {
      *kb = *vb = (int64_t)tb * DH * 2;
    }
  };
  // per-lane byte offsets of this lane's 16 bytes in DMA chunk c (rows 4c + G)
  uint32_t koff[8], voff[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const int r = 4 * c + G;
    koff[c] = (uint32_t)(r * tokb + (((lane & 15) ^ (r & 15)) << 4));
    voff[c] = (uint32_t)(r * tokb + (((lane & 15) ^ (2 * (r & 7))) << 4));
  }
  auto issue = [&](int i) {
    const int tb = t0 + i * RSTEP;
    const uint8_t *slot = ring + (i & 1) * RSLOT;
    int64_t kb0, vb0;
    step_base(tb, &kb0, &vb0);
    if (tb + RSTEP <= Lb) {
      const char *kb = kbase + kb0, *vb = vbase + vb0;
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        // paged: the page base was read from the block table by v_readlane
        if constexpr (PAGED)
          dma16<true>(kb, koff[c], lds_offset(slot + c * 1024));
        else
          dma16_sbase<true>(kb, koff[c], lds_offset(slot + c * 1024));
      }
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        if constexpr (PAGED)
          dma16<true>(vb, voff[c], lds_offset(slot + RTILE + c * 1024));
        else
          dma16_sbase<true>(vb, voff[c], lds_offset(slot + RTILE + c * 1024));
      }
    } else {  // tail: rows past the sequence re-read its last token (masked)
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const int r = 4 * c + G;
        const int64_t row = min(tb + r, Lb - 1) - tb;
        dma16<true>(kbase + kb0 + row * tokb + (((lane & 15) ^ (r & 15)) << 4),
              lds_offset(slot + c * 1024));
      }
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const int r = 4 * c + G;
        const int64_t row = min(tb + r, Lb - 1) - tb;
        dma16<true>(vbase + vb0 + row * tokb + (((lane & 15) ^ (2 * (r & 7))) << 4),
              lds_offset(slot + RTILE + c * 1024));
      }
    }
  };
  // Q^T operand: k-step ks covers head_dim 32 ks + 8 G .. +7 of head n
  u32x4 qf[4];
  {
    const uint16_t *qrow = a.q + ((int64_t)b * a.Hq + hk * Gq + n) * DH;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      qf[ks] = n < Gq ? *(const u32x4 *)(qrow + 32 * ks + 8 * G) : u32x4{0, 0, 0, 0};
  }
  if (PAGED) load_tab(t0 / a.ps);
  // Q and the table land before the first copy is issued
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) settle(qf[ks]);
  if (PAGED) settle(tabv);
  if (nsteps > 0) issue(0);
  if (nsteps > 1) issue(1);
  // LDS read offsets: K A-operand (row n of each 16-key half, unit 4 ks + G),
  // V^T transpose reads (rows 4 G + i, columns 16 mb + 4 q)
  int ka[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) ka[ks] = n * 256 + (((4 * ks + G) ^ n) << 4);
  const int vi = (lane & 15) >> 2, vq = lane & 3;
  const int vrow = 4 * G + vi;

  f32x4 oacc[8];
#pragma unroll
  for (int mb = 0; mb < 8; ++mb) oacc[mb] = f32x4{0, 0, 0, 0};
  float m = kNegFltMax, lsum = 0.0f;
  const float sc = a.scale2;

  for (int i = 0; i < nsteps; ++i) {
    // this step's tiles have landed once only the next step's 16 copies
    // may still be outstanding
    if (i + 1 < nsteps)
      __builtin_amdgcn_s_waitcnt(waitcnt_vm(16));
    else
      __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    const uint8_t *kt = ring + (i & 1) * RSLOT;
    const uint8_t *vt = kt + RTILE;
    const int t = t0 + i * RSTEP;

    f32x4 s[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      s[kb] = f32x4{0, 0, 0, 0};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const u32x4 A = *(const u32x4 *)(kt + kb * 4096 + ka[ks]);
        s[kb] = Bf16Tag::mfma16(as_vec8<bf16x8>(A), as_vec8<bf16x8>(qf[ks]), s[kb]);
      }
    }
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 4; ++r) s[kb][r] *= sc;
    if (t + RSTEP > t1) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (t + 16 * kb + 4 * G + r >= t1) s[kb][r] = -INFINITY;
    }
    float rs, p[8];
    softmax_step(s, i == 0, m, lsum, oacc, p, rs);
    lsum += rs;
    // P^T: k-slot 8 G + j holds key 4 G + j (j < 4) or 16 + 4 G + j - 4
    u32x4 pf;
#pragma unroll
    for (int i2 = 0; i2 < 4; ++i2) pf[i2] = Bf16Tag::pack2(p[2 * i2], p[2 * i2 + 1]);
#pragma unroll
    for (int mb = 0; mb < 8; ++mb) {
      const int col = 32 * (mb ^ (vrow & 7)) + 8 * vq;
      const v4i16 lo = lds_read_tr16(vt + vrow * 256 + col);
      const v4i16 hi = lds_read_tr16(vt + (vrow + 16) * 256 + col);
      const u32x2 a0 = __builtin_bit_cast(u32x2, lo), a1 = __builtin_bit_cast(u32x2, hi);
      const u32x4 A = {a0[0], a0[1], a1[0], a1[1]};
      oacc[mb] = Bf16Tag::mfma16(as_vec8<bf16x8>(A), as_vec8<bf16x8>(pf), oacc[mb]);
    }
    // every read of this slot has returned before it is refilled
    __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
    if (i + 2 < nsteps) issue(i + 2);
  }

  lsum += __shfl_xor(lsum, 16, 64);
  lsum += __shfl_xor(lsum, 32, 64);

  // ---- merge the waves of this split
  __syncthreads();
  float *mo = (float *)smem;              // [RW][16][DH]
  float *mml = mo + RW * 16 * DH;         // [RW][16][2]
  if (n < Gq) {
#pragma unroll
    for (int mb = 0; mb < 8; ++mb)
#pragma unroll
      for (int r = 0; r < 4; ++r) mo[(w * 16 + n) * DH + 16 * mb + 4 * G + r] = oacc[mb][r];
    if (G == 0) {
      mml[(w * 16 + n) * 2 + 0] = m;
      mml[(w * 16 + n) * 2 + 1] = lsum;
    }
  }
  __syncthreads();
  for (int e = tid; e < Gq * DH; e += RT) {
    const int hn = e / DH, d = e % DH;
    float M = kNegFltMax;
#pragma unroll
    for (int ww = 0; ww < RW; ++ww) M = fmaxf(M, mml[(ww * 16 + hn) * 2]);
    float acc = 0.0f, Ls = 0.0f;
#pragma unroll
    for (int ww = 0; ww < RW; ++ww) {
      const float wgt = fast_exp2(mml[(ww * 16 + hn) * 2] - M);
      acc += wgt * mo[(ww * 16 + hn) * DH + d];
      Ls += wgt * mml[(ww * 16 + hn) * 2 + 1];
    }
    const int64_t row = ((int64_t)b * a.Hq + hk * Gq + hn) * a.splits + split;
    a.part_o[row * DH + d] = acc;
    if (d == 0) {
      a.part_ml[row * 2 + 0] = M;
      a.part_ml[row * 2 + 1] = Ls;
    }
  }
}

// fp8-E4M3 KV: K codes straight into registers, V codes through an LDS
// ring. A 32-token step is 4 KiB of K and 4 KiB of V codes; R8P steps are
// in flight. Each lane loads the 64 K codes it feeds to S^T = K.Q^T with
// four non-temporal global_load_dwordx4 into a register buffer (one buffer
// per step in flight), so only V -- which the MFMA needs transposed, by
// ds_read_b64_tr_b8 -- takes LDS: the ring holds R8P V tiles (16 KiB per
// wave) and the register file holds the K tiles, twice the bytes in flight
// of a ring of K and V tiles in the same LDS. Codes are widened to bf16 in
// registers (exact); the per-(token block) K scale folds into the score
// scale and the V scale into P before its bf16 rounding. 32-token steps
// never straddle a scale block (the block is a multiple of 32 and every
// wave range starts on a 32-token boundary). PAGED: the pools are addressed
// through the block table as in decode_partial_ring<true>, and the page is
// the scale block (one K and one V scale per page and kv head).
//   K: lane (n, G) loads rows n and 16 + n of the step, head_dim
//      64 sp + 16 G .. +15 (sp = 0, 1): the A operand of two MFMA k-steps.
//   V tile: 16-byte unit u of row r at u ^ ((r >> 1) & 7); V^T comes from
//      ds_read_b64_tr_b8, whose source lane pair (2i, 2i+1) names the token
//      row of k-slot i, so the rows can follow the P^T key order directly.
// The K loads are inline assembly like the V copies: the compiler counts
// neither, and a load it counted would make it wait for the untracked copies
// issued after it as well. kload_wait() waits for a buffer and ties the
// buffer's registers to that wait, so nothing reads them earlier
// (tests/test_isa_hazards.py checks the compiled code for it).
constexpr int R8W = 1;                      // waves per work-group (LDS-bound occupancy)
constexpr int R8T = 64 * R8W;
constexpr int R8TILE = RSTEP * DH;          // bytes of one V code tile
constexpr int R8P = 4;                      // steps in flight (K buffers, V ring slots)
constexpr int R8WAVE = R8P * R8TILE;
constexpr int R8LDS = R8W * R8WAVE;

typedef int v2i32 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) v2i32 lds_v2i32;

// One non-temporal global_load_dwordx4 into dst: 16 bytes at sbase + voff
// (sbase wave-uniform). The compiler does not count it: the caller waits
// with s_waitcnt and then passes dst through kload_wait before any use.
// s_nop 4: the SGPR base may have been written by a VALU (v_readfirstlane)
// just before, which a VMEM read of that SGPR must not follow within 5 wait
// states.
__device__ inline void kload(u32x4 &dst, const char *sbase, uint32_t voff) {
  asm volatile("s_nop 4\n\tglobal_load_dwordx4 %0, %1, %2 nt"
               : "=&v"(dst)
               : "v"(voff), "s"(uniform_ptr(sbase))
               : "memory");
}
// The same load from a per-lane address (the tail step re-reads the last
// token for rows past the sequence).
__device__ inline void kload(u32x4 &dst, const char *addr) {
  asm volatile("global_load_dwordx4 %0, %1, off nt" : "=&v"(dst) : "v"(addr) : "memory");
}
// After the s_waitcnt that retired a buffer's loads: its registers are
// produced here as far as the compiler knows, so no read of them (and no
// copy) can be scheduled before the wait.
// The statement emits only an assembly comment naming the registers, which
// tests/test_isa_hazards.py matches against the loads' destinations (a copy
// of a buffer before its wait would name other registers).
__device__ inline void kload_wait(u32x4 (&k)[4]) {
  asm volatile("; kload_wait %0 %1 %2 %3"
               : "+v"(k[0]), "+v"(k[1]), "+v"(k[2]), "+v"(k[3])
               :
               : "memory");
}

template <bool PAGED>
__global__ __launch_bounds__(R8T) void decode_partial_ring8(DecArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 15, G = lane >> 4;
  const int id = blockIdx.x;
  int split, b, hk;
  grid_item<PAGED>(a, id, &b, &hk, &split);
  const int bk = b * a.Hk + hk;  // batch * Hk + kv head
  const int Gq = a.group;
  // this sequence's length (paged: its own; out-of-range values clamped)
  const int Lb = PAGED ? min(max(a.seqlens[b], 0), a.L) : a.L;

  const int c0 = split * a.chunk;
  const int c1 = min(c0 + a.chunk, Lb);
  const int wlen = ((a.chunk + R8W * RSTEP - 1) / (R8W * RSTEP)) * RSTEP;
  const int t0 = c0 + w * wlen;
  const int t1 = min(t0 + wlen, c1);
  const int nsteps = t1 > t0 ? (t1 - t0 + RSTEP - 1) / RSTEP : 0;

  const uint8_t *ring = smem + w * R8WAVE;
  // token-row stride in bytes (a code is one byte); contiguous KV: row t of
  // (b, kv head) at (bk * L + t) * DH
  const int64_t tokb = PAGED ? (int64_t)a.tok : DH;
  const char *kbase =
      (const char *)a.k + (PAGED ? (int64_t)hk * a.k_ps[1] : (int64_t)bk * a.L * DH);
  const char *vbase =
      (const char *)a.v + (PAGED ? (int64_t)hk * a.v_ps[1] : (int64_t)bk * a.L * DH);
  // paged: 64 block-table entries held in a register for the copies (lane j
  // holding entry tab0 + j), read with v_readlane, reloaded every 64 pages
  int tab0 = 0, tabv = 0;
  auto load_tab = [&](int first) {
    tab0 = first;
    const int j = first + lane;
    tabv = j < a.maxp ? a.btab[(int64_t)b * a.maxp + j] : 0;
  };
  // bytes from kbase / vbase to the first row of the step at tb (a step
  // never straddles a page; entries outside [0, npages) are clamped)
  auto step_base = [&](int tb, int64_t *kb, int64_t *vb) {
    if (PAGED) {
      const int pi = tb / a.ps;
      if (pi - tab0 >= 64) {
        load_tab(pi);
        settle(tabv);
      }
      int pg = __builtin_amdgcn_readlane(tabv, pi - tab0);
      pg = min(max(pg, 0), a.npages - 1);
      const int64_t in_page = (int64_t)(tb % a.ps) * tokb;
      *kb = (int64_t)pg * a.k_ps[0] + in_page;
      *vb = (int64_t)pg * a.v_ps[0] + in_page;
    } else {
      *kb = *vb = (int64_t)tb * DH;
    }
  };
  // V copy chunk c covers rows 8c .. 8c+7; this lane moves row 8c + lane/8,
  // physical unit lane & 7
  uint32_t off[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int r = 8 * c + (lane >> 3);
    off[c] = (uint32_t)(r * tokb + (((lane & 7) ^ ((r >> 1) & 7)) << 4));
  }
  // K loads: row 16 kb + n, head_dim 64 sp + 16 G (q = 2 kb + sp)
  uint32_t koff[4];
#pragma unroll
  for (int q = 0; q < 4; ++q)
    koff[q] = (uint32_t)((16 * (q >> 1) + n) * tokb + 64 * (q & 1) + 16 * G);

  u32x4 kq[R8P][4];  // K codes of the steps in flight, buffer i % R8P
  // step i's K codes into buffer J (= i % R8P), then its V tile into ring
  // slot J: 8 operations, always in this order
  auto issue = [&](int i, auto J) {
    constexpr int j = decltype(J)::value;
    const int tb = t0 + i * RSTEP;
    const uint8_t *slot = ring + j * R8TILE;
    int64_t kb0, vb0;
    step_base(tb, &kb0, &vb0);
    if (tb + RSTEP <= Lb) {
      const char *kb = kbase + kb0, *vb = vbase + vb0;
#pragma unroll
      for (int q = 0; q < 4; ++q) kload(kq[j][q], kb, koff[q]);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        // paged: the page base was read from the block table by v_readlane
        if constexpr (PAGED)
          dma16<true>(vb, off[c], lds_offset(slot + c * 1024));
        else
          dma16_sbase<true>(vb, off[c], lds_offset(slot + c * 1024));
      }
    } else {  // tail: rows past the sequence re-read its last token (masked)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int r = 16 * (q >> 1) + n;
        const int64_t row = min(tb + r, Lb - 1) - tb;
        kload(kq[j][q], kbase + kb0 + row * tokb + 64 * (q & 1) + 16 * G);
      }
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int r = 8 * c + (lane >> 3);
        const int64_t row = min(tb + r, Lb - 1) - tb;
        const int u = ((lane & 7) ^ ((r >> 1) & 7)) << 4;
        dma16<true>(vbase + vb0 + row * tokb + u, lds_offset(slot + c * 1024));
      }
    }
  };
  // Q^T operand: k-step ks covers head_dim 64 (ks >> 1) + 16 G + 8 (ks & 1) .. +7
  u32x4 qf[4];
  {
    const uint16_t *qrow = a.q + ((int64_t)b * a.Hq + hk * Gq + n) * DH;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int d = 64 * (ks >> 1) + 16 * G + 8 * (ks & 1);
      qf[ks] = n < Gq ? *(const u32x4 *)(qrow + d) : u32x4{0, 0, 0, 0};
    }
  }
  // the K / V scales of 64 scale blocks of this wave's range in registers,
  // lane j holding block blk0 + j: a step takes its scales with v_readlane
  // instead of a memory load; reloaded every 64 blocks. Paged, a block is a
  // page (one scale per page and kv head) and lane j holds the scales of
  // block-table entry blk0 + j: this window is separate from the copies'
  // one, which runs up to R8P - 1 steps ahead of the math
  const int bsz = PAGED ? a.ps : a.sb;  // tokens per scale block
  int blk0 = 0;
  float kscv = 0.0f, vscv = 0.0f;
  auto load_scales = [&](int first) {
    blk0 = first;
    const int j = first + lane;
    if (PAGED) {
      int pg = j < a.maxp ? a.btab[(int64_t)b * a.maxp + j] : 0;
      pg = min(max(pg, 0), a.npages - 1);
      kscv = a.ksc[(int64_t)pg * a.Hk + hk];
      vscv = a.vsc[(int64_t)pg * a.Hk + hk];
    } else {
      kscv = j < a.nsb ? a.ksc[(int64_t)bk * a.nsb + j] : 0.0f;
      vscv = j < a.nsb ? a.vsc[(int64_t)bk * a.nsb + j] : 0.0f;
    }
  };
  load_scales(t0 / bsz);
  if (PAGED) load_tab(t0 / a.ps);
  // scale block of the current step, kept by counting (a step is 32 tokens
  // and a block a multiple of 32, so steps never straddle blocks)
  int blk = t0 / bsz, in_blk = t0 - blk * bsz;
  // Q, the scales and the table land before the first copy is issued
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) settle(qf[ks]);
  settle(kscv);
  settle(vscv);
  if (PAGED) settle(tabv);
  static_for<R8P>([&](auto J) {
    if (decltype(J)::value < nsteps) issue(decltype(J)::value, J);
  });
  // V^T reads: source lane pair (2i, 2i+1) of group G names the token row of
  // k-slot i (keys 4 G + i, then 16 + 4 G + i - 4), 8 bytes each
  const int vi = (lane & 15) >> 1, vhalf = lane & 1;
  const int vrow = (vi < 4 ? 4 * G + vi : 16 + 4 * G + vi - 4);
  const int vrow_off = vrow * DH + 8 * vhalf;
  const int vsw = (vrow >> 1) & 7;

  f32x4 oacc[8];
#pragma unroll
  for (int mb = 0; mb < 8; ++mb) oacc[mb] = f32x4{0, 0, 0, 0};
  float m = kNegFltMax, lsum = 0.0f;

  // waits until at most 8 * later + extra of this wave's operations are
  // outstanding (later: steps issued after this one, each 8 operations)
  auto wait_ops = [&](int later, auto extra) {
    constexpr int X = decltype(extra)::value;
    static_assert(8 * (R8P - 1) + X <= 63, "vmcnt holds at most 63");
    static_for<R8P>([&](auto L) {
      constexpr int l = decltype(L)::value;
      if (later == l) __builtin_amdgcn_s_waitcnt(waitcnt_vm(8 * l + X));
    });
  };
  auto step = [&](int i, auto J) {
    constexpr int j = decltype(J)::value;
    const int later = min(R8P - 1, nsteps - 1 - i);
    // K(i) has landed once only V(i) and the later steps may be outstanding
    wait_ops(later, std::integral_constant<int, 4>{});
    kload_wait(kq[j]);
    const uint8_t *vt = ring + j * R8TILE;
    const int t = t0 + i * RSTEP;

    f32x4 s[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      s[kb] = f32x4{0, 0, 0, 0};
#pragma unroll
      for (int sp = 0; sp < 2; ++sp) {
        const u32x4 c = kq[j][2 * kb + sp];
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2) {
          const u32x2 lo = e4m3x4_to_bf16(c[2 * h2]);
          const u32x2 hi = e4m3x4_to_bf16(c[2 * h2 + 1]);
          const u32x4 A = {lo[0], lo[1], hi[0], hi[1]};
          s[kb] = Bf16Tag::mfma16(as_vec8<bf16x8>(A), as_vec8<bf16x8>(qf[2 * sp + h2]), s[kb]);
        }
      }
    }
    if (blk - blk0 >= 64) {
      load_scales(blk);
      settle(kscv);
      settle(vscv);
    }
    const float sc = a.scale2 * __builtin_bit_cast(
        float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, kscv), blk - blk0));
    const float vsc = __builtin_bit_cast(
        float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, vscv), blk - blk0));
    // scale first, then mask: a zero fp8 scale must not meet -inf
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 4; ++r) s[kb][r] *= sc;
    if (t + RSTEP > t1) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (t + 16 * kb + 4 * G + r >= t1) s[kb][r] = -INFINITY;
    }
    float rs, p[8];
    softmax_step(s, i == 0, m, lsum, oacc, p, rs);
    lsum += rs;
    u32x4 pf;
#pragma unroll
    for (int i2 = 0; i2 < 4; ++i2) pf[i2] = Bf16Tag::pack2(p[2 * i2] * vsc, p[2 * i2 + 1] * vsc);
    // V(i) has landed once only the later steps may be outstanding
    wait_ops(later, std::integral_constant<int, 0>{});
#pragma unroll
    for (int mb = 0; mb < 8; ++mb) {
      const v2i32 c = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
          (lds_v2i32 *)as_lds(vt + vrow_off + ((mb ^ vsw) << 4)));
      const u32x2 lo = e4m3x4_to_bf16((uint32_t)c[0]);
      const u32x2 hi = e4m3x4_to_bf16((uint32_t)c[1]);
      const u32x4 A = {lo[0], lo[1], hi[0], hi[1]};
      oacc[mb] = Bf16Tag::mfma16(as_vec8<bf16x8>(A), as_vec8<bf16x8>(pf), oacc[mb]);
    }
    // every read of this slot has returned before it is refilled
    __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
    if (i + R8P < nsteps) issue(i + R8P, J);
    in_blk += RSTEP;
    if (in_blk == bsz) {
      in_blk = 0;
      ++blk;
    }
  };
  for (int i0 = 0; i0 < nsteps; i0 += R8P)
    static_for<R8P>([&](auto J) {
      if (i0 + decltype(J)::value < nsteps) step(i0 + decltype(J)::value, J);
    });

  lsum += __shfl_xor(lsum, 16, 64);
  lsum += __shfl_xor(lsum, 32, 64);

  __syncthreads();
  float *mo = (float *)smem;              // [R8W][16][DH]
  float *mml = mo + R8W * 16 * DH;         // [R8W][16][2]
  if (n < Gq) {
#pragma unroll
    for (int mb = 0; mb < 8; ++mb)
#pragma unroll
      for (int r = 0; r < 4; ++r) mo[(w * 16 + n) * DH + 16 * mb + 4 * G + r] = oacc[mb][r];
    if (G == 0) {
      mml[(w * 16 + n) * 2 + 0] = m;
      mml[(w * 16 + n) * 2 + 1] = lsum;
    }
  }
  __syncthreads();
  for (int e = tid; e < Gq * DH; e += R8T) {
    const int hn = e / DH, d = e % DH;
    float M = kNegFltMax;
#pragma unroll
    for (int ww = 0; ww < R8W; ++ww) M = fmaxf(M, mml[(ww * 16 + hn) * 2]);
    float acc = 0.0f, Ls = 0.0f;
#pragma unroll
    for (int ww = 0; ww < R8W; ++ww) {
      const float wgt = fast_exp2(mml[(ww * 16 + hn) * 2] - M);
      acc += wgt * mo[(ww * 16 + hn) * DH + d];
      Ls += wgt * mml[(ww * 16 + hn) * 2 + 1];
    }
    const int64_t row = ((int64_t)b * a.Hq + hk * Gq + hn) * a.splits + split;
    a.part_o[row * DH + d] = acc;
    if (d == 0) {
      a.part_ml[row * 2 + 0] = M;
      a.part_ml[row * 2 + 1] = Ls;
    }
  }
}

// One work-group per (batch, query head): combine the splits' partials.
// Every thread (one head_dim element) first issues the loads of its first
// kCombinePre splits' o~, which do not depend on the weights, so their
// latency overlaps that of the (m, l) reads. Wave 0 reads every split's
// (m, l) (one lane per split), reduces M and L across the wave and leaves
// the weights 2^(m_s - M) in LDS; then each thread sums its splits' o~ in
// split order.
constexpr int kCombinePre = 16;

__global__ __launch_bounds__(DH) void decode_combine(const float *part_o,
                                                     const float *part_ml,
                                                     uint16_t *o, float *lse,
                                                     int32_t splits) {
  extern __shared__ float wts[];  // [splits]
  __shared__ float stat[2];
  const int64_t bh = blockIdx.x;
  const int d = threadIdx.x;
  const float *ml = part_ml + bh * splits * 2;
  const float *po = part_o + bh * splits * DH + d;
  float pre[kCombinePre];
#pragma unroll
  for (int s = 0; s < kCombinePre; ++s) pre[s] = s < splits ? po[(int64_t)s * DH] : 0.0f;
  if (d < 64) {
    float M = kNegFltMax;
    for (int s = d; s < splits; s += 64) M = fmaxf(M, ml[2 * s]);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) M = fmaxf(M, __shfl_xor(M, off, 64));
    float Ls = 0.0f;
    for (int s = d; s < splits; s += 64) {
      const float wgt = fast_exp2(ml[2 * s] - M);
      wts[s] = wgt;
      Ls += wgt * ml[2 * s + 1];
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) Ls += __shfl_xor(Ls, off, 64);
    if (d == 0) {
      stat[0] = M;
      stat[1] = Ls;
    }
  }
  __syncthreads();
  float acc = 0.0f;
#pragma unroll
  for (int s = 0; s < kCombinePre; ++s)
    if (s < splits) acc += wts[s] * pre[s];
#pragma unroll 8
  for (int s = kCombinePre; s < splits; ++s) acc += wts[s] * po[(int64_t)s * DH];
  const float Ls = stat[1];
  // an empty sequence (paged decode with length 0) has L = 0: O = 0, lse = -inf
  o[bh * DH + d] = Bf16Tag::from_f32(Ls > 0.0f ? acc / Ls : 0.0f);
  if (d == 0 && lse) lse[bh] = Ls > 0.0f ? (stat[0] + log2f(Ls)) * kLn2 : -INFINITY;
}

// One work-group per (batch, kv head, scale block): amax, scale, codes.
// fp8 KV quantiser, register path: one 256-thread work-group per (batch,
// kv head, scale block) whose block holds at most 256 * QMAX chunks of 8
// elements. The block is read once with non-temporal 16-byte loads into
// registers, reduced to amax, scaled and converted from registers, so HBM
// sees one read of the bf16 source and one write of the codes.
// v_cvt_pk_fp8_f32 is the OCP E4M3 conversion with round to nearest even;
// scaled magnitudes exceed 448 by at most the rounding of 448 / amax, which
// rounds back to 448, so the saturating case of the format never arises.
constexpr int QMAX = 8;

template <int NC>
__global__ __launch_bounds__(256) void kv_quantize_reg(const uint16_t *src, uint8_t *codes,
                                                       float *scales, int32_t L, int32_t D,
                                                       int32_t sb, int32_t nsb) {
  __shared__ float red[4];
  const int blk = blockIdx.x % nsb;
  const int64_t bk = blockIdx.x / nsb;
  const int t0 = blk * sb, t1 = min(t0 + sb, L);
  const int64_t e0 = bk * (int64_t)L * D + (int64_t)t0 * D;
  const int nch = (t1 - t0) * D / 8;
  const u32x4 *in = (const u32x4 *)(src + e0);
  u32x4 v[NC];
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int ch = threadIdx.x + 256 * i;
    v[i] = ch < nch ? __builtin_nontemporal_load(in + ch) : u32x4{0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < 4; ++j)
      amax = fmaxf(amax, fmaxf(fabsf(__uint_as_float(v[i][j] << 16)),
                               fabsf(__uint_as_float(v[i][j] & 0xffff0000u))));
  }
  for (int off = 32; off >= 1; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float inv = amax > 0.0f ? 448.0f / amax : 0.0f;
  if (threadIdx.x == 0) scales[bk * nsb + blk] = amax > 0.0f ? amax / 448.0f : 0.0f;
  u32x2 *out = (u32x2 *)(codes + e0);
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int ch = threadIdx.x + 256 * i;
    if (ch >= nch) break;
    u32x2 c = {0, 0};
    if (amax > 0.0f) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint32_t p0 = v[i][2 * h], p1 = v[i][2 * h + 1];
        int w = __builtin_amdgcn_cvt_pk_fp8_f32(__uint_as_float(p0 << 16) * inv,
                                                __uint_as_float(p0 & 0xffff0000u) * inv, 0, false);
        w = __builtin_amdgcn_cvt_pk_fp8_f32(__uint_as_float(p1 << 16) * inv,
                                            __uint_as_float(p1 & 0xffff0000u) * inv, w, true);
        c[h] = (uint32_t)w;
      }
    }
    out[ch] = c;
  }
}

// general path (any head_dim or alignment, any block size): two passes
// over the block with element loads and the software encoder
__global__ __launch_bounds__(256) void kv_quantize(const uint16_t *src,
                                                   uint8_t *codes,
                                                   float *scales, int32_t L,
                                                   int32_t D, int32_t sb,
                                                   int32_t nsb) {
  __shared__ float red[4];
  const int blk = blockIdx.x % nsb;
  const int64_t bk = blockIdx.x / nsb;
  const int t0 = blk * sb, t1 = min(t0 + sb, L);
  const int64_t base = bk * L * D;
  const int64_t e0 = (int64_t)t0 * D, e1 = (int64_t)t1 * D;
  float amax = 0.0f;
  for (int64_t e = e0 + threadIdx.x; e < e1; e += 256)
    amax = fmaxf(amax, fabsf(Bf16Tag::to_f32(src[base + e])));
  for (int off = 32; off >= 1; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float inv = amax > 0.0f ? 448.0f / amax : 0.0f;
  if (threadIdx.x == 0) scales[bk * nsb + blk] = amax > 0.0f ? amax / 448.0f : 0.0f;
  for (int64_t e = e0 + threadIdx.x; e < e1; e += 256)
    codes[base + e] =
        amax > 0.0f ? f32_to_e4m3(Bf16Tag::to_f32(src[base + e]) * inv) : uint8_t(0);
}

}  // namespace

bool decode_supported(const DecodeLaunch &a, const char **why) {
  if (a.head_dim != DH) {
    *why = "decode supports head_dim 128";
    return false;
  }
  if (a.heads_q / a.heads_kv > 16) {
    *why = "decode supports at most 16 query heads per kv head";
    return false;
  }
  if (a.kv_dtype == 3 && a.scale_block % STEP) {
    *why = "fp8 decode needs scale_block to be a multiple of 32 tokens";
    return false;
  }
  if (a.block_table) {
    if (a.page_size % STEP) {
      *why = "paged decode needs a page size that is a multiple of 32 tokens";
      return false;
    }
    if (a.kv_dtype == 3 && a.scale_block != a.page_size) {
      *why = "paged fp8 decode takes one scale per page (scale_block 0 or page_size)";
      return false;
    }
    const int64_t esize = a.kv_dtype == 3 ? 1 : 2;
    if (a.k_pstride[2] != a.v_pstride[2] || 31 * a.k_pstride[2] * esize + 256 > ((int64_t)1 << 31) ||
        a.num_pages > ((int64_t)1 << 31) - 1 || a.max_pages > ((int64_t)1 << 31) - 1) {
      *why = "paged decode needs equal K/V token strides below 64 MiB and fewer than 2^31 pages";
      return false;
    }
  }
  if (a.seq_kv > (int64_t)1 << 30 ||
      a.batch * a.heads_kv * a.splits > (int64_t)1 << 30) {
    *why = "decode shape too large for one launch";
    return false;
  }
  // the combine keeps one fp32 weight per split in LDS (64 KiB at most)
  if (a.splits > kMaxSplits) {
    *why = "decode supports at most 16384 splits";
    return false;
  }
  return true;
}

hipError_t launch_decode(const DecodeLaunch &L, hipStream_t s) {
  DecArgs a;
  a.q = (const uint16_t *)L.q;
  a.k = L.k;
  a.v = L.v;
  a.ksc = L.k_scale;
  a.vsc = L.v_scale;
  a.part_o = L.part_o;
  a.part_ml = L.part_ml;
  a.Hq = (int32_t)L.heads_q;
  a.Hk = (int32_t)L.heads_kv;
  a.group = (int32_t)(L.heads_q / L.heads_kv);
  a.L = (int32_t)L.seq_kv;
  a.chunk = (int32_t)L.chunk;
  a.splits = (int32_t)L.splits;
  a.nsb = (int32_t)L.n_scale_blocks;
  a.sb = (int32_t)L.scale_block;
  a.scale2 = L.scale_log2;
  const bool paged = L.block_table != nullptr;
  a.btab = L.block_table;
  a.seqlens = L.seq_lens;
  a.ps = (int32_t)L.page_size;
  a.maxp = (int32_t)L.max_pages;
  a.npages = (int32_t)L.num_pages;
  a.tok = (int32_t)L.k_pstride[2];
  a.k_ps[0] = L.k_pstride[0];
  a.k_ps[1] = L.k_pstride[1];
  a.v_ps[0] = L.v_pstride[0];
  a.v_ps[1] = L.v_pstride[1];
  const int grid = (int)(L.batch * L.heads_kv * L.splits);
  // Both rings fit the dynamic LDS every launch may use without a per-kernel
  // attribute (which would have to be set on each device), so none is set.
  static_assert(RLDS <= 48 * 1024 && R8LDS <= 48 * 1024, "decode ring past the default LDS limit");
  if (L.kv_dtype == 3) {
    if (paged)
      hipLaunchKernelGGL(decode_partial_ring8<true>, dim3(grid), dim3(R8T), R8LDS, s, a);
    else
      hipLaunchKernelGGL(decode_partial_ring8<false>, dim3(grid), dim3(R8T), R8LDS, s, a);
  } else {
    if (paged)
      hipLaunchKernelGGL(decode_partial_ring<true>, dim3(grid), dim3(RT), RLDS, s, a);
    else
      hipLaunchKernelGGL(decode_partial_ring<false>, dim3(grid), dim3(RT), RLDS, s, a);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(decode_combine, dim3((unsigned)(L.batch * L.heads_q)), dim3(DH),
                     (size_t)L.splits * sizeof(float), s,
                     (const float *)L.part_o, (const float *)L.part_ml, (uint16_t *)L.o,
                     L.lse, (int32_t)L.splits);
  return hipGetLastError();
}

}  // namespace neptune

// The split partials of neptune_decode_splitk_noalloc. Every GPU the library
// runs on holds its own copy until the process ends. In host code the name
// is only a stand-in: kernels receive the device address decode_scratch
// resolves, never the array itself.
static __device__ __align__(256) unsigned char scratch[neptune::kDecodeScratchBytes];

namespace neptune {

// The scratch address on the device that owns stream s (the null and
// per-thread streams: the current device), resolved once per device with
// that device current.
hipError_t decode_scratch(hipStream_t s, void **ptr) {
  constexpr int kMaxDevices = 64;
  static std::mutex mu;
  static void *addr[kMaxDevices] = {};
  int dev = -1;
  hipError_t e = (s == nullptr || s == hipStreamPerThread) ? hipGetDevice(&dev)
                                                           : hipStreamGetDevice(s, &dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(mu);
  if (!addr[dev]) {
    int cur = -1;
    e = hipGetDevice(&cur);
    if (e != hipSuccess) return e;
    if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess) return e;
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (cur != dev) {
      const hipError_t back = hipSetDevice(cur);
      if (e == hipSuccess) e = back;
    }
    if (e != hipSuccess) return e;
    addr[dev] = p;
  }
  *ptr = addr[dev];
  return hipSuccess;
}

hipError_t launch_kv_quantize(const QuantLaunch &q, hipStream_t s) {
  const int grid = (int)(q.batch * q.heads_kv * q.n_scale_blocks);
  const uint16_t *src = (const uint16_t *)q.src;
  const int32_t L = (int32_t)q.seq_kv, D = (int32_t)q.head_dim, sb = (int32_t)q.scale_block,
                nsb = (int32_t)q.n_scale_blocks;
  const int64_t chunks = q.scale_block * q.head_dim / 8;  // 8-element chunks per full block
  const bool reg = q.head_dim % 8 == 0 && ((uintptr_t)q.src & 15u) == 0 &&
                   ((uintptr_t)q.codes & 7u) == 0 && chunks <= 256 * QMAX;
  if (reg && chunks <= 256 * 4)
    hipLaunchKernelGGL(kv_quantize_reg<4>, dim3(grid), dim3(256), 0, s, src, q.codes, q.scales,
                       L, D, sb, nsb);
  else if (reg)
    hipLaunchKernelGGL(kv_quantize_reg<QMAX>, dim3(grid), dim3(256), 0, s, src, q.codes,
                       q.scales, L, D, sb, nsb);
  else
    hipLaunchKernelGGL(kv_quantize, dim3(grid), dim3(256), 0, s, src, q.codes, q.scales, L, D,
                       sb, nsb);
  return hipGetLastError();
}

}  // namespace neptune
