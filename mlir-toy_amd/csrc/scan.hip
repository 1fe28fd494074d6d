// scan.hip — Mamba-1 selective scan forward on gfx950.
//
// Not in the reference (Evan-Zhao/mlir-toy); the recurrence is the
// selective SSM of Gu & Dao 2023 with mamba_ssm's zero-order-hold
// simplification (B_bar = delta * B):
//   delta = softplus(delta_raw + bias[d])           (torch threshold 20)
//   x_n  <- 2^(delta * A[d,n] * log2 e) x_n + (delta u) B[b,n,l]
//   y     = (sum_n C[b,n,l] x_n + D[d] u) * silu(z)
//
// The per-state update (one exp2, two multiplies, one FMA, one multiply for
// the output term) is VALU/transcendental work: 16 states per (channel,
// step) against 8 bytes of HBM traffic, so the kernel is bound by the VALU,
// not by HBM. The design therefore maximises the number of independent
// wavefronts per SIMD and keeps every other cost off the VALU:
//
// Mapping: a 256-thread work-group owns 16 channels of one batch row; lane
// (wave w, row r = lane / 16, column c = lane % 16) carries the single fp32
// state n = 4 w + r of channel c and walks the sequence in order, so no
// carry crosses lanes. 16-channel work-groups give every CU the same share
// of channels (batch * dim / 16 groups), and one state per lane gives four
// or five resident wavefronts per SIMD to hide the exp2 -> FMA chain.
//
// Per 32-step chunk:
//   stage  each thread loads 2 steps of u / delta_raw / z of one channel
//          (64-byte row segments per wave) and B / C of one state, computes
//          (delta, delta*u) and (B, C) into LDS, and keeps (D*u, silu(z))
//          in registers for its own outputs; the next chunk's loads are
//          issued before the recurrence so their latency is hidden.
//   scan   lanes read (delta, delta*u) of their channel and (B, C) of their
//          state with 16-byte LDS reads covering two steps (broadcast
//          across the lanes that share them) and keep C_n x_n per step.
//   reduce the 16-state sum is a transposed butterfly: v_permlane32_swap
//          then v_permlane16_swap each exchange one register pair and add,
//          leaving every lane with the 4-state sum of 8 of the 32 steps;
//          the four waves' sums meet in LDS.
//   store  each thread adds the four wave sums for its two steps, applies
//          D*u and the gate and stores two bf16 outputs.
//
// Sequence-parallel path. When batch * dim / 16 work-groups cannot fill the
// GPU (few channels, long sequences), the sequence is cut into nch chunks of
// T steps (the last one takes the remainder, T .. 2T - 1 steps) and the
// scan runs in three launches, using y itself as scratch (no workspace):
//   state   every chunk but the last scans from x = 0 without outputs and
//           leaves its end state x_end[16] and its delta sum S (fp32) at the
//           start of its own y segment (T >= 64 steps: 128 bytes >= 68);
//   carry   one lane per (batch, channel, state) walks the chunks in order,
//           x_start[k + 1] = 2^(A S[k] log2 e) x_start[k] + x_end[k] (the
//           decay over a chunk is the product of its steps' decays), and
//           leaves x_start[k] where x_end[k] was;
//   output  every chunk reads its x_start from its own segment, then scans
//           it with outputs, overwriting the segment.
// Each launch touches only its own chunk's segment, so work-groups never
// race on the scratch. The work is about 1.6 times the single pass's (the
// state pass repeats the updates without outputs), which pays once the
// chunks multiply the work-groups enough to fill the GPU.
#include <algorithm>

#include "device_common.h"
#include "kernels.h"

namespace neptune {
namespace {

constexpr int ST = 16;     // d_state covered
constexpr int SCH = 16;    // channels per work-group
constexpr int TT = 32;     // steps per chunk
constexpr int NT = 256;    // threads per work-group
constexpr int TP = TT / 2; // step pairs per chunk

struct ScanArgs {
  const uint16_t *u, *dr, *Bm, *Cm, *z;
  const float *A, *D, *bias;
  uint16_t *y;
  int32_t Dm, L, softplus;
  int32_t vec;  // 4-byte pair access: L even and every base 4-byte aligned
  int32_t T, nch;  // chunk length and count (1 chunk of L: the single pass)
};

// the single pass, and the state and output passes of the chunked path
enum ScanMode { kScanFull = 0, kScanState = 1, kScanOutput = 2 };

// chunk k of channel d of batch row b: its y segment as fp32 scratch
// (x[16], then S)
__device__ inline float *chunk_scratch(const ScanArgs &a, int b, int d, int k) {
  return reinterpret_cast<float *>(a.y + ((int64_t)b * a.Dm + d) * a.L + (int64_t)k * a.T);
}

__device__ inline float lo_bf16(uint32_t p) { return __uint_as_float(p << 16); }
__device__ inline float hi_bf16(uint32_t p) { return __uint_as_float(p & 0xffff0000u); }

// two consecutive bf16 elements of a row as packed bits; t is even and
// elements at or beyond L read as zero
__device__ inline uint32_t load_pair(const uint16_t *row, int t, int L, bool vec) {
  if (vec && t + 1 < L) return *(const uint32_t *)(row + t);
  uint32_t lo = t < L ? row[t] : 0u;
  uint32_t hi = t + 1 < L ? row[t + 1] : 0u;
  return lo | (hi << 16);
}

__device__ inline float softplus_fast(float v) {
  // log(1 + e^v) = ln2 * log2(1 + 2^(v log2 e)); torch returns v above 20
  return v > 20.0f ? v : 0.69314718055994531f * __builtin_amdgcn_logf(1.0f + fast_exp2(v * kLog2e));
}

__device__ inline float silu_fast(float z) {
  return z * __builtin_amdgcn_rcpf(1.0f + fast_exp2(-z * kLog2e));
}

// (lane, lane ^ 32) exchange: returns a_lo + a_hi in the low half and
// b_lo + b_hi in the high half
__device__ inline float fold32(float a, float b) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// row pairs (0,1) and (2,3): returns a summed over the pair in even rows
// and b summed over the pair in odd rows
__device__ inline float fold16(float a, float b) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

template <int MODE>
__global__ __launch_bounds__(NT) void selective_scan_fwd(ScanArgs a) {
  // (delta, delta*u) and (B, C) for two steps per float4; one float4 of
  // padding per row keeps the 16 rows read together in distinct banks
  __shared__ float4 pre[SCH][TP + 1];
  __shared__ float4 bcs[ST][TP + 1];
  // per-wave 4-state sums, [wave][step][channel], padded rows
  __shared__ float part[4][TT][SCH + 1];

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = tid >> 6;
  const int nblk = (a.Dm + SCH - 1) / SCH;
  // work-group -> (batch row, channel block, chunk); the state pass has no
  // work-group for the last chunk, whose end state nothing reads
  const int nwch = MODE == kScanState ? a.nch - 1 : a.nch;
  const int kc = (int)(blockIdx.x % (unsigned)nwch);
  const int grp = (int)(blockIdx.x / (unsigned)nwch);
  const int b = grp / nblk;
  const int d0 = (grp % nblk) * SCH;
  const int tb = kc * a.T;
  const int te = kc == a.nch - 1 ? a.L : tb + a.T;

  // scan identity: channel c, state n
  const int c = lane & 15, r = lane >> 4;
  const int n = 4 * w + r;
  const bool cok = d0 + c < a.Dm;
  const float A2 = cok ? a.A[(int64_t)(d0 + c) * ST + n] * kLog2e : 0.0f;
  // the output pass starts from the carried state the carry pass left in
  // this chunk's segment (read here, before any store overwrites it)
  float x = (MODE == kScanOutput && cok) ? chunk_scratch(a, b, d0 + c, kc)[n] : 0.0f;
  float dsum = 0.0f;  // state pass: this thread's share of the chunk's delta sum

  // stage / store identity: channel sc, steps 2 sp and 2 sp + 1 of a chunk;
  // B / C identity: state tid / 16, same step pair
  const int sc = tid / TP, sp = tid % TP;
  const int sd = d0 + sc;
  const bool sok = sd < a.Dm;
  const int bn = tid / TP;
  const int64_t srow = ((int64_t)b * a.Dm + (sok ? sd : 0)) * a.L;
  const int64_t bcrow = ((int64_t)b * ST + bn) * a.L;
  const float bias = (sok && a.bias) ? a.bias[sd] : 0.0f;
  const float Dd = (sok && a.D) ? a.D[sd] : 0.0f;
  const bool vec = a.vec != 0;

  // the reduced sums a lane holds after the butterfly are for steps
  // 4 m + rs, m = 0..7, with rs = 2 (r & 1) + (r >> 1)
  const int rs = 2 * (r & 1) + (r >> 1);

  uint32_t pu = 0, pdr = 0, pz = 0, pB = 0, pC = 0;
  auto fetch = [&](int t0) {
    const int t = t0 + 2 * sp;
    if (vec && t0 + TT <= a.L) {  // whole chunk in range: one dword per row
      if (sok) {
        pu = *(const uint32_t *)(a.u + srow + t);
        pdr = *(const uint32_t *)(a.dr + srow + t);
        if (MODE != kScanState && a.z) pz = *(const uint32_t *)(a.z + srow + t);
      }
      pB = *(const uint32_t *)(a.Bm + bcrow + t);
      if (MODE != kScanState) pC = *(const uint32_t *)(a.Cm + bcrow + t);
    } else {
      if (sok) {
        pu = load_pair(a.u + srow, t, a.L, vec);
        pdr = load_pair(a.dr + srow, t, a.L, vec);
        pz = (MODE != kScanState && a.z) ? load_pair(a.z + srow, t, a.L, vec) : 0u;
      }
      pB = load_pair(a.Bm + bcrow, t, a.L, vec);
      if (MODE != kScanState) pC = load_pair(a.Cm + bcrow, t, a.L, vec);
    }
  };

  fetch(tb);
  for (int t0 = tb; t0 < te; t0 += TT) {
    // ---- stage
    float du2[2], gate[2];
    {
      const float uu[2] = {lo_bf16(pu), hi_bf16(pu)};
      const float dl[2] = {lo_bf16(pdr), hi_bf16(pdr)};
      const float zz[2] = {lo_bf16(pz), hi_bf16(pz)};
      float4 pv;
      float *pf = reinterpret_cast<float *>(&pv);
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const float v = dl[i] + bias;
        // steps past the end carry delta = 0 and delta*u = 0 (x unchanged)
        const bool in = t0 + 2 * sp + i < a.L;
        const float delta = in ? (a.softplus ? softplus_fast(v) : v) : 0.0f;
        pf[2 * i] = delta;
        pf[2 * i + 1] = delta * uu[i];
        if constexpr (MODE == kScanState) {
          dsum += delta;
        } else {
          du2[i] = Dd * uu[i];
          gate[i] = a.z ? silu_fast(zz[i]) : 1.0f;
        }
      }
      pre[sc][sp] = pv;
      bcs[bn][sp] = make_float4(lo_bf16(pB), lo_bf16(pC), hi_bf16(pB), hi_bf16(pC));
    }
    if (t0 + TT < te) fetch(t0 + TT);
    __syncthreads();

    if constexpr (MODE == kScanState) {
      // the recurrence alone
#pragma unroll
      for (int j = 0; j < TP; ++j) {
        const float4 pd = pre[c][j];
        const float4 q = bcs[n][j];
        x = fmaf(fast_exp2(pd.x * A2), x, pd.y * q.x);
        x = fmaf(fast_exp2(pd.z * A2), x, pd.w * q.z);
      }
      // pre / bcs are rewritten by the next stage only after every wave is
      // done with them
      __syncthreads();
      continue;
    }

    // ---- scan: C_n x_n per step
    float p[TT];
#pragma unroll
    for (int j = 0; j < TP; ++j) {
      const float4 pd = pre[c][j];
      const float4 q = bcs[n][j];
      x = fmaf(fast_exp2(pd.x * A2), x, pd.y * q.x);
      p[2 * j] = q.y * x;
      x = fmaf(fast_exp2(pd.z * A2), x, pd.w * q.z);
      p[2 * j + 1] = q.w * x;
    }
    // ---- reduce over the wave's 4 states (rows): after fold32 lane half h
    // holds steps 2 k + h, after fold16 row r holds steps 4 m + rs
    float h1[TP];
#pragma unroll
    for (int k = 0; k < TP; ++k) h1[k] = fold32(p[2 * k], p[2 * k + 1]);
#pragma unroll
    for (int m = 0; m < TT / 4; ++m) {
      const float s = fold16(h1[2 * m], h1[2 * m + 1]);
      part[w][4 * m + rs][c] = s;
    }
    __syncthreads();

    // ---- store
    if (sok) {
      float yv[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int t = 2 * sp + i;
        const float acc = part[0][t][sc] + part[1][t][sc] + part[2][t][sc] + part[3][t][sc];
        yv[i] = (acc + du2[i]) * gate[i];
      }
      const int t = t0 + 2 * sp;
      uint16_t *yrow = a.y + srow;
      if (vec && t + 1 < a.L) {
        *(uint32_t *)(yrow + t) = Bf16Tag::pack2(yv[0], yv[1]);
      } else {
        if (t < a.L) yrow[t] = Bf16Tag::from_f32(yv[0]);
        if (t + 1 < a.L) yrow[t + 1] = Bf16Tag::from_f32(yv[1]);
      }
    }
    // pre / bcs are rewritten by the next stage only after every wave has
    // passed this chunk's second barrier, and part only after the next
    // chunk's first barrier, which every wave reaches after its stores
  }
  if constexpr (MODE == kScanState) {
    // the chunk's end state and delta sum, at the start of its own segment
    if (cok) chunk_scratch(a, b, d0 + c, kc)[n] = x;
#pragma unroll
    for (int off = 1; off < TP; off <<= 1) dsum += __shfl_xor(dsum, off, 64);
    if (sok && sp == 0) chunk_scratch(a, b, sd, kc)[ST] = dsum;
  }
}

// The carry pass: one lane per (batch row, channel, state) walks the chunks
// in order and leaves each chunk's starting state where its end state was.
__global__ __launch_bounds__(256) void selective_scan_carry(ScanArgs a, int32_t lanes) {
  const int gid = blockIdx.x * 256 + threadIdx.x;
  if (gid >= lanes) return;
  const int n = gid & (ST - 1), bd = gid / ST;
  const int b = bd / a.Dm, d = bd - b * a.Dm;
  const float A2 = a.A[(int64_t)d * ST + n] * kLog2e;
  float carry = 0.0f;
  float *p = chunk_scratch(a, b, d, 0);
  float xe = p[n], S = p[ST];
  for (int k = 0; k + 1 < a.nch; ++k) {
    // the next chunk's summary is read before this chunk's is overwritten
    float *pn = chunk_scratch(a, b, d, k + 1);
    float xe_n = 0.0f, S_n = 0.0f;
    if (k + 2 < a.nch) {
      xe_n = pn[n];
      S_n = pn[ST];
    }
    p[n] = carry;
    carry = fmaf(fast_exp2(A2 * S), carry, xe);
    p = pn;
    xe = xe_n;
    S = S_n;
  }
  p[n] = carry;  // the last chunk's starting state
}

}  // namespace

// Chunking of the sequence-parallel path: used when the single pass would
// launch fewer than kScanFillGroups work-groups (four per CU) and the
// sequence holds at least two 64-step chunks; the chunk count brings the
// launch to about kScanTargetGroups work-groups (five per CU, what the
// single pass gets at config 4). T is a multiple of 32 steps and at least
// 64; the last chunk takes the remainder (T .. 2T - 1 steps). nch = 1: the
// single pass. The chunked path needs the 4-byte pair access (even L).
constexpr int64_t kScanFillGroups = 1024, kScanTargetGroups = 1280, kScanMinChunk = 64;

void scan_chunking(int64_t batch, int64_t dim, int64_t L, bool vec, int32_t *T, int32_t *nch) {
  const int64_t groups = (dim + SCH - 1) / SCH * batch;
  *T = (int32_t)L;
  *nch = 1;
  if (!vec || groups >= kScanFillGroups || L < 2 * kScanMinChunk) return;
  int64_t want = (kScanTargetGroups + groups - 1) / groups;
  want = std::min(want, L / kScanMinChunk);
  if (want < 2) return;
  int64_t t = (L + want - 1) / want;
  t = std::max<int64_t>((t + TT - 1) / TT * TT, kScanMinChunk);
  const int64_t k = L / t;  // the last chunk absorbs the remainder
  if (k < 2) return;
  *T = (int32_t)t;
  *nch = (int32_t)k;
}

bool scan_supported(const ScanLaunch &a, const char **why) {
  if (a.d_state != ST) {
    *why = "selective scan supports d_state 16";
    return false;
  }
  if (a.seq_len > (int64_t)1 << 30 || a.dim > (int64_t)1 << 30 ||
      a.batch * ((a.dim + SCH - 1) / SCH) > (((int64_t)1 << 31) - 1)) {
    *why = "selective scan shape too large for one launch";
    return false;
  }
  return true;
}

hipError_t launch_selective_scan(const ScanLaunch &L, hipStream_t s) {
  ScanArgs a;
  a.u = (const uint16_t *)L.u;
  a.dr = (const uint16_t *)L.delta_raw;
  a.Bm = (const uint16_t *)L.B;
  a.Cm = (const uint16_t *)L.C;
  a.z = (const uint16_t *)L.z;
  a.A = L.A;
  a.D = L.D;
  a.bias = L.delta_bias;
  a.y = (uint16_t *)L.y;
  a.Dm = (int32_t)L.dim;
  a.L = (int32_t)L.seq_len;
  a.softplus = L.delta_softplus;
  auto al4 = [](const void *p) { return ((uintptr_t)p & 3u) == 0; };
  a.vec = (L.seq_len % 2 == 0) && al4(L.u) && al4(L.delta_raw) && al4(L.B) && al4(L.C) &&
          al4(L.y) && (!L.z || al4(L.z));
  const int64_t groups = (L.dim + SCH - 1) / SCH * L.batch;
  scan_chunking(L.batch, L.dim, L.seq_len, a.vec != 0, &a.T, &a.nch);
  if (a.nch <= 1) {
    hipLaunchKernelGGL(selective_scan_fwd<kScanFull>, dim3((unsigned)groups), dim3(NT), 0, s, a);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(selective_scan_fwd<kScanState>, dim3((unsigned)(groups * (a.nch - 1))),
                     dim3(NT), 0, s, a);
  const int64_t lanes = L.batch * L.dim * ST;
  hipLaunchKernelGGL(selective_scan_carry, dim3((unsigned)((lanes + 255) / 256)), dim3(256), 0,
                     s, a, (int32_t)lanes);
  hipLaunchKernelGGL(selective_scan_fwd<kScanOutput>, dim3((unsigned)(groups * a.nch)), dim3(NT),
                     0, s, a);
  return hipGetLastError();
}

}  // namespace neptune
