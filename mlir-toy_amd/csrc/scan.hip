// scan.hip — Mamba-1 selective scan forward on gfx950.
//
// Not in the reference (Evan-Zhao/mlir-toy); the recurrence is the
// selective SSM of Gu & Dao 2023 with mamba_ssm's zero-order-hold
// simplification (B_bar = delta * B):
//   delta = softplus(delta_raw + bias[d])           (torch threshold 20)
//   x_n  <- 2^(delta * A[d,n] * log2 e) x_n + (delta u) B[b,n,l]
//   y     = (sum_n C[b,n,l] x_n + D[d] u) * silu(z)
//
// Mapping: a channel (batch b, inner dim d) is owned by NL adjacent lanes,
// each carrying 16/NL of its fp32 states in registers and walking the
// sequence in order, so no carry ever crosses lanes or work-groups. The
// per-step output reduction over states is an in-row DPP butterfly
// (quad_perm xor1/xor2, row_half_mirror, row_mirror). A 256-thread
// work-group owns 256/NL channels of one batch row and stages 64-step tiles
// through LDS: the channel rows of u / delta_raw / z arrive as coalesced
// 16-byte loads, the per-(channel, step) terms (delta, delta*u, D*u,
// silu(z)) are computed once per tile by the whole group, B and C (shared by
// every channel of the batch row) are read once per tile, and y leaves
// through an LDS tile as coalesced 16-byte stores.
//
// The per-state update (one exp2, one mul, two FMAs) is VALU/transcendental
// work that no layout removes; the kernel is compute-bound, not HBM-bound.
#include "device_common.h"
#include "kernels.h"

namespace neptune {
namespace {

constexpr int ST = 16;     // d_state covered
constexpr int TT = 64;     // steps per LDS tile
constexpr int NT = 256;    // threads per work-group

struct ScanArgs {
  const uint16_t *u, *dr, *Bm, *Cm, *z;
  const float *A, *D, *bias;
  uint16_t *y;
  int32_t Dm, L, softplus;
  int32_t vec;  // rows are 16-byte aligned: L % 8 == 0 and aligned bases
};

template <int CTRL>
__device__ inline float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xf, 0xf, true));
}

// sum over NL adjacent lanes (NL in 1,2,4,8,16), result in every lane
template <int NL>
__device__ inline float group_sum(float x) {
  if (NL >= 2) x += dpp<0xB1>(x);   // quad_perm [1,0,3,2]
  if (NL >= 4) x += dpp<0x4E>(x);   // quad_perm [2,3,0,1]
  if (NL >= 8) x += dpp<0x141>(x);  // row_half_mirror
  if (NL >= 16) x += dpp<0x140>(x); // row_mirror
  return x;
}

template <int NL>
__global__ __launch_bounds__(NT) void selective_scan_fwd(ScanArgs a) {
  constexpr int SPL = ST / NL;     // states per lane
  constexpr int CPB = NT / NL;     // channels per work-group
  constexpr int CPR = TT / 8;      // 16-byte chunks per channel row of a tile
  // rows padded by one element so lanes of different channels / states
  // land in different LDS banks
  __shared__ __attribute__((aligned(16))) float2 pre[CPB][TT + 1];   // (delta, delta*u)
  __shared__ __attribute__((aligned(16))) float2 post[CPB][TT + 1];  // (D*u, silu(z))
  __shared__ __attribute__((aligned(16))) float bc[2][ST][TT + 1];   // B, C
  __shared__ __attribute__((aligned(16))) float yt[CPB][TT + 1];

  const int tid = threadIdx.x;
  const int nblk = (a.Dm + CPB - 1) / CPB;
  const int b = blockIdx.x / nblk;
  const int d0 = (blockIdx.x % nblk) * CPB;

  // compute-phase identity
  const int cw = tid / NL;        // channel within the group
  const int j = tid % NL;         // state slice
  const int dch = d0 + cw;
  float A2[SPL], x[SPL];
#pragma unroll
  for (int s = 0; s < SPL; ++s) {
    A2[s] = dch < a.Dm ? a.A[(int64_t)dch * ST + j * SPL + s] * kLog2e : 0.0f;
    x[s] = 0.0f;
  }

  const int64_t rowbase = ((int64_t)b * a.Dm) * a.L;
  const int64_t bcbase = (int64_t)b * ST * a.L;

  for (int t0 = 0; t0 < a.L; t0 += TT) {
    const int tn = min(TT, a.L - t0);
    // ---- stage: per-(channel, step) terms
    for (int c = tid; c < CPB * CPR; c += NT) {
      const int ch = c / CPR, k8 = c % CPR, dd = d0 + ch;
      const int tt = 8 * k8;
      float uu[8], dl[8], zz[8];
      if (a.vec && dd < a.Dm && t0 + tt + 8 <= a.L) {
        const int64_t off = rowbase + (int64_t)dd * a.L + t0 + tt;
        u32x4 uv = *(const u32x4 *)(a.u + off);
        u32x4 dv = *(const u32x4 *)(a.dr + off);
        u32x4 zv = a.z ? *(const u32x4 *)(a.z + off) : u32x4{0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          uu[2 * i] = __uint_as_float(uv[i] << 16);
          uu[2 * i + 1] = __uint_as_float(uv[i] & 0xffff0000u);
          dl[2 * i] = __uint_as_float(dv[i] << 16);
          dl[2 * i + 1] = __uint_as_float(dv[i] & 0xffff0000u);
          zz[2 * i] = __uint_as_float(zv[i] << 16);
          zz[2 * i + 1] = __uint_as_float(zv[i] & 0xffff0000u);
        }
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          bool ok = dd < a.Dm && t0 + tt + i < a.L;
          int64_t off = rowbase + (int64_t)dd * a.L + t0 + tt + i;
          uu[i] = ok ? Bf16Tag::to_f32(a.u[off]) : 0.0f;
          dl[i] = ok ? Bf16Tag::to_f32(a.dr[off]) : 0.0f;
          zz[i] = ok && a.z ? Bf16Tag::to_f32(a.z[off]) : 0.0f;
        }
      }
      const float bias = (dd < a.Dm && a.bias) ? a.bias[dd] : 0.0f;
      const float Dd = (dd < a.Dm && a.D) ? a.D[dd] : 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float v = dl[i] + bias;
        float delta = a.softplus ? (v > 20.0f ? v : log1pf(__expf(v))) : v;
        float gate = a.z ? zz[i] / (1.0f + __expf(-zz[i])) : 1.0f;
        pre[ch][tt + i] = make_float2(delta, delta * uu[i]);
        post[ch][tt + i] = make_float2(Dd * uu[i], gate);
      }
    }
    for (int c = tid; c < 2 * ST * CPR; c += NT) {
      const int which = c / (ST * CPR), r = (c / CPR) % ST, tt = 8 * (c % CPR);
      const uint16_t *src = which ? a.Cm : a.Bm;
      const int64_t off = bcbase + (int64_t)r * a.L + t0 + tt;
      if (a.vec && t0 + tt + 8 <= a.L) {
        u32x4 v = *(const u32x4 *)(src + off);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          bc[which][r][tt + 2 * i] = __uint_as_float(v[i] << 16);
          bc[which][r][tt + 2 * i + 1] = __uint_as_float(v[i] & 0xffff0000u);
        }
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i)
          bc[which][r][tt + i] = t0 + tt + i < a.L ? Bf16Tag::to_f32(src[off + i]) : 0.0f;
      }
    }
    __syncthreads();

    // ---- recurrence over the tile
    for (int t = 0; t < tn; ++t) {
      const float2 pd = pre[cw][t];
      float acc = 0.0f;
#pragma unroll
      for (int s = 0; s < SPL; ++s) {
        const int nn = j * SPL + s;
        const float da = fast_exp2(pd.x * A2[s]);
        x[s] = fmaf(da, x[s], pd.y * bc[0][nn][t]);
        acc = fmaf(bc[1][nn][t], x[s], acc);
      }
      acc = group_sum<NL>(acc);
      if (j == 0) {
        const float2 po = post[cw][t];
        yt[cw][t] = (acc + po.x) * po.y;
      }
    }
    __syncthreads();

    // ---- y tile out (bf16, coalesced)
    for (int c = tid; c < CPB * CPR; c += NT) {
      const int ch = c / CPR, tt = 8 * (c % CPR), dd = d0 + ch;
      if (dd >= a.Dm) continue;
      const int64_t off = rowbase + (int64_t)dd * a.L + t0 + tt;
      if (a.vec && t0 + tt + 8 <= a.L) {
        u32x4 v;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          v[i] = Bf16Tag::pack2(yt[ch][tt + 2 * i], yt[ch][tt + 2 * i + 1]);
        *(u32x4 *)(a.y + off) = v;
      } else {
        for (int i = 0; i < 8 && t0 + tt + i < a.L; ++i)
          a.y[off + i] = Bf16Tag::from_f32(yt[ch][tt + i]);
      }
    }
    // the next tile's staging writes pre/post/bc only after every wave has
    // finished reading them
    __syncthreads();
  }
}

}  // namespace

constexpr int kScanLanes = 8;

bool scan_supported(const ScanLaunch &a, const char **why) {
  if (a.d_state != ST) {
    *why = "selective scan supports d_state 16";
    return false;
  }
  if (a.seq_len > (int64_t)1 << 30 || a.dim > (int64_t)1 << 30 || a.batch > 65535) {
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
  auto al16 = [](const void *p) { return ((uintptr_t)p & 15u) == 0; };
  a.vec = (L.seq_len % 8 == 0) && al16(L.u) && al16(L.delta_raw) && al16(L.B) &&
          al16(L.C) && al16(L.y) && (!L.z || al16(L.z));
  constexpr int CPB = NT / kScanLanes;
  const int nblk = (int)((L.dim + CPB - 1) / CPB);
  hipLaunchKernelGGL(selective_scan_fwd<kScanLanes>, dim3((unsigned)(nblk * L.batch)), dim3(NT), 0,
                     s, a);
  return hipGetLastError();
}

}  // namespace neptune
