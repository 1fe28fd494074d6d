// scan.hip — Mamba-1 selective scan forward on gfx950.
//
// Not in the reference (Evan-Zhao/mlir-toy); the recurrence is the
// selective SSM of Gu & Dao 2023 with mamba_ssm's zero-order-hold
// simplification (B_bar = delta * B):
//   delta = softplus(delta_raw + bias[d])           (torch threshold 20)
//   x_n  <- 2^(delta * A[d,n] * log2 e) x_n + (delta u) B[b,n,l]
//   y     = (sum_n C[b,n,l] x_n + D[d] u) * silu(z)
//
// The per-state update (one exp2, two multiplies, one FMA) and the output
// term (one FMA per state) are VALU/transcendental work: 16 states per
// (channel, step) against 8 bytes of HBM traffic, so the kernel is bound by
// the VALU, not by HBM, and is laid out to spend as little of it as
// possible beyond those five instructions per state:
//
// Mapping: a 256-thread work-group owns 16 channels of one batch row; wave w
// owns channels 4 w .. 4 w + 3 with all their states: lane (row q = lane /
// 16, column n = lane % 16) carries the fp32 state n of channel 4 w + q and
// walks the sequence in order, so no carry crosses lanes. 16-channel
// work-groups give every CU the same share of channels (batch * dim / 16
// groups) and one state per lane gives five resident wavefronts per SIMD at
// config 4 to hide the exp2 -> FMA chain.
//
// Per 32-step chunk:
//   stage  lane (q, j) loads u, delta_raw and z of its channel at steps j
//          and j + 16, and keeps (delta log2 e, delta u) for the scan and
//          u ln2 and silu(z) for the two outputs it forms itself; B and C of
//          one state and two steps go to LDS, double-buffered by chunk
//          parity, so one barrier per chunk suffices. The next chunk's loads
//          are issued before the scan and first waited for by the next stage.
//          Working in log2 units, delta log2 e is one FMA of delta_raw (plus
//          the softplus, whose exp2 / log2 take it directly), the decay is
//          2^(delta log2 e * A), and the output's D u is (D log2 e)(u ln2)
//          inside one FMA.
//   scan   in two halves of 16 steps: step j's (delta log2 e, delta u) comes
//          from lane j of the row by DPP row broadcast inside the two
//          multiplies that use it (v_mul_f32_dpp row_newbcast: no extra
//          instruction), and after each step the lane writes x to its wave's
//          LDS rows;
//   output lane (q, j) then forms y of its channel at step 16 h + j as
//          sum_n C_n x_n with 16 FMAs over four 16-byte reads of the states
//          and four of C, and applies D*u and the gate; the chunk's two
//          bf16 outputs per lane are stored in the next chunk.
// Every exchange of states stays inside the wave that wrote them (a wave's
// LDS operations execute in order), so the scan and the output need no
// barrier between them, and the output term costs one FMA per state where
// a cross-lane reduction of C_n x_n costs a multiply plus exchanges.
//
// Memory waits: loads and stores share the vector-memory counter, so a wait
// for the fetched data also waits for every store issued before it. The
// chunk loop therefore runs in pairs with two register sets for the loads
// (the parity, and the LDS offsets it selects, are constants), stores each
// chunk's outputs after the next chunk's fetch and barrier, unconditionally
// (a lane without an output stores out of range), and keeps their data
// registers until the stores are old; its barrier orders LDS only, so the
// stores stay in flight across it. Each chunk then waits for its own data
// with the two newest stores still outstanding.
//
// Addressing: u, delta_raw, z, y, B and C go through buffer resources. A
// lane's offset is fixed for the launch; each chunk's resources start at
// its first step and end with the channel block (B, C: the batch row), in
// scalar registers, so the per-chunk address work is scalar and the
// hardware range check reads 0 for a load past the end of the block.
// Steps past the end of the sequence (in its last chunk) are not masked:
// they read the next row of the block, or 0, and scan on. They come after
// every real step of the chunk, their states only reach the LDS rows of
// their own steps, whose outputs are not stored, and the last chunk's end
// state is never read, so whatever they compute goes nowhere.
//
// Sequence-parallel path. When batch * dim / 16 work-groups cannot fill the
// GPU (few channels, long sequences), the sequence is cut into nch chunks of
// nearly equal length (whole 32-step units, at least two per chunk) and the
// scan runs in three launches, using y itself as scratch (no workspace):
//   state   every chunk but the last scans from x = 0 without outputs and
//           leaves its end state x_end[16] and its delta sum S (fp32) at the
//           start of its own y segment (64 steps or more: 128 bytes >= 68);
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
  // chunks of the sequence (1: the single pass): chunk k starts at step
  // chunk_start(k); the first rem hold Tu + 1 units of 32 steps, the others Tu
  // (the last also the partial unit at the end)
  int32_t Tu, rem, nch;
};

// the output kernel as the single pass, and as the chunked path's output pass
enum ScanMode { kScanFull = 0, kScanOutput = 1 };

// chunk k of channel d of batch row b: its y segment as fp32 scratch
// (x[16], then S)
__device__ inline int chunk_start(const ScanArgs &a, int k) {
  return TT * (k * a.Tu + min(k, a.rem));
}
__device__ inline float *chunk_scratch(const ScanArgs &a, int b, int d, int k) {
  return reinterpret_cast<float *>(a.y + ((int64_t)b * a.Dm + d) * a.L + chunk_start(a, k));
}



__device__ inline float silu_fast(float z) {
  return z * __builtin_amdgcn_rcpf(1.0f + fast_exp2(-z * kLog2e));
}

// softplus's linear branch (torch: delta_raw + bias above 20), in log2 units
constexpr float kSoftplusLinear2 = 20.0f * kLog2e;

// The state pass of the chunked path: the recurrence alone, from x = 0, over
// every chunk but the last; leaves the chunk's end state and delta sum at
// the start of its own y segment.
template <bool SOFTPLUS>
__global__ __launch_bounds__(NT) void selective_scan_state(ScanArgs a) {
  // (delta log2 e, delta u) for two steps per float4, and B of one state for
  // two steps, double-buffered by chunk parity (one barrier per chunk); one
  // float4 of padding per row keeps the 16 rows read together in distinct
  // banks
  __shared__ float4 pre[2][SCH][TP + 1];
  __shared__ float2 bsh[2][ST][TP + 2];

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = tid >> 6;
  const int nblk = (a.Dm + SCH - 1) / SCH;
  // work-group -> (batch row, channel block, chunk); no work-group for the
  // last chunk, whose end state nothing reads
  const int nwch = a.nch - 1;
  const int kc = (int)(blockIdx.x % (unsigned)nwch);
  const int grp = (int)(blockIdx.x / (unsigned)nwch);
  const int b = grp / nblk;
  const int d0 = (grp % nblk) * SCH;
  const int tb = chunk_start(a, kc);
  const int te = chunk_start(a, kc + 1);

  // scan identity: channel c, state n; the decay is 2^(delta log2 e * A)
  const int c = lane & 15, r = lane >> 4;
  const int n = 4 * w + r;
  const bool cok = d0 + c < a.Dm;
  const float Ac = cok ? a.A[(int64_t)(d0 + c) * ST + n] : 0.0f;
  float x = 0.0f;
  float dsum = 0.0f;  // this thread's share of the chunk's delta log2 e

  // stage identity: channel sc, steps 2 sp and 2 sp + 1 of a chunk; B
  // identity: state tid / 16, same step pair
  const int sc = tid / TP, sp = tid % TP;
  const int sd = d0 + sc;
  const bool sok = sd < a.Dm;
  const int bn = tid / TP;
  // rows past the last channel read the block's first row (unused)
  const int64_t srow = ((int64_t)b * a.Dm + (sok ? sd : d0)) * a.L;
  const int64_t bcrow = ((int64_t)b * ST + bn) * a.L;
  const float bias2 = (sok && a.bias) ? a.bias[sd] * kLog2e : 0.0f;

  // every chunk of this pass lies inside the sequence, and so does the step
  // pair after it (the last chunk follows), so the loads need no guard; the
  // path needs even L and 4-byte aligned rows, so a step pair is one dword
  uint32_t pu, pdr, pB;
  auto fetch = [&](int t0) {
    const int t = t0 + 2 * sp;
    pu = *(const uint32_t *)(a.u + srow + t);
    pdr = *(const uint32_t *)(a.dr + srow + t);
    pB = *(const uint32_t *)(a.Bm + bcrow + t);
  };

  fetch(tb);
  for (int t0 = tb, par = 0; t0 < te; t0 += TT, par ^= 1) {
    {
      const float uu[2] = {__uint_as_float(pu << 16), __uint_as_float(pu & 0xffff0000u)};
      const float dr[2] = {__uint_as_float(pdr << 16), __uint_as_float(pdr & 0xffff0000u)};
      float4 pv;
      float *pf = reinterpret_cast<float *>(&pv);
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        // (delta_raw + bias) log2 e, and delta log2 e = log2(1 + 2^that)
        // below the linear branch
        const float v2 = fmaf(dr[i], kLog2e, bias2);
        const float d2 =
            SOFTPLUS && !(v2 > kSoftplusLinear2) ? __builtin_amdgcn_logf(1.0f + fast_exp2(v2)) : v2;
        pf[2 * i] = d2;
        pf[2 * i + 1] = d2 * (uu[i] * kLn2);
        dsum += d2;
      }
      pre[par][sc][sp] = pv;
      bsh[par][bn][sp] = make_float2(__uint_as_float(pB << 16), __uint_as_float(pB & 0xffff0000u));
    }
    fetch(t0 + TT);
    // this chunk's buffers are next written two chunks on, behind the next
    // chunk's barrier, which every wave reaches after its reads of this one
    __syncthreads();
#pragma unroll
    for (int j = 0; j < TP; ++j) {
      const float4 pd = pre[par][c][j];
      const float2 q = bsh[par][n][j];
      x = fmaf(fast_exp2(pd.x * Ac), x, pd.y * q.x);
      x = fmaf(fast_exp2(pd.z * Ac), x, pd.w * q.y);
    }
  }
  if (cok) chunk_scratch(a, b, d0 + c, kc)[n] = x;
#pragma unroll
  for (int off = 1; off < TP; off <<= 1) dsum += __shfl_xor(dsum, off, 64);
  if (sok && sp == 0) chunk_scratch(a, b, sd, kc)[ST] = dsum * kLn2;  // natural units
}

// Cross-lane exchange through LDS inside one wave: the wave's LDS
// operations execute in order, so only the compiler must keep the accesses
// on either side of this point in program order.
__device__ inline void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Work-group barrier that orders LDS only. A __syncthreads() fence also
// orders global memory, so it waits for every store issued before it; the
// output kernel's barriers exchange LDS data only, and its stores may stay
// in flight across them.
__device__ inline void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Lane J of each 16-lane row, broadcast to the whole row (DPP row_newbcast);
// folded into the VOP2 that consumes it
template <int J>
__device__ inline float row_bcast(float v) {
  static_assert(J >= 0 && J < 16, "row lane");
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x150 + J, 0xf, 0xf, false));
}

// LDS rows of the output kernel: a wave's states of one step (a step's 64
// writes fill 64 consecutive banks; the output's 16-byte reads of 16 steps
// measure two LDS passes where one is the minimum, and a channel-major
// layout that reads in one pass measured no faster), C of one step, B of one
// state
constexpr int XR = 4 * ST + 4;  // floats per xs row
constexpr int CR = ST + 4;      // floats per C row
constexpr int BR = TT + 4;      // floats per B row

// a pointer the same for every lane of the work-group, read from the first
// lane so that it and what is derived from it stay in scalar registers
template <class T>
__device__ inline T *uniform_ptr(T *p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  return reinterpret_cast<T *>(((uint64_t)__builtin_amdgcn_readfirstlane((uint32_t)(v >> 32)) << 32) |
                               (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)v));
}

// buffer resource over [base, base + bytes) (base and bytes uniform): loads
// at or past the end read 0, stores there are dropped
__device__ inline __amdgpu_buffer_rsrc_t byte_range(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes,
                                           0x00020000);
}

// a byte offset past every output resource (at most 16 rows x 2 x 2^26
// bytes): a store there is dropped by the range check
constexpr uint32_t kDropped = 0x80000000u;

// The single pass (kScanFull), and the output pass of the chunked path;
// SOFTPLUS and GATE (z given) are fixed per launch, and so is PAIRS: B and C
// come in 4-byte step pairs (even seq_len, 4-byte aligned rows), so each
// stage lane fetches its two steps of B and of C with one dword load each
// (a chunk's loads are 8 rather than 10; measured 2% faster at config 4).
// Five work-groups per CU (at most 96 VGPRs): what config 4's 1280
// work-groups need to run in one round.
template <int MODE, bool SOFTPLUS, bool GATE, bool PAIRS>
__global__ __launch_bounds__(NT, 5) void selective_scan_out(ScanArgs a) {
  static_assert(MODE == kScanFull || MODE == kScanOutput, "output kernel modes");
  __shared__ __attribute__((aligned(16))) float xs[4][TT / 2][XR];    // [wave][step][lane]
  __shared__ __attribute__((aligned(16))) float bq[2][ST][BR];        // B [parity][state][step]
  __shared__ __attribute__((aligned(16))) float cs[2][TT][CR];        // C [parity][step][state]

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = tid >> 6;
  const int nblk = (a.Dm + SCH - 1) / SCH;
  // work-group -> (batch row, channel block, chunk)
  // (the divisions run on the vector unit: their results are taken back to
  // scalar registers so that every address derived from them stays scalar)
  const int kc = __builtin_amdgcn_readfirstlane((int)(blockIdx.x % (unsigned)a.nch));
  const int grp = (int)(blockIdx.x / (unsigned)a.nch);
  const int b = __builtin_amdgcn_readfirstlane(grp / nblk);
  const int d0 = __builtin_amdgcn_readfirstlane((grp % nblk) * SCH);
  const int tb = chunk_start(a, kc);
  const int te = kc == a.nch - 1 ? a.L : chunk_start(a, kc + 1);

  const int q = lane >> 4, n = lane & 15;
  const int ch = d0 + 4 * w + q;  // this lane's channel
  const bool cok = ch < a.Dm;
  // the decay 2^(delta log2 e * A) takes A as it is
  const float Ac = cok ? a.A[(int64_t)ch * ST + n] : 0.0f;
  // the output pass starts from the carried state the carry pass left in
  // this chunk's segment; every thread holds it (the load retired, below)
  // before the first barrier, and the work-group's first store follows that
  // barrier
  float x = (MODE == kScanOutput && cok) ? chunk_scratch(a, b, ch, kc)[n] : 0.0f;
  const float bias2 = (cok && a.bias) ? a.bias[ch] * kLog2e : 0.0f;
  const float D2 = (cok && a.D) ? a.D[ch] * kLog2e : 0.0f;  // times u ln2: D u
  // B / C identity: state bn, steps 2 sp and 2 sp + 1
  const int bn = tid >> 4, sp = tid & 15;

  // rows of this channel block (u, delta_raw, z, y) and of this batch row
  // (B, C); lanes past the last channel read the block's first row (their
  // states are never stored)
  const int64_t blk = ((int64_t)b * a.Dm + d0) * a.L, bcb = (int64_t)b * ST * a.L;
  const uint32_t rbytes = (uint32_t)(min(SCH, a.Dm - d0) * 2 * a.L);
  const uint32_t bcbytes = (uint32_t)(ST * 2 * a.L);
  const uint16_t *ub = uniform_ptr(a.u + blk), *drb = uniform_ptr(a.dr + blk);
  const uint16_t *zb = uniform_ptr((GATE ? a.z : a.u) + blk);
  const uint16_t *Bb = uniform_ptr(a.Bm + bcb), *Cb = uniform_ptr(a.Cm + bcb);
  const auto ry = byte_range(uniform_ptr(a.y + blk), rbytes);
  const uint32_t vo = (uint32_t)(((cok ? 4 * w + q : 0) * a.L + n) * 2);
  const uint32_t vbc = (uint32_t)((bn * a.L + 2 * sp) * 2);
  // Two register sets for the loads: a chunk of parity P stages from set P
  // and fetches the next chunk into set 1 - P (the chunk loop runs in pairs,
  // so the parity and every LDS offset derived from it are constants)
  uint32_t fu[2][2], fdr[2][2], fz[2][2], fB[2][2], fC[2][2];
  // (issued unconditionally: past the end of the sequence the resources
  // cover 0 bytes and the loads read 0)
  auto fetch = [&](auto S, int t0) {
    constexpr int set = decltype(S)::value;
    const uint32_t rb = t0 < a.L ? rbytes - 2 * t0 : 0, bcb2 = t0 < a.L ? bcbytes - 2 * t0 : 0;
    const auto ru = byte_range(ub + t0, rb);
    const auto rdr = byte_range(drb + t0, rb);
    const auto rz = byte_range(zb + t0, rb);
    const auto rB = byte_range(Bb + t0, bcb2);
    const auto rC = byte_range(Cb + t0, bcb2);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      fu[set][i] = __builtin_amdgcn_raw_buffer_load_b16(ru, vo + 32 * i, 0, 0);
      fdr[set][i] = __builtin_amdgcn_raw_buffer_load_b16(rdr, vo + 32 * i, 0, 0);
      if constexpr (GATE)
        fz[set][i] = __builtin_amdgcn_raw_buffer_load_b16(rz, vo + 32 * i, 0, 0);
      if constexpr (!PAIRS) {
        fB[set][i] = __builtin_amdgcn_raw_buffer_load_b16(rB, vbc + 2 * i, 0, 0);
        fC[set][i] = __builtin_amdgcn_raw_buffer_load_b16(rC, vbc + 2 * i, 0, 0);
      }
    }
    if constexpr (PAIRS) {  // steps 2 sp and 2 sp + 1 in one dword
      fB[set][0] = __builtin_amdgcn_raw_buffer_load_b32(rB, vbc, 0, 0);
      fC[set][0] = __builtin_amdgcn_raw_buffer_load_b32(rC, vbc, 0, 0);
    }
  };

  float *xw = &xs[w][0][lane];            // this lane's state at step 0
  const float *xr = &xs[w][n][16 * q];    // row of the output at step n

  // A chunk's two outputs per lane are stored in the next chunk, after its
  // fetch and barrier: the next wait on the vector-memory counter (shared by
  // loads and stores) is then a chunk away, so it never waits on a store
  // issued just before it
  // The stores are issued by every lane, unconditionally, so that the
  // compiler counts them exactly: a lane with no output (past the end of
  // the sequence, or past the last channel) stores past the resource's
  // range, where the hardware drops it.
  uint16_t yq[2] = {0, 0};
  auto store_outputs = [&](int tp) {  // tp: the chunk's first step
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const bool live = cok && n < a.L - tp - 16 * h;
      __builtin_amdgcn_raw_buffer_store_b16(yq[h], ry, live ? vo + 32 * h + 2 * tp : kDropped, 0, 0);
    }
  };

  // the 32-step chunk from t0, of parity P; the first one has no previous
  // outputs to store
  auto chunk = [&](auto P, auto FIRST, int t0) {
    constexpr int par = decltype(P)::value;
    // ---- stage
    // (delta log2 e, delta u) of steps n and n + 16 of this row's channel:
    // the scan takes step j's from lane j of the row
    float ul[2], gate[2], dl[2], dlu[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const float uln2 = __uint_as_float(fu[par][i] << 16) * kLn2;
      // (delta_raw + bias) log2 e, and delta log2 e = log2(1 + 2^that)
      // below the linear branch
      const float v2 = fmaf(__uint_as_float(fdr[par][i] << 16), kLog2e, bias2);
      const float d2 =
          SOFTPLUS && !(v2 > kSoftplusLinear2) ? __builtin_amdgcn_logf(1.0f + fast_exp2(v2)) : v2;
      dl[i] = d2;
      dlu[i] = d2 * uln2;
      ul[i] = uln2;
      gate[i] = GATE ? silu_fast(__uint_as_float(fz[par][i] << 16)) : 1.0f;
    }
    // step 2 sp + i of B or C: the high half of the pair's dword (PAIRS), or
    // register i
    auto bc = [&](const uint32_t(&r)[2], int i) {
      return __uint_as_float(PAIRS ? (i ? r[0] & 0xffff0000u : r[0] << 16) : r[i] << 16);
    };
    *(float2 *)&bq[par][bn][2 * sp] = make_float2(bc(fB[par], 0), bc(fB[par], 1));
    cs[par][2 * sp][bn] = bc(fC[par], 0);
    cs[par][2 * sp + 1][bn] = bc(fC[par], 1);
    fetch(std::integral_constant<int, 1 - par>{}, t0 + TT);
    // B / C of this chunk are visible to every wave; cs[par] and bq[par]
    // are next written two chunks on, behind the next chunk's barrier,
    // which every wave reaches after its reads of this chunk
    lds_barrier();
    if constexpr (!decltype(FIRST)::value) store_outputs(t0 - TT);

#pragma unroll
    for (int h = 0; h < 2; ++h) {
      // ---- scan: steps 16 h .. 16 h + 15
      const float dlh = dl[h], dluh = dlu[h];
      float4 bv;
      static_for<16>([&](auto J) {
        constexpr int j = decltype(J)::value;
        if constexpr (j % 4 == 0) bv = *(const float4 *)&bq[par][n][16 * h + j];
        const float bj = j % 4 == 0 ? bv.x : j % 4 == 1 ? bv.y : j % 4 == 2 ? bv.z : bv.w;
        x = fmaf(fast_exp2(row_bcast<j>(dlh) * Ac), x, row_bcast<j>(dluh) * bj);
        xw[j * XR] = x;
      });
      wave_lds_sync();
      // the previous chunk's outputs, stored after this chunk's barrier,
      // keep their registers until here: writing over a store's data
      // register waits for that store
      if (h == 0) asm volatile("" ::"v"(yq[0]), "v"(yq[1]));
      // ---- output: this lane's channel at step 16 h + n
      {
        const float *cr = &cs[par][16 * h + n][0];
        float acc0 = 0.0f, acc1 = 0.0f;
#pragma unroll
        for (int k = 0; k < 4; k += 2) {
          const float4 x0 = *(const float4 *)(xr + 4 * k);
          const float4 c0 = *(const float4 *)(cr + 4 * k);
          const float4 x1 = *(const float4 *)(xr + 4 * k + 4);
          const float4 c1 = *(const float4 *)(cr + 4 * k + 4);
          acc0 = fmaf(c0.x, x0.x, acc0);
          acc1 = fmaf(c1.x, x1.x, acc1);
          acc0 = fmaf(c0.y, x0.y, acc0);
          acc1 = fmaf(c1.y, x1.y, acc1);
          acc0 = fmaf(c0.z, x0.z, acc0);
          acc1 = fmaf(c1.z, x1.z, acc1);
          acc0 = fmaf(c0.w, x0.w, acc0);
          acc1 = fmaf(c1.w, x1.w, acc1);
        }
        const float yv = fmaf(D2, ul[h], acc0 + acc1);
        yq[h] = Bf16Tag::from_f32(GATE ? yv * gate[h] : yv);
        // formed here, not sunk past the next half's scan with its 32
        // operands held live (the store is a chunk away)
        asm volatile("" ::"v"(yq[h]));
      }
      // the next half (or chunk) rewrites xs only after these reads
      wave_lds_sync();
    }
  };

  using P0 = std::integral_constant<int, 0>;
  using P1 = std::integral_constant<int, 1>;
  fetch(P0{}, tb);
  if constexpr (MODE == kScanOutput) asm volatile("" ::"v"(x));  // the load of x has retired
  chunk(P0{}, std::true_type{}, tb);
  for (int t0 = tb + TT; t0 < te; t0 += 2 * TT) {
    chunk(P1{}, std::false_type{}, t0);
    if (t0 + TT < te) chunk(P0{}, std::false_type{}, t0 + TT);
  }
  store_outputs(tb + (te - tb - 1) / TT * TT);  // the last chunk's
}

// The carry pass: one lane per (batch row, channel, state) walks the chunks
// in order and leaves each chunk's starting state where its end state was.
// The walk depends on memory only through the chunk summaries, which do not
// depend on it: they are read KB chunks at a time, one batch ahead of the
// walk, in two register sets, so a sequence cut into hundreds of chunks
// waits on memory about once rather than once per chunk. A batch is read
// before any of its chunks is written (the summary a lane reads and the
// starting state it writes share the chunk's slot n).
constexpr int KB = 16;
__global__ __launch_bounds__(256) void selective_scan_carry(ScanArgs a, int32_t lanes) {
  const int gid = blockIdx.x * 256 + threadIdx.x;
  if (gid >= lanes) return;
  const int n = gid & (ST - 1), bd = gid / ST;
  const int b = bd / a.Dm, d = bd - b * a.Dm;
  const float A2 = a.A[(int64_t)d * ST + n] * kLog2e;
  const int nsum = a.nch - 1;  // chunks with a summary: all but the last
  float xe[2][KB], S[2][KB];
  auto load = [&](auto SET, int k0) {
    constexpr int set = decltype(SET)::value;
#pragma unroll
    for (int i = 0; i < KB; ++i) {
      // past the last summary: re-read it (the value is not used)
      const float *p = chunk_scratch(a, b, d, min(k0 + i, nsum - 1));
      xe[set][i] = p[n];
      S[set][i] = p[ST];
    }
  };
  float carry = 0.0f;
  auto walk = [&](auto SET, int k0) {
    constexpr int set = decltype(SET)::value;
#pragma unroll
    for (int i = 0; i < KB; ++i)
      if (k0 + i < nsum) {
        chunk_scratch(a, b, d, k0 + i)[n] = carry;
        carry = fmaf(fast_exp2(A2 * S[set][i]), carry, xe[set][i]);
      }
  };
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  load(S0{}, 0);
  for (int k0 = 0; k0 < nsum; k0 += 2 * KB) {
    load(S1{}, k0 + KB);
    walk(S0{}, k0);
    load(S0{}, k0 + 2 * KB);
    walk(S1{}, k0 + KB);
  }
  chunk_scratch(a, b, d, nsum)[n] = carry;  // the last chunk's starting state
}

// The carry pass for long chains of chunks (more than 64 summaries): one
// wave per (batch row, channel, state), 64 chunks per pass, one per lane.
// Chunk k maps its starting state x to a_k x + b_k (a_k = 2^(A S_k log2 e),
// b_k its end state from 0); an inclusive scan of these affine maps across
// the lanes (Hillis-Steele, six shuffles) gives every lane the map from the
// pass's starting state to the end of its chunk, so its chunk's starting
// state is the previous lane's map applied to that state. The pass's loads
// are independent, so a chain of hundreds of chunks waits on memory once
// per 64 chunks. Lanes past the last summary carry the identity map.
__global__ __launch_bounds__(256) void selective_scan_carry_wave(ScanArgs a, int32_t rows) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int lane = threadIdx.x & 63;
  const int n = row & (ST - 1), bd = row / ST;
  const int b = bd / a.Dm, d = bd - b * a.Dm;
  const float A2 = a.A[(int64_t)d * ST + n] * kLog2e;
  const int nsum = a.nch - 1;
  float carry = 0.0f;  // the state at the start of the pass (the same in every lane)
  for (int k0 = 0; k0 < nsum; k0 += 64) {
    const int k = k0 + lane;
    const bool live = k < nsum;
    const float *p = chunk_scratch(a, b, d, live ? k : nsum - 1);
    float m = live ? fast_exp2(A2 * p[ST]) : 1.0f;  // this lane's map: x -> m x + c
    float c = live ? p[n] : 0.0f;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      // compose with the map of the lanes before: x -> m (m' x + c') + c
      const float mp = __shfl_up(m, off, 64), cp = __shfl_up(c, off, 64);
      if (lane >= off) {
        c = fmaf(m, cp, c);
        m *= mp;
      }
    }
    // this chunk starts where the lanes before it end
    const float mp = __shfl_up(m, 1, 64), cp = __shfl_up(c, 1, 64);
    const float start = lane == 0 ? carry : fmaf(mp, carry, cp);
    if (live) chunk_scratch(a, b, d, k)[n] = start;
    carry = fmaf(__shfl(m, 63, 64), carry, __shfl(c, 63, 64));
  }
  if (lane == 0) chunk_scratch(a, b, d, nsum)[n] = carry;  // the last chunk's starting state
}

}  // namespace

// Chunking of the sequence-parallel path: used when the single pass would
// launch fewer than kScanFillGroups work-groups (four per CU) and the
// sequence holds at least two 64-step chunks; the chunk count brings the
// launch to about kScanTargetGroups work-groups (five per CU, what the
// single pass gets at config 4). The whole 32-step units of the sequence
// are dealt out evenly: every chunk holds Tu or Tu + 1 units (Tu >= 2), the
// last one also the partial unit at the end, so no chunk holds up its
// launch by more than 32 steps. nch = 1: the single pass. The chunked path
// needs the 4-byte pair access (even L).
constexpr int64_t kScanFillGroups = 1024, kScanTargetGroups = 1280, kScanMinChunk = 64;
constexpr int64_t kScanMaxSeq = (int64_t)1 << 26;  // 16 rows x 2 bytes x 2^26 = 2^31

void scan_chunking(int64_t batch, int64_t dim, int64_t L, bool vec, int32_t *Tu, int32_t *rem,
                   int32_t *nch) {
  const int64_t groups = (dim + SCH - 1) / SCH * batch;
  *Tu = 0;
  *rem = 0;
  *nch = 1;
  if (!vec || groups >= kScanFillGroups || L < 2 * kScanMinChunk) return;
  const int64_t units = L / TT;
  int64_t want = (kScanTargetGroups + groups - 1) / groups;
  want = std::min(want, units / (kScanMinChunk / TT));
  if (want < 2) return;
  *nch = (int32_t)want;
  *Tu = (int32_t)(units / want);
  *rem = (int32_t)(units % want);
}

bool scan_supported(const ScanLaunch &a, const char **why) {
  if (a.d_state != ST) {
    *why = "selective scan supports d_state 16";
    return false;
  }
  // the output kernel addresses a channel block (16 rows) and a batch row of
  // B / C (16 rows) through 32-bit byte offsets
  if (a.seq_len >= kScanMaxSeq) {
    *why = "selective scan supports seq_len below 2^26";
    return false;
  }
  if (a.dim > (int64_t)1 << 30 ||
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
  scan_chunking(L.batch, L.dim, L.seq_len, a.vec != 0, &a.Tu, &a.rem, &a.nch);
  const bool sp = L.delta_softplus != 0, gate = L.z != nullptr;
  // the output kernel for this mode and these options
  auto out = [&](auto mode, unsigned grid) {
    constexpr int M = decltype(mode)::value;
    auto pick = [&](auto PAIRS) {
      constexpr bool P = decltype(PAIRS)::value;
      return sp ? (gate ? selective_scan_out<M, true, true, P> : selective_scan_out<M, true, false, P>)
                : (gate ? selective_scan_out<M, false, true, P> : selective_scan_out<M, false, false, P>);
    };
    auto k = a.vec ? pick(std::true_type{}) : pick(std::false_type{});
    hipLaunchKernelGGL(k, dim3(grid), dim3(NT), 0, s, a);
  };
  if (a.nch <= 1) {
    out(std::integral_constant<int, kScanFull>{}, (unsigned)groups);
    return hipGetLastError();
  }
  const dim3 sgrid((unsigned)(groups * (a.nch - 1)));
  if (L.delta_softplus)
    hipLaunchKernelGGL(selective_scan_state<true>, sgrid, dim3(NT), 0, s, a);
  else
    hipLaunchKernelGGL(selective_scan_state<false>, sgrid, dim3(NT), 0, s, a);
  const int64_t lanes = L.batch * L.dim * ST;
  // a long chain of chunks: one wave per (batch, channel, state); up to 64
  // summaries the per-lane walk measured as fast or faster
  if (a.nch - 1 > 4 * KB)
    hipLaunchKernelGGL(selective_scan_carry_wave, dim3((unsigned)((lanes + 3) / 4)), dim3(256), 0,
                       s, a, (int32_t)lanes);
  else
    hipLaunchKernelGGL(selective_scan_carry, dim3((unsigned)((lanes + 255) / 256)), dim3(256), 0,
                       s, a, (int32_t)lanes);
  out(std::integral_constant<int, kScanOutput>{}, (unsigned)(groups * a.nch));
  return hipGetLastError();
}

}  // namespace neptune
