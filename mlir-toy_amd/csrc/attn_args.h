// attn_args.h — kernel-side argument block of the attention kernels
// (resolved by launch_attn_fwd from the validated AttnLaunch).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace neptune {

struct AttnArgs {
  const void *q, *k, *v;
  void *o;
  float *lse;
  int64_t qs0, qs1, qs2, ks0, ks1, ks2, vs0, vs1, vs2, os0, os1, os2;
  int32_t Hq, group, Sq, Sk, nqb, BH, off;  // off = Sk - Sq (causal diagonal)
  float scale2;                             // log2(e)/sqrt(D) unless given
};

// Launches the head_dim-128 16-bit kernel (attn_fwd_d128.hip); dtype 1 = f16,
// 2 = bf16; stages = LDS slots per operand (1, 2 or 3); kt = K stored
// [.., head_dim, seq] (ks2 is then the head_dim-row stride).
hipError_t launch_attn_d128(const AttnArgs &a, int32_t dtype, bool causal, int stages, bool kt,
                            hipStream_t s);

}  // namespace neptune
