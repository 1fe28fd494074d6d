// lds_dma.h — HBM -> LDS copies on gfx950 (global_load_lds_dwordx4) and the
// LDS pointer helpers the tiled kernels share.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace neptune {

typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) v4i16 lds_v4i16;

__device__ inline lds_void *as_lds(const uint8_t *p) { return (lds_void *)(p); }

// ds_read_b64_tr_b16 of the 8 bytes at p (LDS)
__device__ inline v4i16 lds_read_tr16(const uint8_t *p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16 *)as_lds(p));
}

__device__ inline const char *uniform_ptr(const char *p) {
  const uint64_t v = (uint64_t)(uintptr_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return (const char *)(uintptr_t)(((uint64_t)hi << 32) | lo);
}

// LDS byte address of a pointer into a __shared__ array: the low 32 bits of
// its generic address (no null check), made wave-uniform
__device__ inline uint32_t lds_offset(const uint8_t *p) {
  return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)p);
}

// One global_load_lds_dwordx4: 16 bytes per lane into LDS at lds_addr +
// 16 * lane. Issued as inline assembly because the compiler's wait-count
// pass does not order ds_read_b64_tr_b16 against LDS DMA by address and
// would drain every outstanding load (vmcnt(0)) before each transpose read,
// serialising any prefetch. The compiler therefore does not count these
// loads: callers wait for them explicitly (s_waitcnt vmcnt, plus a barrier
// when other waves read the data) and finish their own reads of a slot
// (lgkmcnt(0)) before refilling it. The LDS address travels in M0 as a tied
// input/output operand, so the compiler sets M0 itself (one s_mov) and knows
// the statement leaves it changed. The compiler does not check hazards
// inside inline assembly, so the statement covers two itself: M0 write ->
// LDS DMA (1 wait state) and, in the SGPR-base form, VALU write of an SGPR
// (v_readfirstlane of the base) -> VMEM read of that SGPR (5 wait states:
// s_nop 4). Without the latter a base computed by a VALU just before the
// copy (a block-table lookup) is read stale.
// NT = true marks the load non-temporal (streamed data read once: keeps it
// from displacing reused lines, and measured on MI355X it sustains ~7.1 TB/s
// against ~6.4 TB/s for plain loads).
template <bool NT = false>
__device__ inline void dma16(const char *sbase, uint32_t voff, uint32_t lds_addr) {
  uint32_t m0;
  if (NT)
    asm volatile("s_nop 4\n\tglobal_load_lds_dwordx4 %1, %2 nt"
                 : "={m0}"(m0)
                 : "v"(voff), "s"(uniform_ptr(sbase)), "0"(__builtin_amdgcn_readfirstlane(lds_addr))
                 : "memory");
  else
    asm volatile("s_nop 4\n\tglobal_load_lds_dwordx4 %1, %2"
                 : "={m0}"(m0)
                 : "v"(voff), "s"(uniform_ptr(sbase)), "0"(__builtin_amdgcn_readfirstlane(lds_addr))
                 : "memory");
}
// The same copy when the base comes from scalar instructions only (kernel
// arguments, work-group ids and uniform loop counters): no VALU writes those
// SGPRs, so only the M0 wait state is needed. Which form a copy needs is a
// property of the compiled code, not of the source: the ISA test in
// tests/test_isa_hazards.py checks every copy of the built kernels.
template <bool NT = false>
__device__ inline void dma16_sbase(const char *sbase, uint32_t voff, uint32_t lds_addr) {
  uint32_t m0;
  if (NT)
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %1, %2 nt"
                 : "={m0}"(m0)
                 : "v"(voff), "s"(uniform_ptr(sbase)), "0"(__builtin_amdgcn_readfirstlane(lds_addr))
                 : "memory");
  else
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
                 : "={m0}"(m0)
                 : "v"(voff), "s"(uniform_ptr(sbase)), "0"(__builtin_amdgcn_readfirstlane(lds_addr))
                 : "memory");
}
template <bool NT = false>
__device__ inline void dma16(const char *addr, uint32_t lds_addr) {
  uint32_t m0;
  if (NT)
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %1, off nt"
                 : "={m0}"(m0)
                 : "v"(addr), "0"(__builtin_amdgcn_readfirstlane(lds_addr))
                 : "memory");
  else
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
                 : "={m0}"(m0)
                 : "v"(addr), "0"(__builtin_amdgcn_readfirstlane(lds_addr))
                 : "memory");
}

// Makes the compiler wait, here, for the loads that produced x (an empty
// statement that reads x). The compiler does not count the copies above, so
// a loop that streams through them must enter with none of the compiler's
// own loads outstanding: a load still pending at the loop head (or issued
// in the loop) gets a vmcnt(0) inside the loop, which also retires every
// copy in flight and so drains the prefetch at each step.
template <typename T>
__device__ inline void settle(const T &x) {
  asm volatile("" ::"v"(x));
}

// s_waitcnt immediates (gfx9 encoding): wait until at most n vector-memory
// operations are outstanding / until all LDS operations have completed.
constexpr int waitcnt_vm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }
constexpr int kWaitLgkm0 = 0xc07f;

}  // namespace neptune
