// Device building blocks of the persistent grouped GEMM shared by gemm.hip (forward kernels) and
// gemm_wgrad.hip (grouped-K weight-gradient kernels): the direct-to-LDS copy and the waits, operand
// fragments, the LDS fragment reads and MFMAs, and the software-pipelined K loop. The kernels of the
// two files are compiled in separate translation units: with both kernel families in one module the
// compiler schedules the forward kernels' scalar address code differently.
#pragma once
#include <type_traits>
#include "common.h"
#include "scan.h"
#include "../../include/mi355moe.h"
#include "gemm.h"
#include "gemm_plan.h"


// Direct global -> LDS copy: lane i of the wave writes its SZ bytes at LDS address M0 + SZ*i
// (SZ = 16) or M0 + 4*i (SZ = 4). Written as inline assembly on purpose: for the compiler's
// builtin, the backend must assume the copy may alias every later LDS read and inserts a wait for
// all outstanding vector-memory loads before the next ds_read, which would drain the whole
// prefetch ring each stage. Completion is tracked here with explicit vmcnt waits (loads of a wave
// retire in order) and made visible to the other waves by the following workgroup barrier.
// M0 is a reserved register that the compiler sets right before each of its own uses, so the
// assembly may overwrite it.
template <int SZ>
MI355_DEV void lds_dma(const void* g, uint32_t lds_off_uniform, uint8_t* smem, int enable = 1) {
  // `enable` (wave-uniform) skips the copy inside the assembly, so a conditional copy adds no
  // branch to the surrounding code and the MFMAs around it keep their place.
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)(smem + lds_off_uniform));
  const int en = __builtin_amdgcn_readfirstlane(enable);
  if constexpr (SZ == 16)
    asm volatile("s_cmp_eq_u32 %2, 0\n\ts_cbranch_scc1 1f\n\ts_mov_b32 m0, %1\n\ts_nop 0\n\t"
                 "global_load_lds_dwordx4 %0, off\n1:" ::"v"(g), "s"(m0), "s"(en) : "memory", "scc");
  else if constexpr (SZ == 4)
    asm volatile("s_cmp_eq_u32 %2, 0\n\ts_cbranch_scc1 1f\n\ts_mov_b32 m0, %1\n\ts_nop 0\n\t"
                 "global_load_lds_dword %0, off\n1:" ::"v"(g), "s"(m0), "s"(en) : "memory", "scc");
  else static_assert(SZ == 16, "unsupported DMA size");
}
// The copy policy of the kernels (see gemm_plan.h).
struct DevDma {
  template <int SZ>
  MI355_DEV static void copy(const void* g, uint32_t lds_off_uniform, uint8_t* smem, int enable) {
    lds_dma<SZ>(g, lds_off_uniform, smem, enable);
  }
};
// Workgroup barrier without the release fence of __syncthreads (which would wait for every
// outstanding global load, including the prefetched stages): LDS reads of this wave are drained,
// the direct-to-LDS loads are ordered by the explicit vmcnt waits.
MI355_DEV void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
}
// Wait until at most n vector-memory loads of this wave are outstanding (loads retire in order).
// n is wave-uniform; the switch maps it onto the immediate of s_waitcnt.
MI355_DEV void wait_vm(int n) {
  switch (n) {
#define GG_WAIT_CASE(N) case N: asm volatile("s_waitcnt vmcnt(" #N ")" ::: "memory"); break;
    GG_WAIT_CASE(1) GG_WAIT_CASE(2) GG_WAIT_CASE(3) GG_WAIT_CASE(4) GG_WAIT_CASE(5) GG_WAIT_CASE(6)
    GG_WAIT_CASE(7) GG_WAIT_CASE(8) GG_WAIT_CASE(9) GG_WAIT_CASE(10) GG_WAIT_CASE(11) GG_WAIT_CASE(12)
    GG_WAIT_CASE(13) GG_WAIT_CASE(14) GG_WAIT_CASE(15) GG_WAIT_CASE(16) GG_WAIT_CASE(17) GG_WAIT_CASE(18)
    GG_WAIT_CASE(19) GG_WAIT_CASE(20) GG_WAIT_CASE(21) GG_WAIT_CASE(22) GG_WAIT_CASE(23) GG_WAIT_CASE(24)
#undef GG_WAIT_CASE
    default:
      if (n <= 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      else asm volatile("s_waitcnt vmcnt(24)" ::: "memory");
  }
}




#ifdef GG_TRACE
__device__ unsigned long long gg_trace[4 * 8 * 64 * 5];
#define GG_T(pt) if (blockIdx.x < 4 && k < 64 && lane == 0) gg_trace[((blockIdx.x * 8 + wave) * 64 + k) * 5 + pt] = __builtin_amdgcn_s_memtime();
extern "C" int mi355_gg_trace_read(void* host) {
  return hipMemcpyFromSymbol(host, HIP_SYMBOL(gg_trace), sizeof(gg_trace)) == hipSuccess ? 0 : -1;
}
#else
#define GG_T(pt)
#endif

// K loop, software-pipelined in each wave: iteration k (after barrier k) refills the ring slots of
// stage k, reads the fragments of stage k+1 into one register set and runs the MFMAs of stage k
// from the other, so LDS reads and DMA issue overlap the matrix cores. Before barrier k every wave
// has waited for its own copies of stage k+1 (so stage k+1 is complete in LDS after the barrier)
// and drained its LDS reads of stage k (read during iteration k-1), so stage k's slots are free.
// A-scale group g+1 (stages 8g+8 ..) is issued at iteration 8g into the slot of group g-1, whose
// last stage was read during iteration 8g-2.
// NM = number of 32-row subtiles this wave computes (0, 1, 2 or 4).
template <class C, bool MX, bool B_KN, int NM, bool LA, bool GK = false>
MI355_DEV void k_loop(const CopyPlan<C>& cp, int nk, int wave, int wm, int wn, int lane, uint8_t* smem,
                      v16f (&acc)[C::MI][C::NI]) {
  // grouped-K mode: A is read K-major like B (and the caller skips groups without rows)
  using D = DevDma;
#include "gemm_kloop_prologue.inc"
  Frags<C, MX, B_KN, GK> f0, f1;
  wait_vm(younger_than<C, LA>(0, -1, nk, la_n, lb_n));
  lds_barrier();
  using SS = StepShape<C, MX, NM, GK>;
  if constexpr (NM > 0) {
    const uint8_t* ASs = smem + C::AS_OFF;
#pragma unroll
    for (int e = 0; e < SS::READS; ++e)
      read_elem<C, MX, B_KN, NM, GK>(f0, e, smem, smem + C::B_OFF, ASs, smem + C::BSR_OFF, wm, wn, lane);
  }
  // one pipelined iteration with a next stage (k + 1 < nk)
  auto step = [&](int k, Frags<C, MX, B_KN, GK>& cur, Frags<C, MX, B_KN, GK>& nxt) {
    __builtin_amdgcn_sched_barrier(0);  // keep the MFMAs of the previous stage above the barrier
    GG_T(0)
    wait_vm(younger_than<C, LA>(k + 1, k - 1, nk, la_n, lb_n));
    GG_T(1)
    lds_barrier();
    __builtin_amdgcn_sched_barrier(0);
    GG_T(2)
    int ln = lane;
    asm volatile("" : "+v"(ln));  // recompute lane-dependent LDS offsets here rather than hold them
    const int kn = k + 1;
    const uint8_t* As = smem + (kn % C::A_SLOTS) * C::A_BYTES;
    const uint8_t* Bs = smem + C::B_OFF + (kn % C::B_SLOTS) * C::B_SLOT;
    const uint8_t* ASs;
    if constexpr (MX && GK) ASs = smem + C::AS_OFF + (kn % C::A_SLOTS) * C::BS_BYTES;  // per-stage column scales
    else ASs = smem + C::AS_OFF + ((kn / C::AS_GROUP) & 1) * C::AS_SLOT + (kn & (C::AS_GROUP - 1)) * 2;
    const uint8_t* BSRs = smem + C::BSR_OFF + ((kn / C::AS_GROUP) & 1) * C::BSR_SLOT + (kn & (C::AS_GROUP - 1)) * 2;
    constexpr int T = SS::MFMAS > 0 ? SS::MFMAS : 1;
#pragma unroll
    for (int t = 0; t < T; ++t) {
#ifndef GG_ABLATE_COMPUTE
      if constexpr (NM > 0) {
        mfma_elem<C, MX, B_KN, NM, GK>(cur, acc, t);
#pragma unroll
        for (int e = t * SS::READS / T; e < (t + 1) * SS::READS / T; ++e)
          read_elem<C, MX, B_KN, NM, GK>(nxt, e, As, Bs, ASs, BSRs, wm, wn, ln);
      }
#endif
#pragma unroll
      for (int it = t * SS::ITEMS / T; it < (t + 1) * SS::ITEMS / T; ++it)
        issue_item<C, MX, B_KN, LA, GK, DevDma>(cp, k, nk, wave, smem, it);
      if (t == T / 2 - 1) { GG_T(3) }
      __builtin_amdgcn_sched_barrier(0);  // keep this interleave order
    }
    issue_scales_item<C, MX, B_KN, LA, DevDma, GK>(cp, k, nk, wave, smem);
    GG_T(4)
  };
  // Stages 0 .. nk-2 are pipelined steps (each reads the next stage), taken in pairs so that the
  // two fragment sets keep fixed registers; an odd count starts with one step and a copy.
  int k = 0;
  if ((nk - 1) & 1) {
    step(0, f0, f1);
    f0 = f1;
    k = 1;
  }
  for (; k < nk - 1; k += 2) {
    step(k, f0, f1);
    step(k + 1, f1, f0);
  }
  // last stage: its fragments are in f0 and it issues no copies
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#ifndef GG_ABLATE_COMPUTE
  if constexpr (NM > 0) {
#pragma unroll
    for (int t = 0; t < SS::MFMAS; ++t) mfma_elem<C, MX, B_KN, NM, GK>(f0, acc, t);
  }
#endif
}

