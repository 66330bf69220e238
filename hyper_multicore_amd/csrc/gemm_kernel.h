// Device building blocks of the persistent grouped GEMM shared by gemm.hip (forward kernels) and
// gemm_wgrad.hip (grouped-K weight-gradient kernels): the direct-to-LDS copy and the waits, the
// software-pipelined K loop, the forward kernel and its launch. The two files are separate
// translation units: with other kernel families in the same module the compiler schedules the
// forward kernels' scalar address code differently.
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
                 "global_load_lds_dwordx4 %0, off\n1:" ::"v"(g), "s"(m0), "s"(en) : "memory", "scc", "m0");
  else if constexpr (SZ == 4)
    asm volatile("s_cmp_eq_u32 %2, 0\n\ts_cbranch_scc1 1f\n\ts_mov_b32 m0, %1\n\ts_nop 0\n\t"
                 "global_load_lds_dword %0, off\n1:" ::"v"(g), "s"(m0), "s"(en) : "memory", "scc", "m0");
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
    wait_vm(younger_than<C, LA>(k + 1, k - 1, nk, la_n, lb_n));
    lds_barrier();
    __builtin_amdgcn_sched_barrier(0);
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
      if constexpr (NM > 0) {
        mfma_elem<C, MX, B_KN, NM, GK>(cur, acc, t);
#pragma unroll
        for (int e = t * SS::READS / T; e < (t + 1) * SS::READS / T; ++e)
          read_elem<C, MX, B_KN, NM, GK>(nxt, e, As, Bs, ASs, BSRs, wm, wn, ln);
      }
#pragma unroll
      for (int it = t * SS::ITEMS / T; it < (t + 1) * SS::ITEMS / T; ++it)
        issue_item<C, MX, B_KN, LA, GK, DevDma>(cp, k, nk, wave, smem, it);
      __builtin_amdgcn_sched_barrier(0);  // keep this interleave order
    }
    issue_scales_item<C, MX, B_KN, LA, DevDma, GK>(cp, k, nk, wave, smem);
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
  if constexpr (NM > 0) {
#pragma unroll
    for (int t = 0; t < SS::MFMAS; ++t) mfma_elem<C, MX, B_KN, NM, GK>(f0, acc, t);
  }
}

template <class C, bool MX, bool B_KN, int EPI>
__global__ __launch_bounds__(C::THREADS, C::WG_PER_CU) void grouped_gemm_kernel(GGParams p) {
  static_assert(!MX || C::AS_N == 2, "MX needs the activation-scale ring");
  static_assert(!(MX && !B_KN) || C::BSR_N == 2, "MX with K-contiguous weights needs the row-scale ring");
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
  int32_t* s_prefix = (int32_t*)(smem + C::PREFIX_OFF);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = (int)((unsigned)wave / C::WGN), wn = (int)((unsigned)wave % C::WGN);
  constexpr bool SWIGLU = (EPI == EPI_SWIGLU_BF16 || EPI == EPI_SWIGLU_MX || EPI == EPI_SWIGLU_BF16_NUM);
  constexpr int ESIZE = MX ? 1 : 2;

  const bool prefix_in_lds = p.G <= C::PREFIX_MAX;
  const int32_t* prefix = prefix_in_lds ? s_prefix : p.tile_prefix;
  if (prefix_in_lds)
    for (int g = tid; g <= p.G; g += C::THREADS) s_prefix[g] = p.tile_prefix[g];
  __syncthreads();
  const int splits = (EPI == EPI_STORE_F32 && p.k_splits > 1) ? p.k_splits : 1;
  const int items = prefix[p.G] * p.n_tiles;
  const int nk = p.K / splits * ESIZE / C::KB;  // stages per work item
  // A partial last round of whole items leaves most CUs idle while it streams its weights: its items
  // run as two column halves each (half the weight lines per item, twice the workgroups), when the
  // halves still fit in one round. Every output element keeps its own K loop, so the results are
  // those of the whole items. SwiGLU GEMMs only: on the plain-store GEMM (decode GMM2, short K) the
  // halves measured 1.3 % slower.
  int tail_from = INT32_MAX;
  if constexpr (C::HALF_TAIL && EPI != EPI_STORE_F32 && EPI != EPI_STORE_BF16) {
    const int full = items / (int)gridDim.x * (int)gridDim.x;
    if (items > full && 2 * (items - full) <= (int)gridDim.x) tail_from = full;
  }
  const int total = splits > 1 ? items * splits : (tail_from < items ? tail_from + 2 * (items - tail_from) : items);
  const int xcd = blockIdx.x & 7;
  const int per_xcd = gridDim.x >> 3;
  const int slot = blockIdx.x >> 3;

  for (int round = 0;; ++round) {
    const int L = round * (int)gridDim.x + xcd * per_xcd + slot;
    if (L >= total) break;
    // ---- decode work item, per-thread copy sources -------------------------------------
#include "gemm_item_fwd.inc"

    v16f acc[C::MI][C::NI];
#pragma unroll
    for (int i = 0; i < C::MI; ++i)
#pragma unroll
      for (int j = 0; j < C::NI; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    __syncthreads();  // the previous item's last stage / epilogue reads are done before refilling
    const int rows_w = rows_valid - wm * C::WM;
    int nm = (C::MI >= 4 && rows_w > 64) ? 4 : ((C::MI >= 2 && rows_w > 32) ? 2 : (rows_w >= 1 ? 1 : 0));
    if (half >= 0 && (wn >> 1) != half) nm = 0;  // a column half: the other half's waves only copy
    // this wave copies A rows wave*A_INSTR*16 .. (and, MX scale waves, scale rows wave*64 .. +63)
    const bool la = wave_copies_a<C>(wave, rows_valid);
    if (la) {
      if (C::MI >= 4 && nm == 4) k_loop<C, MX, B_KN, (C::MI >= 4 ? 4 : 1), true>(cp, nk, wave, wm, wn, lane, smem, acc);
      else if (nm == 2) k_loop<C, MX, B_KN, 2, true>(cp, nk, wave, wm, wn, lane, smem, acc);
      else if (nm == 1) k_loop<C, MX, B_KN, 1, true>(cp, nk, wave, wm, wn, lane, smem, acc);
      else k_loop<C, MX, B_KN, 0, true>(cp, nk, wave, wm, wn, lane, smem, acc);
    } else {
      if (C::MI >= 4 && nm == 4) k_loop<C, MX, B_KN, (C::MI >= 4 ? 4 : 1), false>(cp, nk, wave, wm, wn, lane, smem, acc);
      else if (nm == 2) k_loop<C, MX, B_KN, 2, false>(cp, nk, wave, wm, wn, lane, smem, acc);
      else if (nm == 1) k_loop<C, MX, B_KN, 1, false>(cp, nk, wave, wm, wn, lane, smem, acc);
      else k_loop<C, MX, B_KN, 0, false>(cp, nk, wave, wm, wn, lane, smem, acc);
    }
    __syncthreads();  // all waves are done reading the ring before the epilogue reuses LDS

#include "gemm_epilogue.inc"
  }
}

template <class C, bool MX, bool B_KN, int EPI>
static int launch_gg(const GGParams& p, hipStream_t stream) {
  static bool configured = false;
  auto kern = grouped_gemm_kernel<C, MX, B_KN, EPI>;
  if (!configured) {
    if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, C::TOTAL) != hipSuccess)
      return MI355MOE_ELAUNCH;
    configured = true;
  }
  int grid = (mi355_num_cus() / 8) * 8 * C::WG_PER_CU;
  if (grid < 8) grid = 8;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(C::THREADS), C::TOTAL, stream, p);
  return hipGetLastError() == hipSuccess ? MI355MOE_OK : MI355MOE_ELAUNCH;
}

template <class C>
static int dispatch_gg(const GGParams& p, bool mx, bool b_kn, int epi, hipStream_t stream) {
  if (!mx) {
    if (!b_kn) {
      switch (epi) {
        case EPI_STORE_BF16: return launch_gg<C, false, false, EPI_STORE_BF16>(p, stream);
        case EPI_STORE_F32: return launch_gg<C, false, false, EPI_STORE_F32>(p, stream);
        case EPI_SWIGLU_BF16: return launch_gg<C, false, false, EPI_SWIGLU_BF16>(p, stream);
        case EPI_SWIGLU_BF16_NUM: return launch_gg<C, false, false, EPI_SWIGLU_BF16_NUM>(p, stream);
        default: return MI355MOE_EUNSUPPORTED;
      }
    } else {
      switch (epi) {
        case EPI_STORE_BF16: return launch_gg<C, false, true, EPI_STORE_BF16>(p, stream);
        case EPI_SWIGLU_BF16: return launch_gg<C, false, true, EPI_SWIGLU_BF16>(p, stream);
        case EPI_SWIGLU_BF16_NUM: return launch_gg<C, false, true, EPI_SWIGLU_BF16_NUM>(p, stream);
        default: return MI355MOE_EUNSUPPORTED;
      }
    }
  }
  if constexpr (C::AS_N == 0) {  // a configuration without the MX scale rings
    return MI355MOE_EUNSUPPORTED;
  } else {
    if (!b_kn) {
      if constexpr (C::BSR_N == 0) {
        return MI355MOE_EUNSUPPORTED;
      } else {
        switch (epi) {
          case EPI_STORE_BF16: return launch_gg<C, true, false, EPI_STORE_BF16>(p, stream);
          case EPI_SWIGLU_MX: return launch_gg<C, true, false, EPI_SWIGLU_MX>(p, stream);
          default: return MI355MOE_EUNSUPPORTED;
        }
      }
    }
    switch (epi) {
      case EPI_STORE_BF16: return launch_gg<C, true, true, EPI_STORE_BF16>(p, stream);
      case EPI_SWIGLU_MX: return launch_gg<C, true, true, EPI_SWIGLU_MX>(p, stream);
      default: return MI355MOE_EUNSUPPORTED;
    }
  }
}

