// Persistent grouped GEMM for gfx950 (MI355X), 8-wave ping-pong configuration: bf16 and MXFP8. The
// tile configurations, work-item decode, copy plan, fragment reads, MFMAs and epilogues are the
// policy-typed code of gemm_pp_plan.h (replayed on the CPU by the checker under tests/native); this
// file holds the kernel's stage pipeline and the launch.
//
// Pipeline: the stages of all work items of a workgroup form one stream. The copies of stage q + 1
// go out at the start of the interval in which stage q is used, into the slot that stage q - 1 left;
// copies past the end of the stream re-read the last stage into the free slot, which keeps the
// counts exact. A stage is used in two half-steps of 64 bytes of K (one set of operand fragments in
// registers at a time). Between two barriers the groups alternate on every SIMD: group 0 reads half
// 0 of stage q while group 1 issues the MFMAs of half 1 of stage q - 1, then group 0 issues half 0's
// MFMAs while group 1 reads half 0, and so on, so each SIMD's matrix core is fed alternately by its
// two waves while the other one reads LDS. Before the barrier that ends the interval every wave
// waits for its own copies (loads of a wave retire in order; every wave issues the same copies per
// stage), so the next item's first stage is in flight while the current item finishes.
#include "common.h"
#include "gemm.h"
#include "gemm_pp_plan.h"
#include "../../include/mi355moe.h"

namespace {

using namespace pp;
using O = PpDev;

__device__ __forceinline__ void wait_vm0() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
__device__ __forceinline__ void wait_lgkm0() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }
// Workgroup barrier without a memory fence: the copies are ordered by the explicit vmcnt waits.
__device__ __forceinline__ void barrier() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

template <bool MX, bool B_KN, int EPI, bool TALL, int SEL>
__global__ __launch_bounds__(THREADS, 1) void gg_pp_kernel(GGParams p) {
  using C = Cfg<MX, TALL, sel_skinny<SEL>>;
  constexpr int MI = C::MI, S_SLOT = C::SLOT;
  constexpr bool SWIGLU = EPI == EPI_SWIGLU_BF16 || EPI == EPI_SWIGLU_F32;
  constexpr int ESIZE = MX ? 1 : 2;
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
  int32_t* s_prefix = (int32_t*)(smem + C::PREFIX_OFF);
  int32_t* s_rows = (int32_t*)(smem + C::ROWS_OFF);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = O::uni(tid >> 6);
  const int grp = wave >> 2, wq = C::wq_of(wave), rbo = C::rbo_of(wave);

  // The work list: m-tiles of C::BM rows per group (of the groups SEL takes) and their exclusive
  // prefix, from group_list (the tile height is this kernel's own, so no host-side plan is read).
  // Thread t takes groups PER t ..+PER-1; a scan over the threads gives each its first tile.
  {
    constexpr int PER = (C::PREFIX_MAX + THREADS - 1) / THREADS;
    int cnt[PER];
    int local = 0;
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int g = tid * PER + u;
      cnt[u] = 0;
      if (g < p.G) {
        const int64_t end = p.group_list[g];
        const int64_t rows = end - (g == 0 ? 0 : p.group_list[g - 1]);
        cnt[u] = rows > 0 && sel_takes<SEL, C::BM>(rows) ? (int)((rows + C::BM - 1) / C::BM) : 0;
        s_rows[g] = (int32_t)end;
      }
      local += cnt[u];
    }
    int incl = local;  // inclusive scan within the wave
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int v = __shfl_up(incl, d, 64);
      if (lane >= d) incl += v;
    }
    int32_t* wsum = (int32_t*)(smem + C::EPI_OFF);  // the epilogue staging is free until the first item ends
    if (lane == 63) wsum[wave] = incl;
    __syncthreads();
    int base = 0;
    for (int w = 0; w < wave; ++w) base += wsum[w];
    int run = base + incl - local;
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int g = tid * PER + u;
      if (g < p.G) s_prefix[g] = run;
      run += cnt[u];
    }
    if (tid == THREADS - 1) s_prefix[p.G] = run;
  }
  __syncthreads();
  const int total = O::uni(s_prefix[p.G]) * p.n_tiles;
  const int nk = p.K * ESIZE / KB;
  const int grid = (int)gridDim.x;
  const int L0 = (int)(blockIdx.x & 7) * (grid >> 3) + (int)(blockIdx.x >> 3);
  if (L0 >= total) return;
  const int n_items = (total - L0 + grid - 1) / grid;
  const int nq = n_items * nk;
  const uint32_t lds0 = O::uni((uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)smem);

  // copy cursor: item cL, stage ck
  int cL = L0, ck = 0;
  Item ci;
  decode<C, O>(p, smem, cL, ci);
  Plan<C::CPW_A> pl;
  make_plan<C, B_KN, SWIGLU, O>(p, ci, wave, lane, pl);
  auto issue_next = [&](int q) {
    issue_stage<C, B_KN, SWIGLU, O>(p, pl, ck, lds0 + (uint32_t)((q % S) * S_SLOT), wave, lane);
    if (++ck == nk) {
      if (cL + grid < total) {
        cL += grid;
        decode<C, O>(p, smem, cL, ci);
        make_plan<C, B_KN, SWIGLU, O>(p, ci, wave, lane, pl);
        ck = 0;
      } else {
        ck = nk - 1;  // past the end: repeat the last stage into the free slot
      }
    }
  };

  // compute cursor: item it, stage kk; `live`: this wave's 128 rows hold rows of the item
  int kL = L0, kk = 0;
  Item it;
  decode<C, O>(p, smem, kL, it);
  // row blocks of this wave that hold rows of the item; `live`: any
  auto row_blocks = [&]() {
    const int n = ((it.rows + 31) / 32 - rbo + C::RBS - 1) / C::RBS;
    return O::uni(n < 0 ? 0 : (n > MI ? MI : n));
  };
  int nmi = row_blocks();
  bool live = nmi > 0;
  v16f acc[MI][NI];
#pragma unroll
  for (int mi = 0; mi < MI; ++mi)
#pragma unroll
    for (int ni = 0; ni < NI; ++ni)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[mi][ni][r] = 0.0f;

  auto finish_stage = [&]() {
    if (++kk == nk) {
      if (live) epilogue<C, EPI, O>(p, it, acc, rbo, wq, lane, smem + C::EPI_OFF + wave * C::EPI_BLOCK);
#pragma unroll
      for (int mi = 0; mi < MI; ++mi)
#pragma unroll
        for (int ni = 0; ni < NI; ++ni)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[mi][ni][r] = 0.0f;
      kk = 0;
      kL += grid;
      if (kL < total) {
        decode<C, O>(p, smem, kL, it);
        nmi = row_blocks();
        live = nmi > 0;
      }
    }
  };

  issue_next(0);
  wait_vm0();
  barrier();
  Frags<MX, B_KN, MI> f;
  if (grp == 0) {
    for (int q = 0; q < nq; ++q) {
      issue_next(q + 1);
      const uint8_t* slot = smem + (q % S) * S_SLOT;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        if (live) read_frags<C, B_KN, O>(f, slot, h, rbo, wq, lane, (int)(it.row0 & 3), nmi);
        wait_lgkm0();
        __builtin_amdgcn_sched_barrier(0);
        if (live) mfmas<MX, B_KN, MI, O>(f, acc, nmi);
        __builtin_amdgcn_sched_barrier(0);
      }
      finish_stage();
      wait_vm0();
      barrier();
    }
  } else {
    for (int q = 0; q < nq; ++q) {
      issue_next(q + 1);
      if (q > 0) {  // half 1 of stage q - 1, read before the barrier
        if (live) mfmas<MX, B_KN, MI, O>(f, acc, nmi);
        finish_stage();
      }
      __builtin_amdgcn_sched_barrier(0);
      const uint8_t* slot = smem + (q % S) * S_SLOT;
      if (live) read_frags<C, B_KN, O>(f, slot, 0, rbo, wq, lane, (int)(it.row0 & 3), nmi);
      wait_lgkm0();
      __builtin_amdgcn_sched_barrier(0);
      if (live) mfmas<MX, B_KN, MI, O>(f, acc, nmi);
      __builtin_amdgcn_sched_barrier(0);
      if (live) read_frags<C, B_KN, O>(f, slot, 1, rbo, wq, lane, (int)(it.row0 & 3), nmi);
      wait_lgkm0();
      wait_vm0();
      barrier();
    }
    if (live) mfmas<MX, B_KN, MI, O>(f, acc, nmi);
    finish_stage();
  }
  wait_vm0();  // no copy may still write the LDS when the workgroup ends
}

template <bool MX, bool B_KN, int EPI, bool TALL, int SEL>
int launch_pp_k(const GGParams& p, hipStream_t stream) {
  using C = Cfg<MX, TALL, sel_skinny<SEL>>;
  auto kern = gg_pp_kernel<MX, B_KN, EPI, TALL, SEL>;
  static bool configured = false;
  if (!configured) {
    if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, C::TOTAL) != hipSuccess)
      return MI355MOE_ELAUNCH;
    configured = true;
  }
  int grid = (mi355_num_cus() / 8) * 8;
  if (grid < 8) grid = 8;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(THREADS), C::TOTAL, stream, p);
  return hipGetLastError() == hipSuccess ? MI355MOE_OK : MI355MOE_ELAUNCH;
}

struct DevLaunch {
  hipStream_t stream;
  template <bool MX, bool B_KN, int EPI, bool TALL, int SEL>
  int run(const GGParams& p) {
    return launch_pp_k<MX, B_KN, EPI, TALL, SEL>(p, stream);
  }
};

}  // namespace

bool mi355_gg_pp_applies(const GGParams& p, bool mx, bool b_kn, int epi) {
  if (p.k_splits > 1 || p.c_row_index != nullptr) return false;
  if (p.G > Cfg<false, false>::PREFIX_MAX) return false;  // the work list is in LDS
  if (p.swiglu_limit > 0.0f || p.row_prob != nullptr) return false;  // numerics options: default kernel
  const int esize = mx ? 1 : 2;
  if ((int64_t)p.K * esize % KB != 0) return false;
  if (mx && p.a_scale_stage_stride == 0) return false;  // needs the stage-major activation scales
  // 32-bit copy offsets: the activations and one group's weights below 4 GiB
  const int64_t lim = (int64_t)1 << 32;
  if (p.a_bytes <= 0 || p.a_bytes >= lim || p.b_group_stride >= lim) return false;
  if (mx && (p.a_scale_stage_stride >= lim || p.b_scale_group_stride >= lim)) return false;
  if (mx && !b_kn) return false;  // MX weights: the root's col_data / col_scale layout
  if (mx && p.a_row_index != nullptr && !p.a_scale_routed) return false;  // code planes by routed row
  if (mx) return epi == EPI_STORE_BF16 || epi == EPI_SWIGLU_F32;
  return epi == EPI_STORE_BF16 || epi == EPI_SWIGLU_BF16;
}

bool mi355_gg_pp_usable(int variant, bool mx, bool b_kn, int64_t K, int G, int64_t a_bytes, int64_t b_group_stride) {
  const int v = variant;
  if (v != MI355_GG_VARIANT_DEFAULT && v != MI355_GG_VARIANT_PP) return false;
  if (mx && !b_kn) return false;
  if (G > Cfg<false, false>::PREFIX_MAX || K * (mx ? 1 : 2) % KB != 0) return false;
  const int64_t lim = (int64_t)1 << 32;
  return a_bytes > 0 && a_bytes < lim && b_group_stride > 0 && b_group_stride < lim;
}

int mi355_grouped_gemm_pp(const GGParams& p, bool mx, bool b_kn, int epi, hipStream_t stream) {
  if (!mi355_gg_pp_applies(p, mx, b_kn, epi)) return MI355MOE_EUNSUPPORTED;
  DevLaunch L{stream};
  return pp_select(p, mx, b_kn, epi, L);
}
