// Direct-weight forward grouped GEMM (configuration GGDirect, measurement variant "dv"): weights read
// K-contiguous straight into registers, activations through an 8-slot LDS ring. The pipeline and the
// copy plan are described in gemm_direct_plan.h. Own translation unit, so the default kernels'
// code does not depend on it.
#include "gemm_direct_plan.h"
#include "gemm_kernel.h"

// Memory policy of the kernel: both loads use the scalar-base + 32-bit vector-offset address form.
// Inline assembly for the reason given at lds_dma: with the builtins the compiler would wait for a
// weight load with vmcnt counts that ignore the direct-to-LDS copies issued after it (draining the
// activation ring), and before the LDS reads after a copy it would wait for every copy. The kernel
// issues only loads of stages that exist (which steps issue is fixed at compile time), so `enable`
// is always 1 here. Completion is ordered by the step's s_waitcnt (direct_wait_fixed) before the
// registers are tied (direct_tie) and read, and by the workgroup barrier for the LDS.
struct DevMem {
  MI355_DEV static void load(v4i& dst, const uint8_t* base, uint32_t off, int) {
    asm volatile("global_load_dwordx4 %0, %1, %2" : "=&v"(dst) : "v"(off), "s"(base) : "memory");
  }
  MI355_DEV static void lds(const uint8_t* base, uint32_t off, uint8_t* smem, uint32_t lds_off, int) {
    // LDS address of the destination: the LDS base of the dynamic shared array plus the offset
    const uint32_t m0 = __builtin_amdgcn_readfirstlane(
        (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)smem + lds_off);
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "s"(m0)
                 : "memory");
  }
};

// Registers written by loads that have landed: uses below this point depend on it.
MI355_DEV void direct_tie(v4i& a, v4i& b, v4i& c, v4i& d) { asm volatile("" : "+v"(a), "+v"(b), "+v"(c), "+v"(d)); }
MI355_DEV void direct_tie(v4i& a, v4i& b) { asm volatile("" : "+v"(a), "+v"(b)); }

// One step at ring position P (k % D == P): MFMAs of stage k, fragment reads of stage k + 1 and the
// copies of stage k + D - 1, one copy item after each subtile row.
template <bool MX, int NMI, int P, bool LAST>
MI355_DEV void direct_step(const DirectPlan& d, int k, int nk, int wave, int lane,
                           uint8_t* smem, v4i (&ring)[GGDirect::D][GGDirect::B_LOADS], v4i (&bs_cur)[GGDirect::NI],
                           v4i (&bs_nxt)[GGDirect::NI], DirectFrags<MX>& f, v16f (&acc)[GGDirect::MI][GGDirect::NI]) {
  using C = GGDirect;
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(direct_wait_fixed<MX, P, LAST>()) : "memory");
  direct_tie(ring[P][0], ring[P][1], ring[P][2], ring[P][3]);
  if constexpr (MX && P == 0) direct_tie(bs_nxt[0], bs_nxt[1]);
  lds_barrier();
  __builtin_amdgcn_sched_barrier(0);
  // which steps issue is fixed: every turn but the last issues a stage per step and a scale group
  // at position 0; the last turn only the last stage, at position 0 (direct_wait_fixed counts so)
  constexpr bool ISSUE = !LAST || P == 0;
  if constexpr (MX && P == 0) {
#pragma unroll
    for (int q = 0; q < C::NI; ++q) bs_cur[q] = bs_nxt[q];
    if constexpr (!LAST) direct_issue_scales<DevMem>(d, k / 8 + 1, 1, wave, smem, bs_nxt);
  }
  int ln = lane;
  asm volatile("" : "+v"(ln));  // recompute lane-dependent LDS offsets here rather than hold them
  constexpr int PN = (P + 1) % C::D;
  const uint8_t* As = smem + PN * C::A_BYTES;
  const int grp_n = (k + 1) / C::AS_GROUP;
  const uint8_t* ASs = smem + C::AS_OFF + (grp_n & 1) * C::AS_SLOT + PN * 2;
#pragma unroll
  for (int mi = 0; mi < C::MI; ++mi) {
    if (mi < NMI) {
#pragma unroll
      for (int t = 0; t < direct_mfmas<MX>(); ++t) direct_mfma<MX>(f, mi, t, ring[P], bs_cur, P, ln, acc);
      direct_read_a<MX>(f, mi, As, ASs, ln);
    }
    if constexpr (ISSUE) direct_issue<DevMem>(d, k, nk, wave, smem, ring[(P + C::D - 1) % C::D], mi);
    __builtin_amdgcn_sched_barrier(0);  // keep this interleave order
  }
}

// Steps k0 .. k0 + D - 1 (ring positions 0 .. D - 1).
template <bool MX, int NMI, bool LAST>
MI355_DEV void direct_steps(const DirectPlan& d, int k0, int nk, int wave, int lane, uint8_t* smem,
                            v4i (&ring)[GGDirect::D][GGDirect::B_LOADS], v4i (&bs_cur)[GGDirect::NI],
                            v4i (&bs_nxt)[GGDirect::NI], DirectFrags<MX>& f, v16f (&acc)[GGDirect::MI][GGDirect::NI]) {
  direct_step<MX, NMI, 0, LAST>(d, k0 + 0, nk, wave, lane, smem, ring, bs_cur, bs_nxt, f, acc);
  direct_step<MX, NMI, 1, LAST>(d, k0 + 1, nk, wave, lane, smem, ring, bs_cur, bs_nxt, f, acc);
  direct_step<MX, NMI, 2, LAST>(d, k0 + 2, nk, wave, lane, smem, ring, bs_cur, bs_nxt, f, acc);
  direct_step<MX, NMI, 3, LAST>(d, k0 + 3, nk, wave, lane, smem, ring, bs_cur, bs_nxt, f, acc);
  direct_step<MX, NMI, 4, LAST>(d, k0 + 4, nk, wave, lane, smem, ring, bs_cur, bs_nxt, f, acc);
  direct_step<MX, NMI, 5, LAST>(d, k0 + 5, nk, wave, lane, smem, ring, bs_cur, bs_nxt, f, acc);
  direct_step<MX, NMI, 6, LAST>(d, k0 + 6, nk, wave, lane, smem, ring, bs_cur, bs_nxt, f, acc);
  direct_step<MX, NMI, 7, LAST>(d, k0 + 7, nk, wave, lane, smem, ring, bs_cur, bs_nxt, f, acc);
}

template <bool MX, int NMI>
MI355_DEV void direct_k_loop(const DirectPlan& d, int nk, int wave, int lane,
                             uint8_t* smem, v16f (&acc)[GGDirect::MI][GGDirect::NI]) {
  using C = GGDirect;
  v4i ring[C::D][C::B_LOADS];
  v4i bs_cur[C::NI], bs_nxt[C::NI];
  DirectFrags<MX> f;
  if constexpr (MX) direct_issue_scales<DevMem>(d, 0, 1, wave, smem, bs_nxt);
  // prologue: steps -(D-1) .. -1 issue stages 0 .. D-2 into ring slots 0 .. D-2
#pragma unroll
  for (int s = 0; s < C::D - 1; ++s)
#pragma unroll
    for (int it = 0; it < C::B_LOADS + C::A_INSTR; ++it)
      direct_issue<DevMem>(d, s - (C::D - 1), nk, wave, smem, ring[s], it);
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(direct_wait_first()) : "memory");
  lds_barrier();
  {
    int ln = lane;
    asm volatile("" : "+v"(ln));  // lane-dependent LDS offsets computed here, not held from before
    const uint8_t* ASs = smem + C::AS_OFF;
#pragma unroll
    for (int mi = 0; mi < NMI; ++mi) direct_read_a<MX>(f, mi, smem, ASs, ln);
  }
  // every turn of the ring but the last, then the last (their wait counts differ)
  int k0 = 0;
  for (; k0 + C::D < nk; k0 += C::D) direct_steps<MX, NMI, false>(d, k0, nk, wave, lane, smem, ring, bs_cur, bs_nxt, f, acc);
  direct_steps<MX, NMI, true>(d, k0, nk, wave, lane, smem, ring, bs_cur, bs_nxt, f, acc);
  __builtin_amdgcn_sched_barrier(0);
}

template <bool MX, int EPI>
__global__ __launch_bounds__(GGDirect::THREADS, 1) void grouped_gemm_direct_kernel(GGParams p) {
  using C = GGDirect;
  constexpr bool B_KN = false;
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
  int32_t* s_prefix = (int32_t*)(smem + C::PREFIX_OFF);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = 0, wn = wave;
  constexpr bool SWIGLU = (EPI == EPI_SWIGLU_BF16 || EPI == EPI_SWIGLU_MX || EPI == EPI_SWIGLU_BF16_NUM);
  constexpr int ESIZE = MX ? 1 : 2;

  const bool prefix_in_lds = p.G <= C::PREFIX_MAX;
  const int32_t* prefix = prefix_in_lds ? s_prefix : p.tile_prefix;
  if (prefix_in_lds)
    for (int g = tid; g <= p.G; g += C::THREADS) s_prefix[g] = p.tile_prefix[g];
  __syncthreads();
  const int splits = 1;
  const int total = prefix[p.G] * p.n_tiles;
  const int nk = p.K * ESIZE / C::KB;  // stages per work item (a multiple of D, checked by the host)
  const int xcd = blockIdx.x & 7;
  const int per_xcd = gridDim.x >> 3;
  const int slot = blockIdx.x >> 3;

  for (int round = 0;; ++round) {
    const int L = round * (int)gridDim.x + xcd * per_xcd + slot;
    if (L >= total) break;
    constexpr bool copy_role_a = true, copy_role_b = true;
    constexpr int tail_from = INT32_MAX;  // no column halves in the direct-weight configuration
#include "gemm_item_fwd.inc"
    DirectPlan d = direct_plan(p, g, nt, tile_row0, rows_valid, SWIGLU, MX, wave, lane);
    d.a_base = gg_uniform(d.a_base);
    d.as_base = gg_uniform(d.as_base);
    d.b_base = gg_uniform(d.b_base);
    d.bs_base = gg_uniform(d.bs_base);

    v16f acc[C::MI][C::NI];
#pragma unroll
    for (int i = 0; i < C::MI; ++i)
#pragma unroll
      for (int j = 0; j < C::NI; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    __syncthreads();  // the previous item's epilogue reads of the LDS are done before refilling
    if (rows_valid > 128) direct_k_loop<MX, 8>(d, nk, wave, lane, smem, acc);
    else if (rows_valid > 64) direct_k_loop<MX, 4>(d, nk, wave, lane, smem, acc);
    else if (rows_valid > 32) direct_k_loop<MX, 2>(d, nk, wave, lane, smem, acc);
    else direct_k_loop<MX, 1>(d, nk, wave, lane, smem, acc);
    __syncthreads();  // all waves are done reading the ring before the epilogue reuses LDS

#include "gemm_epilogue.inc"
  }
}

template <bool MX, int EPI>
static int launch_direct(const GGParams& p, hipStream_t stream) {
  static bool configured = false;
  auto kern = grouped_gemm_direct_kernel<MX, EPI>;
  if (!configured) {
    if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, GGDirect::TOTAL) != hipSuccess)
      return MI355MOE_ELAUNCH;
    configured = true;
  }
  int grid = (mi355_num_cus() / 8) * 8;
  if (grid < 8) grid = 8;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(GGDirect::THREADS), GGDirect::TOTAL, stream, p);
  return hipGetLastError() == hipSuccess ? MI355MOE_OK : MI355MOE_ELAUNCH;
}

// Within direct_supported's domain; the fp32 router projection (split K) and the numerics-option
// epilogue stay on the default configuration.
// MXFP8 is refused: on the GPU its outputs were wrong in the second 32-column block of every 64-column
// pair (the even blocks matched the default configuration), which the host-side emulation of the
// scale MFMA operands does not reproduce; the bf16 configuration is bit-identical to the default.
int mi355_grouped_gemm_direct(const GGParams& p, bool mx, bool b_kn, int epi, hipStream_t stream) {
  if (mx || !direct_supported(p, mx, b_kn, epi)) return MI355MOE_EUNSUPPORTED;
  if (epi == EPI_STORE_BF16) return launch_direct<false, EPI_STORE_BF16>(p, stream);
  return launch_direct<false, EPI_SWIGLU_BF16>(p, stream);
}
