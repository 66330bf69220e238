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


// ---- fragment loads (one K step: 16 bf16 or 64 e4m3) ------------------------------------------
MI355_DEV v8bf read_a_bf16(const uint8_t* As, int r, int ks, int lane) {
  return *(const v8bf*)(As + a_chunk_off(r, ks * 2 + (lane >> 5)));
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

// Operand fragments of one stage for one wave (WM rows x WN columns x one stage of K). Values
// that are read in several LDS instructions are kept as the raw pieces and joined only when the
// MFMA consumes them, so that issuing the reads never forces a wait for their data.
template <class C, bool MX, bool B_KN, bool A_KN = false> struct Frags;
template <class C> struct Frags<C, false, false> { v8bf a[2][C::MI], b[2][C::NI]; };  // [ks][mi], [ks][ni]
template <class C> struct Frags<C, false, true> { v8bf a[2][C::MI]; v4s bl[2][C::NI], bh[2][C::NI]; };
template <class C> struct Frags<C, false, true, true> {  // grouped-K: A K-major like B
  v4s al[2][C::MI], ah[2][C::MI], bl[2][C::NI], bh[2][C::NI];
};
template <class C> struct Frags<C, true, true> {
  v4i al[C::MI], ah[C::MI];
  v2i bp[C::NI][4];
  int sa[C::MI], sb[C::NI];
};
template <class C> struct Frags<C, true, true, true> {  // grouped-K MX: A K-major like B
  v2i ap[C::MI][4], bp[C::NI][4];
  int sa[C::MI], sb[C::NI];
};
template <class C> struct Frags<C, true, false> {
  v4i al[C::MI], ah[C::MI], bl[C::NI], bh[C::NI];
  int sa[C::MI], sb[C::NI];
};

// bf16 fragment of 32 rows / columns x 16 K (ks) from a K-major LDS tile (512-byte K rows of 256
// bf16, chunks swizzled with (k & 7) << 1), read with two transposing loads.
MI355_DEV void read_kn16(const uint8_t* S, int base, int ks, int lane, v4s& lo, v4s& hi) {
  const int g16 = lane >> 4, m = lane & 15;
  const int nb = base + (g16 & 1) * 16 + 4 * (m & 3);
  const int k0 = ks * 16 + (g16 >> 1) * 8 + (m >> 2), k1 = k0 + 4;
  const int off0 = k0 * 512 + (((nb >> 3) ^ ((k0 & 7) << 1)) << 4) + (nb & 7) * 2;
  const int off1 = k1 * 512 + (((nb >> 3) ^ ((k1 & 7) << 1)) << 4) + (nb & 7) * 2;
  lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(LDS_PTR(v4s, S + off0));
  hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(LDS_PTR(v4s, S + off1));
}

// Element-wise fragment reads and MFMAs and the copies of one iteration, so that one pipelined
// step can interleave them: MFMA t, then its share of the LDS reads of the next stage
// and of the DMA copies. The wave never stalls on the DMA queue or on the LDS return queue for
// long while the matrix core has work.

template <class C, bool MX, bool B_KN, int NM, bool A_KN = false>
MI355_DEV void read_elem(Frags<C, MX, B_KN, A_KN>& f, int e, const uint8_t* As, const uint8_t* Bs, const uint8_t* ASs,
                         const uint8_t* BSRs, int wm, int wn, int lane) {
  constexpr int NI = C::NI;
  if constexpr (!MX) {
    const int ks = e / (NI + NM), q = e % (NI + NM);
    if (q < NI) {
      if constexpr (!B_KN) {
        const int n = wn * C::WN + q * 32 + (lane & 31);
        f.b[ks][q] = *(const v8bf*)(Bs + a_chunk_off(n, ks * 2 + (lane >> 5)));
      } else {
        const int g16 = lane >> 4, m = lane & 15;
        const int nb = wn * C::WN + q * 32 + (g16 & 1) * 16 + 4 * (m & 3);
        const int k0 = ks * 16 + (g16 >> 1) * 8 + (m >> 2), k1 = k0 + 4;
        const int off0 = k0 * 512 + (((nb >> 3) ^ ((k0 & 7) << 1)) << 4) + (nb & 7) * 2;
        const int off1 = k1 * 512 + (((nb >> 3) ^ ((k1 & 7) << 1)) << 4) + (nb & 7) * 2;
        f.bl[ks][q] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(LDS_PTR(v4s, Bs + off0));
        f.bh[ks][q] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(LDS_PTR(v4s, Bs + off1));
      }
    } else {
      if constexpr (A_KN) read_kn16(As, wm * C::WM + (q - NI) * 32, ks, lane, f.al[ks][q - NI], f.ah[ks][q - NI]);
      else f.a[ks][q - NI] = read_a_bf16(As, wm * C::WM + (q - NI) * 32 + (lane & 31), ks, lane);
    }
  } else {
    if (e < NI) {
      if constexpr (B_KN) {
        const int g16 = lane >> 4, m = lane & 15;
        const int nb = wn * C::WN + e * 32 + (g16 & 1) * 16;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int k = (q >> 1) * 32 + (g16 >> 1) * 16 + (q & 1) * 8 + (m >> 1);
          const int off = k * 256 + (((nb >> 4) ^ (k & 15)) << 4) + 8 * (m & 1);
          f.bp[e][q] = __builtin_amdgcn_ds_read_tr8_b64_v2i32(LDS_PTR(v2i, Bs + off));
        }
        f.sb[e] = Bs[C::B_BYTES + (wn * C::WN + e * 32 + (lane & 31)) * 2 + (lane >> 5)];
      } else {
        // K-contiguous weight rows: same fragment layout as the activations
        const int n = wn * C::WN + e * 32 + (lane & 31);
        const int c0 = lane >> 5;
        f.bl[e] = *(const v4i*)(Bs + a_chunk_off(n, c0));
        f.bh[e] = *(const v4i*)(Bs + a_chunk_off(n, c0 + 2));
        f.sb[e] = BSRs[n * 16 + (lane >> 5)];
      }
    } else if constexpr (A_KN) {
      // grouped-K: A tile K-major (64 rows of 256 bytes), read like the EIO weight tile; the two
      // codes of row m (K rows 0-31 / 32-63 of the stage) follow at ASs + 2m
      const int mi = e - NI;
      const int g16 = lane >> 4, m = lane & 15;
      const int mb = wm * C::WM + mi * 32 + (g16 & 1) * 16;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int k = (q >> 1) * 32 + (g16 >> 1) * 16 + (q & 1) * 8 + (m >> 1);
        const int off = k * 256 + (((mb >> 4) ^ (k & 15)) << 4) + 8 * (m & 1);
        f.ap[mi][q] = __builtin_amdgcn_ds_read_tr8_b64_v2i32(LDS_PTR(v2i, As + off));
      }
      f.sa[mi] = ASs[(wm * C::WM + mi * 32 + (lane & 31)) * 2 + (lane >> 5)];
    } else {
      const int r = wm * C::WM + (e - NI) * 32 + (lane & 31);
      const int c0 = lane >> 5;
      f.al[e - NI] = *(const v4i*)(As + a_chunk_off(r, c0));
      f.ah[e - NI] = *(const v4i*)(As + a_chunk_off(r, c0 + 2));
      f.sa[e - NI] = ASs[r * 16 + (lane >> 5)];
    }
  }
}

template <class C, bool MX, bool B_KN, int NM, bool A_KN = false>
MI355_DEV void mfma_elem(const Frags<C, MX, B_KN, A_KN>& f, v16f (&acc)[C::MI][C::NI], int t) {
  constexpr int NI = C::NI;
  if constexpr (!MX) {
    const int ks = t / (NM * NI), mi = (t / NI) % NM, ni = t % NI;
    v8bf b;
    if constexpr (!B_KN) b = f.b[ks][ni];
    else b = __builtin_bit_cast(v8bf, __builtin_shufflevector(f.bl[ks][ni], f.bh[ks][ni], 0, 1, 2, 3, 4, 5, 6, 7));
    v8bf a;
    if constexpr (A_KN) a = __builtin_bit_cast(v8bf, __builtin_shufflevector(f.al[ks][mi], f.ah[ks][mi], 0, 1, 2, 3, 4, 5, 6, 7));
    else a = f.a[ks][mi];
    acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[mi][ni], 0, 0, 0);
  } else {
    const int mi = t / NI, ni = t % NI;
    v8i a;
    if constexpr (A_KN) {
      const v4i a01 = __builtin_shufflevector(f.ap[mi][0], f.ap[mi][1], 0, 1, 2, 3);
      const v4i a23 = __builtin_shufflevector(f.ap[mi][2], f.ap[mi][3], 0, 1, 2, 3);
      a = __builtin_shufflevector(a01, a23, 0, 1, 2, 3, 4, 5, 6, 7);
    } else {
      a = __builtin_shufflevector(f.al[mi], f.ah[mi], 0, 1, 2, 3, 4, 5, 6, 7);
    }
    v8i b;
    if constexpr (B_KN) {
      const v4i b01 = __builtin_shufflevector(f.bp[ni][0], f.bp[ni][1], 0, 1, 2, 3);
      const v4i b23 = __builtin_shufflevector(f.bp[ni][2], f.bp[ni][3], 0, 1, 2, 3);
      b = __builtin_shufflevector(b01, b23, 0, 1, 2, 3, 4, 5, 6, 7);
    } else {
      b = __builtin_shufflevector(f.bl[ni], f.bh[ni], 0, 1, 2, 3, 4, 5, 6, 7);
    }
    acc[mi][ni] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, acc[mi][ni], 0, 0, 0, f.sa[mi], 0, f.sb[ni]);
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

