// Persistent grouped GEMM for gfx950 (MI355X): bf16 and MXFP8 (e4m3 + e8m0 per 32 along K).
//
// Work list: the row segments of the groups (experts) are cut into BM-row tiles; every
// (group, m-tile, n-tile) is one work item. tile_prefix[g] (computed on the device from the
// group row counts) gives the first m-tile of group g, so the work list needs no host round
// trip. The grid is one workgroup per CU; workgroup i runs on XCD i % 8 and walks the work list
// in rounds so that each XCD takes a contiguous run of items per round (m fastest): items that
// share a weight slice run at the same time on one XCD and share its L2.
//
// Workgroup: 256 threads = 4 wavefronts, one per SIMD, in a 2 (M) x 2 (N) grid; tile BM=256 x
// BN=256; each wavefront computes 128 x 128 with 4 x 4 32x32 MFMAs (bf16:
// v_mfma_f32_32x32x16_bf16; MXFP8: v_mfma_scale_f32_32x32x64_f8f6f4 with per-lane e8m0 scales:
// lane r + 32b supplies the scale of 32-block b of row / column r, and its operand bytes 0-15 /
// 16-31 hold K = 16b + i / 32 + 16b + i of the 64-K step). With one wave per SIMD each wave owns
// 512 registers: the accumulators live in the AGPRs, two stages of operand fragments in VGPRs.
// A stage holds 64 bytes of K per row (32 bf16 or 64 e4m3). Global -> LDS copies use the
// direct-to-LDS loads into decoupled rings (activations 3 slots, weights 5 slots). Each K step is
// software-pipelined inside the wave: after the stage barrier the wave interleaves the MFMAs of
// stage k with the LDS fragment reads of stage k+1 and with its share of the copies that refill
// the slots of stage k, so the matrix cores, the LDS and the copy engine work at the same time.
//
// LDS layouts (16-byte chunk granularity, XOR swizzled against bank conflicts):
//   K-contiguous operand rows (A always; B in EOI layout): row r at r*64, chunk c stored at
//     c ^ ((r >> 2) & 3); read with ds_read_b128.
//   N-contiguous B (EIO bf16 / MX col_data): row k holds 256 columns; bf16 chunk c stored at
//     c ^ ((k & 7) << 1) (512-byte rows), e4m3 chunk c at c ^ (k & 15) (256-byte rows); read
//     with the transposing ds_read_b64_tr_b16 / ds_read_b64_tr_b8.
//   MX scales: A rows get 16 codes (8 stages) per copy into a 2-slot ring; B in EIO layout the two
//     codes of every tile column per stage (col_scale's [.., N, 2] pairs) with the B stage; B in
//     EOI layout 16 codes per column per 8 stages, like A.
//
// Epilogues: bf16 store, fp32 store (router logits, optional row scatter), SwiGLU -> bf16 and
// SwiGLU -> MXFP8 requant. For SwiGLU the B tile columns are gate/up interleaved in 64-column
// groups so that each lane holds the gate and up value of the same output element.
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
    const v8i a = __builtin_shufflevector(f.al[mi], f.ah[mi], 0, 1, 2, 3, 4, 5, 6, 7);
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
  using SS = StepShape<C, MX, NM>;
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
    const uint8_t* ASs = smem + C::AS_OFF + ((kn / C::AS_GROUP) & 1) * C::AS_SLOT + (kn & (C::AS_GROUP - 1)) * 2;
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
    issue_scales_item<C, MX, B_KN, LA, DevDma>(cp, k, nk, wave, smem);
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

template <class C, bool MX, bool B_KN, int EPI>
__global__ __launch_bounds__(C::THREADS, C::WG_PER_CU) void grouped_gemm_kernel(GGParams p) {
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
  const int total = prefix[p.G] * p.n_tiles * splits;
  const int nk = p.K / splits * ESIZE / C::KB;  // stages per work item
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
    const int nm = (C::MI >= 4 && rows_w > 64) ? 4 : ((C::MI >= 2 && rows_w > 32) ? 2 : (rows_w >= 1 ? 1 : 0));
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

    // ---- epilogue -----------------------------------------------------------------------
    // acc[mi][ni][r] holds row wm*WM + mi*32 + 8*(r/4) + 4*(lane/32) + r%4,
    // column wn*WN + ni*32 + lane%32 of the tile.
    if (EPI == EPI_STORE_F32) {
      float* outp = (float*)p.C;
#pragma unroll
      for (int mi = 0; mi < C::MI; ++mi)
#pragma unroll
        for (int ni = 0; ni < C::NI; ++ni) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            int row = wm * C::WM + mi * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            int col = nt * C::BN + wn * C::WN + ni * 32 + (lane & 31);
            if (row < rows_valid && col < p.N) {
              int64_t routed = tile_row0 + row;
              int64_t orow = p.c_row_index ? (int64_t)p.c_row_index[routed] : routed;
              outp[split * p.c_split_stride + orow * p.ldc + col] = acc[mi][ni][r];
            }
          }
          __builtin_amdgcn_sched_barrier(0);
        }
    } else if (EPI == EPI_STORE_BF16) {
      constexpr int RS = C::EPI_RS_BF16;  // staged row stride (bytes)
#pragma unroll
      for (int mi = 0; mi < C::MI; ++mi)
#pragma unroll
        for (int ni = 0; ni < C::NI; ++ni) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            int row = wm * C::WM + mi * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            int col = wn * C::WN + ni * 32 + (lane & 31);
            *(uint16_t*)(smem + row * RS + col * 2) = f32_to_bf16(acc[mi][ni][r]);
          }
          __builtin_amdgcn_sched_barrier(0);  // one 32x32 block at a time: bounded register use
        }
      __syncthreads();
      uint16_t* outp = (uint16_t*)p.C;
      for (int id = tid; id < C::BM * (C::BN / 8); id += C::THREADS) {
        int row = id >> 5, ch = id & 31;
        int col = nt * C::BN + ch * 8;
        if (row < rows_valid && col < p.N)
          *(uint4*)(outp + (tile_row0 + row) * p.ldc + col) = *(const uint4*)(smem + row * RS + ch * 16);
      }
      __syncthreads();
    } else {
      // SwiGLU: subtiles ni < NI/2 hold gate, ni + NI/2 the matching up columns.
      constexpr int RS = C::EPI_RS_ACT;  // fp32 staged act row stride
#pragma unroll
      for (int mi = 0; mi < C::MI; ++mi)
#pragma unroll
        for (int ni = 0; ni < C::NI / 2; ++ni) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            int row = wm * C::WM + mi * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            int col = wn * (C::WN / 2) + ni * 32 + (lane & 31);
            float gte = bf16_to_f32(f32_to_bf16(acc[mi][ni][r]));
            float up = bf16_to_f32(f32_to_bf16(acc[mi][ni + C::NI / 2][r]));
            float act;
            if (EPI == EPI_SWIGLU_BF16_NUM && p.swiglu_limit > 0.0f) {
              // MegaMoeNumericsOptions clamp: up to [-L, L]; gate to <= L before SiLU, or SiLU(gate)
              // to <= L after it
              const float L = p.swiglu_limit;
              up = fminf(fmaxf(up, -L), L);
              if (p.swiglu_after_silu) act = fminf(gte / (1.0f + __expf(-gte)), L) * up;
              else {
                const float gc = fminf(gte, L);
                act = gc / (1.0f + __expf(-gc)) * up;
              }
            } else {
              act = gte / (1.0f + __expf(-gte)) * up;
            }
            *(float*)(smem + row * RS + col * 4) = act;
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      __syncthreads();
      if (EPI == EPI_SWIGLU_BF16 || EPI == EPI_SWIGLU_BF16_NUM) {
        uint16_t* outp = (uint16_t*)p.C;
        for (int id = tid; id < C::BM * 16; id += C::THREADS) {
          int row = id >> 4, ch = id & 15;
          if (row < rows_valid) {
            const float* s = (const float*)(smem + row * RS + ch * 32);
            uint4 o;
            if (EPI == EPI_SWIGLU_BF16_NUM) {
              float v[8];
#pragma unroll
              for (int i = 0; i < 8; ++i) v[i] = s[i];
              if (p.row_prob != nullptr) {
                // probabilities before FC2: bf16(fp32(bf16(act)) * p) (two roundings, the reference
                // contract); row r of the tile is slot a_row_index[r]
                const float pr = p.row_prob[p.a_row_index[tile_row0 + row]];
#pragma unroll
                for (int i = 0; i < 8; ++i) v[i] = bf16_to_f32(f32_to_bf16(v[i])) * pr;
              }
              o.x = f32_to_bf16(v[0]) | ((uint32_t)f32_to_bf16(v[1]) << 16);
              o.y = f32_to_bf16(v[2]) | ((uint32_t)f32_to_bf16(v[3]) << 16);
              o.z = f32_to_bf16(v[4]) | ((uint32_t)f32_to_bf16(v[5]) << 16);
              o.w = f32_to_bf16(v[6]) | ((uint32_t)f32_to_bf16(v[7]) << 16);
            } else {
              o.x = f32_to_bf16(s[0]) | ((uint32_t)f32_to_bf16(s[1]) << 16);
              o.y = f32_to_bf16(s[2]) | ((uint32_t)f32_to_bf16(s[3]) << 16);
              o.z = f32_to_bf16(s[4]) | ((uint32_t)f32_to_bf16(s[5]) << 16);
              o.w = f32_to_bf16(s[6]) | ((uint32_t)f32_to_bf16(s[7]) << 16);
            }
            *(uint4*)(outp + (tile_row0 + row) * p.ldc + nt * (C::BN / 2) + ch * 8) = o;
          }
        }
      } else {
        uint8_t* outp = (uint8_t*)p.C;
        for (int id = tid; id < C::BM * 4; id += C::THREADS) {
          int row = id >> 2, blk = id & 3;
          if (row < rows_valid) {
            const float* s = (const float*)(smem + row * RS + blk * 128);
            float amax = 0.0f;
#pragma unroll
            for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(s[i]));
            uint32_t code = mx_scale_code(amax);
            uint32_t w[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
              uint32_t b0 = f32_to_e4m3(mx_apply_inv_scale(s[4 * i + 0], code));
              uint32_t b1 = f32_to_e4m3(mx_apply_inv_scale(s[4 * i + 1], code));
              uint32_t b2 = f32_to_e4m3(mx_apply_inv_scale(s[4 * i + 2], code));
              uint32_t b3 = f32_to_e4m3(mx_apply_inv_scale(s[4 * i + 3], code));
              w[i] = b0 | (b1 << 8) | (b2 << 16) | (b3 << 24);
            }
            uint8_t* dst = outp + (tile_row0 + row) * p.ldc + nt * (C::BN / 2) + blk * 32;
            *(uint4*)dst = make_uint4(w[0], w[1], w[2], w[3]);
            *(uint4*)(dst + 16) = make_uint4(w[4], w[5], w[6], w[7]);
            p.c_scale[(tile_row0 + row) * p.c_scale_ld + nt * 4 + blk] = (uint8_t)code;
          }
        }
      }
      __syncthreads();
    }
  }
}

// Grouped-K GEMM (weight gradients): C_g[m, n] = sum over the rows r of group g (group_list) of
// A[r, m] * B[r, n], bf16 in, fp32 accumulate, C_g = C + g * c_group_stride (fp32 or bf16 store).
// Both operands are read K-major (rows = K) into the same LDS layout as an EIO weight tile and
// read with transposing loads; rows past a group's end come from a zero row, so groups of any
// size (including none: C_g = 0) are exact. Work items are (group, m-tile, n-tile), m fastest.
template <class C, int EPI>
__global__ __launch_bounds__(C::THREADS, C::WG_PER_CU) void grouped_gemm_wgrad_kernel(GGParams p) {
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = (int)((unsigned)wave / C::WGN), wn = (int)((unsigned)wave % C::WGN);
  const int per_g = p.m_tiles * p.n_tiles;
  const int total = p.G * per_g;
  const int xcd = blockIdx.x & 7;
  const int per_xcd = gridDim.x >> 3;
  const int slot = blockIdx.x >> 3;
  for (int round = 0;; ++round) {
    const int L = round * (int)gridDim.x + xcd * per_xcd + slot;
    if (L >= total) break;
#include "gemm_item_wgrad.inc"

    v16f acc[C::MI][C::NI];
#pragma unroll
    for (int i = 0; i < C::MI; ++i)
#pragma unroll
      for (int j = 0; j < C::NI; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    __syncthreads();  // the previous item's epilogue reads are done before refilling
    if (nk > 0) {
      const int rows_w = rows_valid - wm * C::WM;
      const int nm = (C::MI >= 4 && rows_w > 64) ? 4 : ((C::MI >= 2 && rows_w > 32) ? 2 : (rows_w >= 1 ? 1 : 0));
      if (C::MI >= 4 && nm == 4) k_loop<C, false, true, (C::MI >= 4 ? 4 : 1), true, true>(cp, nk, wave, wm, wn, lane, smem, acc);
      else if (nm == 2) k_loop<C, false, true, 2, true, true>(cp, nk, wave, wm, wn, lane, smem, acc);
      else if (nm == 1) k_loop<C, false, true, 1, true, true>(cp, nk, wave, wm, wn, lane, smem, acc);
      else k_loop<C, false, true, 0, true, true>(cp, nk, wave, wm, wn, lane, smem, acc);
    }
    __syncthreads();  // all waves are done reading the ring before the epilogue reuses LDS

    // acc[mi][ni][r] holds row (m) wm*WM + mi*32 + 8*(r/4) + 4*(lane/32) + r%4 and column (n)
    // wn*WN + ni*32 + lane%32 of the tile
    if constexpr (EPI == EPI_STORE_F32) {
      float* outp = (float*)p.C + (int64_t)g * p.c_group_stride;
#pragma unroll
      for (int mi = 0; mi < C::MI; ++mi)
#pragma unroll
        for (int ni = 0; ni < C::NI; ++ni) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int row = wm * C::WM + mi * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            const int col = nt * C::BN + wn * C::WN + ni * 32 + (lane & 31);
            if (row < rows_valid && col < p.N) outp[(int64_t)(m0 + row) * p.ldc + col] = acc[mi][ni][r];
          }
          __builtin_amdgcn_sched_barrier(0);
        }
    } else {
      constexpr int RS = C::EPI_RS_BF16;
#pragma unroll
      for (int mi = 0; mi < C::MI; ++mi)
#pragma unroll
        for (int ni = 0; ni < C::NI; ++ni) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int row = wm * C::WM + mi * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            const int col = wn * C::WN + ni * 32 + (lane & 31);
            *(uint16_t*)(smem + row * RS + col * 2) = f32_to_bf16(acc[mi][ni][r]);
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      __syncthreads();
      uint16_t* outp = (uint16_t*)p.C + (int64_t)g * p.c_group_stride;
      for (int id = tid; id < C::BM * (C::BN / 8); id += C::THREADS) {
        const int row = id >> 5, ch = id & 31;
        const int col = nt * C::BN + ch * 8;
        if (row < rows_valid && col < p.N)
          *(uint4*)(outp + (int64_t)(m0 + row) * p.ldc + col) = *(const uint4*)(smem + row * RS + ch * 16);
      }
      __syncthreads();
    }
  }
}

// tile_prefix[g] = sum_{g' < g} ceil(rows_g' / BM) from an inclusive group_list.
__global__ __launch_bounds__(1024) void plan_tiles_kernel(const int64_t* group_list, int G, int bm,
                                                          int32_t* tile_prefix) {
  __shared__ int64_t vals[4096];
  __shared__ int64_t wsum[17];
  for (int g = threadIdx.x; g < G; g += 1024) {
    int64_t prev = g == 0 ? 0 : group_list[g - 1];
    int64_t rows = group_list[g] - prev;
    vals[g] = rows > 0 ? (rows + bm - 1) / bm : 0;
  }
  __syncthreads();
  int64_t total = block_exclusive_scan_1024(vals, G, wsum);
  for (int g = threadIdx.x; g < G; g += 1024) tile_prefix[g] = (int32_t)vals[g];
  if (threadIdx.x == 0) tile_prefix[G] = (int32_t)total;
}

// CU count of the current device, cached per device (the persistent grids are sized from it).
static int g_num_cus[64] = {};
static int num_cus() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  if (g_num_cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    g_num_cus[dev] = n;
  }
  return g_num_cus[dev];
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
  int grid = (num_cus() / 8) * 8 * C::WG_PER_CU;
  if (grid < 8) grid = 8;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(C::THREADS), C::TOTAL, stream, p);
  return hipGetLastError() == hipSuccess ? MI355MOE_OK : MI355MOE_ELAUNCH;
}

int mi355_plan_tiles(const int64_t* group_list, int G, int32_t* tile_prefix, hipStream_t stream, bool small) {
  hipLaunchKernelGGL(plan_tiles_kernel, dim3(1), dim3(1024), 0, stream, group_list, G, mi355_gg_bm(small), tile_prefix);
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
  if (!b_kn) {
    switch (epi) {
      case EPI_STORE_BF16: return launch_gg<C, true, false, EPI_STORE_BF16>(p, stream);
      case EPI_SWIGLU_MX: return launch_gg<C, true, false, EPI_SWIGLU_MX>(p, stream);
      default: return MI355MOE_EUNSUPPORTED;
    }
  }
  switch (epi) {
    case EPI_STORE_BF16: return launch_gg<C, true, true, EPI_STORE_BF16>(p, stream);
    case EPI_SWIGLU_MX: return launch_gg<C, true, true, EPI_SWIGLU_MX>(p, stream);
    default: return MI355MOE_EUNSUPPORTED;
  }
}

template <class C, int EPI>
static int launch_wgrad(const GGParams& p, hipStream_t stream) {
  static bool configured = false;
  auto kern = grouped_gemm_wgrad_kernel<C, EPI>;
  if (!configured) {
    if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, C::TOTAL) != hipSuccess)
      return MI355MOE_ELAUNCH;
    configured = true;
  }
  int grid = (num_cus() / 8) * 8 * C::WG_PER_CU;
  if (grid < 8) grid = 8;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(C::THREADS), C::TOTAL, stream, p);
  return hipGetLastError() == hipSuccess ? MI355MOE_OK : MI355MOE_ELAUNCH;
}

int mi355_grouped_gemm_wgrad(const GGParams& p, int epi, hipStream_t stream) {
  if (p.m_rows % 8 || p.N % 8 || p.m_tiles != (p.m_rows + GGBig::BM - 1) / GGBig::BM ||
      p.n_tiles != (p.N + GGBig::BN - 1) / GGBig::BN || p.zero_row == nullptr)
    return MI355MOE_EINVAL;
  switch (epi) {
    case EPI_STORE_F32: return launch_wgrad<GGBig, EPI_STORE_F32>(p, stream);
    case EPI_STORE_BF16: return launch_wgrad<GGBig, EPI_STORE_BF16>(p, stream);
    default: return MI355MOE_EUNSUPPORTED;
  }
}

// Internal dispatcher used by the C-ABI entry points. `small` selects the 64-row tile
// configuration (the tile prefix must have been planned with the same one).
int mi355_grouped_gemm(const GGParams& p, bool mx, bool b_kn, int epi, hipStream_t stream, bool small) {
  if (epi == EPI_SWIGLU_BF16_NUM) return MI355MOE_EINVAL;  // internal: chosen from the options below
  if (epi == EPI_SWIGLU_BF16 && (p.swiglu_limit > 0.0f || p.row_prob != nullptr)) epi = EPI_SWIGLU_BF16_NUM;
  if (small) {
    // the EPI_STORE_F32 router projection keeps the big tiles
    if (epi == EPI_STORE_F32) return MI355MOE_EUNSUPPORTED;
    return dispatch_gg<GGSmall>(p, mx, b_kn, epi, stream);
  }
  return dispatch_gg<GGBig>(p, mx, b_kn, epi, stream);
}

int mi355_gg_bm(bool small) { return small ? GGSmall::BM : GGBig::BM; }
int mi355_gg_bn() { return GGBig::BN; }
