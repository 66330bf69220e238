// Grouped GEMM copy plan: tile configurations, the per-lane global sources of the direct-to-LDS
// copies and the order in which each wave issues them.
//
// Everything here is __host__ __device__ and takes the copy instruction as a policy type `D`
// (`D::template copy<SZ>(global, lds_offset, smem, enable)`, one lane's share of a wave-wide
// copy): the kernels in gemm.hip instantiate it with the direct-to-LDS load, and the host-side
// copy checker under tests/native instantiates the same code with a recorder that bounds-checks
// every source and LDS destination, compares it with the element the LDS reads expect, and replays
// the vmcnt waits and the ring-slot reuse. The work-item decode and the copy-plan set-up are the
// statement fragments gemm_item_fwd.inc / gemm_item_wgrad.inc and the K-loop prologue is
// gemm_kloop_prologue.inc, included as text by both. A change of the copy schedule is therefore
// checked on the CPU before it runs on a GPU.
#pragma once
#include "common.h"
#include "gemm.h"


// Tile configurations (compile time). Both use 4 waves, tiles of BN = 256 weight columns and
// 64-byte K stages (32 bf16 or 64 e4m3 per row):
//   GGBig   - BM = 256, one workgroup per CU, waves in a 2 x 2 grid of 128 x 128 wave tiles (one
//             wave per SIMD owning all 512 registers); prefill shapes.
//   GGSmall - BM = 64, two workgroups per CU (the weight stream of one CU then runs through two
//             independent pipelines), waves in a 1 x 4 grid of 64 x 64 wave tiles; decode shapes
//             where experts see a few rows each.
// AS_N_ / BSR_N_: slots of the MX activation-scale ring and of the MX EOI weight row-scale ring
// (2, or 0 for a configuration that never runs those paths and spends the LDS on its rings).
template <int BM_, int WGM_, int A_SLOTS_, int B_SLOTS_, int PREFIX_MAX_, int WG_PER_CU_, int AS_N_ = 2, int BSR_N_ = 2>
struct GGCfg {
  static constexpr int BM = BM_;
  static constexpr int BN = 256;
  static constexpr int KB = 64;                        // bytes of K per stage per row
  static constexpr int WAVES = 4;
  static constexpr int THREADS = 64 * WAVES;
  static constexpr int WG_PER_CU = WG_PER_CU_;
  static constexpr int WGM = WGM_, WGN = WAVES / WGM_; // wave grid
  static constexpr int WM = BM / WGM, WN = BN / WGN;   // wave tile
  static constexpr int MI = WM / 32, NI = WN / 32;     // 32 x 32 MFMA subtiles per wave
  // Decoupled rings: activations A (re-read from L2 by the tiles of one expert) and weights B
  // (streamed once from HBM, so it gets the deeper ring).
  static constexpr int A_BYTES = BM * KB;
  static constexpr int B_BYTES = BN * KB;              // 16 KB
  static constexpr int BS_BYTES = BN * 2;              // 512 B (MX EIO: two codes per column)
  static constexpr int B_SLOT = B_BYTES + BS_BYTES;
  static constexpr int A_SLOTS = A_SLOTS_;             // A(k + A_SLOTS) issued at iteration k
  static constexpr int B_SLOTS = B_SLOTS_;             // B(k + B_SLOTS) issued at iteration k
  static constexpr int AS_GROUP = 8;                   // MX: scale codes fetched per 8 stages
  static constexpr int AS_SLOT = BM * 16;              // 16 codes per row
  static constexpr int B_OFF = A_SLOTS * A_BYTES;
  static constexpr int AS_N = AS_N_, BSR_N = BSR_N_;
  static constexpr int AS_OFF = B_OFF + B_SLOTS * B_SLOT;
  static constexpr int PREFIX_MAX = PREFIX_MAX_;       // groups whose tile prefix is kept in LDS
  static constexpr int BSR_SLOT = BN * 16;             // MX EOI weights: 16 scale codes per column
  static constexpr int BSR_OFF = AS_OFF + AS_N * AS_SLOT;
  static constexpr int PREFIX_OFF = BSR_OFF + BSR_N * BSR_SLOT;
  static constexpr int TOTAL = PREFIX_OFF + (PREFIX_MAX + 1) * 4;
  // DMA instructions per wave per stage (64 lanes x 16 bytes each)
  static constexpr int A_INSTR = BM * (KB / 16) / 64 / WAVES;
  static constexpr int B_INSTR = BN * (KB / 16) / 64 / WAVES;
  static constexpr int AS_WAVES = BM / 64;             // waves that fetch A scale rows (64 each)
  // Every wave copies its share of both operands.
  static constexpr int A_PER = A_INSTR;  // activation copies per wave and stage
  static constexpr int B_PER = B_INSTR;  // weight copies per wave and stage
  // the 64-row decode configuration runs the items of a partial last round as column halves
  static constexpr bool HALF_TAIL = BM == 64;
  // epilogue staging (overlays the rings and the scale slots, never the tile prefix)
  static constexpr int EPI_RS_BF16 = BN * 2 + 16;      // bf16 row stride
  static constexpr int EPI_RS_ACT = (BN / 2) * 4 + 16; // SwiGLU fp32 row stride
  static_assert(A_SLOTS >= 3 && A_SLOTS <= B_SLOTS, "ring depths");
  static_assert(!HALF_TAIL || (WGM == 1 && WN == 64), "column halves: wave tiles 2 h and 2 h + 1 of 64 columns");
  static_assert(BM * EPI_RS_BF16 <= PREFIX_OFF, "bf16 epilogue staging must fit");
  static_assert(BM * EPI_RS_ACT <= PREFIX_OFF, "SwiGLU epilogue staging must fit");
  static_assert(TOTAL * WG_PER_CU <= 160 * 1024, "LDS budget");
  static_assert(AS_WAVES >= 1 && AS_WAVES <= WAVES && WAVES * 64 == BN, "scale copies: 64 rows / columns a wave");
  static_assert(A_INSTR >= 1 && NI % 2 == 0 && MI >= 1, "tile shape");
  static_assert(AS_N == 0 || A_SLOTS * BS_BYTES <= AS_N * AS_SLOT,
                "grouped-K MX: per-stage A column scales fit the AS area");
  static_assert((AS_N == 0 || AS_N == 2) && (BSR_N == 0 || BSR_N == 2), "scale rings have two slots or none");
};
using GGBig = GGCfg<256, 2, 3, 5, 1024, 1>;
using GGSmall = GGCfg<64, 1, 3, 3, 256, 2>;

// Tile column j (0..BN-1) -> weight column. SwiGLU: the columns of each wave tile (WN wide) are
// WN/2 gate columns followed by the matching WN/2 up columns, so a lane holds gate and up of the
// same output element.
template <class C>
MI355_HD int tile_col_to_weight_col(int j, int nt, int I, bool swiglu, int gu = 0) {
  if (!swiglu) return nt * C::BN + j;
  constexpr int H = C::WN / 2;
  static_assert(C::WN == 128 || C::WN == 64, "wave tile width");
  int q = j >> (C::WN == 128 ? 7 : 6), jj = j & (C::WN - 1);
  int base = nt * (C::BN / 2) + q * H;
  return gate_up_col(jj < H ? base + jj : I + base + (jj - H), I, gu);
}

MI355_HD int a_chunk_off(int r, int c) { return r * 64 + ((c ^ ((r >> 2) & 3)) << 4); }

// ---- copy plan -------------------------------------------------------------------------------
// Per stage each wave issues A_INSTR + B_INSTR 16-byte DMA instructions; MX adds the B scale codes
// (EIO weights: waves 0 and 1, one 4-byte DMA for 128 columns each, per stage) and, every 8
// stages, 16 scale codes per A row (AS_WAVES waves, 64 rows each) and, for EOI weights, per B
// column (every wave, 64 columns each).
template <class C>
struct CopyPlan {
  const uint8_t* a[C::A_PER];
  const uint8_t* b[C::B_PER];
  const uint8_t* s;        // MX: A scale row (waves < AS_WAVES)
  const uint8_t* bs;       // MX EIO: B scale column pair (waves 0 and 1)
  const uint8_t* bsr;      // MX EOI: B scale row (tile column wave*64 + lane)
  int64_t b_stage_stride;  // bytes to advance B per stage
  int64_t bs_stage_stride; // bytes to advance the B scales per stage
  // grouped-K mode: a[j] / b[j] point at the copy's column of row 0, rows are K
  const uint8_t* zero;     // zero row read by copies past the group's last row
  int64_t lda_k, ldb_k;    // row strides (bytes)
  int a_k[C::A_INSTR], b_k[C::B_INSTR];      // K row of each copy within a stage
  int a_col[C::A_INSTR], b_col[C::B_INSTR];  // byte column of each copy
  int k0, k_end;           // routed-row range of the group
  int64_t as_stage_stride; // grouped-K MX: bytes to advance the A column scales per stage
};

// Waves 0 and 1 copy the per-stage MX weight scales (EIO layout).
MI355_HD bool is_bs_wave(int wave) { return wave < 2; }
// Grouped-K MX: waves 2 and 3 copy the per-stage column scales of A (as waves 0 and 1 do for B).
MI355_HD bool is_as_wave(int wave) { return wave >= 2; }
// Grouped-K mode: routed rows (K) per stage - 32 bf16 rows or 64 e4m3 rows of 256 columns.
template <bool MX>
constexpr int gk_rows() { return MX ? 64 : 32; }

// Source of copy j at stage kt.
template <class C, bool GK, bool MX = false>
MI355_HD const uint8_t* a_src(const CopyPlan<C>& cp, int j, int kt) {
  if constexpr (!GK) {
    return cp.a[j] + (int64_t)kt * C::KB;
  } else {
    const int r = cp.k0 + kt * gk_rows<MX>() + cp.a_k[j];
    return r < cp.k_end ? cp.a[j] + (int64_t)r * cp.lda_k : cp.zero + cp.a_col[j];
  }
}
template <class C, bool GK, bool MX = false>
MI355_HD const uint8_t* b_src(const CopyPlan<C>& cp, int j, int kt) {
  if constexpr (!GK) {
    return cp.b[j] + (int64_t)kt * cp.b_stage_stride;
  } else {
    const int r = cp.k0 + kt * gk_rows<MX>() + cp.b_k[j];
    return r < cp.k_end ? cp.b[j] + (int64_t)r * cp.ldb_k : cp.zero + cp.b_col[j];
  }
}

// ---- copy issue order --------------------------------------------------------------------------
template <class C, bool MX, bool GK, class D>
MI355_HD void issue_a(const CopyPlan<C>& cp, int kt, int wave, uint8_t* smem) {
  const uint32_t base = (kt % C::A_SLOTS) * C::A_BYTES;
#pragma unroll
  for (int j = 0; j < C::A_PER; ++j)
    D::template copy<16>(a_src<C, GK, MX>(cp, j, kt), base + (wave * C::A_PER + j) * 1024, smem, 1);
  if constexpr (MX && GK)
    if (is_as_wave(wave))
      D::template copy<4>(cp.s + kt * cp.as_stage_stride, C::AS_OFF + (kt % C::A_SLOTS) * C::BS_BYTES + (wave & 1) * 256,
                          smem, 1);
}
template <class C, bool MX, bool B_KN, bool GK, class D>
MI355_HD void issue_b(const CopyPlan<C>& cp, int kt, int wave, uint8_t* smem) {
  // (MX with K-contiguous weights has no per-stage scale copy: its scales come in groups)
  const uint32_t base = C::B_OFF + (kt % C::B_SLOTS) * C::B_SLOT;
  if constexpr (!GK) {
    const int64_t boff = (int64_t)kt * cp.b_stage_stride;
#pragma unroll
    for (int j = 0; j < C::B_PER; ++j) D::template copy<16>(cp.b[j] + boff, base + (wave * C::B_PER + j) * 1024, smem, 1);
  } else {
#pragma unroll
    for (int j = 0; j < C::B_INSTR; ++j)
      D::template copy<16>(b_src<C, GK, MX>(cp, j, kt), base + (wave * C::B_INSTR + j) * 1024, smem, 1);
  }
  if (MX && B_KN && is_bs_wave(wave)) D::template copy<4>(cp.bs + kt * cp.bs_stage_stride, base + C::B_BYTES + wave * 256, smem, 1);
}
// MX: A scale codes of stages 8*grp .. 8*grp+7 (16 bytes per row) into AS slot grp & 1.
template <class C, class D>
MI355_HD void issue_as(const CopyPlan<C>& cp, int grp, int wave, uint8_t* smem) {
  if (wave < C::AS_WAVES) D::template copy<16>(cp.s + grp * 16, C::AS_OFF + (grp & 1) * C::AS_SLOT + wave * 1024, smem, 1);
}

// Work of one pipelined K step of a wave that computes NM 32-row subtiles: MFMAs, LDS fragment
// reads of the next stage and copy items (issue_item), interleaved by the K loop.
template <class C, bool MX, int NM, bool GK = false> struct StepShape {
  static constexpr int MFMAS = MX ? NM * C::NI : 2 * NM * C::NI;
  static constexpr int READS = MX ? C::NI + NM : 2 * (C::NI + NM);  // fragment elements of a stage
  // B copies, B scales, A copies (grouped-K MX: and the A column scales)
  static constexpr int ITEMS = C::B_PER + 1 + C::A_PER + ((MX && GK) ? 1 : 0);
};

// Copy item it of iteration i (same order as issue_iteration: B copies, B scales, A copies, and in
// grouped-K MX mode the A column scales).
template <class C, bool MX, bool B_KN, bool LA, bool GK, class D>
MI355_HD void issue_item(const CopyPlan<C>& cp, int i, int nk, int wave, uint8_t* smem, int it) {
  constexpr int DA = C::A_SLOTS, DB = C::B_SLOTS;
  if (it < C::B_PER) {
    const int kt = i + DB;
    D::template copy<16>(b_src<C, GK, MX>(cp, it, kt),
                         C::B_OFF + (kt % C::B_SLOTS) * C::B_SLOT + (wave * C::B_PER + it) * 1024, smem, kt < nk);
  } else if (it == C::B_PER) {
    const int kt = i + DB;
    if constexpr (MX && B_KN)
      D::template copy<4>(cp.bs + kt * cp.bs_stage_stride,
                          C::B_OFF + (kt % C::B_SLOTS) * C::B_SLOT + C::B_BYTES + (wave & 1) * 256, smem,
                          is_bs_wave(wave) && kt < nk);
  } else if constexpr (LA) {
    const int j = it - C::B_PER - 1;
    const int kt = i + DA;
    if (!(MX && GK) || j < C::A_PER) {
      D::template copy<16>(a_src<C, GK, MX>(cp, j, kt),
                           (kt % C::A_SLOTS) * C::A_BYTES + (wave * C::A_PER + j) * 1024, smem, kt < nk);
    } else if constexpr (MX && GK) {
      D::template copy<4>(cp.s + kt * cp.as_stage_stride,
                          C::AS_OFF + (kt % C::A_SLOTS) * C::BS_BYTES + (wave & 1) * 256, smem,
                          is_as_wave(wave) && kt < nk);
    }
  }
}

// MX: the scale groups due at iteration i (every AS_GROUP stages: A rows and, for K-contiguous
// weights, B rows), each as one conditional copy.
template <class C, bool MX, bool B_KN, bool LA, class D, bool GK = false>
MI355_HD void issue_scales_item(const CopyPlan<C>& cp, int i, int nk, int wave, uint8_t* smem) {
  if constexpr (MX && !GK) {
    const int grp = i / C::AS_GROUP + 1;
    const bool due = (i & (C::AS_GROUP - 1)) == 0 && i + C::AS_GROUP < nk;
    if constexpr (LA) {
      D::template copy<16>(cp.s + grp * 16, C::AS_OFF + (grp & 1) * C::AS_SLOT + (wave & 3) * 1024, smem,
                           due && wave < C::AS_WAVES);
    }
    if constexpr (!B_KN)
      D::template copy<16>(cp.bsr + grp * 16, C::BSR_OFF + (grp & 1) * C::BSR_SLOT + (wave & 3) * 1024, smem, due);
  }
}

// Loads of stage j still allowed in flight (younger than stage j's last load) once iterations
// up to `last` have issued. Iteration i issues B(i + DB), then A(i + DA) (DB = B_SLOTS >= DA =
// A_SLOTS; the prologue runs iterations -DB .. -1), each only below nk. Stage j's last load is A(j)
// (iteration j - DA; B(j) came earlier) for a wave that copies A, else B(j) (iteration j - DB).
// Scale groups issued between are not counted, which only makes the wait stricter. Loads of one
// wave retire in order.
template <class C, bool LA>
MI355_HD int younger_than(int j, int last, int nk, int la_n, int lb_n) {
  constexpr int DA = C::A_SLOTS, DB = C::B_SLOTS;
  const int from = (LA ? j - DA : j - DB) + 1;
  // iterations i in [from, last] with i + DB < nk, and (A) with 0 <= i + DA < nk
  const int lb = last < nk - DB - 1 ? last : nk - DB - 1;
  const int nb = lb - from + 1;
  int n = (nb > 0 ? nb : 0) * lb_n;
  if (LA) {
    const int la = last < nk - DA - 1 ? last : nk - DA - 1;
    const int fa = from > -DA ? from : -DA;
    const int na = la - fa + 1;
    n += (na > 0 ? na : 0) * la_n;
  }
  return n;
}

template <class C, bool MX, bool B_KN, bool LA, bool GK, class D>
MI355_HD void issue_iteration(const CopyPlan<C>& cp, int i, int nk, int wave, uint8_t* smem) {
  constexpr int DA = C::A_SLOTS, DB = C::B_SLOTS;
  if (i + DB < nk) issue_b<C, MX, B_KN, GK, D>(cp, i + DB, wave, smem);
  if (LA && i + DA >= 0 && i + DA < nk) {
    if (MX && !GK && i + DA == 0) issue_as<C, D>(cp, 0, wave, smem);
    issue_a<C, MX, GK, D>(cp, i + DA, wave, smem);
  }
  if (LA && MX && !GK && i >= 0 && (i & (C::AS_GROUP - 1)) == 0 && i + C::AS_GROUP < nk)
    issue_as<C, D>(cp, i / C::AS_GROUP + 1, wave, smem);
}

// Whether a wave copies activation rows: waves whose A rows all lie past the tile's valid rows
// issue no A copies (and no A scale copies).
template <class C>
MI355_HD bool wave_copies_a(int wave, int rows_valid) {
  return wave * (C::A_PER * 16) < rows_valid;
}

// ---- LDS fragment reads and MFMAs ---------------------------------------------------------------
// The transposing LDS loads and the MFMAs (the lane-crossing instructions) go through a policy type
// `O`: DevOps issues the gfx950 instructions; the host-side checker under tests/native runs the same
// fragment code with an emulation of those instructions to compute whole tiles on the CPU.
struct DevOps {
  MI355_DEV static v4s tr16(const uint8_t* p) { return __builtin_amdgcn_ds_read_tr16_b64_v4i16(LDS_PTR(v4s, p)); }
  MI355_DEV static v2i tr8(const uint8_t* p) { return __builtin_amdgcn_ds_read_tr8_b64_v2i32(LDS_PTR(v2i, p)); }
  MI355_DEV static void mfma_bf16(v8bf a, v8bf b, v16f& acc) {
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc, 0, 0, 0);
  }
  MI355_DEV static void mfma_f8(v8i a, v8i b, v16f& acc, int sa, int sb) {
    acc = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, acc, 0, 0, 0, sa, 0, sb);
  }
};

// fragment loads (one K step: 16 bf16 or 64 e4m3)
template <class O = DevOps>
MI355_HD v8bf read_a_bf16(const uint8_t* As, int r, int ks, int lane) {
  return *(const v8bf*)(As + a_chunk_off(r, ks * 2 + (lane >> 5)));
}

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
template <class O = DevOps>
MI355_HD void read_kn16(const uint8_t* S, int base, int ks, int lane, v4s& lo, v4s& hi) {
  const int g16 = lane >> 4, m = lane & 15;
  const int nb = base + (g16 & 1) * 16 + 4 * (m & 3);
  const int k0 = ks * 16 + (g16 >> 1) * 8 + (m >> 2), k1 = k0 + 4;
  const int off0 = k0 * 512 + (((nb >> 3) ^ ((k0 & 7) << 1)) << 4) + (nb & 7) * 2;
  const int off1 = k1 * 512 + (((nb >> 3) ^ ((k1 & 7) << 1)) << 4) + (nb & 7) * 2;
  lo = O::tr16(S + off0);
  hi = O::tr16(S + off1);
}

// Element-wise fragment reads and MFMAs and the copies of one iteration, so that one pipelined
// step can interleave them: MFMA t, then its share of the LDS reads of the next stage
// and of the DMA copies. The wave never stalls on the DMA queue or on the LDS return queue for
// long while the matrix core has work.

template <class C, bool MX, bool B_KN, int NM, bool A_KN = false, class O = DevOps>
MI355_HD void read_elem(Frags<C, MX, B_KN, A_KN>& f, int e, const uint8_t* As, const uint8_t* Bs, const uint8_t* ASs,
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
        f.bl[ks][q] = O::tr16(Bs + off0);
        f.bh[ks][q] = O::tr16(Bs + off1);
      }
    } else {
      if constexpr (A_KN) read_kn16<O>(As, wm * C::WM + (q - NI) * 32, ks, lane, f.al[ks][q - NI], f.ah[ks][q - NI]);
      else f.a[ks][q - NI] = read_a_bf16<O>(As, wm * C::WM + (q - NI) * 32 + (lane & 31), ks, lane);
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
          f.bp[e][q] = O::tr8(Bs + off);
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
        f.ap[mi][q] = O::tr8(As + off);
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

template <class C, bool MX, bool B_KN, int NM, bool A_KN = false, class O = DevOps>
MI355_HD void mfma_elem(const Frags<C, MX, B_KN, A_KN>& f, v16f (&acc)[C::MI][C::NI], int t) {
  constexpr int NI = C::NI;
  if constexpr (!MX) {
    const int ks = t / (NM * NI), mi = (t / NI) % NM, ni = t % NI;
    v8bf b;
    if constexpr (!B_KN) b = f.b[ks][ni];
    else b = __builtin_bit_cast(v8bf, __builtin_shufflevector(f.bl[ks][ni], f.bh[ks][ni], 0, 1, 2, 3, 4, 5, 6, 7));
    v8bf a;
    if constexpr (A_KN) a = __builtin_bit_cast(v8bf, __builtin_shufflevector(f.al[ks][mi], f.ah[ks][mi], 0, 1, 2, 3, 4, 5, 6, 7));
    else a = f.a[ks][mi];
    O::mfma_bf16(a, b, acc[mi][ni]);
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
    O::mfma_f8(a, b, acc[mi][ni], f.sa[mi], f.sb[ni]);
  }
}

