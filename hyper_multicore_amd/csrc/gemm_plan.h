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

#define MI355_HD __host__ __device__ __forceinline__

// Tile configurations (compile time). Both use 4 waves, tiles of BN = 256 weight columns and
// 64-byte K stages (32 bf16 or 64 e4m3 per row):
//   GGBig   - BM = 256, one workgroup per CU, waves in a 2 x 2 grid of 128 x 128 wave tiles (one
//             wave per SIMD owning all 512 registers); prefill shapes.
//   GGSmall - BM = 64, two workgroups per CU (the weight stream of one CU then runs through two
//             independent pipelines), waves in a 1 x 4 grid of 64 x 64 wave tiles; decode shapes
//             where experts see a few rows each.
template <int BM_, int WGM_, int A_SLOTS_, int B_SLOTS_, int PREFIX_MAX_, int WG_PER_CU_>
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
  static constexpr int AS_OFF = B_OFF + B_SLOTS * B_SLOT;
  static constexpr int PREFIX_MAX = PREFIX_MAX_;       // groups whose tile prefix is kept in LDS
  static constexpr int BSR_SLOT = BN * 16;             // MX EOI weights: 16 scale codes per column
  static constexpr int BSR_OFF = AS_OFF + 2 * AS_SLOT;
  static constexpr int PREFIX_OFF = BSR_OFF + 2 * BSR_SLOT;
  static constexpr int TOTAL = PREFIX_OFF + (PREFIX_MAX + 1) * 4;
  // DMA instructions per wave per stage (64 lanes x 16 bytes each)
  static constexpr int A_INSTR = BM * (KB / 16) / 64 / WAVES;
  static constexpr int B_INSTR = BN * (KB / 16) / 64 / WAVES;
  static constexpr int AS_WAVES = BM / 64;             // waves that fetch A scale rows (64 each)
  // epilogue staging (overlays the rings and the scale slots, never the tile prefix)
  static constexpr int EPI_RS_BF16 = BN * 2 + 16;      // bf16 row stride
  static constexpr int EPI_RS_ACT = (BN / 2) * 4 + 16; // SwiGLU fp32 row stride
  static_assert(A_SLOTS >= 3 && A_SLOTS <= B_SLOTS, "ring depths");
  static_assert(BM * EPI_RS_BF16 <= PREFIX_OFF, "bf16 epilogue staging must fit");
  static_assert(BM * EPI_RS_ACT <= PREFIX_OFF, "SwiGLU epilogue staging must fit");
  static_assert(TOTAL * WG_PER_CU <= 160 * 1024, "LDS budget");
  static_assert(AS_WAVES >= 1 && AS_WAVES <= WAVES && WAVES * 64 == BN, "scale copies: 64 rows / columns a wave");
  static_assert(A_INSTR >= 1 && NI % 2 == 0 && MI >= 1, "tile shape");
  static_assert(A_SLOTS * BS_BYTES <= 2 * AS_SLOT, "grouped-K MX: per-stage A column scales fit the AS area");
};
using GGBig = GGCfg<256, 2, 3, 5, 1024, 1>;
using GGSmall = GGCfg<64, 1, 3, 3, 256, 2>;

// Tile column j (0..BN-1) -> weight column. SwiGLU: the columns of each wave tile (WN wide) are
// WN/2 gate columns followed by the matching WN/2 up columns, so a lane holds gate and up of the
// same output element.
template <class C>
MI355_HD int tile_col_to_weight_col(int j, int nt, int I, bool swiglu) {
  if (!swiglu) return nt * C::BN + j;
  constexpr int H = C::WN / 2;
  static_assert(C::WN == 128 || C::WN == 64, "wave tile width");
  int q = j >> (C::WN == 128 ? 7 : 6), jj = j & (C::WN - 1);
  int base = nt * (C::BN / 2) + q * H;
  return jj < H ? base + jj : I + base + (jj - H);
}

MI355_HD int a_chunk_off(int r, int c) { return r * 64 + ((c ^ ((r >> 2) & 3)) << 4); }

// ---- copy plan -------------------------------------------------------------------------------
// Per stage each wave issues A_INSTR + B_INSTR 16-byte DMA instructions; MX adds the B scale codes
// (EIO weights: waves 0 and 1, one 4-byte DMA for 128 columns each, per stage) and, every 8
// stages, 16 scale codes per A row (AS_WAVES waves, 64 rows each) and, for EOI weights, per B
// column (every wave, 64 columns each).
template <class C>
struct CopyPlan {
  const uint8_t* a[C::A_INSTR];
  const uint8_t* b[C::B_INSTR];
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
#ifdef GG_ABLATE_DMA
  if (wave < 64) return;
#endif
  const uint32_t base = (kt % C::A_SLOTS) * C::A_BYTES;
#pragma unroll
  for (int j = 0; j < C::A_INSTR; ++j)
    D::template copy<16>(a_src<C, GK, MX>(cp, j, kt), base + (wave * C::A_INSTR + j) * 1024, smem, 1);
  if constexpr (MX && GK)
    if (is_as_wave(wave))
      D::template copy<4>(cp.s + kt * cp.as_stage_stride, C::AS_OFF + (kt % C::A_SLOTS) * C::BS_BYTES + (wave & 1) * 256,
                          smem, 1);
}
template <class C, bool MX, bool B_KN, bool GK, class D>
MI355_HD void issue_b(const CopyPlan<C>& cp, int kt, int wave, uint8_t* smem) {
  // (MX with K-contiguous weights has no per-stage scale copy: its scales come in groups)
#ifdef GG_ABLATE_DMA
  if (wave < 64) return;
#endif
  const uint32_t base = C::B_OFF + (kt % C::B_SLOTS) * C::B_SLOT;
  if constexpr (!GK) {
    const int64_t boff = (int64_t)kt * cp.b_stage_stride;
#pragma unroll
    for (int j = 0; j < C::B_INSTR; ++j)
      D::template copy<16>(cp.b[j] + boff, base + (wave * C::B_INSTR + j) * 1024, smem, 1);
  } else {
#pragma unroll
    for (int j = 0; j < C::B_INSTR; ++j)
      D::template copy<16>(b_src<C, GK, MX>(cp, j, kt), base + (wave * C::B_INSTR + j) * 1024, smem, 1);
  }
  if (MX && B_KN && is_bs_wave(wave))
    D::template copy<4>(cp.bs + kt * cp.bs_stage_stride, base + C::B_BYTES + wave * 256, smem, 1);
}
// MX: A scale codes of stages 8*grp .. 8*grp+7 (16 bytes per row) into AS slot grp & 1.
template <class C, class D>
MI355_HD void issue_as(const CopyPlan<C>& cp, int grp, int wave, uint8_t* smem) {
#ifdef GG_ABLATE_DMA
  if (wave < 64) return;
#endif
  if (wave < C::AS_WAVES)
    D::template copy<16>(cp.s + grp * 16, C::AS_OFF + (grp & 1) * C::AS_SLOT + wave * 1024, smem, 1);
}

// Work of one pipelined K step of a wave that computes NM 32-row subtiles: MFMAs, LDS fragment
// reads of the next stage and copy items (issue_item), interleaved by the K loop.
template <class C, bool MX, int NM, bool GK = false> struct StepShape {
  static constexpr int MFMAS = MX ? NM * C::NI : 2 * NM * C::NI;
  static constexpr int READS = MX ? C::NI + NM : 2 * (C::NI + NM);  // fragment elements of a stage
  // B copies, B scales, A copies (grouped-K MX: and the A column scales)
  static constexpr int ITEMS = C::B_INSTR + 1 + C::A_INSTR + ((MX && GK) ? 1 : 0);
};

// Copy item it of iteration i (same order as issue_iteration: B copies, B scales, A copies, and in
// grouped-K MX mode the A column scales).
template <class C, bool MX, bool B_KN, bool LA, bool GK, class D>
MI355_HD void issue_item(const CopyPlan<C>& cp, int i, int nk, int wave, uint8_t* smem, int it) {
#ifdef GG_ABLATE_DMA
  if (wave < 64) return;
#endif
  constexpr int DA = C::A_SLOTS, DB = C::B_SLOTS;
  if (it < C::B_INSTR) {
    const int kt = i + DB;
    D::template copy<16>(b_src<C, GK, MX>(cp, it, kt),
                         C::B_OFF + (kt % C::B_SLOTS) * C::B_SLOT + (wave * C::B_INSTR + it) * 1024, smem, kt < nk);
  } else if (it == C::B_INSTR) {
    const int kt = i + DB;
    if constexpr (MX && B_KN)
      D::template copy<4>(cp.bs + kt * cp.bs_stage_stride,
                          C::B_OFF + (kt % C::B_SLOTS) * C::B_SLOT + C::B_BYTES + (wave & 1) * 256, smem,
                          is_bs_wave(wave) && kt < nk);
  } else if constexpr (LA) {
    const int j = it - C::B_INSTR - 1;
    const int kt = i + DA;
    if (!(MX && GK) || j < C::A_INSTR) {
      D::template copy<16>(a_src<C, GK, MX>(cp, j, kt),
                           (kt % C::A_SLOTS) * C::A_BYTES + (wave * C::A_INSTR + j) * 1024, smem, kt < nk);
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
#ifdef GG_ABLATE_DMA
  if (wave < 64) return;
#endif
  if constexpr (MX && !GK) {
    const int grp = i / C::AS_GROUP + 1;
    const bool due = (i & (C::AS_GROUP - 1)) == 0 && i + C::AS_GROUP < nk;
    if constexpr (LA)
      D::template copy<16>(cp.s + grp * 16, C::AS_OFF + (grp & 1) * C::AS_SLOT + (wave & 3) * 1024, smem,
                           due && wave < C::AS_WAVES);
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
MI355_HD bool wave_copies_a(int wave, int rows_valid) { return wave * (C::A_INSTR * 16) < rows_valid; }
