// Direct-weight configuration of the forward grouped GEMM (measurement variant "dv").
//
// For weights stored K-contiguous (bf16 EOI [G, N, K]; MXFP8 row_data [G, N, K] with row scales
// [G * N, ld]) every wave loads its weight fragments straight from global memory into registers,
// already in the MFMA operand layout, through a ring of D stages; only the activation tile goes
// through the LDS, in a ring of D slots. The LDS then holds no weight bytes, so the whole 160 KB
// serves the activation ring, and the weight bytes in flight per CU are bounded by the register
// ring (4 waves x (D - 1) stages x 4 KB) rather than by LDS slots.
//
// Workgroup: 4 waves in a 1 (M) x 4 (N) grid, tile BM = 256 x BN = 256, wave tile 256 x 64 (8 x 2
// MFMA subtiles of 32 x 32): each wave owns 64 weight columns, so no weight byte is loaded twice in
// a workgroup, and each wave reads the whole activation stage from the LDS (the same LDS read
// traffic per stage as a 2 x 2 grid of 128 x 128 wave tiles). A stage is 64 bytes of K per row.
//
// Step j of a work item issues, in this order: (MX, j % 8 == 0) the scale group of stages
// j + 8 .. j + 15; the weight fragments of stage j + D - 1 (4 loads into the register ring slot that
// stage j - 1 used); the activation copies of stage j + D - 1 (4 direct-to-LDS loads into the LDS slot
// that stage j - 1 used). Loads past the last stage are not issued: with the stage count a multiple
// of D, every turn of the ring but the last issues at every step, the last turn only at its first. Before step k a wave waits until
// its weight fragments of stage k and its activation copies of stage k + 1 have landed; the
// workgroup barrier that follows makes stage k + 1 complete in the LDS for every wave, whose
// fragments the wave then reads while running the MFMAs of stage k (one register set: the
// fragments of subtile row mi are re-read right after their last MFMA).
//
// Everything here is __host__ __device__ with the instructions behind policy types, like
// gemm_plan.h: the kernel (gemm_direct.hip) uses DevDma / DevLoad / DevOps, the host-side checker
// under tests/native records the issue order, checks the waits and emulates the data path.
#pragma once
#include "gemm_plan.h"

struct GGDirect {
  static constexpr int BM = 256;
  static constexpr int BN = 256;
  static constexpr int KB = 64;                         // bytes of K per stage per row
  static constexpr int WAVES = 4;
  static constexpr int THREADS = 64 * WAVES;
  static constexpr int WG_PER_CU = 1;
  static constexpr int WGM = 1, WGN = 4;                // wave grid
  static constexpr int WM = BM / WGM, WN = BN / WGN;    // wave tile 256 x 64
  static constexpr int MI = WM / 32, NI = WN / 32;      // 8 x 2 MFMA subtiles
  static constexpr int D = 8;                           // ring depth (stages)
  static constexpr int A_SLOTS = D;
  static constexpr int A_BYTES = BM * KB;               // 16 KB
  static constexpr int A_INSTR = BM * (KB / 16) / 64 / WAVES;
  static constexpr int B_INSTR = 1;                     // (weight copies of the LDS plan: unused)
  static constexpr bool SPLIT = false, OFFS = false;    // (the LDS plan's copy roles and addressing: unused)
  static constexpr int A_PER = A_INSTR, B_PER = B_INSTR;
  static constexpr int B_LOADS = 2 * NI;                // 16-byte weight loads per stage and lane
  static constexpr int AS_GROUP = 8;                    // MX: scale codes per fetch = 8 stages
  static constexpr int AS_SLOT = BM * 16;
  static constexpr int AS_WAVES = BM / 64;
  static constexpr int AS_OFF = A_SLOTS * A_BYTES;
  static constexpr int PREFIX_MAX = 1024;
  static constexpr int PREFIX_OFF = AS_OFF + 2 * AS_SLOT;
  static constexpr int TOTAL = PREFIX_OFF + (PREFIX_MAX + 1) * 4;
  static constexpr int EPI_RS_BF16 = BN * 2 + 16;
  static constexpr int EPI_RS_ACT = (BN / 2) * 4 + 16;
  static constexpr int LOADS_STAGE = A_INSTR + B_LOADS; // vector-memory loads per stage and wave
  static constexpr int LOADS_SCALE = 1 + NI;            // MX: per scale group, A-scale copy + weight scales
  static_assert(D == AS_GROUP, "ring positions and scale groups share the unrolled step index");
  static_assert(AS_WAVES == WAVES, "every wave copies 64 activation-scale rows");
  static_assert(BM * EPI_RS_BF16 <= PREFIX_OFF && BM * EPI_RS_ACT <= PREFIX_OFF, "epilogue staging fits");
  static_assert(TOTAL <= 160 * 1024, "LDS budget");
  static_assert(A_INSTR == 4 && B_LOADS == 4, "one copy item per subtile row: 4 weight loads, 4 activation copies");
};

// The GEMMs the direct configuration runs (otherwise the caller keeps the default configuration):
// K-contiguous weights, a whole number of D-stage ring turns, the bf16 store and SwiGLU epilogues,
// 32-bit byte offsets within A, one group's weights and the scale rows, and 16-byte scale rows (MX).
MI355_HD bool direct_supported(const GGParams& p, bool mx, bool b_kn, int epi) {
  using C = GGDirect;
  if (b_kn || p.K <= 0 || (int64_t)p.K * (mx ? 1 : 2) % (C::KB * C::D) != 0) return false;
  if (mx ? (epi != EPI_STORE_BF16 && epi != EPI_SWIGLU_MX) : (epi != EPI_STORE_BF16 && epi != EPI_SWIGLU_BF16))
    return false;
  const int64_t lim = (int64_t)1 << 32;
  if (p.a_bytes <= 0 || p.a_bytes >= lim || (int64_t)p.Ntot * p.b_row_bytes >= lim) return false;
  if (mx && (p.a_scale_ld % 16 != 0 || p.b_scale_ld % 16 != 0 || p.a_bytes / p.lda_bytes * p.a_scale_ld >= lim ||
             (int64_t)p.Ntot * p.b_scale_ld >= lim))
    return false;
  return true;
}

// This lane's copy plan for one work item: uniform bases and per-lane 32-bit byte offsets (the
// loads use the scalar-base + vector-offset address form, which keeps one register per stream).
struct DirectPlan {
  const uint8_t* a_base;                 // A (uniform)
  const uint8_t* as_base;                // MX: A scales
  const uint8_t* b_base;                 // this group's weights
  const uint8_t* bs_base;                // MX: this group's weight row scales
  uint32_t a[GGDirect::A_INSTR];         // activation copy j: this lane's 16 bytes of stage 0
  uint32_t as;                           // MX: this lane's activation-scale row (rows wave * 64 + lane)
  uint32_t b[GGDirect::NI];              // weight subtile q: this lane's column at K byte 16 * (lane / 32)
  uint32_t bs[GGDirect::NI];             // MX: the column's row scales (16 codes = 8 stages per group)
};

// Subtile q of wave w covers tile columns w * WN + 32 q .. + 31; activation copy j of wave w covers
// the 16-byte chunks (w * A_INSTR + j) * 64 + lane of the stage (row chunk / 4, XOR-swizzled as the
// LDS fragment reads expect, rows past the tile's valid rows repeat its last row).
MI355_HD DirectPlan direct_plan(const GGParams& p, int g, int nt, int64_t tile_row0, int rows_valid, bool swiglu,
                                bool mx, int wave, int lane) {
  using C = GGDirect;
  DirectPlan d;
  d.a_base = p.A;
  d.as_base = p.a_scale;
  d.b_base = p.B + (int64_t)g * p.b_group_stride;
  d.bs_base = mx ? p.b_scale + (int64_t)g * p.Ntot * p.b_scale_ld : nullptr;
#pragma unroll
  for (int j = 0; j < C::A_INSTR; ++j) {
    const int L16 = (wave * C::A_INSTR + j) * 64 + lane;
    const int r = L16 >> 2, cs = L16 & 3;
    const int c = cs ^ ((r >> 2) & 3);
    const int rr = r < rows_valid ? r : rows_valid - 1;
    const int64_t routed = tile_row0 + rr;
    const int64_t src = p.a_row_index ? (int64_t)(p.a_row_index[routed] / p.a_row_div) : routed;
    d.a[j] = (uint32_t)(src * p.lda_bytes + c * 16);
  }
  d.as = 0;
  if (mx) {
    const int r = wave * 64 + lane;
    const int rr = r < rows_valid ? r : rows_valid - 1;
    const int64_t routed = tile_row0 + rr;
    const int64_t src = p.a_row_index ? (int64_t)(p.a_row_index[routed] / p.a_row_div) : routed;
    d.as = (uint32_t)(src * p.a_scale_ld);
  }
#pragma unroll
  for (int q = 0; q < C::NI; ++q) {
    int wc = tile_col_to_weight_col<C>(wave * C::WN + q * 32 + (lane & 31), nt, p.N, swiglu, p.gate_up_interleaved);
    if (wc >= p.Ntot) wc = p.Ntot - 1;
    d.b[q] = (uint32_t)((int64_t)wc * p.b_row_bytes + 16 * (lane >> 5));
    d.bs[q] = mx ? (uint32_t)((int64_t)wc * p.b_scale_ld) : 0u;
  }
  return d;
}

// Copy item `it` of step j (stage j + D - 1): it < B_LOADS loads 16 weight bytes of subtile it / 2,
// K half it % 2 (bf16: K step 0 / 1 of the stage; MX: operand bytes 0-15 / 16-31) into bslot[it];
// the others copy activation chunks (it - B_LOADS) of the stage into its LDS slot. M is the memory
// policy: M::lds(base, offset, smem, lds_offset, enable) copies 16 bytes per lane to
// smem + lds_offset + 16 * lane, M::load(dst, base, offset, enable) loads 16 bytes into dst.
template <class M>
MI355_HD void direct_issue(const DirectPlan& d, int j, int nk, int wave, uint8_t* smem, v4i (&bslot)[GGDirect::B_LOADS],
                           int it) {
  using C = GGDirect;
  const int kt = j + C::D - 1;
  const int en = kt < nk;
  if (it < C::B_LOADS) {
    M::load(bslot[it], d.b_base + (int64_t)kt * C::KB + (it & 1) * 32, d.b[it >> 1], en);
  } else {
    const int jj = it - C::B_LOADS;
    M::lds(d.a_base + (int64_t)kt * C::KB, d.a[jj], smem,
           (uint32_t)((kt % C::A_SLOTS) * C::A_BYTES + (wave * C::A_INSTR + jj) * 1024), en);
  }
}

// MX: scale group grp (stages 8 grp .. 8 grp + 7): the activation rows' 16 codes into AS slot grp & 1
// and this lane's two weight columns' 16 codes into bs.
template <class M>
MI355_HD void direct_issue_scales(const DirectPlan& d, int grp, int en, int wave, uint8_t* smem, v4i (&bs)[GGDirect::NI]) {
  using C = GGDirect;
  M::lds(d.as_base + grp * 16, d.as, smem, (uint32_t)(C::AS_OFF + (grp & 1) * C::AS_SLOT + wave * 1024), en);
#pragma unroll
  for (int q = 0; q < C::NI; ++q) M::load(bs[q], d.bs_base + grp * 16, d.bs[q], en);
}

// Loads issued by steps a .. b (prologue steps are negative; a step issues its stage's loads only
// below nk, and MX scale groups at steps 0, 8, .. while a later group exists).
template <bool MX>
MI355_HD int direct_loads(int a, int b, int nk) {
  using C = GGDirect;
  const int hb = b < nk - C::D ? b : nk - C::D;
  int n = (hb >= a ? hb - a + 1 : 0) * C::LOADS_STAGE;
  if (MX) {
    const int lo = a > 0 ? a : 0;
    const int hs = b < nk - 9 ? b : nk - 9;
    if (hs >= lo) {
      const int cnt = hs / 8 - (lo + 7) / 8 + 1;
      n += (cnt > 0 ? cnt : 0) * C::LOADS_SCALE;
    }
  }
  return n;
}
// Loads allowed in flight at the wait before step k (steps up to k - 1 issued), so that the weight
// fragments of stage k and the activation copies of stage k + 1 have landed. The activation copies
// of stage s are the last loads of step s - D + 1, after its weight loads; in the last step only the
// weight fragments of stage k are needed, followed in their step by the A_INSTR copies of stage k.
// k = -1 gives the wait before the prologue's read of stage 0 (after prologue step -1).
template <bool MX>
MI355_HD int direct_wait(int k, int nk) {
  using C = GGDirect;
  if (k < 0) return direct_loads<MX>(2 - C::D, -1, nk);
  if (k + 1 < nk) return direct_loads<MX>(k + 3 - C::D, k - 1, nk);
  return C::A_INSTR + direct_loads<MX>(k - C::D + 2, k - 1, nk);
}

// direct_wait as compile-time counts by ring position (the kernel's waits; the checker verifies
// them against direct_wait for every step). With nk a multiple of D: in every turn of the ring but
// the last, five whole steps, plus the scale group of step 8 i at steps 8 i + 1 .. 8 i + 5; in the
// last turn only the steps whose stage exists (none issue scale groups), and the copies of stage k
// at its last step; before the prologue's read of stage 0, the D - 2 prologue steps after the first.
template <bool MX, int P, bool LAST>
constexpr int direct_wait_fixed() {
  using C = GGDirect;
  if constexpr (!LAST) return (C::D - 3) * C::LOADS_STAGE + ((MX && P >= 1 && P <= C::D - 3) ? C::LOADS_SCALE : 0);
  if constexpr (P == C::D - 1) return C::A_INSTR;
  constexpr int steps = (C::D - 2 - P) < (C::D - 3) ? (C::D - 2 - P) : (C::D - 3);
  return steps * C::LOADS_STAGE;
}
constexpr int direct_wait_first() { return (GGDirect::D - 2) * GGDirect::LOADS_STAGE; }

// Activation fragments of one stage (single register set, re-read subtile row by subtile row).
template <bool MX> struct DirectFrags;
template <> struct DirectFrags<false> { v8bf a[GGDirect::MI][2]; };  // [mi][ks]
template <> struct DirectFrags<true> {
  v4i al[GGDirect::MI], ah[GGDirect::MI];
  int sa[GGDirect::MI];
};

// Subtile row mi of the activation stage at As (A-scale codes of the stage at ASs).
template <bool MX, class O = DevOps>
MI355_HD void direct_read_a(DirectFrags<MX>& f, int mi, const uint8_t* As, const uint8_t* ASs, int lane) {
  const int r = mi * 32 + (lane & 31);
  if constexpr (!MX) {
    f.a[mi][0] = read_a_bf16<O>(As, r, 0, lane);
    f.a[mi][1] = read_a_bf16<O>(As, r, 1, lane);
  } else {
    const int c0 = lane >> 5;
    f.al[mi] = *(const v4i*)(As + a_chunk_off(r, c0));
    f.ah[mi] = *(const v4i*)(As + a_chunk_off(r, c0 + 2));
    f.sa[mi] = ASs[r * 16 + (lane >> 5)];
  }
}

// e8m0 code of this lane's weight column for K block lane / 32 of the stage at position pos of its
// scale group (codes 2 pos, 2 pos + 1 of the 16 loaded).
MI355_HD int direct_b_scale(const v4i& bs, int pos, int lane) {
  return (bs[pos >> 1] >> (16 * (pos & 1) + 8 * (lane >> 5))) & 0xff;
}

// MFMAs per subtile row and stage: bf16 2 K steps x NI; MX NI.
template <bool MX>
constexpr int direct_mfmas() { return MX ? GGDirect::NI : 2 * GGDirect::NI; }

// MFMA t of subtile row mi with the weight fragments in bslot (bf16: t = ks * NI + q; MX: t = q).
template <bool MX, class O = DevOps>
MI355_HD void direct_mfma(const DirectFrags<MX>& f, int mi, int t, const v4i (&bslot)[GGDirect::B_LOADS],
                          const v4i (&bs)[GGDirect::NI], int pos, int lane, v16f (&acc)[GGDirect::MI][GGDirect::NI]) {
  using C = GGDirect;
  if constexpr (!MX) {
    const int ks = t / C::NI, q = t % C::NI;
    O::mfma_bf16(f.a[mi][ks], __builtin_bit_cast(v8bf, bslot[q * 2 + ks]), acc[mi][q]);
  } else {
    const int q = t;
    const v8i a = __builtin_shufflevector(f.al[mi], f.ah[mi], 0, 1, 2, 3, 4, 5, 6, 7);
    const v8i b = __builtin_shufflevector(bslot[q * 2], bslot[q * 2 + 1], 0, 1, 2, 3, 4, 5, 6, 7);
    O::mfma_f8(a, b, acc[mi][q], f.sa[mi], direct_b_scale(bs[q], pos, lane));
  }
}
