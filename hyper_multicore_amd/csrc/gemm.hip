// Persistent grouped GEMM for gfx950 (MI355X): bf16 and MXFP8 (e4m3 + e8m0 per 32 along K).
//
// Work list: the row segments of the groups (experts) are cut into BM-row tiles; every
// (group, m-tile, n-tile) is one work item. tile_prefix[g] (computed on the device from the
// group row counts) gives the first m-tile of group g, so the work list needs no host round
// trip. The grid is one workgroup per CU; workgroup i runs on XCD i % 8 and walks the work list
// in rounds so that each XCD takes a contiguous run of items per round (m fastest): items that
// share a weight slice run at the same time on one XCD and share its L2.
//
// Workgroup: 512 threads = 8 wavefronts (two per SIMD, which both the HBM stream and the LDS
// read rate need) in a 4 (M) x 2 (N) grid; tile BM=256 x BN=256; each wavefront computes
// 64 x 128 with 2 x 4 32x32 MFMAs (bf16: v_mfma_f32_32x32x16_bf16; MXFP8:
// v_mfma_scale_f32_32x32x64_f8f6f4 with per-lane e8m0 scales: lane r + 32b supplies the scale
// of 32-block b of row / column r, and its operand bytes 0-15 / 16-31 hold K = 16b + i /
// 32 + 16b + i of the 64-K step). A stage holds 64 bytes of K per row (32 bf16 or 64 e4m3);
// global -> LDS copies use the direct-to-LDS loads into a 4-deep ring (three stages in flight).
//
// LDS layouts (16-byte chunk granularity, XOR swizzled against bank conflicts):
//   K-contiguous operand rows (A always; B in EOI layout): row r at r*64, chunk c stored at
//     c ^ ((r >> 2) & 3); read with ds_read_b128.
//   N-contiguous B (EIO bf16 / MX col_data): row k holds 256 columns; bf16 chunk c stored at
//     c ^ ((k & 7) << 1) (512-byte rows), e4m3 chunk c at c ^ (k & 15) (256-byte rows); read
//     with the transposing ds_read_b64_tr_b16 / ds_read_b64_tr_b8.
//   MX scales per stage: A one dword per row (the row's two e8m0 codes, 2-byte DMA zero-extends),
//     B the two codes of every tile column (col_scale's [.., N, 2] pairs).
//
// Epilogues: bf16 store, fp32 store (router logits, optional row scatter), SwiGLU -> bf16 and
// SwiGLU -> MXFP8 requant. For SwiGLU the B tile columns are gate/up interleaved in 64-column
// groups so that each lane holds the gate and up value of the same output element.
#include <type_traits>
#include "common.h"
#include "scan.h"
#include "../../include/mi355moe.h"
#include "gemm.h"

#define GG_BM 256
#define GG_BN 256
#define GG_KB 64  // bytes of K per stage per row
#define GG_THREADS 512
#define GG_WAVES 8

struct GGLds {
  // Decoupled rings: activations A (re-read from L2 by the tiles of one expert) and weights B
  // (streamed once from HBM, so it gets the deeper ring: five stages = 80 KB in flight per CU).
  static constexpr int A_BYTES = GG_BM * GG_KB;        // 16 KB
  static constexpr int B_BYTES = GG_BN * GG_KB;        // 16 KB
  static constexpr int BS_BYTES = GG_BN * 2;           // 512 B (MX: two codes per column)
  static constexpr int B_SLOT = B_BYTES + BS_BYTES;
  static constexpr int A_SLOTS = 3;                    // A(k+2) issued at iteration k
  static constexpr int B_SLOTS = 6;                    // B(k+5) issued at iteration k
  static constexpr int AS_GROUP = 8;                   // MX: A scale codes fetched per 8 stages
  static constexpr int AS_SLOT = GG_BM * 16;           // 4 KB: 16 codes per row
  static constexpr int B_OFF = A_SLOTS * A_BYTES;
  static constexpr int AS_OFF = B_OFF + B_SLOTS * B_SLOT;
  static constexpr int PREFIX_MAX = 1024;              // groups whose tile prefix is kept in LDS
  static constexpr int PREFIX_OFF = AS_OFF + 2 * AS_SLOT;
  static constexpr int TOTAL = PREFIX_OFF + (PREFIX_MAX + 1) * 4;
  static_assert(GG_BM * (GG_BN * 2 + 16) <= AS_OFF, "bf16 epilogue staging must fit the rings");
  static_assert(GG_BM * (128 * 4 + 16) <= AS_OFF, "SwiGLU epilogue staging must fit the rings");
  static_assert(TOTAL <= 160 * 1024, "LDS budget");
};

template <int SZ>
MI355_DEV void lds_dma(const void* g, uint32_t lds_off_uniform, uint8_t* smem) {
  auto* dst = (__attribute__((address_space(3))) void*)(smem + lds_off_uniform);
  if constexpr (SZ == 16) __builtin_amdgcn_global_load_lds(g, dst, 16, 0, 0);
  else if constexpr (SZ == 4) __builtin_amdgcn_global_load_lds(g, dst, 4, 0, 0);
  else if constexpr (SZ == 2) __builtin_amdgcn_global_load_lds(g, dst, 2, 0, 0);
  else static_assert(SZ == 16, "unsupported DMA size");
}
// Workgroup barrier without the release fence of __syncthreads (which would wait for every
// outstanding global load, including the prefetched stages): LDS reads of this wave are drained,
// the direct-to-LDS loads are ordered by the explicit vmcnt waits.
MI355_DEV void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
}
// Wait until at most N vector-memory loads of this wave are outstanding (loads retire in order).
template <int N>
MI355_DEV void wait_vm_le() {
  if constexpr (N == 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  else if constexpr (N == 2) asm volatile("s_waitcnt vmcnt(2)" ::: "memory");
  else if constexpr (N == 4) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
  else if constexpr (N == 6) asm volatile("s_waitcnt vmcnt(6)" ::: "memory");
  else if constexpr (N == 8) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
  else static_assert(N == 0, "unsupported vmcnt");
}

// Tile column j (0..255) -> weight column. SwiGLU: per 128-column half h, 64 gate then 64 up.
MI355_DEV int tile_col_to_weight_col(int j, int nt, int I, bool swiglu) {
  if (!swiglu) return nt * GG_BN + j;
  int h = j >> 7, jj = j & 127;
  int base = nt * 128 + h * 64;
  return jj < 64 ? base + jj : I + base + (jj - 64);
}

MI355_DEV int a_chunk_off(int r, int c) { return r * GG_KB + ((c ^ ((r >> 2) & 3)) << 4); }

// ---- fragment loads (one K step: 16 bf16 or 64 e4m3) ------------------------------------------
MI355_DEV v8bf read_a_bf16(const uint8_t* As, int r, int ks, int lane) {
  return *(const v8bf*)(As + a_chunk_off(r, ks * 2 + (lane >> 5)));
}
template <bool B_KN>
MI355_DEV v8bf read_b_bf16(const uint8_t* Bs, int wn, int ni, int ks, int lane) {
  if (!B_KN) {
    int n = wn * 128 + ni * 32 + (lane & 31);
    return *(const v8bf*)(Bs + a_chunk_off(n, ks * 2 + (lane >> 5)));
  }
  int g16 = lane >> 4, m = lane & 15;
  int nb = wn * 128 + ni * 32 + (g16 & 1) * 16 + 4 * (m & 3);
  int k0 = ks * 16 + (g16 >> 1) * 8 + (m >> 2);
  int k1 = k0 + 4;
  int off0 = k0 * 512 + (((nb >> 3) ^ ((k0 & 7) << 1)) << 4) + (nb & 7) * 2;
  int off1 = k1 * 512 + (((nb >> 3) ^ ((k1 & 7) << 1)) << 4) + (nb & 7) * 2;
  v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(LDS_PTR(v4s, Bs + off0));
  v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(LDS_PTR(v4s, Bs + off1));
  typedef __attribute__((ext_vector_type(8))) short v8s;
  v8s both = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  return __builtin_bit_cast(v8bf, both);
}
MI355_DEV v8i read_a_mx(const uint8_t* As, int r, int lane) {
  int c0 = lane >> 5;
  v4i lo = *(const v4i*)(As + a_chunk_off(r, c0));
  v4i hi = *(const v4i*)(As + a_chunk_off(r, c0 + 2));
  return (v8i){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}
MI355_DEV v8i read_b_mx(const uint8_t* Bs, int wn, int ni, int lane) {
  int g16 = lane >> 4, m = lane & 15;
  int nb = wn * 128 + ni * 32 + (g16 & 1) * 16;
  int parts[8];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    int k = (q >> 1) * 32 + (g16 >> 1) * 16 + (q & 1) * 8 + (m >> 1);
    int off = k * 256 + (((nb >> 4) ^ (k & 15)) << 4) + 8 * (m & 1);
    v2i v = __builtin_amdgcn_ds_read_tr8_b64_v2i32(LDS_PTR(v2i, Bs + off));
    parts[2 * q] = v[0];
    parts[2 * q + 1] = v[1];
  }
  return (v8i){parts[0], parts[1], parts[2], parts[3], parts[4], parts[5], parts[6], parts[7]};
}

// ---- copy plan -------------------------------------------------------------------------------
// Per stage the workgroup copies A 16 KB and B 16 KB: each wave issues 2 + 2 16-byte DMA
// instructions; MX adds the B scale codes (waves 4-5, one 4-byte DMA for 128 columns each) and,
// every 8 stages, 16 A scale codes per row (waves 0-3, one 16-byte DMA for 64 rows each).
struct CopyPlan {
  const uint8_t* a[2];
  const uint8_t* b[2];
  const uint8_t* s;        // MX: A scale row (waves 0-3) or B scale column pair (waves 4-5)
  int64_t b_stage_stride;  // bytes to advance B per stage
  int64_t bs_stage_stride; // bytes to advance the B scales per stage
};

template <bool MX>
MI355_DEV void issue_a(const CopyPlan& cp, int kt, int wave, uint8_t* smem) {
#ifdef GG_ABLATE_DMA
  if (wave < 64) return;
#endif
  const uint32_t base = (kt % GGLds::A_SLOTS) * GGLds::A_BYTES;
  const int64_t koff = (int64_t)kt * GG_KB;
#pragma unroll
  for (int j = 0; j < 2; ++j) lds_dma<16>(cp.a[j] + koff, base + (wave * 2 + j) * 1024, smem);
}
template <bool MX>
MI355_DEV void issue_b(const CopyPlan& cp, int kt, int wave, uint8_t* smem) {
#ifdef GG_ABLATE_DMA
  if (wave < 64) return;
#endif
  const uint32_t base = GGLds::B_OFF + (kt % GGLds::B_SLOTS) * GGLds::B_SLOT;
  const int64_t boff = (int64_t)kt * cp.b_stage_stride;
#pragma unroll
  for (int j = 0; j < 2; ++j) lds_dma<16>(cp.b[j] + boff, base + (wave * 2 + j) * 1024, smem);
  if (MX && (wave == 4 || wave == 5))
    lds_dma<4>(cp.s + kt * cp.bs_stage_stride, base + GGLds::B_BYTES + (wave - 4) * 256, smem);
}
// MX: A scale codes of stages 8*grp .. 8*grp+7 (16 bytes per row) into AS slot grp & 1.
MI355_DEV void issue_as(const CopyPlan& cp, int grp, int wave, uint8_t* smem) {
#ifdef GG_ABLATE_DMA
  if (wave < 64) return;
#endif
  if (wave < 4) lds_dma<16>(cp.s + grp * 16, GGLds::AS_OFF + (grp & 1) * GGLds::AS_SLOT + wave * 1024, smem);
}

// K loop. Issue order (per wave): B0 B1 B2 AS0 A0 B3 A1 B4 | A2 B5 [AS1] | A3 B6 | ... : iteration
// k issues A(k+2), B(k+5) and, every 8 stages, the next A scale group. At the top of iteration k
// the loads younger than A(k) are B(k+3), A(k+1), B(k+4) (plus scale groups on waves 0-3), so
// waiting for at most that many keeps A(k), B(k) and the scale group of stage k complete.
// A wave whose 32 A rows (and 64 scale rows) all lie past the tile's last valid row copies no
// A at all (LA = false, decode and ragged tiles); it waits on its B groups alone: younger than
// B(k) are B(k+1) .. B(k+4).
// NM = number of valid 32-row subtiles this wave computes (0..2).
template <int N>
MI355_DEV void wait_vm_b_only(int ahead) {
  // ahead = number of later B groups issued (0..4), 2 loads each at least
  if (ahead >= 4) wait_vm_le<8>();
  else if (ahead == 3) wait_vm_le<6>();
  else if (ahead == 2) wait_vm_le<4>();
  else if (ahead == 1) wait_vm_le<2>();
  else wait_vm_le<0>();
}
template <bool MX, bool B_KN, int NM, bool LA>
MI355_DEV void k_loop(const CopyPlan& cp, int nk, int wave, int wm, int wn, int lane, uint8_t* smem,
                      v16f (&acc)[2][4]) {
  for (int j = 0; j < 3 && j < nk; ++j) issue_b<MX>(cp, j, wave, smem);
  if (LA) {
    if (MX) issue_as(cp, 0, wave, smem);
    issue_a<MX>(cp, 0, wave, smem);
  }
  if (nk > 3) issue_b<MX>(cp, 3, wave, smem);
  if (LA && nk > 1) issue_a<MX>(cp, 1, wave, smem);
  if (nk > 4) issue_b<MX>(cp, 4, wave, smem);
  for (int k = 0; k < nk; ++k) {
    if (LA) {
      if (k + 4 < nk) wait_vm_le<6>();
      else if (k + 3 < nk) wait_vm_le<4>();
      else if (k + 1 < nk) wait_vm_le<2>();
      else wait_vm_le<0>();
    } else {
      wait_vm_b_only<0>(nk - 1 - k < 4 ? nk - 1 - k : 4);
    }
    lds_barrier();
    if (LA && k + 2 < nk) issue_a<MX>(cp, k + 2, wave, smem);
    if (k + 5 < nk) issue_b<MX>(cp, k + 5, wave, smem);
    if (LA && MX && (k & (GGLds::AS_GROUP - 1)) == 0 && k + GGLds::AS_GROUP < nk)
      issue_as(cp, k / GGLds::AS_GROUP + 1, wave, smem);
#ifdef GG_ABLATE_COMPUTE
    if (wave < 64) continue;
#endif
    if constexpr (NM > 0) {
      const uint8_t* As = smem + (k % GGLds::A_SLOTS) * GGLds::A_BYTES;
      const uint8_t* Bs = smem + GGLds::B_OFF + (k % GGLds::B_SLOTS) * GGLds::B_SLOT;
      if constexpr (!MX) {
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          v8bf a[2], b[4];
#pragma unroll
          for (int ni = 0; ni < 4; ++ni) b[ni] = read_b_bf16<B_KN>(Bs, wn, ni, ks, lane);
#pragma unroll
          for (int mi = 0; mi < NM; ++mi) a[mi] = read_a_bf16(As, wm * 64 + mi * 32 + (lane & 31), ks, lane);
#pragma unroll
          for (int mi = 0; mi < NM; ++mi)
#pragma unroll
            for (int ni = 0; ni < 4; ++ni)
              acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[mi], b[ni], acc[mi][ni], 0, 0, 0);
        }
      } else {
        const uint8_t* BSs = Bs + GGLds::B_BYTES;
        const uint8_t* ASs = smem + GGLds::AS_OFF + ((k / GGLds::AS_GROUP) & 1) * GGLds::AS_SLOT +
                             (k & (GGLds::AS_GROUP - 1)) * 2;
        v8i a[2], b[4];
        int sa[2], sb[4];
#pragma unroll
        for (int ni = 0; ni < 4; ++ni) {
          b[ni] = read_b_mx(Bs, wn, ni, lane);
          sb[ni] = BSs[(wn * 128 + ni * 32 + (lane & 31)) * 2 + (lane >> 5)];
        }
#pragma unroll
        for (int mi = 0; mi < NM; ++mi) {
          int r = wm * 64 + mi * 32 + (lane & 31);
          a[mi] = read_a_mx(As, r, lane);
          sa[mi] = ASs[r * 16 + (lane >> 5)];
        }
#pragma unroll
        for (int mi = 0; mi < NM; ++mi)
#pragma unroll
          for (int ni = 0; ni < 4; ++ni)
            acc[mi][ni] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a[mi], b[ni], acc[mi][ni], 0, 0, 0, sa[mi],
                                                                           0, sb[ni]);
      }
    }
  }
}

template <bool MX, bool B_KN, int EPI>
__global__ __launch_bounds__(GG_THREADS, 1) void grouped_gemm_kernel(GGParams p) {
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
  int32_t* s_prefix = (int32_t*)(smem + GGLds::PREFIX_OFF);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  constexpr bool SWIGLU = (EPI == EPI_SWIGLU_BF16 || EPI == EPI_SWIGLU_MX);
  constexpr int ESIZE = MX ? 1 : 2;

  const bool prefix_in_lds = p.G <= GGLds::PREFIX_MAX;
  const int32_t* prefix = prefix_in_lds ? s_prefix : p.tile_prefix;
  if (prefix_in_lds)
    for (int g = tid; g <= p.G; g += GG_THREADS) s_prefix[g] = p.tile_prefix[g];
  __syncthreads();
  const int splits = (EPI == EPI_STORE_F32 && p.k_splits > 1) ? p.k_splits : 1;
  const int total = prefix[p.G] * p.n_tiles * splits;
  const int nk = p.K / splits * ESIZE / GG_KB;  // stages per work item
  const int xcd = blockIdx.x & 7;
  const int per_xcd = gridDim.x >> 3;
  const int slot = blockIdx.x >> 3;

  for (int round = 0;; ++round) {
    const int L = round * (int)gridDim.x + xcd * per_xcd + slot;
    if (L >= total) break;
    // ---- decode work item -------------------------------------------------------------
    const int split = splits > 1 ? L % splits : 0;
    const int LT = splits > 1 ? L / splits : L;
    int lo = 0, hi = p.G - 1;
    while (lo < hi) {  // largest g with prefix[g]*n_tiles <= LT
      int mid = (lo + hi + 1) >> 1;
      if (prefix[mid] * p.n_tiles <= LT) lo = mid; else hi = mid - 1;
    }
    const int g = lo;
    const int mtiles = prefix[g + 1] - prefix[g];
    const int local = LT - prefix[g] * p.n_tiles;
    const int nt = local / mtiles;
    const int mt = local - nt * mtiles;
    const int64_t row_begin = (g == 0 ? 0 : p.group_list[g - 1]);
    const int64_t row_end = p.group_list[g];
    const int64_t tile_row0 = row_begin + (int64_t)mt * GG_BM;
    const int rows_valid = (int)((row_end - tile_row0) < GG_BM ? (row_end - tile_row0) : GG_BM);

    // ---- per-thread copy sources ------------------------------------------------------
    CopyPlan cp;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      int L16 = wave * 128 + j * 64 + lane;
      int r = L16 >> 2, cs = L16 & 3;
      int c = cs ^ ((r >> 2) & 3);
      int rr = r < rows_valid ? r : rows_valid - 1;
      int64_t routed = tile_row0 + rr;
      int64_t src = p.a_row_index ? (int64_t)(p.a_row_index[routed] / p.a_row_div) : routed;
      cp.a[j] = p.A + src * p.lda_bytes + c * 16;
    }
    const uint8_t* bgrp = p.B + (int64_t)g * p.b_group_stride;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      int L16 = wave * 128 + j * 64 + lane;
      if (!B_KN) {
        int r = L16 >> 2, cs = L16 & 3;
        int c = cs ^ ((r >> 2) & 3);
        int wc = tile_col_to_weight_col(r, nt, p.N, SWIGLU);
        if (wc >= p.Ntot) wc = p.Ntot - 1;
        cp.b[j] = bgrp + (int64_t)wc * p.b_row_bytes + c * 16;
      } else if (MX) {
        int k = L16 >> 4, cs = L16 & 15;
        int c = cs ^ (k & 15);
        int wc = tile_col_to_weight_col(c * 16, nt, p.N, SWIGLU);
        if (wc >= p.Ntot) wc = p.Ntot - 16;
        cp.b[j] = bgrp + (int64_t)k * p.b_row_bytes + wc;
      } else {
        int k = L16 >> 5, cs = L16 & 31;
        int c = cs ^ ((k & 7) << 1);
        int wc = tile_col_to_weight_col(c * 8, nt, p.N, SWIGLU);
        if (wc >= p.Ntot) wc = p.Ntot - 8;
        cp.b[j] = bgrp + (int64_t)k * p.b_row_bytes + (int64_t)wc * 2;
      }
    }
    cp.b_stage_stride = B_KN ? (int64_t)(GG_KB / ESIZE) * p.b_row_bytes : GG_KB;
    if (splits > 1) {
      const int64_t k0_stages = (int64_t)split * nk;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        cp.a[j] += k0_stages * GG_KB;
        cp.b[j] += k0_stages * cp.b_stage_stride;
      }
    }
    cp.s = nullptr;
    cp.bs_stage_stride = 0;
    if (MX) {
      if (wave < 4) {
        // A scales: row wave*64 + lane (16 codes = 8 stages per fetch)
        int r = wave * 64 + lane;
        int rr = r < rows_valid ? r : rows_valid - 1;
        int64_t routed = tile_row0 + rr;
        int64_t src = p.a_row_index ? (int64_t)(p.a_row_index[routed] / p.a_row_div) : routed;
        cp.s = p.a_scale + src * p.a_scale_ld;
      } else {
        // B scales: tile columns ((wave-4)*64 + lane)*2 .. +1, one col_scale group per stage
        int j = ((wave & 1) * 64 + lane) * 2;
        int wc = tile_col_to_weight_col(j, nt, p.N, SWIGLU);
        if (wc >= p.Ntot) wc = p.Ntot - 2;
        cp.s = p.b_scale + (int64_t)g * p.b_scale_group_stride + (int64_t)wc * 2;
        cp.bs_stage_stride = (int64_t)p.Ntot * 2;
      }
    }

    v16f acc[2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    __syncthreads();  // the previous item's last stage / epilogue reads are done before refilling
    const int rows_w = rows_valid - wm * 64;
    const int nm = rows_w >= 33 ? 2 : (rows_w >= 1 ? 1 : 0);
    // this wave copies A rows wave*32 .. +31 (and, MX waves 0-3, scale rows wave*64 .. +63)
    const bool la = wave * 32 < rows_valid;
    if (la) {
      if (nm == 2) k_loop<MX, B_KN, 2, true>(cp, nk, wave, wm, wn, lane, smem, acc);
      else if (nm == 1) k_loop<MX, B_KN, 1, true>(cp, nk, wave, wm, wn, lane, smem, acc);
      else k_loop<MX, B_KN, 0, true>(cp, nk, wave, wm, wn, lane, smem, acc);
    } else {
      if (nm == 2) k_loop<MX, B_KN, 2, false>(cp, nk, wave, wm, wn, lane, smem, acc);
      else if (nm == 1) k_loop<MX, B_KN, 1, false>(cp, nk, wave, wm, wn, lane, smem, acc);
      else k_loop<MX, B_KN, 0, false>(cp, nk, wave, wm, wn, lane, smem, acc);
    }
    __syncthreads();  // all waves are done reading the ring before the epilogue reuses LDS

    // ---- epilogue -----------------------------------------------------------------------
    // acc[mi][ni][r] holds row wm*64 + mi*32 + 8*(r/4) + 4*(lane/32) + r%4,
    // column wn*128 + ni*32 + lane%32 of the tile.
    if (EPI == EPI_STORE_F32) {
      float* C = (float*)p.C;
#pragma unroll
      for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < 4; ++ni)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            int row = wm * 64 + mi * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            int col = nt * GG_BN + wn * 128 + ni * 32 + (lane & 31);
            if (row < rows_valid && col < p.N) {
              int64_t routed = tile_row0 + row;
              int64_t orow = p.c_row_index ? (int64_t)p.c_row_index[routed] : routed;
              C[split * p.c_split_stride + orow * p.ldc + col] = acc[mi][ni][r];
            }
          }
    } else if (EPI == EPI_STORE_BF16) {
      constexpr int RS = GG_BN * 2 + 16;  // staged row stride (bytes)
#pragma unroll
      for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < 4; ++ni)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            int row = wm * 64 + mi * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            int col = wn * 128 + ni * 32 + (lane & 31);
            *(uint16_t*)(smem + row * RS + col * 2) = f32_to_bf16(acc[mi][ni][r]);
          }
      __syncthreads();
      uint16_t* C = (uint16_t*)p.C;
      for (int id = tid; id < GG_BM * (GG_BN / 8); id += GG_THREADS) {
        int row = id >> 5, ch = id & 31;
        int col = nt * GG_BN + ch * 8;
        if (row < rows_valid && col < p.N)
          *(uint4*)(C + (tile_row0 + row) * p.ldc + col) = *(const uint4*)(smem + row * RS + ch * 16);
      }
      __syncthreads();
    } else {
      // SwiGLU: subtiles ni=0,1 hold gate, ni=2,3 the matching up columns.
      constexpr int RS = 128 * 4 + 16;  // fp32 staged act row stride
#pragma unroll
      for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < 2; ++ni)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            int row = wm * 64 + mi * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            int col = wn * 64 + ni * 32 + (lane & 31);
            float gte = bf16_to_f32(f32_to_bf16(acc[mi][ni][r]));
            float up = bf16_to_f32(f32_to_bf16(acc[mi][ni + 2][r]));
            float act = gte / (1.0f + __expf(-gte)) * up;
            *(float*)(smem + row * RS + col * 4) = act;
          }
      __syncthreads();
      if (EPI == EPI_SWIGLU_BF16) {
        uint16_t* C = (uint16_t*)p.C;
        for (int id = tid; id < GG_BM * 16; id += GG_THREADS) {
          int row = id >> 4, ch = id & 15;
          if (row < rows_valid) {
            const float* s = (const float*)(smem + row * RS + ch * 32);
            uint4 o;
            o.x = f32_to_bf16(s[0]) | ((uint32_t)f32_to_bf16(s[1]) << 16);
            o.y = f32_to_bf16(s[2]) | ((uint32_t)f32_to_bf16(s[3]) << 16);
            o.z = f32_to_bf16(s[4]) | ((uint32_t)f32_to_bf16(s[5]) << 16);
            o.w = f32_to_bf16(s[6]) | ((uint32_t)f32_to_bf16(s[7]) << 16);
            *(uint4*)(C + (tile_row0 + row) * p.ldc + nt * 128 + ch * 8) = o;
          }
        }
      } else {
        uint8_t* C = (uint8_t*)p.C;
        for (int id = tid; id < GG_BM * 4; id += GG_THREADS) {
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
            uint8_t* dst = C + (tile_row0 + row) * p.ldc + nt * 128 + blk * 32;
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

static int g_num_cus = 0;
static int num_cus() {
  if (g_num_cus == 0) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    g_num_cus = n;
  }
  return g_num_cus;
}

template <bool MX, bool B_KN, int EPI>
static int launch_gg(const GGParams& p, hipStream_t stream) {
  static bool configured = false;
  auto kern = grouped_gemm_kernel<MX, B_KN, EPI>;
  if (!configured) {
    if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, GGLds::TOTAL) != hipSuccess)
      return MI355MOE_ELAUNCH;
    configured = true;
  }
  int grid = (num_cus() / 8) * 8;
  if (grid < 8) grid = 8;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(GG_THREADS), GGLds::TOTAL, stream, p);
  return hipGetLastError() == hipSuccess ? MI355MOE_OK : MI355MOE_ELAUNCH;
}

int mi355_plan_tiles(const int64_t* group_list, int G, int32_t* tile_prefix, hipStream_t stream) {
  hipLaunchKernelGGL(plan_tiles_kernel, dim3(1), dim3(1024), 0, stream, group_list, G, GG_BM, tile_prefix);
  return hipGetLastError() == hipSuccess ? MI355MOE_OK : MI355MOE_ELAUNCH;
}

// Internal dispatcher used by the C-ABI entry points.
// kind: 0 plain bf16 out, 1 fp32 out, 2 swiglu bf16, 3 swiglu mx
int mi355_grouped_gemm(const GGParams& p, bool mx, bool b_kn, int epi, hipStream_t stream) {
  if (!mx) {
    if (!b_kn) {
      switch (epi) {
        case EPI_STORE_BF16: return launch_gg<false, false, EPI_STORE_BF16>(p, stream);
        case EPI_STORE_F32: return launch_gg<false, false, EPI_STORE_F32>(p, stream);
        case EPI_SWIGLU_BF16: return launch_gg<false, false, EPI_SWIGLU_BF16>(p, stream);
        default: return MI355MOE_EUNSUPPORTED;
      }
    } else {
      switch (epi) {
        case EPI_STORE_BF16: return launch_gg<false, true, EPI_STORE_BF16>(p, stream);
        case EPI_SWIGLU_BF16: return launch_gg<false, true, EPI_SWIGLU_BF16>(p, stream);
        default: return MI355MOE_EUNSUPPORTED;
      }
    }
  }
  if (!b_kn) return MI355MOE_EUNSUPPORTED;
  switch (epi) {
    case EPI_STORE_BF16: return launch_gg<true, true, EPI_STORE_BF16>(p, stream);
    case EPI_SWIGLU_MX: return launch_gg<true, true, EPI_SWIGLU_MX>(p, stream);
    default: return MI355MOE_EUNSUPPORTED;
  }
}

int mi355_gg_bm() { return GG_BM; }
int mi355_gg_bn() { return GG_BN; }
