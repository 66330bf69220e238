// Persistent grouped GEMM for gfx950 (MI355X): bf16 and MXFP8 (e4m3 + e8m0 per 32 along K).
//
// Work list: the row segments of the groups (experts) are cut into BM-row tiles; every
// (group, m-tile, n-tile) is one work item. tile_prefix[g] (computed on the device from the
// group row counts) gives the first m-tile of group g, so the work list needs no host round
// trip. The grid is one workgroup per CU; workgroup i runs on XCD i % 8 and walks the work list
// in rounds so that each XCD takes a contiguous run of items per round (m fastest): items that
// share a weight slice run at the same time on one XCD and share its L2.
//
// Workgroup: 256 threads = 4 wavefronts in a 2 (M) x 2 (N) grid; tile BM=128 x BN=256; each
// wavefront computes 64 x 128 with 32x32 MFMA (bf16: v_mfma_f32_32x32x16_bf16; MXFP8:
// v_mfma_scale_f32_32x32x64_f8f6f4 with per-lane e8m0 scales: lane r + 32b supplies the scale
// of 32-block b of row / column r, and its operand bytes 0-15 / 16-31 hold K = 16b + i /
// 32 + 16b + i of the 64-K step). K advances 128 bytes per stage
// (64 bf16 or 128 e4m3). Global -> LDS copies use the direct-to-LDS 16-byte loads; two LDS
// stages are double buffered.
//
// LDS layouts (16-byte chunk granularity, XOR swizzled against bank conflicts):
//   K-contiguous operand rows (A always; B in EOI layout): row r at r*128, chunk c stored at
//     c ^ ((r >> 1) & 7); read with ds_read_b128.
//   N-contiguous B (EIO bf16 / MX col_data): row k holds 256 columns; bf16 chunk c stored at
//     c ^ ((k & 7) << 1) (512-byte rows), e4m3 chunk c at c ^ (k & 15) (256-byte rows); read
//     with the transposing ds_read_b64_tr_b16 / ds_read_b64_tr_b8.
//
// Epilogues: bf16 store, fp32 store (router logits, optional row scatter), SwiGLU -> bf16 and
// SwiGLU -> MXFP8 requant. For SwiGLU the B tile columns are gate/up interleaved in 64-column
// groups so that each lane holds the gate and up value of the same output element.
#include "common.h"
#include "scan.h"
#include "../../include/mi355moe.h"
#include "gemm.h"

#define GG_BM 128
#define GG_BN 256
#define GG_KB 128  // bytes of K per stage per row
#define GG_THREADS 256

struct GGLds {
  static constexpr int A_BYTES = GG_BM * GG_KB;        // 16 KB
  static constexpr int B_BYTES = GG_BN * GG_KB;        // 32 KB
  static constexpr int AS_BYTES = GG_BM * 4;           // 512 B
  static constexpr int BS_BYTES = 2 * GG_BN * 2;       // 1 KB
  static constexpr int STAGE = A_BYTES + B_BYTES + AS_BYTES + BS_BYTES;
  static constexpr int NSTAGE = 3;
  static constexpr int PREFIX_MAX = 1024;              // groups whose tile prefix is kept in LDS
  static constexpr int PREFIX_OFF = NSTAGE * STAGE;
  static constexpr int TOTAL = PREFIX_OFF + (PREFIX_MAX + 1) * 4;
};

MI355_DEV void lds_load16(const void* g, uint32_t lds_off_uniform, uint8_t* smem) {
  __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)(smem + lds_off_uniform), 16, 0, 0);
}
MI355_DEV void lds_load4(const void* g, uint32_t lds_off_uniform, uint8_t* smem) {
  __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)(smem + lds_off_uniform), 4, 0, 0);
}
// Wait until at most N vector-memory loads of this wave are outstanding (loads retire in order).
// Workgroup barrier without the release fence of __syncthreads (which would wait for every
// outstanding global load, including the prefetched stages): LDS reads of this wave are drained,
// the direct-to-LDS loads are ordered by the explicit vmcnt waits.
MI355_DEV void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
}
template <int N>
MI355_DEV void wait_vm_le() {
  if constexpr (N == 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  else if constexpr (N == 12) asm volatile("s_waitcnt vmcnt(12)" ::: "memory");
  else if constexpr (N == 13) asm volatile("s_waitcnt vmcnt(13)" ::: "memory");
  else static_assert(N == 0, "unsupported vmcnt");
}

// Tile column j (0..255) -> weight column. SwiGLU: per 128-column half h, 64 gate then 64 up.
MI355_DEV int tile_col_to_weight_col(int j, int nt, int I, bool swiglu) {
  if (!swiglu) return nt * GG_BN + j;
  int h = j >> 7, jj = j & 127;
  int base = nt * 128 + h * 64;
  return jj < 64 ? base + jj : I + base + (jj - 64);
}

struct FragBF16 {
  v8bf a[2];
  v8bf b[4];
};
struct FragMX {
  v8i a[2];
  v8i b[4];
  int sa[2];
  int sb[4];
};

template <bool B_KN>
MI355_DEV void load_frag_bf16(const uint8_t* As, const uint8_t* Bs, int ks, int wm, int wn, int lane, FragBF16& f) {
#pragma unroll
  for (int mi = 0; mi < 2; ++mi) {
    int r = wm * 64 + mi * 32 + (lane & 31);
    int c = (ks * 2 + (lane >> 5)) ^ ((r >> 1) & 7);
    f.a[mi] = *(const v8bf*)(As + r * 128 + c * 16);
  }
#pragma unroll
  for (int ni = 0; ni < 4; ++ni) {
    if (!B_KN) {
      int n = wn * 128 + ni * 32 + (lane & 31);
      int c = (ks * 2 + (lane >> 5)) ^ ((n >> 1) & 7);
      f.b[ni] = *(const v8bf*)(Bs + n * 128 + c * 16);
    } else {
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
      f.b[ni] = __builtin_bit_cast(v8bf, both);
    }
  }
}

// Scaled-MFMA operand order: lane r + 32g holds bytes 0-15 = K 16g + i and bytes 16-31 =
// K 32 + 16g + i of the 64-K step, and supplies the e8m0 scale of 32-block g.
MI355_DEV void load_frag_mx(const uint8_t* As, const uint8_t* Bs, const uint8_t* ASs, const uint8_t* BSs, int ks,
                            int wm, int wn, int lane, FragMX& f) {
#pragma unroll
  for (int mi = 0; mi < 2; ++mi) {
    int r = wm * 64 + mi * 32 + (lane & 31);
    int c0 = ks * 4 + (lane >> 5);
    v4i lo = *(const v4i*)(As + r * 128 + ((c0 ^ ((r >> 1) & 7)) << 4));
    v4i hi = *(const v4i*)(As + r * 128 + (((c0 + 2) ^ ((r >> 1) & 7)) << 4));
    f.a[mi] = (v8i){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    f.sa[mi] = ASs[r * 4 + ks * 2 + (lane >> 5)];
  }
#pragma unroll
  for (int ni = 0; ni < 4; ++ni) {
    int g16 = lane >> 4, m = lane & 15;
    int nb = wn * 128 + ni * 32 + (g16 & 1) * 16;
    int parts[8];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      int k = ks * 64 + (q >> 1) * 32 + (g16 >> 1) * 16 + (q & 1) * 8 + (m >> 1);
      int off = k * 256 + (((nb >> 4) ^ (k & 15)) << 4) + 8 * (m & 1);
      v2i v = __builtin_amdgcn_ds_read_tr8_b64_v2i32(LDS_PTR(v2i, Bs + off));
      parts[2 * q] = v[0];
      parts[2 * q + 1] = v[1];
    }
    f.b[ni] = (v8i){parts[0], parts[1], parts[2], parts[3], parts[4], parts[5], parts[6], parts[7]};
    int n = wn * 128 + ni * 32 + (lane & 31);
    f.sb[ni] = BSs[ks * 512 + n * 2 + (lane >> 5)];
  }
}

template <int NM>
MI355_DEV void mfma_bf16(v16f (&acc)[2][4], const FragBF16& f) {
#pragma unroll
  for (int mi = 0; mi < NM; ++mi)
#pragma unroll
    for (int ni = 0; ni < 4; ++ni)
      acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.a[mi], f.b[ni], acc[mi][ni], 0, 0, 0);
}
template <int NM>
MI355_DEV void mfma_mx(v16f (&acc)[2][4], const FragMX& f) {
#pragma unroll
  for (int mi = 0; mi < NM; ++mi)
#pragma unroll
    for (int ni = 0; ni < 4; ++ni)
      acc[mi][ni] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(f.a[mi], f.b[ni], acc[mi][ni], 0, 0, 0, f.sa[mi],
                                                                     0, f.sb[ni]);
}

// Per-thread copy plan of one work item (global sources of this thread's 16-byte chunks).
struct CopyPlan {
  const uint8_t* a[4];
  const uint8_t* b[8];
  const uint8_t* s[2];
};

template <bool MX, bool B_KN>
MI355_DEV void issue_stage(const GGParams& p, const CopyPlan& cp, int kt, int stage, int wave, uint8_t* smem) {
  constexpr int ESIZE = MX ? 1 : 2;
  const uint32_t base = stage * GGLds::STAGE;
  const int64_t koff = (int64_t)kt * GG_KB;
#pragma unroll
  for (int j = 0; j < 4; ++j) lds_load16(cp.a[j] + koff, base + (wave * 4 + j) * 1024, smem);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint8_t* src = B_KN ? cp.b[j] + (int64_t)kt * (GG_KB / ESIZE) * p.b_row_bytes : cp.b[j] + koff;
    lds_load16(src, base + GGLds::A_BYTES + (wave * 8 + j) * 1024, smem);
  }
  if (MX) {
    if (wave < 2) {
      lds_load4(cp.s[0] + kt * 4, base + GGLds::A_BYTES + GGLds::B_BYTES + wave * 256, smem);
    } else {
      const int64_t ks = (int64_t)kt * 2 * p.Ntot * 2;  // two 64-K groups per stage
#pragma unroll
      for (int h = 0; h < 2; ++h)
        lds_load4(cp.s[h] + ks, base + GGLds::A_BYTES + GGLds::B_BYTES + GGLds::AS_BYTES + (wave - 2) * 512 + h * 256,
                  smem);
    }
  }
}

// K loop over a 3-stage LDS ring; NM = number of valid 32-row subtiles this wave computes.
template <bool MX, bool B_KN, int NM>
MI355_DEV void k_loop(const GGParams& p, const CopyPlan& cp, int nk, int wave, int wm, int wn, int lane, uint8_t* smem,
                      v16f (&acc)[2][4]) {
  constexpr int LOADS = MX ? 13 : 12;  // minimum loads per wave per stage
  issue_stage<MX, B_KN>(p, cp, 0, 0, wave, smem);
  if (nk > 1) issue_stage<MX, B_KN>(p, cp, 1, 1, wave, smem);
  int stage = 0;
  for (int kt = 0; kt < nk; ++kt) {
    if (kt + 1 < nk) wait_vm_le<LOADS>(); else wait_vm_le<0>();
    lds_barrier();
    if (kt + 2 < nk) {
      int s2 = stage + 2;
      if (s2 >= 3) s2 -= 3;
      issue_stage<MX, B_KN>(p, cp, kt + 2, s2, wave, smem);
    }
    const uint8_t* As = smem + stage * GGLds::STAGE;
    const uint8_t* Bs = As + GGLds::A_BYTES;
    if constexpr (NM > 0) {
      if constexpr (!MX) {
        FragBF16 f[2];
        load_frag_bf16<B_KN>(As, Bs, 0, wm, wn, lane, f[0]);
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          if (ks + 1 < 4) load_frag_bf16<B_KN>(As, Bs, ks + 1, wm, wn, lane, f[(ks + 1) & 1]);
          mfma_bf16<NM>(acc, f[ks & 1]);
        }
      } else {
        const uint8_t* ASs = Bs + GGLds::B_BYTES;
        const uint8_t* BSs = ASs + GGLds::AS_BYTES;
        FragMX f[2];
        load_frag_mx(As, Bs, ASs, BSs, 0, wm, wn, lane, f[0]);
        load_frag_mx(As, Bs, ASs, BSs, 1, wm, wn, lane, f[1]);
        mfma_mx<NM>(acc, f[0]);
        mfma_mx<NM>(acc, f[1]);
      }
    }
    stage = stage == 2 ? 0 : stage + 1;
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
  const int total = prefix[p.G] * p.n_tiles;
  const int nk = p.K * ESIZE / GG_KB;
  const int xcd = blockIdx.x & 7;
  const int per_xcd = gridDim.x >> 3;
  const int slot = blockIdx.x >> 3;

  for (int round = 0;; ++round) {
    const int L = round * (int)gridDim.x + xcd * per_xcd + slot;
    if (L >= total) break;
    // ---- decode work item -------------------------------------------------------------
    int lo = 0, hi = p.G - 1;
    while (lo < hi) {  // largest g with prefix[g]*n_tiles <= L
      int mid = (lo + hi + 1) >> 1;
      if (prefix[mid] * p.n_tiles <= L) lo = mid; else hi = mid - 1;
    }
    const int g = lo;
    const int mtiles = prefix[g + 1] - prefix[g];
    const int local = L - prefix[g] * p.n_tiles;
    const int nt = local / mtiles;
    const int mt = local - nt * mtiles;
    const int64_t row_begin = (g == 0 ? 0 : p.group_list[g - 1]);
    const int64_t row_end = p.group_list[g];
    const int64_t tile_row0 = row_begin + (int64_t)mt * GG_BM;
    const int rows_valid = (int)((row_end - tile_row0) < GG_BM ? (row_end - tile_row0) : GG_BM);

    // ---- per-thread copy sources ------------------------------------------------------
    CopyPlan cp;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      int L16 = wave * 256 + j * 64 + lane;
      int r = L16 >> 3, cs = L16 & 7;
      int c = cs ^ ((r >> 1) & 7);
      int rr = r < rows_valid ? r : rows_valid - 1;
      int64_t routed = tile_row0 + rr;
      int64_t src = p.a_row_index ? (int64_t)(p.a_row_index[routed] / p.a_row_div) : routed;
      cp.a[j] = p.A + src * p.lda_bytes + c * 16;
    }
    const uint8_t* bgrp = p.B + (int64_t)g * p.b_group_stride;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      int L16 = wave * 512 + j * 64 + lane;
      if (!B_KN) {
        int r = L16 >> 3, cs = L16 & 7;
        int c = cs ^ ((r >> 1) & 7);
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
    // MX scales: waves 0/1 copy A scale dwords (rows 0..63 / 64..127), waves 2/3 copy the two
    // 64-K groups of B scales (256 columns x 2 bytes = 128 dwords = 2 instructions each).
    cp.s[0] = cp.s[1] = nullptr;
    if (MX) {
      if (wave < 2) {
        int r = wave * 64 + lane;
        int rr = r < rows_valid ? r : rows_valid - 1;
        int64_t routed = tile_row0 + rr;
        int64_t src = p.a_row_index ? (int64_t)(p.a_row_index[routed] / p.a_row_div) : routed;
        cp.s[0] = p.a_scale + src * (p.K / 32);
      } else {
        int gi = wave - 2;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          int j = (h * 64 + lane) * 2;  // tile column pair (j, j+1)
          int wc = tile_col_to_weight_col(j, nt, p.N, SWIGLU);
          if (wc >= p.Ntot) wc = p.Ntot - 2;
          cp.s[h] = p.b_scale + (int64_t)g * p.b_scale_group_stride + ((int64_t)gi * p.Ntot + wc) * 2;
        }
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
    const int nm = wm * 64 + 32 < rows_valid ? 2 : (wm * 64 < rows_valid ? 1 : 0);
    if (nm == 2) k_loop<MX, B_KN, 2>(p, cp, nk, wave, wm, wn, lane, smem, acc);
    else if (nm == 1) k_loop<MX, B_KN, 1>(p, cp, nk, wave, wm, wn, lane, smem, acc);
    else k_loop<MX, B_KN, 0>(p, cp, nk, wave, wm, wn, lane, smem, acc);
    __syncthreads();  // all waves are done reading the ring before the epilogue reuses LDS

    // ---- epilogue -----------------------------------------------------------------------
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
              C[orow * p.ldc + col] = acc[mi][ni][r];
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
            p.c_scale[(tile_row0 + row) * (p.N / 32) + nt * 4 + blk] = (uint8_t)code;
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
