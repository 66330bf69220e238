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
#include "gemm_kernel.h"

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
int mi355_num_cus() {
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
  int grid = (mi355_num_cus() / 8) * 8 * C::WG_PER_CU;
  if (grid < 8) grid = 8;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(C::THREADS), C::TOTAL, stream, p);
  return hipGetLastError() == hipSuccess ? MI355MOE_OK : MI355MOE_ELAUNCH;
}

int mi355_plan_tiles(const int64_t* group_list, int G, int32_t* tile_prefix, hipStream_t stream, bool small) {
  hipLaunchKernelGGL(plan_tiles_kernel, dim3(1), dim3(1024), 0, stream, group_list, G, mi355_gg_bm(small), tile_prefix);
  return hipGetLastError() == hipSuccess ? MI355MOE_OK : MI355MOE_ELAUNCH;
}

int mi355_plan_row_blocks(const int64_t* group_list, int G, int rows, int32_t* block_prefix, hipStream_t stream) {
  hipLaunchKernelGGL(plan_tiles_kernel, dim3(1), dim3(1024), 0, stream, group_list, G, rows, block_prefix);
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
