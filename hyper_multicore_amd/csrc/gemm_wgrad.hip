// Grouped-K GEMM kernels (weight gradients of the expert backward), bf16 and MXFP8; built on the
// shared K loop of gemm_kernel.h (see gemm.hip for the pipeline and the LDS layouts).
#include "gemm_kernel.h"

// Grouped-K GEMM (weight gradients): C_g[m, n] = sum over the rows r of group g (group_list) of
// A[r, m] * B[r, n], bf16 or MXFP8 in, fp32 accumulate, C_g = C + g * c_group_stride (fp32 or bf16
// store). Both operands are read K-major (rows = K) into the same LDS layout as an EIO weight tile
// and read with transposing loads; rows past a group's end come from a zero row, so groups of any
// size (including none: C_g = 0) are exact. MXFP8: e4m3 operands quantised along the routed rows
// in 32-row blocks from each group's first row, with the grouped packed column scales (two codes
// per column per 64-row stage), fed to the scaled MFMA. Work items are (group, m-tile, n-tile),
// m fastest.
template <class C, bool MX, int EPI>
__global__ __launch_bounds__(C::THREADS, C::WG_PER_CU) void grouped_gemm_wgrad_kernel(GGParams p) {
  static_assert(!MX || C::AS_N == 2, "MX needs the AS area for the per-stage column scales of A");
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
      if (C::MI >= 4 && nm == 4) k_loop<C, MX, true, (C::MI >= 4 ? 4 : 1), true, true>(cp, nk, wave, wm, wn, lane, smem, acc);
      else if (nm == 2) k_loop<C, MX, true, 2, true, true>(cp, nk, wave, wm, wn, lane, smem, acc);
      else if (nm == 1) k_loop<C, MX, true, 1, true, true>(cp, nk, wave, wm, wn, lane, smem, acc);
      else k_loop<C, MX, true, 0, true, true>(cp, nk, wave, wm, wn, lane, smem, acc);
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

template <class C, bool MX, int EPI>
static int launch_wgrad(const GGParams& p, hipStream_t stream) {
  static bool configured = false;
  auto kern = grouped_gemm_wgrad_kernel<C, MX, EPI>;
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

int mi355_grouped_gemm_wgrad(const GGParams& p, int epi, hipStream_t stream, bool mx) {
  const int align = mx ? 16 : 8;  // 16-byte copies of e4m3 / bf16 columns
  if (p.m_rows % align || p.N % align || p.m_tiles != (p.m_rows + GGBig::BM - 1) / GGBig::BM ||
      p.n_tiles != (p.N + GGBig::BN - 1) / GGBig::BN || p.zero_row == nullptr)
    return MI355MOE_EINVAL;
  if (mx && (p.a_scale == nullptr || p.b_scale == nullptr)) return MI355MOE_EINVAL;
  switch (epi) {
    case EPI_STORE_F32:
      return mx ? launch_wgrad<GGBig, true, EPI_STORE_F32>(p, stream) : launch_wgrad<GGBig, false, EPI_STORE_F32>(p, stream);
    case EPI_STORE_BF16:
      return mx ? launch_wgrad<GGBig, true, EPI_STORE_BF16>(p, stream)
                : launch_wgrad<GGBig, false, EPI_STORE_BF16>(p, stream);
    default: return MI355MOE_EUNSUPPORTED;
  }
}

