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
#include <cstdlib>
#include <cstring>
#include "gemm_kernel.h"

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

int mi355_plan_tiles(const int64_t* group_list, int G, int32_t* tile_prefix, hipStream_t stream, bool small) {
  hipLaunchKernelGGL(plan_tiles_kernel, dim3(1), dim3(1024), 0, stream, group_list, G, mi355_gg_bm(small), tile_prefix);
  return hipGetLastError() == hipSuccess ? MI355MOE_OK : MI355MOE_ELAUNCH;
}

int mi355_plan_row_blocks(const int64_t* group_list, int G, int rows, int32_t* block_prefix, hipStream_t stream) {
  hipLaunchKernelGGL(plan_tiles_kernel, dim3(1), dim3(1024), 0, stream, group_list, G, rows, block_prefix);
  return hipGetLastError() == hipSuccess ? MI355MOE_OK : MI355MOE_ELAUNCH;
}

// Internal dispatcher used by the C-ABI entry points. `small` selects the 64-row tile
// configuration (the tile prefix must have been planned with the same one).
int mi355_grouped_gemm(const GGParams& p, bool mx, bool b_kn, int epi, hipStream_t stream, bool small) {
  if (epi == EPI_SWIGLU_BF16_NUM) return MI355MOE_EINVAL;  // internal: chosen from the options below
  if (epi == EPI_SWIGLU_BF16 && (p.swiglu_limit > 0.0f || p.row_prob != nullptr)) epi = EPI_SWIGLU_BF16_NUM;
  if (small) return dispatch_gg<GGSmall>(p, mx, b_kn, epi, stream);
  const int variant = p.variant;
  // the 8-wave configuration first (the default); the 4-wave kernels below for what it does not take
  if (variant == MI355_GG_VARIANT_DEFAULT || variant == MI355_GG_VARIANT_PP) {
    const int rc = mi355_grouped_gemm_pp(p, mx, b_kn, epi, stream);
    if (rc != MI355MOE_EUNSUPPORTED) return rc;
  }
  // stage-major MX scales are read and written by the 8-wave configuration only
  if (p.a_scale_stage_stride != 0 || p.c_scale_stage_stride != 0) return MI355MOE_EUNSUPPORTED;
  return dispatch_gg<GGBig>(p, mx, b_kn, epi, stream);
}


int mi355_gg_bm(bool small) { return small ? GGSmall::BM : GGBig::BM; }
int mi355_gg_bn() { return GGBig::BN; }
