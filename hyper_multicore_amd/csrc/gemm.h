// Internal interface of the persistent grouped GEMM (gemm.hip) and the other kernel files.
#pragma once
#include "common.h"

// EPI_SWIGLU_BF16_NUM is EPI_SWIGLU_BF16 with the numerics options (clamp, probabilities before FC2);
// callers ask for EPI_SWIGLU_BF16 and the dispatcher picks it when one of the options is set.
// EPI_SWIGLU_F32 (8-wave configuration, MX inputs): the fp32 SwiGLU output, for mi355_mx_quant_act.
enum { EPI_STORE_BF16 = 0, EPI_STORE_F32 = 1, EPI_SWIGLU_BF16 = 2, EPI_SWIGLU_MX = 3, EPI_SWIGLU_BF16_NUM = 4,
       EPI_SWIGLU_F32 = 5 };

struct GGParams {
  const uint8_t* A;          // [rowsA, K] elements (bf16 or e4m3), row stride lda_bytes
  int64_t lda_bytes;
  const int32_t* a_row_index;  // routed row -> index (or NULL: identity)
  int32_t a_row_div;           // source row = a_row_index[r] / a_row_div
  const uint8_t* a_scale;    // MX: [rowsA, K/32] with row stride a_scale_ld (multiple of 16 bytes)
  int64_t a_scale_ld;
  const uint8_t* B;          // per group: NK [Ntot, K] or KN [K, Ntot]
  int64_t b_group_stride;    // bytes
  int64_t b_row_bytes;       // NK: K*esize ; KN: Ntot*esize
  const uint8_t* b_scale;    // MX, KN: col_scale [G, K/64, Ntot, 2]; NK: row scales [G*Ntot, K/32]
  int64_t b_scale_group_stride;  // bytes (KN: (K/64)*Ntot*2; NK: Ntot*b_scale_ld)
  int64_t b_scale_ld;        // MX NK: row stride of the row scales (multiple of 16 bytes)
  int32_t K;                 // reduction length (elements)
  int32_t N;                 // output columns (SwiGLU: I; otherwise Ntot)
  int32_t Ntot;              // weight columns (SwiGLU: 2I)
  int32_t n_tiles;
  int32_t G;
  const int64_t* group_list; // inclusive cumulative rows per group
  const int32_t* tile_prefix;  // [G+1]
  void* C;
  int64_t ldc;               // elements (bf16/f32) or bytes (e4m3)
  const int32_t* c_row_index;  // optional output row scatter (EPI_STORE_F32)
  uint8_t* c_scale;          // EPI_SWIGLU_MX: [rows, N/32] with row stride c_scale_ld
  int64_t c_scale_ld;
  float swiglu_limit;        // EPI_SWIGLU_BF16: > 0 clamps the SwiGLU inputs (0: no clamp)
  int32_t swiglu_after_silu; // EPI_SWIGLU_BF16: clamp SiLU(gate) instead of gate
  const float* row_prob;     // EPI_SWIGLU_BF16: probability of slot a_row_index[r] multiplies row r
  int32_t k_splits;          // EPI_STORE_F32 only: >1 splits K; split s writes C + s * c_split_stride
  int64_t c_split_stride;    // elements
  // Grouped-K mode (weight gradients): C_g[m, n] = sum over the routed rows r of group g of
  // A[r, m] * B[r, n]; A [rows, m_rows] (row stride lda_bytes) and B [rows, N] (b_row_bytes) are
  // both read K-major, group_list gives the row ranges, C_g = C + g * c_group_stride (elements).
  int32_t m_rows;
  int32_t m_tiles;
  int64_t c_group_stride;
  const uint8_t* zero_row;   // >= 2 * max(m_rows, N) zero bytes (rows past a group's end)
  // Bytes of the activation tensor A (0: not given). The direct-weight configuration addresses A
  // with 32-bit offsets and runs only when this is set and below 4 GiB. Last member, so the other
  // members keep their kernel-argument offsets.
  int64_t a_bytes;
  // Stage-major MX scales (the 8-wave configuration, gemm_pp.hip): when a_scale_stage_stride (bytes
  // per 128-K stage) is set, a_scale holds code planes [K/128][4][P] (P = a_scale_stage_stride / 4):
  // code j of stage s of routed row r at a_scale[s * stride + j * P + r], so a tile's codes of a
  // stage are four contiguous runs. When c_scale_stage_stride is set, the MX SwiGLU epilogue writes
  // c_scale in that form. The planes are indexed by routed row (a_scale_routed must be set when
  // a_row_index gathers the rows), and hold at least 512 bytes past the last row (a tile reads two
  // 256-byte runs per plane from the 4-aligned row at or below its first row).
  int64_t a_scale_stage_stride;
  int64_t c_scale_stage_stride;
  int32_t a_scale_routed;
  // Tile-configuration variant of this call (MI355_GG_VARIANT_*; 0: the default).
  int32_t variant;
  // Rows of the whole GEMM when the caller knows them (0: not given); the 8-wave bf16 configuration
  // picks its tile height from their average per group.
  int64_t rows_hint;
  // SwiGLU GEMMs: the weight's gate and up columns are interleaved in 64-column blocks (block b:
  // gate columns 64 b ..+63, then up columns 64 b ..+63), so a tile's gate and up columns are one
  // contiguous run per K row, and each 64 output columns' gate and up one 128-byte line of an MX
  // weight row (0: gate columns [0, I) then up columns [I, 2I)).
  int32_t gate_up_interleaved;
};

// Physical weight column of projection column c (gate: c < I, up: c >= I) in the gate/up
// interleaved layout (identity when `gu` is 0).
__host__ __device__ __forceinline__ int gate_up_col(int c, int I, int gu) {
  const int up = (c >= I) ? 1 : 0;
  const int cc = c - (up ? I : 0);
  const int il = ((cc >> 6) << 7) + (up << 6) + (cc & 63);
  return gu ? il : c;
}


int mi355_grouped_gemm(const GGParams& p, bool mx, bool b_kn, int epi, hipStream_t stream, bool small = false);
// Grouped-K GEMM (weight gradients), EPI_STORE_F32 or EPI_STORE_BF16; bf16 operands, or with `mx`
// e4m3 operands with grouped packed column scales in a_scale / b_scale.
int mi355_grouped_gemm_wgrad(const GGParams& p, int epi, hipStream_t stream, bool mx = false);
int mi355_plan_tiles(const int64_t* group_list, int G, int32_t* tile_prefix, hipStream_t stream, bool small = false);
int mi355_gg_bm(bool small = false);
// block_prefix[g] = sum_{g' < g} ceil(rows_g' / rows) (rows-row blocks per group), [G] = the total.
int mi355_plan_row_blocks(const int64_t* group_list, int G, int rows, int32_t* block_prefix, hipStream_t stream);
// Routed-row MX quantisation for the MXFP8 backward (quant.hip): the row axis (blocks of 32 columns,
// scales [R, row_scale_ld]) and / or the grouped column axis (blocks of 32 rows from each group's
// first row; packed scales [(R + 63) / 64 + G, C, 2], group g's pairs from 64-row group
// start_g / 64 + g) of a routed matrix [R, C] whose values are:
//   MX_Q_BF16        bf16 rows src[(gather ? gather[r] / gather_div : r) * src_ld + c]
//   MX_Q_SWIGLU      silu(g) * u of U [R, 2C] (the forward's fp32 activation), C = I
//   MX_Q_SWIGLU_BWD  [da u s (1 + g (1 - s)) | da g s] from U [R, C] and da [R, C / 2], fp32
enum { MX_Q_BF16 = 0, MX_Q_SWIGLU = 1, MX_Q_SWIGLU_BWD = 2 };
struct MxGroupedQuant {
  int mode;
  const uint16_t* src;
  const int32_t* gather;
  int32_t gather_div;
  int64_t src_ld;
  const uint16_t* U;
  const uint16_t* da;
  int64_t R;
  int32_t C;
  int32_t G;
  const int64_t* group_list;
  const int32_t* block_prefix;  // mi355_plan_row_blocks(..., 32, ...)
  uint8_t* row_data;
  uint8_t* row_scale;
  int64_t row_scale_ld;
  uint8_t* col_data;
  uint8_t* col_scale;
};
int mi355_mx_quant_grouped(const MxGroupedQuant& q, hipStream_t stream);
int mi355_num_cus();  // CU count of the current device (cached per device)
// Forward tile configurations, chosen per call (GGParams::variant): DEFAULT - the 8-wave configuration
// where it applies, the 64-row tiles for decode-shaped GEMMs, else the 4-wave one; PP - the 8-wave
// configuration where it applies for every row count, else the 4-wave one; W4 - the 4-wave one.
// Values 1-4 are retired (configurations of earlier revisions) and refused.
enum { MI355_GG_VARIANT_DEFAULT = 0, MI355_GG_VARIANT_PP = 5, MI355_GG_VARIANT_W4 = 6 };
bool mi355_gg_variant_valid(int variant);
// The 8-wave ping-pong configuration (gemm_pp.hip); MI355MOE_EUNSUPPORTED outside its domain
// (mi355_gg_pp_applies). Tile plans are those of the 256-row configuration.
bool mi355_gg_pp_applies(const GGParams& p, bool mx, bool b_kn, int epi);
// Whether the 8-wave configuration takes forward GEMMs of these extents under the current variant
// (the caller then lays the MX activation scales out stage-major).
bool mi355_gg_pp_usable(int variant, bool mx, bool b_kn, int64_t K, int G, int64_t a_bytes, int64_t b_group_stride);
int mi355_grouped_gemm_pp(const GGParams& p, bool mx, bool b_kn, int epi, hipStream_t stream);
#include "features.h"
inline bool mi355_use_small_tiles(int64_t rows, int groups, int variant) {
  // a variant named explicitly keeps the 256-row tiles
  return mi355_small_tiles_enabled() && variant == 0 && rows <= (int64_t)groups * 32;
}
int mi355_gg_bn();
int mi355_dispatch_enqueue(const void* ids, int dtype, int64_t num_tokens, int top_k, int E, int32_t* counts,
                           int64_t* expert_offsets, int64_t* group_list, int32_t* mapping, int32_t* gather_index,
                           int32_t* error_flag, void* workspace, hipStream_t stream);
// mi355_dispatch_enqueue that also writes the grouped GEMM's tile plan at tile height bm (what
// mi355_plan_tiles computes from group_list), in the same launches.
int mi355_dispatch_plan_enqueue(const void* ids, int dtype, int64_t num_tokens, int top_k, int E, int32_t* counts,
                                int64_t* group_list, int32_t* mapping, int32_t* gather_index, int32_t* error_flag,
                                void* workspace, int32_t* tile_prefix, int bm, hipStream_t stream);
// The decode prologue (dispatch + MX token quantisation) in one launch (decode_prep.h); dprep::applies
// must hold.
namespace dprep { struct Args; }
int mi355_decode_prep_enqueue(const dprep::Args& a, int dtype, hipStream_t stream);
int mi355_zero_enqueue(void* p, size_t bytes, hipStream_t st);
int mi355_permute_rows_enqueue(const uint16_t* x, int64_t slots, int K, int H, const int32_t* mapping,
                                uint16_t* routed, hipStream_t st);
int mi355_unpermute_enqueue(const uint16_t* y, const int32_t* mapping, const float* probs, int64_t T, int K, int H,
                            uint16_t* out, hipStream_t stream);
// scale_stage_stride > 0 writes the scales as stage-major code planes ([cols/128][4][stride / 4]); with
// `mapping`, to the routed rows mapping[r * fanout + k] of each row r (negative entries skipped).
// MX quantisation of fp32 rows (the SwiGLU output of EPI_SWIGLU_F32) into e4m3 [rows, cols] and the
// stage-major code planes [cols/128][4][stage_stride / 4] (tiles of 64 rows x 256 columns).
int mi355_mx_quant_act(const float* act, int64_t rows, int cols, uint8_t* q, uint8_t* planes, int64_t stage_stride,
                       hipStream_t st);
// MX quantisation of token rows into q [tokens, cols] and per-token codes [tokens, cols/32] (scratch),
// then the stage-major code planes by routed row (gather: routed row -> slot, fanout slots per token).
int mi355_mx_quant_tokens_to_planes(const uint16_t* x, int64_t tokens, int cols, uint8_t* q, uint8_t* codes,
                                    const int32_t* gather, int fanout, const int64_t* group_list, int groups,
                                    uint8_t* planes, int64_t stage_stride, hipStream_t st);
int mi355_mx_quant_rows(const uint16_t* x, int64_t rows, int cols, uint8_t* q, uint8_t* scale, int64_t scale_ld,
                        hipStream_t st, int64_t scale_stage_stride = 0, const int32_t* mapping = nullptr,
                        int fanout = 1);
// Row stride (bytes) of the internal MX activation-scale buffers: K/32 rounded up to 16 so the
// GEMM can fetch 16 codes (8 K stages) of a row with one 16-byte load.
inline int64_t mi355_mx_scale_ld(int64_t k) { return ((k / 32 + 15) / 16) * 16; }
