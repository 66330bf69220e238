// OCP MX (v1.0) quantisation kernels: e4m3fn elements, one e8m0 shared exponent per 32 values.
// scale exponent = floor(log2(amax)) - 8 (8 = exponent of the largest e4m3 power of two), element
// = round-to-nearest-even(v / 2^scale) saturated to +-448.
// Row axis follows the quant_x task (ops/common/mega_moe/adapters/arch35/quantization/
// dual_axis_mxfp8_worker.h:39-66, blocks along the hidden dimension); the column form writes the
// forward MX weight root (modules/mega_moe/backends/mxfp8/weights.py:61-86: col_data [G,K,N],
// col_scale [G,K/64,N,2], 32-blocks along K for every column).
#include "common.h"
#include "gemm.h"
#include "../../include/mi355moe.h"

// One thread per 32-element block of a row.
// scale_stage_stride = 0: scales [rows, scale_ld]; otherwise stage-major code planes
// [cols/128][4][P] (P = scale_stage_stride / 4 rows per plane; code j of a 128-column stage of row r
// at plane j, the 8-wave GEMM's activation-scale layout). With `mapping` (slot -> routed row, `fanout`
// slots per row) the codes of row r go to the routed rows mapping[r * fanout + k] instead, so a GEMM
// over routed rows reads them in order.
__global__ __launch_bounds__(256) void mx_quant_rows_kernel(const uint16_t* x, int64_t rows, int cols,
                                                            uint8_t* q, uint8_t* scale, int64_t scale_ld,
                                                            int64_t scale_stage_stride, const int32_t* mapping,
                                                            int fanout) {
  const int nb = cols / 32;
  const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= rows * nb) return;
  const int64_t r = id / nb;
  const int b = (int)(id - r * nb);
  const uint4* src = (const uint4*)(x + r * cols + b * 32);
  float v[32];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint4 u = src[i];
    uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[i * 8 + 2 * j] = bf16_to_f32((uint16_t)(w[j] & 0xffff));
      v[i * 8 + 2 * j + 1] = bf16_to_f32((uint16_t)(w[j] >> 16));
    }
  }
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(v[i]));
  uint32_t code = mx_scale_code(amax);
  uint32_t out[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    out[i] = f32_to_e4m3_inrange(mx_apply_inv_scale(v[4 * i], code)) |
             (f32_to_e4m3_inrange(mx_apply_inv_scale(v[4 * i + 1], code)) << 8) |
             (f32_to_e4m3_inrange(mx_apply_inv_scale(v[4 * i + 2], code)) << 16) |
             (f32_to_e4m3_inrange(mx_apply_inv_scale(v[4 * i + 3], code)) << 24);
  }
  uint4* dst = (uint4*)(q + r * cols + b * 32);
  dst[0] = make_uint4(out[0], out[1], out[2], out[3]);
  dst[1] = make_uint4(out[4], out[5], out[6], out[7]);
  if (scale_stage_stride) {
    uint8_t* plane = scale + (b >> 2) * scale_stage_stride + (b & 3) * (scale_stage_stride >> 2);
    if (mapping != nullptr) {
      for (int k = 0; k < fanout; ++k) {
        const int32_t rr = mapping[r * fanout + k];
        if (rr >= 0) plane[rr] = (uint8_t)code;
      }
    } else {
      plane[r] = (uint8_t)code;
    }
  } else {
    scale[r * scale_ld + b] = (uint8_t)code;
  }
}

// One thread per (group, 32-row block along K, column).
__global__ __launch_bounds__(256) void mx_quant_cols_kernel(const uint16_t* w, int G, int K, int N,
                                                            uint8_t* col_data, uint8_t* col_scale) {
  const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int kb_n = K / 32;
  if (id >= (int64_t)G * kb_n * N) return;
  const int n = (int)(id % N);
  const int64_t gk = id / N;
  const int kb = (int)(gk % kb_n);
  const int g = (int)(gk / kb_n);
  const uint16_t* src = w + ((int64_t)g * K + kb * 32) * N + n;
  float v[32];
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    v[i] = bf16_to_f32(src[(int64_t)i * N]);
    amax = fmaxf(amax, fabsf(v[i]));
  }
  uint32_t code = mx_scale_code(amax);
  uint8_t* dst = col_data + ((int64_t)g * K + kb * 32) * N + n;
#pragma unroll
  for (int i = 0; i < 32; ++i) dst[(int64_t)i * N] = (uint8_t)f32_to_e4m3_inrange(mx_apply_inv_scale(v[i], code));
  col_scale[(((int64_t)g * (K / 64) + kb / 2) * N + n) * 2 + (kb & 1)] = (uint8_t)code;
}

// MX quantisation of the fp32 SwiGLU rows into e4m3 and the stage-major code planes. A workgroup
// takes a tile of 64 rows x 256 columns (8 blocks of 32): each wave quantises 16 of its rows, a row as
// one coalesced 1 KB read (lane l: columns 4l .. 4l+3, so lanes 8b .. 8b+7 hold block b and its
// amax is a reduction over 8 lanes) and one 256-byte code write. The tile's scale codes go through
// LDS so that each block's codes of the 64 rows are written as one 64-byte run of its plane.
constexpr int QA_ROWS = 64;
__global__ __launch_bounds__(256) void mx_quant_act_kernel(const float* act, int64_t rows, int cols, uint8_t* q,
                                                          uint8_t* planes, int64_t stage_stride) {
  __shared__ __align__(16) uint8_t codes[8][QA_ROWS];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t r0 = (int64_t)blockIdx.x * QA_ROWS;
  const int c0 = blockIdx.y * 256;
  const int col = c0 + 4 * lane;
  const bool live = col < cols;  // a last chunk of 128 columns uses lanes 0 .. 31
  constexpr int BATCH = 4;  // rows whose loads are issued together
  for (int i0 = 0; i0 < QA_ROWS / 4; i0 += BATCH) {
    v4f v[BATCH];
#pragma unroll
    for (int b = 0; b < BATCH; ++b) {
      const int64_t r = r0 + wave * (QA_ROWS / 4) + i0 + b;
      v[b] = (live && r < rows) ? *(const v4f*)(act + r * cols + col) : v4f{0.0f, 0.0f, 0.0f, 0.0f};
    }
#pragma unroll
    for (int b = 0; b < BATCH; ++b) {
      const int lr = wave * (QA_ROWS / 4) + i0 + b;
      const int64_t r = r0 + lr;
      if (r >= rows) break;  // wave-uniform
      float amax = fmaxf(fmaxf(fabsf(v[b][0]), fabsf(v[b][1])), fmaxf(fabsf(v[b][2]), fabsf(v[b][3])));
      amax = fmaxf(amax, __shfl_xor(amax, 1));
      amax = fmaxf(amax, __shfl_xor(amax, 2));
      amax = fmaxf(amax, __shfl_xor(amax, 4));
      const uint32_t code = mx_scale_code(amax);
      const uint32_t w = f32_to_e4m3_inrange(mx_apply_inv_scale(v[b][0], code)) |
                         (f32_to_e4m3_inrange(mx_apply_inv_scale(v[b][1], code)) << 8) |
                         (f32_to_e4m3_inrange(mx_apply_inv_scale(v[b][2], code)) << 16) |
                         (f32_to_e4m3_inrange(mx_apply_inv_scale(v[b][3], code)) << 24);
      if (live) {
        *(uint32_t*)(q + r * cols + col) = w;
        if ((lane & 7) == 0) codes[lane >> 3][lr] = (uint8_t)code;
      }
    }
  }
  __syncthreads();
  // block j of the tile (global block b = c0 / 32 + j): rows r0 .. r0 + 63 of plane (b >> 2, b & 3),
  // 4 bytes per thread
  const int j = threadIdx.x >> 4, k = (threadIdx.x & 15) * 4;
  const int b = c0 / 32 + j;
  if (j < 8 && c0 + 32 * j < cols) {
    uint8_t* plane = planes + (b >> 2) * stage_stride + (b & 3) * (stage_stride >> 2) + r0;
    if (r0 + k + 4 <= rows && ((uintptr_t)(plane + k) & 3) == 0) {
      *(uint32_t*)(plane + k) = *(const uint32_t*)&codes[j][k];
    } else {  // the last rows, or planes whose row count is not a multiple of 4
      for (int t = 0; t < 4 && r0 + k + t < rows; ++t) plane[k + t] = codes[j][k + t];
    }
  }
}

int mi355_mx_quant_act(const float* act, int64_t rows, int cols, uint8_t* q, uint8_t* planes, int64_t stage_stride,
                       hipStream_t st) {
  if (rows == 0) return MI355MOE_OK;
  if (cols % 128) return MI355MOE_EINVAL;
  const dim3 grid((unsigned)((rows + QA_ROWS - 1) / QA_ROWS), (unsigned)((cols + 255) / 256));
  hipLaunchKernelGGL(mx_quant_act_kernel, grid, dim3(256), 0, st, act, rows, cols, q, planes, stage_stride);
  return hipGetLastError() == hipSuccess ? MI355MOE_OK : MI355MOE_ELAUNCH;
}

// Stage-major code planes by routed row from per-token codes [tokens, nb]: one thread per 4
// consecutive routed rows and BPT consecutive 32-blocks (BPT of the code planes; BPT = 8, or 4 when
// nb % 8 != 0), rows fastest: a thread reads the 4 rows' gather entries once and each row's BPT codes
// as one load, and writes 4 bytes to each of its planes (a wavefront: 256 consecutive bytes of each).
// Routed row rr holds the codes of token gather[rr] / fanout; rows at or past the routed-row count
// (group_list[groups - 1]) get code 0 (nothing reads them as rows of a group).
template <int BPT>
__global__ __launch_bounds__(256) void mx_codes_to_planes_kernel(const uint8_t* codes, int nb, const int32_t* gather,
                                                                 int fanout, const int64_t* group_list, int groups,
                                                                 int64_t R, uint8_t* planes, int64_t stage_stride) {
  const int64_t R4 = (R + 3) / 4;
  const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= R4 * (nb / BPT)) return;
  const int b0 = (int)(id / R4) * BPT;
  const int64_t r0 = (id - (b0 / BPT) * R4) * 4;
  const int64_t valid = group_list[groups - 1];
  uint32_t w[BPT] = {};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t rr = r0 + i;
    uint64_t c8 = 0;
    if (rr < valid && rr < R) {
      const int32_t src = gather[rr];
      if (src >= 0) {
        const uint8_t* c = codes + (int64_t)(src / fanout) * nb + b0;
        c8 = BPT == 8 ? *(const uint64_t*)c : *(const uint32_t*)c;
      }
    }
#pragma unroll
    for (int j = 0; j < BPT; ++j) w[j] |= (uint32_t)((c8 >> (8 * j)) & 0xff) << (8 * i);
  }
#pragma unroll
  for (int j = 0; j < BPT; ++j) {
    const int b = b0 + j;
    uint8_t* plane = planes + (b >> 2) * stage_stride + (b & 3) * (stage_stride >> 2);
    if (r0 + 4 <= R && ((uintptr_t)(plane + r0) & 3) == 0) {
      *(uint32_t*)(plane + r0) = w[j];
    } else {
      for (int i = 0; i < 4 && r0 + i < R; ++i) plane[r0 + i] = (uint8_t)(w[j] >> (8 * i));
    }
  }
}

int mi355_mx_quant_tokens_to_planes(const uint16_t* x, int64_t tokens, int cols, uint8_t* q, uint8_t* codes,
                                    const int32_t* gather, int fanout, const int64_t* group_list, int groups,
                                    uint8_t* planes, int64_t stage_stride, hipStream_t st) {
  const int nb = cols / 32;
  const int64_t n = tokens * nb;
  if (n == 0) return MI355MOE_OK;
  hipLaunchKernelGGL(mx_quant_rows_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, x, tokens, cols, q,
                     codes, (int64_t)nb, (int64_t)0, (const int32_t*)nullptr, 1);
  if (hipGetLastError() != hipSuccess) return MI355MOE_ELAUNCH;
  const int64_t R = tokens * fanout;
  if (nb % 4) return MI355MOE_EINVAL;  // cols % 128 == 0
  const int bpt = nb % 8 == 0 ? 8 : 4;
  const int64_t m = (R + 3) / 4 * (nb / bpt);
  if (bpt == 8)
    hipLaunchKernelGGL(mx_codes_to_planes_kernel<8>, dim3((unsigned)((m + 255) / 256)), dim3(256), 0, st, codes, nb,
                       gather, fanout, group_list, groups, R, planes, stage_stride);
  else
    hipLaunchKernelGGL(mx_codes_to_planes_kernel<4>, dim3((unsigned)((m + 255) / 256)), dim3(256), 0, st, codes, nb,
                       gather, fanout, group_list, groups, R, planes, stage_stride);
  return hipGetLastError() == hipSuccess ? MI355MOE_OK : MI355MOE_ELAUNCH;
}

int mi355_mx_quant_rows(const uint16_t* x, int64_t rows, int cols, uint8_t* q, uint8_t* scale, int64_t scale_ld,
                        hipStream_t st, int64_t scale_stage_stride, const int32_t* mapping, int fanout) {
  int64_t n = rows * (cols / 32);
  if (n == 0) return MI355MOE_OK;
  hipLaunchKernelGGL(mx_quant_rows_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, x, rows, cols, q,
                     scale, scale_ld, scale_stage_stride, mapping, fanout);
  return hipGetLastError() == hipSuccess ? MI355MOE_OK : MI355MOE_ELAUNCH;
}

extern "C" int mi355moe_mx_quantize_rows(const uint16_t* x, int64_t rows, int32_t cols, uint8_t* q,
                                         uint8_t* scale, void* stream) {
  if (rows < 0 || cols <= 0 || cols % 32) return MI355MOE_EINVAL;
  if (rows > 0 && (x == nullptr || q == nullptr || scale == nullptr)) return MI355MOE_EINVAL;
  return mi355_mx_quant_rows(x, rows, cols, q, scale, cols / 32, (hipStream_t)stream);
}

extern "C" int mi355moe_mx_quantize_cols(const uint16_t* w, int32_t groups, int32_t kdim, int32_t cols,
                                         uint8_t* col_data, uint8_t* col_scale, void* stream) {
  if (groups <= 0 || kdim <= 0 || kdim % 64 || cols <= 0) return MI355MOE_EINVAL;
  if (w == nullptr || col_data == nullptr || col_scale == nullptr) return MI355MOE_EINVAL;
  int64_t n = (int64_t)groups * (kdim / 32) * cols;
  hipLaunchKernelGGL(mx_quant_cols_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, w,
                     groups, kdim, cols, col_data, col_scale);
  return hipGetLastError() == hipSuccess ? MI355MOE_OK : MI355MOE_ELAUNCH;
}

// ---- dual-axis MX weight quantisation ---------------------------------------------------------
// One workgroup per (group, 32-row block, 256-column block); thread c owns column n0 + c. Column
// axis: the thread's 32 values form one block (scale [G, M/64, N, 2]). Row axis: the 32 threads of
// a half-wave own 32 consecutive columns, so each row's block amax is a 32-lane reduction
// (scale [G, M, N/64, 2] = [G*M, N/32] codes). Loads and stores are row-contiguous across threads.
// Both axes use the same code / element conversions as mx_quant_rows_kernel and
// mx_quant_cols_kernel, so each axis equals what those kernels write.
__global__ __launch_bounds__(256) void mx_quant_weight_dual_kernel(const uint16_t* w, int M, int N, uint8_t* col_data,
                                                                   uint8_t* col_scale, uint8_t* row_data,
                                                                   uint8_t* row_scale) {
  const int g = blockIdx.z, mb = blockIdx.y;
  const int n = blockIdx.x * 256 + threadIdx.x;
  const bool live = n < N;  // N % 32 == 0: a half-wave is all live or all dead
  const int64_t base = ((int64_t)g * M + mb * 32) * N;
  float v[32];
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    v[i] = live ? bf16_to_f32(w[base + (int64_t)i * N + n]) : 0.0f;
    amax = fmaxf(amax, fabsf(v[i]));
  }
  if (col_data != nullptr) {
    const uint32_t code = mx_scale_code(amax);
    if (live) {
#pragma unroll
      for (int i = 0; i < 32; ++i) col_data[base + (int64_t)i * N + n] = (uint8_t)f32_to_e4m3_inrange(mx_apply_inv_scale(v[i], code));
      col_scale[(((int64_t)g * (M / 64) + mb / 2) * N + n) * 2 + (mb & 1)] = (uint8_t)code;
    }
  }
  if (row_data != nullptr) {
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      float a = fabsf(v[i]);
#pragma unroll
      for (int m = 16; m >= 1; m >>= 1) a = fmaxf(a, __shfl_xor(a, m, 64));
      const uint32_t code = mx_scale_code(a);
      if (live) {
        row_data[base + (int64_t)i * N + n] = (uint8_t)f32_to_e4m3_inrange(mx_apply_inv_scale(v[i], code));
        if ((threadIdx.x & 31) == 0) row_scale[((int64_t)g * M + mb * 32 + i) * (N / 32) + n / 32] = (uint8_t)code;
      }
    }
  }
}

extern "C" int mi355moe_mx_quantize_weight(const uint16_t* w, int32_t groups, int32_t rows, int32_t cols,
                                           uint8_t* col_data, uint8_t* col_scale, uint8_t* row_data,
                                           uint8_t* row_scale, void* stream) {
  if (groups <= 0 || groups > 65535 || rows <= 0 || cols <= 0 || rows % 64 || cols % 64) return MI355MOE_EINVAL;
  if (w == nullptr || (col_data == nullptr) != (col_scale == nullptr) || (row_data == nullptr) != (row_scale == nullptr))
    return MI355MOE_EINVAL;
  if (col_data == nullptr && row_data == nullptr) return MI355MOE_EINVAL;
  if (!mi355_mx_weight_prep_enabled()) return MI355MOE_EUNSUPPORTED;
  hipLaunchKernelGGL(mx_quant_weight_dual_kernel, dim3((cols + 255) / 256, rows / 32, groups), dim3(256), 0,
                     (hipStream_t)stream, w, rows, cols, col_data, col_scale, row_data, row_scale);
  return hipGetLastError() == hipSuccess ? MI355MOE_OK : MI355MOE_ELAUNCH;
}

// ---- routed-row MX quantisation (MXFP8 backward) ---------------------------------------------
// One workgroup per (32-row block of a group, 256 columns); thread c owns column c0 + c, as in the
// dual weight kernel: the column block is in-thread, each row block a 32-lane reduction.
template <int MODE>
MI355_DEV float mx_q_value(const MxGroupedQuant& q, int64_t r, int c) {
  if constexpr (MODE == MX_Q_BF16) {
    const int64_t sr = q.gather != nullptr ? (int64_t)(q.gather[r] / q.gather_div) : r;
    return bf16_to_f32(q.src[sr * q.src_ld + c]);
  } else if constexpr (MODE == MX_Q_SWIGLU) {
    const int I = q.C;
    const float gte = bf16_to_f32(q.U[r * 2 * I + c]);
    const float up = bf16_to_f32(q.U[r * 2 * I + I + c]);
    return gte / (1.0f + __expf(-gte)) * up;
  } else {
    const int I = q.C / 2;
    const int cc = c < I ? c : c - I;
    const float g = bf16_to_f32(q.U[r * 2 * I + cc]);
    const float a = bf16_to_f32(q.da[r * I + cc]);
    const float s = 1.0f / (1.0f + __expf(-g));
    if (c < I) return a * bf16_to_f32(q.U[r * 2 * I + I + cc]) * s * (1.0f + g * (1.0f - s));
    return a * (g * s);
  }
}

template <int MODE>
__global__ __launch_bounds__(256) void mx_quant_grouped_kernel(MxGroupedQuant q) {
  const int bi = blockIdx.y;
  if (bi >= q.block_prefix[q.G]) return;
  int lo = 0, hi = q.G - 1;
  while (lo < hi) {  // largest g with block_prefix[g] <= bi
    const int mid = (lo + hi + 1) >> 1;
    if (q.block_prefix[mid] <= bi) lo = mid; else hi = mid - 1;
  }
  const int g = lo;
  const int64_t start = g == 0 ? 0 : q.group_list[g - 1];
  const int64_t n = q.group_list[g] - start;
  const int b = bi - q.block_prefix[g];
  const int64_t r0 = start + 32 * (int64_t)b;
  const int nrows = (int)((n - 32 * (int64_t)b) < 32 ? (n - 32 * (int64_t)b) : 32);
  const int c = blockIdx.x * 256 + threadIdx.x;
  const bool live = c < q.C;  // C % 32 == 0: half-waves are uniformly live or dead
  float v[32];
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    v[i] = (live && i < nrows) ? mx_q_value<MODE>(q, r0 + i, c) : 0.0f;
    amax = fmaxf(amax, fabsf(v[i]));
  }
  if (q.col_data != nullptr && live) {
    const uint32_t code = mx_scale_code(amax);
#pragma unroll
    for (int i = 0; i < 32; ++i)
      if (i < nrows) q.col_data[(r0 + i) * q.C + c] = (uint8_t)f32_to_e4m3_inrange(mx_apply_inv_scale(v[i], code));
    uint8_t* pair = q.col_scale + ((start / 64 + g + b / 2) * q.C + c) * 2;
    pair[b & 1] = (uint8_t)code;
    if (!(b & 1) && 32 * (int64_t)(b + 1) >= n) pair[1] = 0;  // the pair's second block lies past the group
  }
  if (q.row_data != nullptr) {
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      float a = fabsf(v[i]);
#pragma unroll
      for (int m = 16; m >= 1; m >>= 1) a = fmaxf(a, __shfl_xor(a, m, 64));
      const uint32_t code = mx_scale_code(a);
      if (live && i < nrows) {
        q.row_data[(r0 + i) * q.C + c] = (uint8_t)f32_to_e4m3_inrange(mx_apply_inv_scale(v[i], code));
        if ((threadIdx.x & 31) == 0) q.row_scale[(r0 + i) * q.row_scale_ld + c / 32] = (uint8_t)code;
      }
    }
  }
}

int mi355_mx_quant_grouped(const MxGroupedQuant& q, hipStream_t st) {
  if (q.R <= 0) return MI355MOE_OK;
  if (q.C <= 0 || q.C % 32 || q.G <= 0 || q.group_list == nullptr || q.block_prefix == nullptr) return MI355MOE_EINVAL;
  const int64_t max_blocks = (q.R + 31) / 32 + q.G;  // the device-planned count never exceeds this
  if (max_blocks > 65535) return MI355MOE_EUNSUPPORTED;
  const dim3 grid((unsigned)((q.C + 255) / 256), (unsigned)max_blocks);
  switch (q.mode) {
    case MX_Q_BF16: hipLaunchKernelGGL(mx_quant_grouped_kernel<MX_Q_BF16>, grid, dim3(256), 0, st, q); break;
    case MX_Q_SWIGLU: hipLaunchKernelGGL(mx_quant_grouped_kernel<MX_Q_SWIGLU>, grid, dim3(256), 0, st, q); break;
    case MX_Q_SWIGLU_BWD:
      hipLaunchKernelGGL(mx_quant_grouped_kernel<MX_Q_SWIGLU_BWD>, grid, dim3(256), 0, st, q);
      break;
    default: return MI355MOE_EINVAL;
  }
  return hipGetLastError() == hipSuccess ? MI355MOE_OK : MI355MOE_ELAUNCH;
}

// ---- MX weight re-layout: [G, K, N] (+ col_scale [G, K/64, N, 2]) -> [G, N, K] (+ [G, N, ld]) ----
// One 64 (K) x 64 (N) byte tile per workgroup, transposed through LDS.
__global__ __launch_bounds__(256) void mx_weight_to_eoi_kernel(const uint8_t* src, int K, int N, uint8_t* dst) {
  __shared__ uint8_t tile[64][64 + 4];
  const int g = blockIdx.z, k0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
  const uint8_t* s = src + (int64_t)g * K * N;
  for (int i = threadIdx.x; i < 64 * 64; i += 256) {
    const int kk = i / 64, nn = i % 64;
    tile[kk][nn] = (k0 + kk < K && n0 + nn < N) ? s[(int64_t)(k0 + kk) * N + n0 + nn] : 0;
  }
  __syncthreads();
  uint8_t* d = dst + (int64_t)g * N * K;
  for (int i = threadIdx.x; i < 64 * 64; i += 256) {
    const int nn = i / 64, kk = i % 64;
    if (k0 + kk < K && n0 + nn < N) d[(int64_t)(n0 + nn) * K + k0 + kk] = tile[kk][nn];
  }
}

__global__ __launch_bounds__(256) void mx_weight_scale_to_eoi_kernel(const uint8_t* col_scale, int G, int K, int N,
                                                                     int64_t ld, uint8_t* scale) {
  const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= (int64_t)G * N * ld) return;
  const int64_t c = id % ld, gn = id / ld;
  const int n = (int)(gn % N), g = (int)(gn / N);
  uint8_t v = 0;
  if (c < K / 32) v = col_scale[(((int64_t)g * (K / 64) + c / 2) * N + n) * 2 + (c & 1)];
  scale[id] = v;
}

extern "C" int64_t mi355moe_mx_weight_scale_ld(int32_t kdim) { return kdim > 0 ? mi355_mx_scale_ld(kdim) : 0; }

extern "C" int mi355moe_mx_weight_to_eoi(const uint8_t* col_data, const uint8_t* col_scale, int32_t groups,
                                         int32_t kdim, int32_t cols, uint8_t* data, uint8_t* scale, void* stream) {
  if (groups <= 0 || kdim <= 0 || cols <= 0 || kdim % 64 || groups > 65535) return MI355MOE_EINVAL;
  if (col_data == nullptr || col_scale == nullptr || data == nullptr || scale == nullptr) return MI355MOE_EINVAL;
  hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL(mx_weight_to_eoi_kernel, dim3((cols + 63) / 64, (kdim + 63) / 64, groups), dim3(256), 0, st,
                     col_data, kdim, cols, data);
  if (hipGetLastError() != hipSuccess) return MI355MOE_ELAUNCH;
  const int64_t ld = mi355_mx_scale_ld(kdim);
  const int64_t n = (int64_t)groups * cols * ld;
  hipLaunchKernelGGL(mx_weight_scale_to_eoi_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, col_scale,
                     groups, kdim, cols, ld, scale);
  return hipGetLastError() == hipSuccess ? MI355MOE_OK : MI355MOE_ELAUNCH;
}

// ---- gate/up interleave of the GMM1 weight (layout EIO_GU) ------------------------------------
// One thread per 16-byte chunk of a row: a chunk lies inside one 64-column block (64 columns are
// >= 64 bytes), so it moves whole to gate_up_col of its first column.
__global__ __launch_bounds__(256) void interleave_gate_up_kernel(const uint4* src, int64_t rows, int I, int elem_bytes,
                                                                 uint4* dst) {
  const int64_t chunks_per_row = (int64_t)2 * I * elem_bytes / 16;
  const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= rows * chunks_per_row) return;
  const int64_t row = id / chunks_per_row;
  const int chunk = (int)(id - row * chunks_per_row);
  const int col = chunk * 16 / elem_bytes;
  const int to = gate_up_col(col, I, 1) * elem_bytes / 16;
  dst[row * chunks_per_row + to] = src[id];
}

extern "C" int mi355moe_interleave_gate_up(const void* src, int64_t rows, int32_t intermediate_size,
                                           int32_t elem_bytes, void* dst, void* stream) {
  if (rows < 0 || intermediate_size <= 0 || intermediate_size % 128 || (elem_bytes != 1 && elem_bytes != 2))
    return MI355MOE_EINVAL;
  if (rows == 0) return MI355MOE_OK;
  if (src == nullptr || dst == nullptr || ((uintptr_t)src | (uintptr_t)dst) % 16) return MI355MOE_EINVAL;
  const int64_t row_bytes = (int64_t)2 * intermediate_size * elem_bytes;
  const char* s = (const char*)src;
  const char* d = (const char*)dst;
  if (s < d + rows * row_bytes && d < s + rows * row_bytes) return MI355MOE_EINVAL;  // overlap
  const int64_t n = rows * (row_bytes / 16);
  if ((n + 255) / 256 > INT32_MAX) return MI355MOE_EINVAL;
  hipLaunchKernelGGL(interleave_gate_up_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     (const uint4*)src, rows, intermediate_size, elem_bytes, (uint4*)dst);
  return hipGetLastError() == hipSuccess ? MI355MOE_OK : MI355MOE_ELAUNCH;
}
