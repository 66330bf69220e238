// C-ABI entry points that chain the kernels: router projection, grouped GEMM, and the MegaMoE
// expert forward at EP=1 (dispatch -> [MX quant] -> GMM1+SwiGLU[+MX requant] -> GMM2 -> combine).
// All launches are enqueued on the caller's stream; nothing synchronises the host.
#include "common.h"
#include "gemm.h"
#include "decode_prep.h"
#include <cmath>
#include <algorithm>
#include <mutex>
#include "../../include/mi355moe.h"

static size_t al256(size_t v) { return (v + 255) & ~(size_t)255; }

extern "C" int mi355moe_abi_version(void) { return MI355MOE_ABI_VERSION; }
extern "C" int mi355moe_features(void) {
  return (mi355_mx_eoi_enabled() ? MI355MOE_FEATURE_MX_EOI : 0) |
         (mi355_numerics_options_enabled() ? MI355MOE_FEATURE_NUMERICS : 0) |
         (mi355_small_tiles_enabled() ? MI355MOE_FEATURE_DECODE_TILES : 0) |
         (mi355_backward_enabled() ? MI355MOE_FEATURE_BACKWARD : 0) |
         (mi355_route_grad_enabled() ? MI355MOE_FEATURE_ROUTE_GRAD : 0) |
         (mi355_mx_weight_prep_enabled() ? MI355MOE_FEATURE_MX_WEIGHT_PREP : 0) |
         (mi355_mx_backward_enabled() ? MI355MOE_FEATURE_MX_BACKWARD : 0);
}

bool mi355_gg_variant_valid(int variant) {
  return variant == MI355_GG_VARIANT_DEFAULT || variant == MI355_GG_VARIANT_PP || variant == MI355_GG_VARIANT_W4;
}

// ---------------------------------------------------------------------------------------------
// Router projection
// ---------------------------------------------------------------------------------------------
__global__ void mask_to_ids_kernel(const uint8_t* mask, int64_t T, int32_t* ids) {
  int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t < T) ids[t] = mask[t] ? 1 : 0;
}

// One group of `rows` rows: its group_list and its tile plan at tile height bm, in one launch.
__global__ void single_group_plan_kernel(int64_t rows, int bm, int64_t* group_list, int32_t* tile_prefix) {
  group_list[0] = rows;
  tile_prefix[0] = 0;
  tile_prefix[1] = (int32_t)((rows + bm - 1) / bm);
}

// Decode-sized batches (few tokens) project on the 64-row tiles (two workgroups per CU): a 256-row
// tile would be mostly padding.
static bool router_small(int64_t T) { return T <= 256; }

// Split-K factor of the router projection: one work item per workgroup slot (one per CU for the
// 256 x 256 tiles, where T=8192 gives only 32 tiles; two per CU for the 64-row tiles), each split at
// least 4 K stages of 32. More items would add a second round and partial tiles to write and read
// back. Deterministic: split s writes its own partial buffer and the reduction adds them in a fixed
// order.
static int router_splits(int64_t T, int H, int E) {
  const int bm = mi355_gg_bm(router_small(T));
  const int64_t tiles = ((T + bm - 1) / bm) * ((E + 255) / 256);
  const int kst = H / 32;
  const int target = mi355_num_cus() * (router_small(T) ? 2 : 1);
  int best = 1;
  for (int s = 1; s <= kst / 4; ++s) {
    if (kst % s) continue;
    best = s;
    if (tiles * s >= target) break;
  }
  return best;
}

extern "C" size_t mi355moe_gate_logits_workspace_size(int64_t num_tokens, int32_t hidden_size, int32_t num_experts) {
  // ids[T] + mapping[T] + gather[T] + group_list[2] + tile_prefix[3] + dispatch workspace + partials
  size_t base = al256((size_t)num_tokens * 4) * 3 + 256 + 256 + mi355moe_dispatch_workspace_size(num_tokens, 1, 2);
  if (hidden_size <= 0 || num_experts <= 0) return base;
  int s = router_splits(num_tokens, hidden_size, num_experts);
  return base + (s > 1 ? al256((size_t)s * num_tokens * num_experts * 4) : 0);
}

// logits[t, e] = sum over s of partial[s, row(t), e] (row(t) = routed row of token t), in a fixed
// order: a workgroup takes 64 elements; its 4 waves add the splits s = w, w + 4, w + 8, ... in
// ascending order, and wave 0 adds the four sums in wave order (so each load chain is a quarter of
// the splits long).
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* partial, int splits, int64_t split_stride,
                                                            int64_t T, int E, const int32_t* row_of_token_inv,
                                                            float* out) {
  __shared__ float sums[4][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t i = (int64_t)blockIdx.x * 64 + lane;
  const bool live = i < T * E;
  float acc = 0.0f;
  if (live) {
    if (w < splits) acc = partial[w * split_stride + i];
    for (int s = w + 4; s < splits; s += 4) acc += partial[s * split_stride + i];
  }
  sums[w][lane] = acc;
  __syncthreads();
  if (w != 0 || !live) return;
  float total = sums[0][lane];
  for (int q = 1; q < 4 && q < splits; ++q) total += sums[q][lane];
  const int64_t r = i / E;
  const int e = (int)(i - r * E);
  const int64_t orow = row_of_token_inv ? (int64_t)row_of_token_inv[r] : r;
  out[orow * E + e] = total;
}

extern "C" int mi355moe_gate_logits(const uint16_t* x, int64_t num_tokens, int32_t hidden_size, const uint16_t* w,
                                    const uint16_t* w_vision, const uint8_t* image_mask, int32_t num_experts,
                                    float* logits, void* workspace, size_t workspace_size, void* stream) {
  if (num_tokens < 0 || hidden_size <= 0 || num_experts <= 0 || num_experts > 4096) return MI355MOE_EINVAL;
  if (hidden_size % 128) return MI355MOE_EUNSUPPORTED;
  if (num_tokens == 0) return MI355MOE_OK;
  if (x == nullptr || w == nullptr || logits == nullptr) return MI355MOE_EINVAL;
  if (num_tokens > INT32_MAX / 2) return MI355MOE_EINVAL;
  const bool dual = w_vision != nullptr && image_mask != nullptr;
  if (workspace == nullptr ||
      workspace_size < mi355moe_gate_logits_workspace_size(num_tokens, hidden_size, num_experts))
    return -4;
  hipStream_t st = (hipStream_t)stream;
  char* ws = (char*)workspace;
  int32_t* ids = (int32_t*)ws;
  int32_t* mapping = (int32_t*)(ws + al256((size_t)num_tokens * 4));
  int32_t* gather = (int32_t*)(ws + 2 * al256((size_t)num_tokens * 4));
  int64_t* group_list = (int64_t*)(ws + 3 * al256((size_t)num_tokens * 4));
  int32_t* tile_prefix = (int32_t*)(ws + 3 * al256((size_t)num_tokens * 4) + 256);
  void* dws = ws + 3 * al256((size_t)num_tokens * 4) + 512;
  float* partial = (float*)(ws + 3 * al256((size_t)num_tokens * 4) + 512 +
                            mi355moe_dispatch_workspace_size(num_tokens, 1, 2));
  const int splits = router_splits(num_tokens, hidden_size, num_experts);
  int rc;
  GGParams p = {};
  p.A = (const uint8_t*)x;
  p.lda_bytes = (int64_t)hidden_size * 2;
  p.B = (const uint8_t*)w;
  p.b_row_bytes = (int64_t)hidden_size * 2;
  p.K = hidden_size;
  p.N = num_experts;
  p.Ntot = num_experts;
  p.n_tiles = (num_experts + mi355_gg_bn() - 1) / mi355_gg_bn();
  p.C = splits > 1 ? (void*)partial : (void*)logits;
  p.ldc = num_experts;
  p.k_splits = splits;
  p.c_split_stride = (int64_t)num_tokens * num_experts;
  if (dual) {
    hipLaunchKernelGGL(mask_to_ids_kernel, dim3((unsigned)((num_tokens + 255) / 256)), dim3(256), 0, st, image_mask,
                       num_tokens, ids);
    rc = mi355_dispatch_enqueue(ids, MI355MOE_IDS_INT32, num_tokens, 1, 2, nullptr, nullptr, group_list, mapping,
                                gather, nullptr, dws, st);
    if (rc) return rc;
    p.G = 2;
    p.b_group_stride = (int64_t)((const char*)w_vision - (const char*)w);
    p.a_row_index = gather;
    p.a_row_div = 1;
    // with split-K the partials stay in routed order and the reduction scatters them
    p.c_row_index = splits > 1 ? nullptr : gather;
  } else {
    p.G = 1;
    p.a_row_div = 1;
  }
  p.group_list = group_list;
  p.tile_prefix = tile_prefix;
  const bool small = router_small(num_tokens);
  if (dual) {
    rc = mi355_plan_tiles(group_list, p.G, tile_prefix, st, small);
    if (rc) return rc;
  } else {
    hipLaunchKernelGGL(single_group_plan_kernel, dim3(1), dim3(1), 0, st, num_tokens, mi355_gg_bm(small), group_list,
                       tile_prefix);
  }
  rc = mi355_grouped_gemm(p, false, false, EPI_STORE_F32, st, small);
  if (rc || splits == 1) return rc;
  const int64_t n = num_tokens * num_experts;
  hipLaunchKernelGGL(splitk_reduce_kernel, dim3((unsigned)((n + 63) / 64)), dim3(256), 0, st, partial, splits,
                     p.c_split_stride, num_tokens, num_experts, dual ? gather : nullptr, logits);
  return hipGetLastError() == hipSuccess ? MI355MOE_OK : MI355MOE_ELAUNCH;
}

// ---------------------------------------------------------------------------------------------
// Plain grouped GEMM (bf16 in/out)
// ---------------------------------------------------------------------------------------------
extern "C" size_t mi355moe_grouped_gemm_workspace_size(int32_t num_groups) {
  return al256((size_t)(num_groups + 1) * 4);
}

// Argument checks of the bf16 grouped GEMM shared by both entry points (workspace aside).
static int grouped_gemm_bf16_check(const uint16_t* x, int64_t rows, int32_t kdim, const uint16_t* w, int32_t layout,
                                   int32_t num_groups, int32_t ndim, const int64_t* group_list, uint16_t* out,
                                   int32_t gemm_variant) {
  if (!mi355_gg_variant_valid(gemm_variant)) return MI355MOE_EUNSUPPORTED;
  if (rows < 0 || kdim <= 0 || ndim <= 0 || num_groups <= 0 || num_groups > 4096) return MI355MOE_EINVAL;
  if (layout != MI355MOE_LAYOUT_EIO && layout != MI355MOE_LAYOUT_EOI) return MI355MOE_EINVAL;
  if (kdim % 64 || ndim % 8) return MI355MOE_EUNSUPPORTED;
  if (rows == 0) return MI355MOE_OK;
  if (x == nullptr || w == nullptr || group_list == nullptr || out == nullptr) return MI355MOE_EINVAL;
  return MI355MOE_OK;
}

// Plans the tiles into tile_prefix ([num_groups + 1] int32, fully written) and launches the GEMM.
static int grouped_gemm_bf16_launch(const uint16_t* x, int64_t rows, int32_t kdim, const uint16_t* w,
                                    int32_t layout, int32_t num_groups, int32_t ndim, const int64_t* group_list,
                                    uint16_t* out, int32_t gemm_variant, int32_t* tile_prefix, hipStream_t st) {
  GGParams p = {};
  p.variant = gemm_variant;
  p.rows_hint = rows;
  p.A = (const uint8_t*)x;
  p.lda_bytes = (int64_t)kdim * 2;
  p.a_bytes = rows * kdim * 2;
  p.a_row_div = 1;
  p.B = (const uint8_t*)w;
  p.b_group_stride = (int64_t)kdim * ndim * 2;
  p.b_row_bytes = layout == MI355MOE_LAYOUT_EOI ? (int64_t)kdim * 2 : (int64_t)ndim * 2;
  p.K = kdim;
  p.N = ndim;
  p.Ntot = ndim;
  p.n_tiles = (ndim + mi355_gg_bn() - 1) / mi355_gg_bn();
  p.G = num_groups;
  p.group_list = group_list;
  p.tile_prefix = tile_prefix;
  p.C = out;
  p.ldc = ndim;
  const bool small = mi355_use_small_tiles(rows, num_groups, gemm_variant);
  int rc = mi355_plan_tiles(group_list, num_groups, tile_prefix, st, small);
  if (rc) return rc;
  return mi355_grouped_gemm(p, false, layout == MI355MOE_LAYOUT_EIO, EPI_STORE_BF16, st, small);
}

extern "C" int mi355moe_grouped_gemm_bf16(const uint16_t* x, int64_t rows, int32_t kdim, const uint16_t* w,
                                          int32_t layout, int32_t num_groups, int32_t ndim,
                                          const int64_t* group_list, uint16_t* out, int32_t gemm_variant,
                                          void* workspace, size_t workspace_size, void* stream) {
  int rc = grouped_gemm_bf16_check(x, rows, kdim, w, layout, num_groups, ndim, group_list, out, gemm_variant);
  if (rc || rows == 0) return rc;
  if (workspace == nullptr || workspace_size < mi355moe_grouped_gemm_workspace_size(num_groups)) return -4;
  return grouped_gemm_bf16_launch(x, rows, kdim, w, layout, num_groups, ndim, group_list, out, gemm_variant,
                                  (int32_t*)workspace, (hipStream_t)stream);
}

// The no-allocation variant's tile plan: one array per GPU (its own copy at its own address),
// held until the process ends. Host code never passes `scratch` itself (its host-side name is not a
// device address); it uses the per-device address from hipGetSymbolAddress below.
static __device__ __align__(256) int32_t scratch[MI355MOE_NOALLOC_MAX_GROUPS + 1];
static constexpr int kMaxDevices = 64;
static void* g_scratch_ptr[kMaxDevices] = {};
static std::mutex g_scratch_mutex;

// The current device's address of `scratch`, looked up once per device with that device current.
static int32_t* scratch_on_current_device() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || ptr == nullptr) return nullptr;
    g_scratch_ptr[dev] = ptr;
  }
  return (int32_t*)g_scratch_ptr[dev];
}

extern "C" int mi355moe_grouped_gemm_bf16_noalloc(const uint16_t* x, int64_t rows, int32_t kdim, const uint16_t* w,
                                                  int32_t layout, int32_t num_groups, int32_t ndim,
                                                  const int64_t* group_list, uint16_t* out, int32_t gemm_variant,
                                                  void* stream) {
  if (num_groups > MI355MOE_NOALLOC_MAX_GROUPS) return MI355MOE_EWORKSPACE;
  int rc = grouped_gemm_bf16_check(x, rows, kdim, w, layout, num_groups, ndim, group_list, out, gemm_variant);
  if (rc || rows == 0) return rc;
  int32_t* plan = scratch_on_current_device();
  if (plan == nullptr) return MI355MOE_ELAUNCH;
  return grouped_gemm_bf16_launch(x, rows, kdim, w, layout, num_groups, ndim, group_list, out, gemm_variant, plan,
                                  (hipStream_t)stream);
}

extern "C" int mi355moe_grouped_gemm_mxfp8(const uint8_t* xq, const uint8_t* x_scale, int64_t rows, int32_t kdim,
                                           const uint8_t* col_data, const uint8_t* col_scale, int32_t layout,
                                           int32_t num_groups, int32_t ndim, const int64_t* group_list, uint16_t* out,
                                           int32_t gemm_variant, void* workspace, size_t workspace_size,
                                           void* stream) {
  if (!mi355_gg_variant_valid(gemm_variant)) return MI355MOE_EUNSUPPORTED;
  if (rows < 0 || kdim <= 0 || ndim <= 0 || num_groups <= 0 || num_groups > 4096) return MI355MOE_EINVAL;
  if (layout != MI355MOE_LAYOUT_EIO && layout != MI355MOE_LAYOUT_EOI) return MI355MOE_EINVAL;
  const bool eoi = layout == MI355MOE_LAYOUT_EOI;
  if (eoi && !mi355_mx_eoi_enabled()) return MI355MOE_EUNSUPPORTED;
  // the GEMM fetches 16 activation scale codes per row at a time: K/32 must be a multiple of 16
  if (kdim % 512 || ndim % 16) return MI355MOE_EUNSUPPORTED;
  if (rows == 0) return MI355MOE_OK;
  if (xq == nullptr || x_scale == nullptr || col_data == nullptr || col_scale == nullptr || group_list == nullptr ||
      out == nullptr)
    return MI355MOE_EINVAL;
  if (workspace == nullptr || workspace_size < mi355moe_grouped_gemm_workspace_size(num_groups)) return -4;
  hipStream_t st = (hipStream_t)stream;
  GGParams p = {};
  p.variant = gemm_variant;
  p.A = xq;
  p.lda_bytes = kdim;
  p.a_bytes = rows * kdim;
  p.a_row_div = 1;
  p.a_scale = x_scale;
  p.a_scale_ld = kdim / 32;
  p.B = col_data;
  p.b_group_stride = (int64_t)kdim * ndim;
  p.b_row_bytes = eoi ? kdim : ndim;
  p.b_scale = col_scale;
  p.b_scale_ld = mi355_mx_scale_ld(kdim);
  p.b_scale_group_stride = eoi ? (int64_t)ndim * p.b_scale_ld : (int64_t)(kdim / 64) * ndim * 2;
  p.K = kdim;
  p.N = ndim;
  p.Ntot = ndim;
  p.n_tiles = (ndim + mi355_gg_bn() - 1) / mi355_gg_bn();
  p.G = num_groups;
  p.group_list = group_list;
  p.tile_prefix = (int32_t*)workspace;
  p.C = out;
  p.ldc = ndim;
  const bool small = mi355_use_small_tiles(rows, num_groups, gemm_variant);
  int rc = mi355_plan_tiles(group_list, num_groups, (int32_t*)workspace, st, small);
  if (rc) return rc;
  return mi355_grouped_gemm(p, true, !eoi, EPI_STORE_BF16, st, small);
}

// ---------------------------------------------------------------------------------------------
// MegaMoE expert forward
// ---------------------------------------------------------------------------------------------
struct FwdLayout {
  size_t dispatch, counts, group_list, mapping, gather, tile_prefix, act, act_scale, act_f32, y, xq, xs, tok_codes,
      total;
};

static FwdLayout fwd_layout(const MI355MoeForwardArgs& a) {
  FwdLayout L = {};
  const size_t T = (size_t)a.num_tokens, K = (size_t)a.top_k, E = (size_t)a.num_experts;
  const size_t H = (size_t)a.hidden_size, I = (size_t)a.intermediate_size, R = T * K;
  const bool mx = a.precision == MI355MOE_PRECISION_MXFP8;
  size_t off = 0;
  auto take = [&](size_t bytes) { size_t o = off; off += al256(bytes); return o; };
  L.dispatch = take(mi355moe_dispatch_workspace_size(a.num_tokens, a.top_k, a.num_experts));
  L.counts = take(E * 4);
  L.group_list = take(E * 8);
  L.mapping = take(R * 4);
  L.gather = take(R * 4);
  L.tile_prefix = take((E + 1) * 4);
  L.act = take(R * I * (mx ? 1 : 2));
  L.act_scale = mx ? take(std::max(R * mi355_mx_scale_ld(I), R * (I / 32) + 512)) : 0;
  L.act_f32 = mx ? take(R * I * 4) : 0;  // 8-wave MX path: fp32 SwiGLU output before its quantisation
  L.y = take(R * H * 2);
  L.xq = mx ? take(T * H) : 0;
  // MX token scales: [T, ld] for the 4-wave GEMM, or stage-major over the routed rows [H/128][R][4]
  L.xs = mx ? take(std::max(T * mi355_mx_scale_ld(H), R * (H / 32) + 512)) : 0;
  L.tok_codes = mx ? take(T * (H / 32)) : 0;  // per-token codes before they go to the routed rows' planes
  L.total = off;
  return L;
}

static int validate_fwd(const MI355MoeForwardArgs& a) {
  if (a.num_tokens < 0 || a.hidden_size <= 0 || a.intermediate_size <= 0 || a.num_experts <= 0 || a.top_k <= 0)
    return MI355MOE_EINVAL;
  if (a.num_experts > 4096 || a.top_k > 64 || a.top_k > a.num_experts) return MI355MOE_EINVAL;
  if (a.ids_dtype != MI355MOE_IDS_INT32 && a.ids_dtype != MI355MOE_IDS_INT64) return MI355MOE_EINVAL;
  if (a.precision != MI355MOE_PRECISION_BF16 && a.precision != MI355MOE_PRECISION_MXFP8) return MI355MOE_EINVAL;
  if (!mi355_gg_variant_valid(a.gemm_variant)) return MI355MOE_EUNSUPPORTED;
  if (a.weight_layout != MI355MOE_LAYOUT_EIO && a.weight_layout != MI355MOE_LAYOUT_EOI &&
      a.weight_layout != MI355MOE_LAYOUT_EIO_GU)
    return MI355MOE_EINVAL;
  if (a.num_tokens * (int64_t)a.top_k > INT32_MAX) return MI355MOE_EINVAL;
  if (a.numerics_flags & ~(MI355MOE_NUMERICS_CLAMP_AFTER_SILU | MI355MOE_NUMERICS_PROBS_BEFORE_FC2))
    return MI355MOE_EINVAL;
  if (!(a.swiglu_limit >= 0.0f) || a.swiglu_limit == INFINITY) return MI355MOE_EINVAL;  // NaN, negative, inf
  const bool options = a.swiglu_limit > 0.0f || (a.numerics_flags & MI355MOE_NUMERICS_PROBS_BEFORE_FC2);
  if (options && a.precision == MI355MOE_PRECISION_MXFP8) return MI355MOE_EINVAL;  // module.py:132
  if (options && !mi355_numerics_options_enabled()) return MI355MOE_EUNSUPPORTED;
  if (a.precision == MI355MOE_PRECISION_MXFP8) {
    if (a.weight_layout == MI355MOE_LAYOUT_EOI && !mi355_mx_eoi_enabled()) return MI355MOE_EUNSUPPORTED;
    if (a.hidden_size % 128 || a.intermediate_size % 128) return MI355MOE_EUNSUPPORTED;
  } else {
    if (a.hidden_size % 64 || a.intermediate_size % 64) return MI355MOE_EUNSUPPORTED;
  }
  // GMM1 produces I columns in 128-column tiles; GMM2 produces H columns in 256-column tiles.
  if (a.intermediate_size % 128 || a.hidden_size % 8) return MI355MOE_EUNSUPPORTED;
  if (a.num_tokens > 0) {
    if (a.hidden == nullptr || a.topk_ids == nullptr || a.topk_weights == nullptr || a.w1 == nullptr ||
        a.w2 == nullptr || a.out == nullptr)
      return MI355MOE_EINVAL;
    if (a.precision == MI355MOE_PRECISION_MXFP8 && (a.w1_scale == nullptr || a.w2_scale == nullptr))
      return MI355MOE_EINVAL;
  }
  return MI355MOE_OK;
}

extern "C" size_t mi355moe_moe_forward_workspace_size(const MI355MoeForwardArgs* args) {
  if (args == nullptr || validate_fwd(*args) != MI355MOE_OK) return 0;
  return fwd_layout(*args).total;
}

extern "C" int mi355moe_moe_forward(const MI355MoeForwardArgs* args, void* workspace, size_t workspace_size,
                                    void* stream) {
  if (args == nullptr) return MI355MOE_EINVAL;
  const MI355MoeForwardArgs& a = *args;
  int rc = validate_fwd(a);
  if (rc) return rc;
  if (a.num_tokens == 0) return MI355MOE_OK;
  FwdLayout L = fwd_layout(a);
  if (workspace == nullptr || workspace_size < L.total) return -4;
  if (a.num_stage_events < 0 || a.num_stage_events > 5 || (a.num_stage_events > 0 && a.stage_events == nullptr))
    return MI355MOE_EINVAL;
  hipStream_t st = (hipStream_t)stream;
  auto mark = [&](int i) {
    if (i < a.num_stage_events && a.stage_events[i] != nullptr) hipEventRecord((hipEvent_t)a.stage_events[i], st);
  };
  mark(0);
  char* ws = (char*)workspace;
  const int64_t T = a.num_tokens;
  const int K = a.top_k, E = a.num_experts, H = a.hidden_size, I = a.intermediate_size;
  const bool mx = a.precision == MI355MOE_PRECISION_MXFP8;
  const bool eoi = a.weight_layout == MI355MOE_LAYOUT_EOI;

  int32_t* counts = (int32_t*)(ws + L.counts);
  int64_t* group_list = (int64_t*)(ws + L.group_list);
  int32_t* mapping = (int32_t*)(ws + L.mapping);
  int32_t* gather = (int32_t*)(ws + L.gather);
  int32_t* tile_prefix = (int32_t*)(ws + L.tile_prefix);
  // decode shapes (few routed rows per expert) use the 64-row tiles; the dispatch scan writes their plan
  const bool small = mi355_use_small_tiles(T * K, E, a.gemm_variant);
  const uint8_t* a1 = (const uint8_t*)a.hidden;
  // MX on the 8-wave GEMM: activation scales stage-major (one 4-byte copy per row and 128-K stage);
  // the 64-row tiles read row-major scales and a tile plan in 64-row units
  const bool pp_mx = mx && !eoi && !small &&
                     mi355_gg_pp_usable(a.gemm_variant, true, true, H, E, T * H, (int64_t)H * 2 * I) &&
                     mi355_gg_pp_usable(a.gemm_variant, true, true, I, E, T * K * I, (int64_t)I * H);
  // decode: the dispatch and the token quantisation in one launch
  const bool one_launch = small && mi355_decode_prep_enabled() && dprep::applies(T * K, E);
  if (one_launch) {
    dprep::Args d = {};
    d.ids = a.topk_ids;
    d.slots = T * K;
    d.E = E;
    d.counts = counts;
    d.group_list = group_list;
    d.mapping = mapping;
    d.gather = gather;
    d.error_flag = a.error_flag;
    d.tile_prefix = tile_prefix;
    d.bm = mi355_gg_bm(true);
    if (mx) {
      d.x = a.hidden;
      d.rows = T;
      d.cols = H;
      d.q = (uint8_t*)(ws + L.xq);
      d.scale = (uint8_t*)(ws + L.xs);
      d.scale_ld = mi355_mx_scale_ld(H);
    }
    rc = mi355_decode_prep_enqueue(d, a.ids_dtype, st);
  } else {
    rc = mi355_dispatch_plan_enqueue(a.topk_ids, a.ids_dtype, T, K, E, counts, group_list, mapping, gather,
                                     a.error_flag, ws + L.dispatch, tile_prefix, mi355_gg_bm(small), st);
  }
  if (rc) return rc;
  if (mx && one_launch) {
    a1 = (const uint8_t*)(ws + L.xq);
  } else if (mx) {
    // with the 8-wave GEMM the token scales go to each token's routed rows (read in tile order)
    if (pp_mx)
      rc = mi355_mx_quant_tokens_to_planes(a.hidden, T, H, (uint8_t*)(ws + L.xq), (uint8_t*)(ws + L.tok_codes), gather,
                                           K, group_list, E, (uint8_t*)(ws + L.xs), T * K * 4, st);
    else
      rc = mi355_mx_quant_rows(a.hidden, T, H, (uint8_t*)(ws + L.xq), (uint8_t*)(ws + L.xs), mi355_mx_scale_ld(H),
                               st);
    if (rc) return rc;
    a1 = (const uint8_t*)(ws + L.xq);
  }
  mark(1);
  const int esize = mx ? 1 : 2;
  // GMM1: [R, H] x [H, 2I] -> SwiGLU -> act [R, I]
  GGParams p1 = {};
  p1.variant = a.gemm_variant;
  p1.rows_hint = T * K;
  p1.A = a1;
  p1.lda_bytes = (int64_t)H * esize;
  p1.a_bytes = T * H * esize;
  p1.a_row_index = gather;
  p1.a_row_div = K;
  p1.a_scale = mx ? (const uint8_t*)(ws + L.xs) : nullptr;
  p1.a_scale_ld = mi355_mx_scale_ld(H);
  p1.B = (const uint8_t*)a.w1;
  p1.b_group_stride = (int64_t)H * 2 * I * esize;
  p1.b_row_bytes = eoi ? (int64_t)H * esize : (int64_t)2 * I * esize;
  p1.b_scale = a.w1_scale;
  p1.b_scale_ld = mi355_mx_scale_ld(H);
  p1.b_scale_group_stride = eoi ? (int64_t)2 * I * p1.b_scale_ld : (int64_t)(H / 64) * 2 * I * 2;
  p1.K = H;
  p1.N = I;
  p1.Ntot = 2 * I;
  p1.n_tiles = I / 128;
  p1.G = E;
  p1.group_list = group_list;
  p1.tile_prefix = tile_prefix;
  p1.gate_up_interleaved = a.weight_layout == MI355MOE_LAYOUT_EIO_GU;
  p1.C = ws + L.act;
  p1.ldc = I;
  p1.c_scale = mx ? (uint8_t*)(ws + L.act_scale) : nullptr;
  p1.c_scale_ld = mi355_mx_scale_ld(I);
  if (pp_mx) {
    p1.a_scale_stage_stride = T * K * 4;
    p1.a_scale_routed = 1;
  }
  const bool before_fc2 = (a.numerics_flags & MI355MOE_NUMERICS_PROBS_BEFORE_FC2) != 0;
  p1.swiglu_limit = a.swiglu_limit;
  p1.swiglu_after_silu = (a.numerics_flags & MI355MOE_NUMERICS_CLAMP_AFTER_SILU) != 0;
  p1.row_prob = before_fc2 ? a.topk_weights : nullptr;
  if (pp_mx) {
    // SwiGLU output in fp32, then its MX quantisation into act (e4m3) and the code planes
    p1.C = ws + L.act_f32;
    p1.ldc = I;
    // the quantisation belongs to GMM2's stage (as the token quantisation precedes GMM1's), so the
    // GMM1 stage events bracket the GEMM kernel alone
    rc = mi355_grouped_gemm(p1, true, true, EPI_SWIGLU_F32, st, small);
    if (rc) return rc;
    mark(2);
    rc = mi355_mx_quant_act((const float*)(ws + L.act_f32), T * K, I, (uint8_t*)(ws + L.act),
                            (uint8_t*)(ws + L.act_scale), T * K * 4, st);
    if (rc) return rc;
  } else {
    rc = mi355_grouped_gemm(p1, mx, !eoi, mx ? EPI_SWIGLU_MX : EPI_SWIGLU_BF16, st, small);
    if (rc) return rc;
    mark(2);
  }
  // GMM2: [R, I] x [I, H] -> y [R, H] bf16
  GGParams p2 = {};
  p2.variant = a.gemm_variant;
  p2.rows_hint = T * K;
  p2.A = (const uint8_t*)(ws + L.act);
  p2.lda_bytes = (int64_t)I * esize;
  p2.a_bytes = T * K * I * esize;
  p2.a_row_div = 1;
  p2.a_scale = mx ? (const uint8_t*)(ws + L.act_scale) : nullptr;
  p2.a_scale_ld = mi355_mx_scale_ld(I);
  if (pp_mx) p2.a_scale_stage_stride = T * K * 4;
  p2.B = (const uint8_t*)a.w2;
  p2.b_group_stride = (int64_t)I * H * esize;
  p2.b_row_bytes = eoi ? (int64_t)I * esize : (int64_t)H * esize;
  p2.b_scale = a.w2_scale;
  p2.b_scale_ld = mi355_mx_scale_ld(I);
  p2.b_scale_group_stride = eoi ? (int64_t)H * p2.b_scale_ld : (int64_t)(I / 64) * H * 2;
  p2.K = I;
  p2.N = H;
  p2.Ntot = H;
  p2.n_tiles = (H + mi355_gg_bn() - 1) / mi355_gg_bn();
  p2.G = E;
  p2.group_list = group_list;
  p2.tile_prefix = tile_prefix;
  p2.C = ws + L.y;
  p2.ldc = H;
  rc = mi355_grouped_gemm(p2, mx, !eoi, EPI_STORE_BF16, st, small);
  if (rc) return rc;
  mark(3);
  // probabilities applied before FC2 are not applied again: the combine sums the K rows
  rc = mi355_unpermute_enqueue((const uint16_t*)(ws + L.y), mapping, before_fc2 ? nullptr : a.topk_weights, T, K, H,
                               a.out, st);
  mark(4);
  return rc;
}
