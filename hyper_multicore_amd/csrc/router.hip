// MegaGate route kernel for gfx950: fp32 scoring, correction bias (text / vision), optional
// group-limited selection, top-k with lowest-index tie-break, gather, renormalisation and scale.
//
// Semantics follow MegaGate._torch_forward (hyper_multicore/modules/mega_gate/module.py:189-227)
// and the native route pipeline order (ops/hyper_mega_gate/op_kernel/route_pipeline.h:73-562):
//   score   = softmax(l) | sigmoid(l) | sqrt(softplus(l))   (softplus: l>20 ? l : compensated log1p)
//   biased  = score + (mask[t] ? bias_vl : bias)
//   idx     = top-k of biased (group-limited when groups > 1)
//   w       = score[idx];  K>1: w = w / (sum_k w + 1e-20);  w = w * routed_scaling_factor
// One 64-lane wavefront owns one token row; expert e lives in lane e % 64, register slot e / 64.
// The selected experts are emitted in descending biased score, ties broken by lower expert id.
#pragma clang fp contract(off)
#include "common.h"
#include "detmath.h"
#include "features.h"
#include "../../include/mi355moe.h"

#define ROUTER_MAX_SLOTS 16  // E <= 1024
#define ROUTER_FAST_GROUPS 16  // group-limited routing with at most this many groups takes the fast path

MI355_DEV float score_fn(float l, int scoring) {
  if (scoring == MI355MOE_SCORE_SIGMOID) {
    return 1.0f / (1.0f + det_expf(-l));
  }
  // sqrt(softplus(l)) in the route pipeline's compensated order (route_pipeline.h:104-130)
  float e = det_expf(fminf(l, 20.0f));
  float u = e + 1.0f;
  float sp;
  if (u == 1.0f) {
    sp = e;
  } else {
    float ratio = e / (u - 1.0f);
    sp = det_logf(u) * ratio;
  }
  if (l > 20.0f) sp = l;
  return sqrtf(sp);
}

MI355_DEV void argmax_step(float& v, int& i, float ov, int oi) {
  const bool take = (ov > v) || (ov == v && oi < i);
  v = take ? ov : v;
  i = take ? oi : i;
}
template <int CTRL>
MI355_DEV void argmax_dpp(float& v, int& i) {
  const float ov = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
  const int oi = __builtin_amdgcn_mov_dpp(i, CTRL, 0xF, 0xF, false);
  argmax_step(v, i, ov, oi);
}
// (largest v, ties -> lowest i) over the wavefront, in every lane. The order is total, so the pairing
// pattern does not change the result: within each 16-lane row, DPP moves (lane ^ 1, lane ^ 2, the
// half-row mirror 7 - x, the row mirror 15 - x), then shuffles across rows (lane ^ 16, lane ^ 32).
MI355_DEV void wave_argmax(float& v, int& i) {
  argmax_dpp<0xB1>(v, i);   // quad_perm [1, 0, 3, 2]
  argmax_dpp<0x4E>(v, i);   // quad_perm [2, 3, 0, 1]
  argmax_dpp<0x141>(v, i);  // row_half_mirror
  argmax_dpp<0x140>(v, i);  // row_mirror
#pragma unroll
  for (int m = 16; m <= 32; m <<= 1) {
    const float ov = __shfl_xor(v, m, 64);
    const int oi = __shfl_xor(i, m, 64);
    argmax_step(v, i, ov, oi);
  }
}

// SL: per-lane expert slots compiled in (expert e lives in lane e % 64, slot e / 64); the smallest of
// 1, 2, 4, 8, 16 that holds E, so the unrolled per-slot loops carry no slots past E.
template <int SL>
__global__ __launch_bounds__(256) void mi355_route_kernel(MI355MoeRouteArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= a.num_tokens) return;
  const int E = a.num_experts;
  const int slots = (E + 63) >> 6;
  const float* lrow = a.logits + t * (int64_t)a.logits_row_stride;
  const float* bias = a.bias;
  if (a.image_mask != nullptr && a.bias_vl != nullptr && a.image_mask[t]) bias = a.bias_vl;

  float score[SL];
  float biased[SL];
  const float NEG_INF = -__builtin_inff();

  if (a.scoring == MI355MOE_SCORE_SOFTMAX) {
    float lv[SL];
    float mx = NEG_INF;
#pragma unroll
    for (int j = 0; j < SL; ++j) {
      int e = j * 64 + lane;
      lv[j] = (j < slots && e < E) ? lrow[e] : NEG_INF;
      mx = fmaxf(mx, lv[j]);
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) mx = fmaxf(mx, __shfl_xor(mx, m, 64));
    float part = 0.0f;
#pragma unroll
    for (int j = 0; j < SL; ++j) {
      int e = j * 64 + lane;
      if (j < slots && e < E) {
        lv[j] = det_expf(lv[j] - mx);
        part = part + lv[j];
      }
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) part = part + __shfl_xor(part, m, 64);
#pragma unroll
    for (int j = 0; j < SL; ++j) {
      int e = j * 64 + lane;
      score[j] = (j < slots && e < E) ? lv[j] / part : 0.0f;
    }
  } else {
#pragma unroll
    for (int j = 0; j < SL; ++j) {
      int e = j * 64 + lane;
      score[j] = (j < slots && e < E) ? score_fn(lrow[e], a.scoring) : 0.0f;
    }
  }
#pragma unroll
  for (int j = 0; j < SL; ++j) {
    int e = j * 64 + lane;
    bool valid = j < slots && e < E;
    biased[j] = valid ? score[j] + bias[e] : NEG_INF;
    if (valid && a.scores_out != nullptr) a.scores_out[t * (int64_t)E + e] = score[j];
  }

  // Group-limited selection (DeepSeek-V3 form): group score = sum of the two largest biased
  // scores in the group; keep the top `topk_groups` groups (ties -> lower group id).
  const int G = a.num_groups;
  const int S = E / G;
  if (G > 1 && G <= ROUTER_FAST_GROUPS && S <= 64 && 64 % S == 0 && E % 64 == 0) {
    // Groups of S | 64 experts: slot j of lanes q S .. q S + S - 1 holds group j (64 / S) + q, so the
    // top-2 reductions of all groups run at once (one independent chain per slot, xor steps inside
    // the S-lane segments); the group scores go through the wave's LDS row to every lane, and each
    // lane picks the top groups in registers (largest score, ties -> lower group id). The top-2
    // merge and the sum are those of the general path below, so the scores are the same.
    __shared__ float gscore[4][ROUTER_FAST_GROUPS];
    const int wave = threadIdx.x >> 6;
    float t1[SL], t2[SL];
#pragma unroll
    for (int j = 0; j < SL; ++j) {
      t1[j] = j < slots ? biased[j] : NEG_INF;
      t2[j] = NEG_INF;
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
      if (m >= S) continue;  // wave-uniform
#pragma unroll
      for (int j = 0; j < SL; ++j) {
        const float o1 = __shfl_xor(t1[j], m, 64), o2 = __shfl_xor(t2[j], m, 64);
        float n1, n2;
        if (t1[j] >= o1) { n1 = t1[j]; n2 = fmaxf(t2[j], o1); } else { n1 = o1; n2 = fmaxf(t1[j], o2); }
        t1[j] = n1; t2[j] = n2;
      }
    }
    const int per_slot = 64 / S;
#pragma unroll
    for (int j = 0; j < SL; ++j)
      if (j < slots && lane % S == 0) gscore[wave][j * per_slot + lane / S] = t1[j] + t2[j];
    __builtin_amdgcn_wave_barrier();
    float gs[ROUTER_FAST_GROUPS];
#pragma unroll
    for (int g = 0; g < ROUTER_FAST_GROUPS; ++g) gs[g] = g < G ? gscore[wave][g] : NEG_INF;
    uint32_t keep = 0;
    for (int r = 0; r < a.topk_groups; ++r) {
      float bv = NEG_INF;
      int bi = -1;
#pragma unroll
      for (int g = 0; g < ROUTER_FAST_GROUPS; ++g)
        if (g < G && !((keep >> g) & 1u) && (bi < 0 || gs[g] > bv)) { bv = gs[g]; bi = g; }
      keep |= 1u << bi;
    }
#pragma unroll
    for (int j = 0; j < SL; ++j) {
      int e = j * 64 + lane;
      if (j < slots && e < E && !((keep >> (e / S)) & 1u)) biased[j] = NEG_INF;
    }
  } else if (G > 1) {
    float my_gscore = NEG_INF;  // lane g holds the score of group g
    for (int g = 0; g < G; ++g) {
      float t1 = NEG_INF, t2 = NEG_INF;
#pragma unroll
      for (int j = 0; j < SL; ++j) {
        int e = j * 64 + lane;
        if (j < slots && e < E && e / S == g) {
          float v = biased[j];
          if (v > t1) { t2 = t1; t1 = v; } else if (v > t2) { t2 = v; }
        }
      }
#pragma unroll
      for (int m = 32; m >= 1; m >>= 1) {
        float o1 = __shfl_xor(t1, m, 64), o2 = __shfl_xor(t2, m, 64);
        float n1, n2;
        if (t1 >= o1) { n1 = t1; n2 = fmaxf(t2, o1); } else { n1 = o1; n2 = fmaxf(t1, o2); }
        t1 = n1; t2 = n2;
      }
      if (lane == g) my_gscore = t1 + t2;
    }
    uint64_t keep = 0;
    for (int r = 0; r < a.topk_groups; ++r) {
      float v = (lane < G && !((keep >> lane) & 1ull)) ? my_gscore : NEG_INF;
      int i = lane < G && !((keep >> lane) & 1ull) ? lane : 0x7fffffff;
      wave_argmax(v, i);
      if (i < G) keep |= 1ull << i;
    }
#pragma unroll
    for (int j = 0; j < SL; ++j) {
      int e = j * 64 + lane;
      if (j < slots && e < E && !((keep >> (e / S)) & 1ull)) biased[j] = NEG_INF;
    }
  }

  // Top-k by repeated wave argmax; lane k keeps the k-th selection.
  const int K = a.top_k;
  uint32_t taken = 0;
  int my_idx = -1;
  float my_w = 0.0f;
  for (int k = 0; k < K; ++k) {
    float bv = NEG_INF;
    int bi = 0x7fffffff;
#pragma unroll
    for (int j = 0; j < SL; ++j) {
      int e = j * 64 + lane;
      if (j < slots && e < E && !((taken >> j) & 1u)) {
        if (biased[j] > bv || bi == 0x7fffffff) { bv = biased[j]; bi = e; }
      }
    }
    wave_argmax(bv, bi);
    if ((bi & 63) == lane) {
      int j = bi >> 6;
      taken |= 1u << j;
    }
    // the owner lane broadcasts the unbiased score
    float sel = 0.0f;
#pragma unroll
    for (int j = 0; j < SL; ++j) if ((bi >> 6) == j) sel = score[j];
    sel = __shfl(sel, bi & 63, 64);
    if (lane == k) { my_idx = bi; my_w = sel; }
  }
  float w = my_w;
  if (K > 1) {
    float sum = 0.0f;
    for (int k = 0; k < K; ++k) sum = sum + __shfl(my_w, k, 64);
    float denom = sum + 1.0e-20f;
    w = my_w / denom;
  }
  w = w * a.routed_scaling_factor;
  if (lane < K) {
    a.weights_out[t * K + lane] = w;
    if (a.indices_out != nullptr) a.indices_out[t * K + lane] = (int64_t)my_idx;
    if (a.indices32_out != nullptr) a.indices32_out[t * K + lane] = my_idx;
  }
}

extern "C" int mi355moe_gate_route(const MI355MoeRouteArgs* args, void* stream_) {
  hipStream_t stream = (hipStream_t)stream_;
  if (args == nullptr) return MI355MOE_EINVAL;
  const MI355MoeRouteArgs& a = *args;
  if (a.num_tokens < 0 || a.num_experts <= 0 || a.num_experts > 64 * ROUTER_MAX_SLOTS) return MI355MOE_EINVAL;
  if (a.top_k <= 0 || a.top_k > a.num_experts || a.top_k > 64) return MI355MOE_EINVAL;
  if (a.scoring != MI355MOE_SCORE_SOFTMAX && a.scoring != MI355MOE_SCORE_SIGMOID &&
      a.scoring != MI355MOE_SCORE_SQRTSOFTPLUS) return MI355MOE_EINVAL;
  if (a.num_groups < 1 || a.num_groups > 64 || a.num_experts % a.num_groups) return MI355MOE_EINVAL;
  if (a.num_groups > 1) {
    if (a.num_experts / a.num_groups < 2) return MI355MOE_EINVAL;
    if (a.topk_groups < 1 || a.topk_groups > a.num_groups) return MI355MOE_EINVAL;
    if (a.topk_groups * (a.num_experts / a.num_groups) < a.top_k) return MI355MOE_EINVAL;
  }
  if (a.logits == nullptr || a.bias == nullptr || a.weights_out == nullptr) return MI355MOE_EINVAL;
  if (a.indices_out == nullptr && a.indices32_out == nullptr) return MI355MOE_EINVAL;
  if (a.logits_row_stride < a.num_experts) return MI355MOE_EINVAL;
  if (a.num_tokens == 0) return MI355MOE_OK;
  dim3 grid((unsigned)((a.num_tokens + 3) / 4));
  const int slots = (a.num_experts + 63) / 64;
  if (slots <= 1) hipLaunchKernelGGL(mi355_route_kernel<1>, grid, dim3(256), 0, stream, a);
  else if (slots <= 2) hipLaunchKernelGGL(mi355_route_kernel<2>, grid, dim3(256), 0, stream, a);
  else if (slots <= 4) hipLaunchKernelGGL(mi355_route_kernel<4>, grid, dim3(256), 0, stream, a);
  else if (slots <= 8) hipLaunchKernelGGL(mi355_route_kernel<8>, grid, dim3(256), 0, stream, a);
  else hipLaunchKernelGGL(mi355_route_kernel<ROUTER_MAX_SLOTS>, grid, dim3(256), 0, stream, a);
  return hipGetLastError() == hipSuccess ? MI355MOE_OK : MI355MOE_ELAUNCH;
}

// ---------------------------------------------------------------------------------------------
// RouteGrad: one wavefront per token row, lane k < K owns selected slot k, expert e lives in lane
// e % 64, slot e / 64 (as in the forward). The operation order is the torch-autograd order of the
// routing-weight expression that the reference's RouteGrad pipeline reproduces
// (ops/hyper_mega_gate_grad/op_kernel/route_grad_pipeline.h:138-189: Muls, the div backward cross
// term -k0 * ((sel / D) / D), ReduceSum over K, the direct term k0 / D, Add; then
// op_api/hyper_mega_gate_route_grad_post.cpp: ScatterElementsV2 add into zeros, Muls 2, RealDiv,
// SoftplusV2Grad(beta 1, threshold 20)); the K sums run in ascending k.
__global__ __launch_bounds__(256) void mi355_route_grad_kernel(MI355MoeRouteGradArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= a.num_tokens) return;
  const int E = a.num_experts, K = a.top_k;
  const float* srow = a.scores + t * (int64_t)E;
  const float* lrow = a.logits + t * a.logits_row_stride;
  float* orow = a.grad_logits + t * (int64_t)E;
  // selected slot k = lane
  int id = -1;
  float gw = 0.0f, sel = 0.0f;
  if (lane < K) {
    const int64_t v = a.indices != nullptr ? a.indices[t * K + lane] : (int64_t)a.indices32[t * K + lane];
    if (v >= 0 && v < E) {
      id = (int)v;
      sel = a.selected_scores != nullptr ? a.selected_scores[t * K + lane] : srow[id];
    }
    gw = a.grad_weights[t * K + lane];
  }
  const float scale = a.routed_scaling_factor;
  float g;
  if (K == 1) {
    g = gw * scale;
  } else {
    float sum = 0.0f;
    for (int k = 0; k < K; ++k) sum = sum + __shfl(sel, k, 64);
    const float D = a.denominator != nullptr ? a.denominator[t] : sum + 1.0e-20f;
    const float k0 = gw * scale;
    const float cross = (-k0) * ((sel / D) / D);
    float row = 0.0f;
    for (int k = 0; k < K; ++k) row = row + __shfl(cross, k, 64);
    g = k0 / D + row;
  }
  float dot = 0.0f;
  if (a.scoring == MI355MOE_SCORE_SOFTMAX)
    for (int k = 0; k < K; ++k) dot = dot + __shfl(g, k, 64) * __shfl(sel, k, 64);
  const int slots = (E + 63) >> 6;
  for (int j = 0; j < slots; ++j) {
    const int e = j * 64 + lane;
    // scatter-add of the selected-score gradients into zeros
    float sg = 0.0f;
    for (int k = 0; k < K; ++k) {
      const int ik = __shfl(id, k, 64);
      const float gk = __shfl(g, k, 64);
      if (ik == e) sg = sg + gk;
    }
    if (e >= E) continue;
    const float s = srow[e];
    float r;
    if (a.scoring == MI355MOE_SCORE_SQRTSOFTPLUS) {
      const float q = sg / (2.0f * s);
      const float l = lrow[e];
      if (l > 20.0f) {
        r = q;
      } else {
        const float z = det_expf(l);
        r = (q * z) / (z + 1.0f);
      }
    } else if (a.scoring == MI355MOE_SCORE_SIGMOID) {
      r = (sg * (1.0f - s)) * s;
    } else {
      r = s * (sg - dot);
    }
    orow[e] = a.accumulate ? orow[e] + r : r;
  }
}

extern "C" int mi355moe_gate_route_grad(const MI355MoeRouteGradArgs* args, void* stream_) {
  if (args == nullptr) return MI355MOE_EINVAL;
  const MI355MoeRouteGradArgs& a = *args;
  if (a.num_tokens < 0 || a.num_experts <= 0 || a.num_experts > 64 * ROUTER_MAX_SLOTS) return MI355MOE_EINVAL;
  if (a.top_k <= 0 || a.top_k > a.num_experts || a.top_k > 64) return MI355MOE_EINVAL;
  if (a.scoring != MI355MOE_SCORE_SOFTMAX && a.scoring != MI355MOE_SCORE_SIGMOID &&
      a.scoring != MI355MOE_SCORE_SQRTSOFTPLUS)
    return MI355MOE_EINVAL;
  if (a.scores == nullptr || a.grad_weights == nullptr || a.grad_logits == nullptr) return MI355MOE_EINVAL;
  if (a.indices == nullptr && a.indices32 == nullptr) return MI355MOE_EINVAL;
  if (a.scoring == MI355MOE_SCORE_SQRTSOFTPLUS && (a.logits == nullptr || a.logits_row_stride < a.num_experts))
    return MI355MOE_EINVAL;
  if (!mi355_route_grad_enabled()) return MI355MOE_EUNSUPPORTED;
  if (a.num_tokens == 0) return MI355MOE_OK;
  hipLaunchKernelGGL(mi355_route_grad_kernel, dim3((unsigned)((a.num_tokens + 3) / 4)), dim3(256), 0,
                     (hipStream_t)stream_, a);
  return hipGetLastError() == hipSuccess ? MI355MOE_OK : MI355MOE_ELAUNCH;
}
