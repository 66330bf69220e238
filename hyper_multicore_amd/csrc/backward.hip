// MegaMoE expert backward at EP=1 (bf16): recompute the forward intermediates with the grouped
// GEMM, then
//   combine backward   dY[r] = bf16(p[s] * dOut[t]),  dp[s] = sum_h y[r, h] * dOut[t, h]
//   down backward      gA = bf16(dY @ W2^T),           dW2_e = act_e^T dY_e
//   SwiGLU backward    dU = [bf16(gA * u * s * (1 + g * (1 - s))) | bf16(gA * silu(g))]
//   up backward        dXr = bf16(dU @ W1^T),          dW1_e = X_e^T dU_e
//   permute backward   dX[t] = bf16(sum_k dXr[mapping[t * K + k]])
// for the routed row r of slot s = (t, k). The data-gradient GEMMs are the forward's grouped GEMM
// with the weight read in the transposed orientation; the weight gradients use its grouped-K mode.
// Reference: backends/bf16/autograd.py:672-760 (MegaMoeFunction.backward),
// tests/common/multicore/fp32_expert_reference.py:27-35 (rounding points).
#pragma clang fp contract(off)
#include "common.h"
#include "gemm.h"
#include "../../include/mi355moe.h"

namespace {

MI355_DEV float silu_f(float g) { return g / (1.0f + __expf(-g)); }

// act[r, c] = bf16(silu(g) * u) from the bf16 halves of U[r] (the values the forward epilogue uses).
__global__ __launch_bounds__(256) void swiglu_fwd_kernel(const uint16_t* U, int64_t R, int I, uint16_t* act) {
  const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int per_row = I / 8;
  if (id >= R * per_row) return;
  const int64_t r = id / per_row;
  const int c = (int)(id - r * per_row) * 8;
  const uint4 gq = *(const uint4*)(U + r * 2 * I + c);
  const uint4 uq = *(const uint4*)(U + r * 2 * I + I + c);
  const uint32_t gw[4] = {gq.x, gq.y, gq.z, gq.w}, uw[4] = {uq.x, uq.y, uq.z, uq.w};
  uint32_t ow[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float g0 = bf16_to_f32((uint16_t)(gw[i] & 0xffff)), g1 = bf16_to_f32((uint16_t)(gw[i] >> 16));
    const float u0 = bf16_to_f32((uint16_t)(uw[i] & 0xffff)), u1 = bf16_to_f32((uint16_t)(uw[i] >> 16));
    ow[i] = f32_to_bf16(silu_f(g0) * u0) | ((uint32_t)f32_to_bf16(silu_f(g1) * u1) << 16);
  }
  *(uint4*)(act + r * I + c) = make_uint4(ow[0], ow[1], ow[2], ow[3]);
}

// dY[r] = bf16(p * dOut[t]) and dp[s] = sum_h y[r, h] * dOut[t, h] for routed row r of slot s = t*K + k.
// BY_SLOT false: one block per routed row r, index = gather (row -> slot). BY_SLOT true: one block per
// slot s, index = mapping (slot -> row); a slot whose row lies outside [0, R) writes no row and dp 0.
template <bool BY_SLOT>
__global__ __launch_bounds__(256) void dy_dp_kernel(const uint16_t* y, const uint16_t* dout, const float* probs,
                                                    const int32_t* index, int K, int H, int64_t R, uint16_t* dy,
                                                    float* dp) {
  __shared__ float part[4];
  int64_t r;
  int32_t s;
  if constexpr (BY_SLOT) {
    s = (int32_t)blockIdx.x;
    r = index[s];
    if (r < 0 || r >= R) {
      if (dp != nullptr && threadIdx.x == 0) dp[s] = 0.0f;
      return;
    }
  } else {
    r = blockIdx.x;
    s = index[r];
  }
  const int64_t t = s / K;
  const float p = probs[s];
  float acc = 0.0f;
  for (int v = threadIdx.x; v < H / 8; v += blockDim.x) {
    const uint4 dq = ((const uint4*)(dout + t * H))[v];
    const uint4 yq = ((const uint4*)(y + r * H))[v];
    const uint32_t dw[4] = {dq.x, dq.y, dq.z, dq.w}, yw[4] = {yq.x, yq.y, yq.z, yq.w};
    uint32_t ow[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float d0 = bf16_to_f32((uint16_t)(dw[i] & 0xffff)), d1 = bf16_to_f32((uint16_t)(dw[i] >> 16));
      const float y0 = bf16_to_f32((uint16_t)(yw[i] & 0xffff)), y1 = bf16_to_f32((uint16_t)(yw[i] >> 16));
      ow[i] = f32_to_bf16(d0 * p) | ((uint32_t)f32_to_bf16(d1 * p) << 16);
      acc = acc + y0 * d0;
      acc = acc + y1 * d1;
    }
    ((uint4*)(dy + r * H))[v] = make_uint4(ow[0], ow[1], ow[2], ow[3]);
  }
  if (dp == nullptr) return;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    float sum = 0.0f;
    for (int w = 0; w < (int)(blockDim.x >> 6); ++w) sum = sum + part[w];
    dp[s] = sum;
  }
}

// dU = [bf16(gA * u * s * (1 + g * (1 - s))) | bf16(gA * silu(g))] with s = sigmoid(g).
__global__ __launch_bounds__(256) void swiglu_bwd_kernel(const uint16_t* gA, const uint16_t* U, int64_t R, int I,
                                                         uint16_t* dU) {
  const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int per_row = I / 8;
  if (id >= R * per_row) return;
  const int64_t r = id / per_row;
  const int c = (int)(id - r * per_row) * 8;
  const uint4 aq = *(const uint4*)(gA + r * I + c);
  const uint4 gq = *(const uint4*)(U + r * 2 * I + c);
  const uint4 uq = *(const uint4*)(U + r * 2 * I + I + c);
  const uint32_t aw[4] = {aq.x, aq.y, aq.z, aq.w}, gw[4] = {gq.x, gq.y, gq.z, gq.w}, uw[4] = {uq.x, uq.y, uq.z, uq.w};
  uint32_t gg[4], gu[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint16_t og[2], ou[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const float a = bf16_to_f32((uint16_t)(aw[i] >> (16 * h)));
      const float g = bf16_to_f32((uint16_t)(gw[i] >> (16 * h)));
      const float u = bf16_to_f32((uint16_t)(uw[i] >> (16 * h)));
      const float sg = 1.0f / (1.0f + __expf(-g));
      og[h] = f32_to_bf16(a * u * sg * (1.0f + g * (1.0f - sg)));
      ou[h] = f32_to_bf16(a * (g * sg));
    }
    gg[i] = og[0] | ((uint32_t)og[1] << 16);
    gu[i] = ou[0] | ((uint32_t)ou[1] << 16);
  }
  *(uint4*)(dU + r * 2 * I + c) = make_uint4(gg[0], gg[1], gg[2], gg[3]);
  *(uint4*)(dU + r * 2 * I + I + c) = make_uint4(gu[0], gu[1], gu[2], gu[3]);
}

size_t al256(size_t v) { return (v + 255) & ~(size_t)255; }

struct BwdLayout {
  size_t dispatch, counts, group_list, mapping, gather, tile_prefix, xg, u, act, y, dy, ga, du, zero, total;
};

BwdLayout bwd_layout(const MI355MoeBackwardArgs& a) {
  BwdLayout L = {};
  const size_t T = (size_t)a.num_tokens, K = (size_t)a.top_k, E = (size_t)a.num_experts;
  const size_t H = (size_t)a.hidden_size, I = (size_t)a.intermediate_size, R = T * K;
  size_t off = 0;
  auto take = [&](size_t bytes) { size_t o = off; off += al256(bytes); return o; };
  L.dispatch = take(mi355moe_dispatch_workspace_size(a.num_tokens, a.top_k, a.num_experts));
  L.counts = take(E * 4);
  L.group_list = take(E * 8);
  L.mapping = take(R * 4);
  L.gather = take(R * 4);
  L.tile_prefix = take((E + 1) * 4);
  L.xg = take(R * H * 2);
  L.u = take(R * 2 * I * 2);
  L.act = take(R * I * 2);
  L.y = take(R * H * 2);  // expert outputs, then the routed input gradients
  L.dy = take(R * H * 2);
  L.ga = take(R * I * 2);
  L.du = take(R * 2 * I * 2);
  L.zero = take((H > 2 * I ? H : 2 * I) * 2);
  L.total = off;
  return L;
}

int validate_bwd(const MI355MoeBackwardArgs& a) {
  if (a.num_tokens < 0 || a.hidden_size <= 0 || a.intermediate_size <= 0 || a.num_experts <= 0 || a.top_k <= 0)
    return MI355MOE_EINVAL;
  if (a.num_experts > 4096 || a.top_k > 64 || a.top_k > a.num_experts) return MI355MOE_EINVAL;
  if (a.ids_dtype != MI355MOE_IDS_INT32 && a.ids_dtype != MI355MOE_IDS_INT64) return MI355MOE_EINVAL;
  if (a.weight_layout == MI355MOE_LAYOUT_EIO_GU) return MI355MOE_EUNSUPPORTED;  // forward-only layout
  if (a.weight_layout != MI355MOE_LAYOUT_EIO && a.weight_layout != MI355MOE_LAYOUT_EOI) return MI355MOE_EINVAL;
  if (a.weight_grad_dtype != MI355MOE_GRAD_BF16 && a.weight_grad_dtype != MI355MOE_GRAD_FP32) return MI355MOE_EINVAL;
  if (a.num_tokens * (int64_t)a.top_k > INT32_MAX) return MI355MOE_EINVAL;
  if (a.precision != MI355MOE_PRECISION_BF16 && a.precision != MI355MOE_PRECISION_MXFP8) return MI355MOE_EINVAL;
  if (a.hidden_size % 64 || a.intermediate_size % 128) return MI355MOE_EUNSUPPORTED;
  if (a.precision == MI355MOE_PRECISION_MXFP8) {
    // EIO roots only; the data-gradient GEMMs fetch 16 row-scale codes of the weights at a time
    if (a.weight_layout != MI355MOE_LAYOUT_EIO) return MI355MOE_EUNSUPPORTED;
    if (a.hidden_size % 512 || a.intermediate_size % 256) return MI355MOE_EUNSUPPORTED;
    if (!mi355_mx_backward_enabled()) return MI355MOE_EUNSUPPORTED;
    if (a.num_tokens > 0 && (a.w1_scale == nullptr || a.w2_scale == nullptr || a.w1_row == nullptr ||
                             a.w2_row == nullptr || a.w1_row_scale == nullptr || a.w2_row_scale == nullptr))
      return MI355MOE_EINVAL;
  } else if (!mi355_backward_enabled()) {
    return MI355MOE_EUNSUPPORTED;
  }
  if (a.grad_w1 == nullptr || a.grad_w2 == nullptr) return MI355MOE_EINVAL;
  if (a.num_tokens > 0 &&
      (a.hidden == nullptr || a.topk_ids == nullptr || a.topk_weights == nullptr || a.w1 == nullptr ||
       a.w2 == nullptr || a.grad_out == nullptr || a.grad_hidden == nullptr))
    return MI355MOE_EINVAL;
  return MI355MOE_OK;
}

int launch_rows(void (*kern)(const uint16_t*, int64_t, int, uint16_t*), const uint16_t* in, int64_t R, int I,
                uint16_t* out, hipStream_t st) {
  const int64_t n = R * (I / 8);
  if (n == 0) return MI355MOE_OK;
  hipLaunchKernelGGL(kern, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, in, R, I, out);
  return hipGetLastError() == hipSuccess ? MI355MOE_OK : MI355MOE_ELAUNCH;
}

// ---- MXFP8 -------------------------------------------------------------------------------------
struct MxBwdLayout {
  size_t dispatch, counts, group_list, mapping, gather, tile_prefix, block_prefix, xq, xs, u, aq, as, acol, acs, y,
      dy, dyq, dys, dycol, dycs, da, duq, dus, ducol, ducs, xcol, xcs, zero, total;
};

MxBwdLayout mx_bwd_layout(const MI355MoeBackwardArgs& a) {
  MxBwdLayout L = {};
  const size_t T = (size_t)a.num_tokens, K = (size_t)a.top_k, E = (size_t)a.num_experts;
  const size_t H = (size_t)a.hidden_size, I = (size_t)a.intermediate_size, R = T * K;
  const size_t CG = (R + 63) / 64 + E;  // 64-row scale groups of the grouped column axis
  size_t off = 0;
  auto take = [&](size_t bytes) { size_t o = off; off += al256(bytes); return o; };
  L.dispatch = take(mi355moe_dispatch_workspace_size(a.num_tokens, a.top_k, a.num_experts));
  L.counts = take(E * 4);
  L.group_list = take(E * 8);
  L.mapping = take(R * 4);
  L.gather = take(R * 4);
  L.tile_prefix = take((E + 1) * 4);
  L.block_prefix = take((E + 1) * 4);
  L.xq = take(T * H);                                  // x along H (GMM1 recompute)
  L.xs = take(T * (size_t)mi355_mx_scale_ld(H));
  L.u = take(R * 2 * I * 2);                           // U bf16
  L.aq = take(R * I);                                  // act along I (GMM2 recompute)
  L.as = take(R * (size_t)mi355_mx_scale_ld(I));
  L.acol = take(R * I);                                // act along the routed rows (dW2)
  L.acs = take(CG * I * 2);
  L.y = take(R * H * 2);                               // y, later the routed input gradients
  L.dy = take(R * H * 2);
  L.dyq = take(R * H);                                 // dY along H (gA)
  L.dys = take(R * (size_t)mi355_mx_scale_ld(H));
  L.dycol = take(R * H);                               // dY along the routed rows (dW2)
  L.dycs = take(CG * H * 2);
  L.da = take(R * I * 2);                              // gA bf16
  L.duq = take(R * 2 * I);                             // dU along 2I (dX)
  L.dus = take(R * (size_t)mi355_mx_scale_ld(2 * I));
  L.ducol = take(R * 2 * I);                           // dU along the routed rows (dW1)
  L.ducs = take(CG * 2 * I * 2);
  L.xcol = take(R * H);                                // X along the routed rows (dW1)
  L.xcs = take(CG * H * 2);
  L.zero = take(H > 2 * I ? H : 2 * I);
  L.total = off;
  return L;
}

int mx_backward(const MI355MoeBackwardArgs& a, char* ws, const MxBwdLayout& L, hipStream_t st) {
  const int64_t T = a.num_tokens;
  const int K = a.top_k, E = a.num_experts, H = a.hidden_size, I = a.intermediate_size;
  const int64_t R = T * K;
  const bool f32 = a.weight_grad_dtype == MI355MOE_GRAD_FP32;
  int64_t* group_list = (int64_t*)(ws + L.group_list);
  int32_t* mapping = (int32_t*)(ws + L.mapping);
  int32_t* gather = (int32_t*)(ws + L.gather);
  int32_t* tile_prefix = (int32_t*)(ws + L.tile_prefix);
  int32_t* block_prefix = (int32_t*)(ws + L.block_prefix);
  uint16_t* u = (uint16_t*)(ws + L.u);
  uint16_t* y = (uint16_t*)(ws + L.y);
  uint16_t* dy = (uint16_t*)(ws + L.dy);
  uint16_t* da = (uint16_t*)(ws + L.da);
  const uint8_t* zero = (const uint8_t*)(ws + L.zero);
  const int64_t ldH = mi355_mx_scale_ld(H), ldI = mi355_mx_scale_ld(I), ld2I = mi355_mx_scale_ld(2 * I);

  int rc = mi355_dispatch_enqueue(a.topk_ids, a.ids_dtype, T, K, E, (int32_t*)(ws + L.counts), nullptr, group_list,
                                  mapping, gather, a.error_flag, ws + L.dispatch, st);
  if (rc) return rc;
  if ((rc = mi355_plan_tiles(group_list, E, tile_prefix, st))) return rc;
  if ((rc = mi355_plan_row_blocks(group_list, E, 32, block_prefix, st))) return rc;
  if ((rc = mi355_zero_enqueue(ws + L.zero, (size_t)(H > 2 * I ? H : 2 * I), st))) return rc;
  if ((rc = mi355_mx_quant_rows(a.hidden, T, H, (uint8_t*)(ws + L.xq), (uint8_t*)(ws + L.xs), ldH, st))) return rc;

  // MX grouped GEMM over the routed rows: out [R, N] bf16 = A [R, Kd] (row scales a_ld) @ W_g.
  // Forward weights: col_data [E, Kd, N] with col_scale (b_kn); backward weights: row_data of the
  // transposed product, [E, N, Kd] K-contiguous with row scales [E * N, Kd / 32].
  auto gmm = [&](const uint8_t* A, const uint8_t* As, int64_t a_ld, const int32_t* a_index, int a_div, int Kd,
                 const uint8_t* W, const uint8_t* Ws, bool b_kn, int N, uint16_t* out) {
    GGParams p = {};
    p.A = A;
    p.lda_bytes = Kd;
    p.a_bytes = (a_index != nullptr ? T : R) * Kd;  // A holds the tokens when gathered, else the routed rows
    p.a_row_index = a_index;
    p.a_row_div = a_div;
    p.a_scale = As;
    p.a_scale_ld = a_ld;
    p.B = W;
    p.b_group_stride = (int64_t)Kd * N;
    p.b_row_bytes = b_kn ? N : Kd;
    p.b_scale = Ws;
    p.b_scale_ld = b_kn ? 0 : Kd / 32;
    p.b_scale_group_stride = b_kn ? (int64_t)(Kd / 64) * N * 2 : (int64_t)N * (Kd / 32);
    p.K = Kd;
    p.N = N;
    p.Ntot = N;
    p.n_tiles = (N + mi355_gg_bn() - 1) / mi355_gg_bn();
    p.G = E;
    p.group_list = group_list;
    p.tile_prefix = tile_prefix;
    p.C = out;
    p.ldc = N;
    return mi355_grouped_gemm(p, true, b_kn, EPI_STORE_BF16, st);
  };
  // Weight gradient C_g [M, N] = Q_rows(A)_g^T Q_rows(B)_g (grouped packed column scales).
  auto wgrad = [&](const uint8_t* A, const uint8_t* As, int M, const uint8_t* B, const uint8_t* Bs, int N, void* out) {
    GGParams p = {};
    p.A = A;
    p.lda_bytes = M;
    p.a_scale = As;
    p.B = B;
    p.b_row_bytes = N;
    p.b_scale = Bs;
    p.N = N;
    p.Ntot = N;
    p.m_rows = M;
    p.m_tiles = (M + mi355_gg_bm() - 1) / mi355_gg_bm();
    p.n_tiles = (N + mi355_gg_bn() - 1) / mi355_gg_bn();
    p.G = E;
    p.group_list = group_list;
    p.C = out;
    p.ldc = N;
    p.c_group_stride = (int64_t)M * N;
    p.zero_row = zero;
    return mi355_grouped_gemm_wgrad(p, f32 ? EPI_STORE_F32 : EPI_STORE_BF16, st, true);
  };
  auto quant = [&](int mode, const uint16_t* src, const int32_t* g_index, int g_div, int64_t src_ld, int C,
                   size_t rowq, size_t rows, int64_t row_ld, size_t colq, size_t cols) {
    MxGroupedQuant q = {};
    q.mode = mode;
    q.src = src;
    q.gather = g_index;
    q.gather_div = g_div;
    q.src_ld = src_ld;
    q.U = u;
    q.da = da;
    q.R = R;
    q.C = C;
    q.G = E;
    q.group_list = group_list;
    q.block_prefix = block_prefix;
    q.row_data = rowq ? (uint8_t*)(ws + rowq) : nullptr;
    q.row_scale = rowq ? (uint8_t*)(ws + rows) : nullptr;
    q.row_scale_ld = row_ld;
    q.col_data = colq ? (uint8_t*)(ws + colq) : nullptr;
    q.col_scale = colq ? (uint8_t*)(ws + cols) : nullptr;
    return mi355_mx_quant_grouped(q, st);
  };
  const uint8_t* w1 = (const uint8_t*)a.w1;
  const uint8_t* w2 = (const uint8_t*)a.w2;
  // forward recompute: U = Q(x) W1 (rows gathered from the tokens), act, y = Q(act) W2
  if ((rc = gmm((const uint8_t*)(ws + L.xq), (const uint8_t*)(ws + L.xs), ldH, gather, K, H, w1, a.w1_scale, true,
                2 * I, u)))
    return rc;
  if ((rc = quant(MX_Q_SWIGLU, nullptr, nullptr, 1, 0, I, L.aq, L.as, ldI, L.acol, L.acs))) return rc;
  if ((rc = gmm((const uint8_t*)(ws + L.aq), (const uint8_t*)(ws + L.as), ldI, nullptr, 1, I, w2, a.w2_scale, true, H,
                y)))
    return rc;
  // combine backward: dY = bf16(p dOut), dp = <y, dOut>
  // one block per slot through slot -> row (a slot with an id outside [0, E) has no row)
  hipLaunchKernelGGL(dy_dp_kernel<true>, dim3((unsigned)R), dim3(256), 0, st, y, a.grad_out, a.topk_weights, mapping, K,
                     H, R, dy, a.grad_topk_weights);
  if (hipGetLastError() != hipSuccess) return MI355MOE_ELAUNCH;
  if ((rc = quant(MX_Q_BF16, dy, nullptr, 1, H, H, L.dyq, L.dys, ldH, L.dycol, L.dycs))) return rc;
  // dW2 [E, I, H] = Q_rows(act)^T Q_rows(dY);  gA = bf16(Q_H(dY) W2_row^T)
  if ((rc = wgrad((const uint8_t*)(ws + L.acol), (const uint8_t*)(ws + L.acs), I, (const uint8_t*)(ws + L.dycol),
                  (const uint8_t*)(ws + L.dycs), H, a.grad_w2)))
    return rc;
  if ((rc = gmm((const uint8_t*)(ws + L.dyq), (const uint8_t*)(ws + L.dys), ldH, nullptr, 1, H, a.w2_row,
                a.w2_row_scale, false, I, da)))
    return rc;
  // SwiGLU gradient, quantised along 2I and along the routed rows; X along the routed rows
  if ((rc = quant(MX_Q_SWIGLU_BWD, nullptr, nullptr, 1, 0, 2 * I, L.duq, L.dus, ld2I, L.ducol, L.ducs))) return rc;
  if ((rc = quant(MX_Q_BF16, a.hidden, gather, K, H, H, 0, 0, 0, L.xcol, L.xcs))) return rc;
  // dW1 [E, H, 2I] = Q_rows(X)^T Q_rows(dU);  dX_routed = bf16(Q_2I(dU) W1_row^T) (into y)
  if ((rc = wgrad((const uint8_t*)(ws + L.xcol), (const uint8_t*)(ws + L.xcs), H, (const uint8_t*)(ws + L.ducol),
                  (const uint8_t*)(ws + L.ducs), 2 * I, a.grad_w1)))
    return rc;
  if ((rc = gmm((const uint8_t*)(ws + L.duq), (const uint8_t*)(ws + L.dus), ld2I, nullptr, 1, 2 * I, a.w1_row,
                a.w1_row_scale, false, H, y)))
    return rc;
  return mi355_unpermute_enqueue(y, mapping, nullptr, T, K, H, a.grad_hidden, st);
}

}  // namespace

extern "C" int mi355moe_token_unpermute_grad(const uint16_t* permuted, const uint16_t* grad_out, const int32_t* mapping,
                                             const float* probs, int64_t num_tokens, int32_t top_k,
                                             int32_t hidden_size, uint16_t* grad_permuted, float* grad_probs,
                                             void* stream) {
  if (num_tokens < 0 || top_k <= 0 || hidden_size <= 0 || hidden_size % 8) return MI355MOE_EINVAL;
  const int64_t R = num_tokens * top_k;
  if (R > 0x7fffffff) return MI355MOE_EUNSUPPORTED;  // one block per slot
  if (num_tokens > 0) {
    if (permuted == nullptr || grad_out == nullptr || mapping == nullptr || probs == nullptr ||
        grad_permuted == nullptr)
      return MI355MOE_EINVAL;
    if (((uintptr_t)permuted | (uintptr_t)grad_out | (uintptr_t)grad_permuted) & 15) return MI355MOE_EINVAL;
  }
  if (!mi355_backward_enabled()) return MI355MOE_EUNSUPPORTED;
  if (R == 0) return MI355MOE_OK;
  hipLaunchKernelGGL(dy_dp_kernel<true>, dim3((unsigned)R), dim3(256), 0, (hipStream_t)stream, permuted, grad_out,
                     probs, mapping, top_k, hidden_size, R, grad_permuted, grad_probs);
  return hipGetLastError() == hipSuccess ? MI355MOE_OK : MI355MOE_ELAUNCH;
}

extern "C" size_t mi355moe_moe_backward_workspace_size(const MI355MoeBackwardArgs* args) {
  if (args == nullptr || validate_bwd(*args) != MI355MOE_OK) return 0;
  if (args->precision == MI355MOE_PRECISION_MXFP8) return mx_bwd_layout(*args).total;
  return bwd_layout(*args).total;
}

extern "C" int mi355moe_moe_backward(const MI355MoeBackwardArgs* args, void* workspace, size_t workspace_size,
                                     void* stream) {
  if (args == nullptr) return MI355MOE_EINVAL;
  const MI355MoeBackwardArgs& a = *args;
  int rc = validate_bwd(a);
  if (rc) return rc;
  const int64_t T = a.num_tokens;
  const int K = a.top_k, E = a.num_experts, H = a.hidden_size, I = a.intermediate_size;
  const int64_t R = T * K;
  hipStream_t st = (hipStream_t)stream;
  const bool f32 = a.weight_grad_dtype == MI355MOE_GRAD_FP32;
  const size_t wsz = f32 ? 4 : 2;
  if (T == 0) {  // no rows: the weight gradients are zero
    const int rz = mi355_zero_enqueue(a.grad_w1, (size_t)E * H * 2 * I * wsz, st);
    return rz ? rz : mi355_zero_enqueue(a.grad_w2, (size_t)E * I * H * wsz, st);
  }
  if (a.precision == MI355MOE_PRECISION_MXFP8) {
    const MxBwdLayout ML = mx_bwd_layout(a);
    if (workspace == nullptr || workspace_size < ML.total) return MI355MOE_EWORKSPACE_CODE;
    return mx_backward(a, (char*)workspace, ML, st);
  }
  BwdLayout L = bwd_layout(a);
  if (workspace == nullptr || workspace_size < L.total) return MI355MOE_EWORKSPACE_CODE;
  char* ws = (char*)workspace;
  const bool eoi = a.weight_layout == MI355MOE_LAYOUT_EOI;
  int64_t* group_list = (int64_t*)(ws + L.group_list);
  int32_t* mapping = (int32_t*)(ws + L.mapping);
  int32_t* gather = (int32_t*)(ws + L.gather);
  int32_t* tile_prefix = (int32_t*)(ws + L.tile_prefix);
  uint16_t* xg = (uint16_t*)(ws + L.xg);
  uint16_t* u = (uint16_t*)(ws + L.u);
  uint16_t* act = (uint16_t*)(ws + L.act);
  uint16_t* y = (uint16_t*)(ws + L.y);
  uint16_t* dy = (uint16_t*)(ws + L.dy);
  uint16_t* ga = (uint16_t*)(ws + L.ga);
  uint16_t* du = (uint16_t*)(ws + L.du);
  const uint8_t* zero = (const uint8_t*)(ws + L.zero);

  rc = mi355_dispatch_enqueue(a.topk_ids, a.ids_dtype, T, K, E, (int32_t*)(ws + L.counts), nullptr, group_list,
                              mapping, gather, a.error_flag, ws + L.dispatch, st);
  if (rc) return rc;
  rc = mi355_plan_tiles(group_list, E, tile_prefix, st);
  if (rc) return rc;
  rc = mi355_zero_enqueue(ws + L.zero, (size_t)(H > 2 * I ? H : 2 * I) * 2, st);
  if (rc) return rc;
  rc = mi355_permute_rows_enqueue(a.hidden, R, K, H, mapping, xg, st);  // X in routed order
  if (rc) return rc;

  // A grouped GEMM over the routed rows: out[R, N] = A[R, Kd] @ W_g with W_g read as NK or KN.
  auto gmm = [&](const uint16_t* A, int Kd, const uint16_t* W, bool w_kn, int64_t w_row, int64_t w_group, int N,
                 uint16_t* out) {
    GGParams p = {};
    p.A = (const uint8_t*)A;
    p.lda_bytes = (int64_t)Kd * 2;
    p.a_bytes = R * Kd * 2;
    p.a_row_div = 1;
    p.B = (const uint8_t*)W;
    p.b_group_stride = w_group * 2;
    p.b_row_bytes = w_row * 2;
    p.K = Kd;
    p.N = N;
    p.Ntot = N;
    p.n_tiles = (N + mi355_gg_bn() - 1) / mi355_gg_bn();
    p.G = E;
    p.group_list = group_list;
    p.tile_prefix = tile_prefix;
    p.C = out;
    p.ldc = N;
    return mi355_grouped_gemm(p, false, w_kn, EPI_STORE_BF16, st);
  };
  // Weight gradient: C_g[m, n] = sum_r A[r, m] B[r, n] over the rows of group g.
  auto wgrad = [&](const uint16_t* A, int M, const uint16_t* B, int N, void* out) {
    GGParams p = {};
    p.A = (const uint8_t*)A;
    p.lda_bytes = (int64_t)M * 2;
    p.B = (const uint8_t*)B;
    p.b_row_bytes = (int64_t)N * 2;
    p.N = N;
    p.Ntot = N;
    p.m_rows = M;
    p.m_tiles = (M + mi355_gg_bm() - 1) / mi355_gg_bm();
    p.n_tiles = (N + mi355_gg_bn() - 1) / mi355_gg_bn();
    p.G = E;
    p.group_list = group_list;
    p.C = out;
    p.ldc = N;
    p.c_group_stride = (int64_t)M * N;
    p.zero_row = zero;
    return mi355_grouped_gemm_wgrad(p, f32 ? EPI_STORE_F32 : EPI_STORE_BF16, st);
  };
  const int64_t w1_group = (int64_t)H * 2 * I, w2_group = (int64_t)I * H;
  // forward recompute: U = X W1, act = swiglu(U), y = act W2
  rc = gmm(xg, H, a.w1, !eoi, eoi ? H : 2 * I, w1_group, 2 * I, u);
  if (rc) return rc;
  rc = launch_rows(swiglu_fwd_kernel, u, R, I, act, st);
  if (rc) return rc;
  rc = gmm(act, I, a.w2, !eoi, eoi ? I : H, w2_group, H, y);
  if (rc) return rc;
  // combine backward
  // one block per slot through slot -> row (a slot with an id outside [0, E) has no row)
  hipLaunchKernelGGL(dy_dp_kernel<true>, dim3((unsigned)R), dim3(256), 0, st, y, a.grad_out, a.topk_weights, mapping, K,
                     H, R, dy, a.grad_topk_weights);
  if (hipGetLastError() != hipSuccess) return MI355MOE_ELAUNCH;
  // down backward: gA = dY W2^T (W2 read transposed: EIO [I, H] rows are the N index -> NK)
  rc = gmm(dy, H, a.w2, eoi, eoi ? I : H, w2_group, I, ga);
  if (rc) return rc;
  rc = wgrad(eoi ? dy : act, eoi ? H : I, eoi ? act : dy, eoi ? I : H, a.grad_w2);
  if (rc) return rc;
  // SwiGLU backward
  const int64_t n = R * (I / 8);
  hipLaunchKernelGGL(swiglu_bwd_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, ga, u, R, I, du);
  if (hipGetLastError() != hipSuccess) return MI355MOE_ELAUNCH;
  // up backward: dXr = dU W1^T (into the buffer of y), dW1
  rc = gmm(du, 2 * I, a.w1, eoi, eoi ? H : 2 * I, w1_group, H, y);
  if (rc) return rc;
  rc = wgrad(eoi ? du : xg, eoi ? 2 * I : H, eoi ? xg : du, eoi ? H : 2 * I, a.grad_w1);
  if (rc) return rc;
  // permute backward: dX[t] = sum_k dXr[mapping[t * K + k]]
  return mi355_unpermute_enqueue(y, mapping, nullptr, T, K, H, a.grad_hidden, st);
}
