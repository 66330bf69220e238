/*
 * mi355moe.h - C ABI of the MI355X (gfx950) MegaGate -> MegaMoE forward path, expert-parallel
 * degree 1 (every expert on one GPU).
 *
 * Conventions (all entry points):
 *   - Pointers are device pointers unless stated otherwise; tensors are dense row-major.
 *   - `stream` is a hipStream_t passed as void*; work is enqueued asynchronously on it and no
 *     entry point synchronises the host.
 *   - Return 0 on success, a negative MI355MOE_E* code on invalid arguments or launch failure.
 *     Nothing is enqueued when an argument check fails.
 *   - bf16 is passed as uint16_t storage; e4m3 (OCP fp8 e4m3fn) and e8m0 as uint8_t.
 *
 * The reference interfaces each entry point replaces are cited per declaration
 * (paths relative to the hyper-multicore source tree).
 */
#ifndef MI355MOE_H_
#define MI355MOE_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MI355MOE_ABI_VERSION 7

enum {
  MI355MOE_OK_CODE = 0,
  MI355MOE_EINVAL_CODE = -1,      /* invalid argument / shape / alignment */
  MI355MOE_ELAUNCH_CODE = -2,     /* HIP launch error */
  MI355MOE_EUNSUPPORTED_CODE = -3, /* valid request outside what this build implements */
  MI355MOE_EWORKSPACE_CODE = -4   /* workspace missing or too small */
};

enum { MI355MOE_SCORE_SOFTMAX = 0, MI355MOE_SCORE_SIGMOID = 1, MI355MOE_SCORE_SQRTSOFTPLUS = 2 };
enum { MI355MOE_IDS_INT32 = 0, MI355MOE_IDS_INT64 = 1 };
enum { MI355MOE_PRECISION_BF16 = 0, MI355MOE_PRECISION_MXFP8 = 1 };
/* Expert weight layouts (modules/mega_moe/module.py:276-279):
 *   EIO: w1 [E, H, 2I], w2 [E, I, H]   (input-major rows, output contiguous)
 *   EOI: w1 [E, 2I, H], w2 [E, H, I]   (output-major rows, input contiguous)
 *   EIO_GU (no reference counterpart; forward only): EIO, with w1's gate and up columns
 *   interleaved in 64-column blocks by mi355moe_interleave_gate_up (and, for MXFP8, w1_scale's
 *   columns the same way); w2 is plain EIO. */
enum { MI355MOE_LAYOUT_EIO = 0, MI355MOE_LAYOUT_EOI = 1, MI355MOE_LAYOUT_EIO_GU = 2 };

/* ---------------------------------------------------------------------------------------------
 * ABI version of the loaded library (no reference counterpart; used by the loader check).
 */
int mi355moe_abi_version(void);

/* Optional paths this build has switched on (no reference counterpart): a bit set of
 * MI355MOE_FEATURE_*. A path whose bit is clear answers MI355MOE_EUNSUPPORTED. */
enum {
  MI355MOE_FEATURE_MX_EOI = 1,        /* MXFP8 GEMMs on re-laid-out (K-contiguous) weights */
  MI355MOE_FEATURE_NUMERICS = 2,      /* BF16 SwiGLU clamp / probabilities before FC2 */
  MI355MOE_FEATURE_DECODE_TILES = 4,  /* 64-row tiles for groups averaging <= 32 rows */
  MI355MOE_FEATURE_BACKWARD = 8,      /* mi355moe_moe_backward */
  MI355MOE_FEATURE_ROUTE_GRAD = 16,   /* mi355moe_gate_route_grad */
  MI355MOE_FEATURE_MX_WEIGHT_PREP = 32, /* mi355moe_mx_quantize_weight */
  MI355MOE_FEATURE_MX_BACKWARD = 64,  /* mi355moe_moe_backward with precision MXFP8 */
  /* bits 128 and 256 are retired (grouped-GEMM configurations of ABI 6 and earlier) and never set */
};
int mi355moe_features(void);

/* Grouped-GEMM configuration of a call (the gemm_variant argument of the grouped GEMMs and of
 * MI355MoeForwardArgs; a measurement control with no counterpart in the reference, whose GEMM tiling
 * is fixed by its tuning tables). The library holds no variant state: every call names its own.
 *   MI355MOE_GEMM_DEFAULT: the 8-wave 256 x 256 configuration where it applies, except that GEMMs
 *     whose groups average at most 32 rows (decode shapes) run on the 64-row tiles; else the 4-wave
 *     one;
 *   MI355MOE_GEMM_PP: the 8-wave configuration where it applies, also for decode shapes (so the MX
 *     forward keeps the stage-major activation scales there); else the 4-wave one;
 *   MI355MOE_GEMM_W4: the 4-wave 256 x 256 configuration (128 x 128 wave tiles).
 * Values 1-4 named configurations of ABI 6 and earlier; they, and any other value, make the call
 * answer MI355MOE_EUNSUPPORTED. The expert backward always uses the default. */
enum { MI355MOE_GEMM_DEFAULT = 0, MI355MOE_GEMM_PP = 5, MI355MOE_GEMM_W4 = 6 };

/* ---------------------------------------------------------------------------------------------
 * Router projection: logits[t, e] = sum_h x[t, h] * w[e, h], bf16 inputs, fp32 accumulate and
 * fp32 output (deterministic split-K: fixed K chunks summed in ascending order). H % 128 == 0. Replaces the fp32 projection F.linear(x.float(), W.float())
 * (modules/mega_gate/function.py:176-178, modules/mega_gate/module.py:195-198); bf16 x bf16
 * products are exact in fp32, only the summation order differs from the reference.
 * When w_vision and image_mask are given, tokens with image_mask[t] != 0 use w_vision instead of
 * w (per-modality router matrices). `workspace` must hold
 * mi355moe_gate_logits_workspace_size() bytes.
 */
size_t mi355moe_gate_logits_workspace_size(int64_t num_tokens, int32_t hidden_size, int32_t num_experts);
int mi355moe_gate_logits(const uint16_t* x, int64_t num_tokens, int32_t hidden_size,
                         const uint16_t* w, const uint16_t* w_vision, const uint8_t* image_mask,
                         int32_t num_experts, float* logits, void* workspace,
                         size_t workspace_size, void* stream);

/* ---------------------------------------------------------------------------------------------
 * Route: scores, correction bias, (group-limited) top-k, gather, renormalise, scale.
 * Replaces hyper_multicore::mega_gate_route / aclnnHyperMegaGateRoute
 * (torch/csrc/mega_gate_registration.cpp:16-42, torch/csrc/mega_gate.cpp:65-82,
 *  ops/hyper_mega_gate/op_kernel/route_pipeline.h:73-562) and the torch path
 * MegaGate._torch_forward (modules/mega_gate/module.py:189-227) for softmax / sigmoid.
 * Output order within a row: descending biased score, ties by lower expert id.
 * num_groups == 1 selects plain top-k; num_groups > 1 selects the DeepSeek-V3 group-limited form
 * (group score = sum of the top-2 biased scores of the group; keep topk_groups groups).
 */
typedef struct MI355MoeRouteArgs {
  const float* logits;        /* [T, E] fp32, row stride logits_row_stride elements */
  int64_t logits_row_stride;
  const float* bias;          /* [E] fp32 correction bias (text tokens) */
  const float* bias_vl;       /* [E] fp32 vision bias or NULL */
  const uint8_t* image_mask;  /* [T] bool or NULL: nonzero selects bias_vl */
  float* weights_out;         /* [T, K] fp32 routing weights */
  int64_t* indices_out;       /* [T, K] int64 expert ids (NULL allowed if indices32_out given) */
  int32_t* indices32_out;     /* [T, K] int32 expert ids or NULL */
  float* scores_out;          /* [T, E] fp32 unbiased scores or NULL */
  int64_t num_tokens;
  int32_t num_experts;        /* <= 1024 */
  int32_t top_k;              /* <= min(E, 64) */
  int32_t scoring;            /* MI355MOE_SCORE_* */
  int32_t num_groups;         /* 1 = no grouping; divides E */
  int32_t topk_groups;
  float routed_scaling_factor;
} MI355MoeRouteArgs;
int mi355moe_gate_route(const MI355MoeRouteArgs* args, void* stream);

/* ---------------------------------------------------------------------------------------------
 * RouteGrad: the gradient of the routing weights of mi355moe_gate_route with respect to the fp32
 * logits, for the selected experts `indices` and upstream grad_weights [T, K]:
 *   g_k  = K == 1 ? gw_k * scale : k0_k / D + sum_j -k0_j * ((sel_j / D) / D),  k0 = gw * scale,
 *          sel = scores[idx], D = sum_k sel_k + 1e-20   (sums in ascending k)
 *   sg_e = g_k where e = idx_k, else 0
 *   sqrt-softplus: grad = l > 20 ? q : (q * exp(l)) / (exp(l) + 1),  q = sg / (2 * score)
 *   sigmoid:       grad = (sg * (1 - score)) * score
 *   softmax:       grad = score * (sg - sum_k g_k * sel_k)
 * scores are the forward's unbiased scores (scores_out of mi355moe_gate_route); the group-limited
 * selection and the correction biases do not enter the gradient. With accumulate != 0 the result
 * is added to grad_logits (a gradient already held for the logits output), else it overwrites it.
 * An expert whose score is 0 (sqrt-softplus with softplus(l) == 0) gets 0 / 0 = NaN, as in the
 * reference's RealDiv. Ids outside [0, E) select nothing.
 * Replaces hyper_multicore::mega_gate_route_grad -> aclnnHyperMegaGateRouteGrad
 * (torch/csrc/mega_gate.cpp:182-197, ops/hyper_mega_gate_grad/op_host/op_api/
 * hyper_mega_gate_route_grad.cpp:94-120, op_kernel/route_grad_pipeline.h:138-189), which takes the
 * selected scores and the denominator as inputs; here they are recomputed from scores and indices
 * with the forward's summation order. The sigmoid / softmax forms are torch autograd of
 * MegaGate._torch_forward (modules/mega_gate/module.py:199-227), the reference's path for those.
 */
typedef struct MI355MoeRouteGradArgs {
  const float* logits;        /* [T, E] fp32, row stride logits_row_stride (read for sqrt-softplus) */
  int64_t logits_row_stride;
  const float* scores;        /* [T, E] fp32 forward scores, row stride E */
  const int64_t* indices;     /* [T, K] int64 expert ids (or NULL with indices32) */
  const int32_t* indices32;   /* [T, K] int32 expert ids or NULL */
  const float* grad_weights;  /* [T, K] fp32 */
  float* grad_logits;         /* [T, E] fp32 out, row stride E */
  int32_t accumulate;
  int32_t scoring;            /* MI355MOE_SCORE_* */
  int64_t num_tokens;
  int32_t num_experts;        /* <= 1024 */
  int32_t top_k;              /* <= min(E, 64) */
  float routed_scaling_factor;
  int32_t reserved;
  /* Optional forward diagnostics (the reference's selected_scores / normalization_denominator
   * outputs of mega_gate_route, consumed by its RouteGrad): selected scores [T, K] fp32 and the
   * normalisation denominator [T] fp32 (sum of the selected scores + 1e-20). When given they are
   * used as they are; when NULL they are recomputed from scores and indices in the forward's order. */
  const float* selected_scores;
  const float* denominator;
} MI355MoeRouteGradArgs;
int mi355moe_gate_route_grad(const MI355MoeRouteGradArgs* args, void* stream);

/* ---------------------------------------------------------------------------------------------
 * Dispatch metadata: per-expert histogram (LDS atomics), exclusive scan and the stable
 * permutation of the T*K routed slots (slot s = t*K + k) by expert id.
 * Replaces _resolve_counts / bincount (modules/mega_moe/route.py:186-211), the EP=1 case of
 * _compute_route_metadata (route.py:309-390) and the mapping half of moe_token_permute_out /
 * npu_moe_token_permute (route.py:281-306, torch/csrc/moe_token_permute_out.cpp:50-60).
 *   counts[e]          number of slots routed to e                           (int32)
 *   expert_offsets[e]  exclusive prefix of counts = dispatch_src_off at EP=1  (int64, optional)
 *   group_list[e]      inclusive prefix of counts                             (int64, optional)
 *   mapping[s]         routed row of slot s (scatter map), -1 for an id outside [0, E)
 *   gather_index[r]    slot held by routed row r                              (optional)
 *   error_flag         set to 1 when any id is outside [0, E) (optional, int32)
 * Routed rows are expert-major; within an expert they keep ascending slot order.
 */
typedef struct MI355MoeDispatchArgs {
  const void* topk_ids;       /* [T, K] int32 or int64 */
  int32_t ids_dtype;          /* MI355MOE_IDS_* */
  int32_t top_k;
  int64_t num_tokens;
  int32_t num_experts;        /* <= 4096 */
  int32_t* counts;
  int64_t* expert_offsets;
  int64_t* group_list;
  int32_t* mapping;
  int32_t* gather_index;
  int32_t* error_flag;
} MI355MoeDispatchArgs;
size_t mi355moe_dispatch_workspace_size(int64_t num_tokens, int32_t top_k, int32_t num_experts);
int mi355moe_dispatch(const MI355MoeDispatchArgs* args, void* workspace, size_t workspace_size,
                      void* stream);

/* ---------------------------------------------------------------------------------------------
 * Token permute: routed[mapping[t*K+k]] = x[t]; also writes `mapping` (int32 [T*K]).
 * Replaces hyper_multicore::moe_token_permute_out(tokens, indices, out!, mapping!)
 * (torch/csrc/registration.cpp:15-16, torch/csrc/moe_token_permute_out.cpp:25-72).
 */
int mi355moe_token_permute(const uint16_t* x, int64_t num_tokens, int32_t hidden_size,
                           const void* topk_ids, int32_t ids_dtype, int32_t top_k,
                           int32_t num_experts, uint16_t* routed, int32_t* mapping,
                           void* workspace, size_t workspace_size, void* stream);

/* ---------------------------------------------------------------------------------------------
 * Token unpermute (combine): out[t] = bf16( sum_{k=0..K-1} p[t,k] * y[mapping[t*K+k]] ), fp32
 * accumulation in ascending k, a single bf16 rounding; slots with mapping < 0 contribute 0;
 * probs == NULL means p = 1.
 * Replaces npu_moe_token_unpermute(y, mapping, probs) as used by restore_topk_output
 * (modules/mega_moe/route.py:1029-1051, backends/mxfp8/execution.py:103).
 */
int mi355moe_token_unpermute(const uint16_t* y, const int32_t* mapping, const float* probs,
                             int64_t num_tokens, int32_t top_k, int32_t hidden_size,
                             uint16_t* out, void* stream);

/* ---------------------------------------------------------------------------------------------
 * Token unpermute gradient: for every slot s = t*K + k with routed row r = mapping[s],
 *   grad_permuted[r] = bf16( p[s] * grad_out[t] )   and   grad_probs[s] = sum_h y[r,h] * grad_out[t,h]
 * (fp32 products and accumulation). y = permuted [T*K, H] bf16, grad_out [T, H] bf16, probs fp32 [T, K];
 * rows 16-byte aligned (H % 8 == 0). A slot whose row lies outside [0, T*K) writes no row and
 * grad_probs 0; grad_probs may be NULL. Part of the expert backward (MI355MOE_FEATURE_BACKWARD;
 * -3 while that is switched off).
 * Replaces hyper_multicore::mega_moe_unpermute_grad_out -> aclnnMoeTokenUnpermuteGrad, non-padded
 * (torch/csrc/mega_moe_unpermute.cpp:56-62, registration.cpp:17-20).
 */
int mi355moe_token_unpermute_grad(const uint16_t* permuted, const uint16_t* grad_out, const int32_t* mapping,
                                  const float* probs, int64_t num_tokens, int32_t top_k, int32_t hidden_size,
                                  uint16_t* grad_permuted, float* grad_probs, void* stream);

/* ---------------------------------------------------------------------------------------------
 * MX (OCP MX v1.0) quantisation, e4m3fn elements with one e8m0 scale per 32 elements:
 * scale = 2^(floor(log2(amax)) - 8), element = RNE(v / scale) saturated to +-448.
 * rows:  x [M, N] bf16 -> q [M, N] e4m3, scale [M, N/32] e8m0 (blocks along N).
 *        Replaces the row axis of DynamicMxQuantWithDualAxis (quant_x task,
 *        ops/common/mega_moe/adapters/arch35/quantization/dual_axis_mxfp8_worker.h:39-66).
 * cols:  w [G, Kd, N] bf16 -> col_data [G, Kd, N] e4m3, col_scale [G, Kd/64, N, 2] e8m0
 *        (blocks of 32 along Kd per column) - the forward MX weight root layout
 *        (modules/mega_moe/backends/mxfp8/weights.py:61-86).
 */
int mi355moe_mx_quantize_rows(const uint16_t* x, int64_t rows, int32_t cols, uint8_t* q,
                              uint8_t* scale, void* stream);
int mi355moe_mx_quantize_cols(const uint16_t* w, int32_t groups, int32_t kdim, int32_t cols,
                              uint8_t* col_data, uint8_t* col_scale, void* stream);

/* ---------------------------------------------------------------------------------------------
 * Dual-axis MX weight quantisation: the physical fields of an MXFP8 expert-weight root
 * (modules/mega_moe/backends/mxfp8/weights.py:24-97) from a bf16 weight w [G, M, N] in one pass:
 *   col_data [G, M, N] e4m3, col_scale [G, M/64, N, 2]  (blocks of 32 along M for every column;
 *                                                        the forward axis, = mi355moe_mx_quantize_cols)
 *   row_data [G, M, N] e4m3, row_scale [G, M, N/64, 2]  (blocks of 32 along N for every row; the
 *                                                        backward axis, = mi355moe_mx_quantize_rows
 *                                                        of the [G*M, N] view)
 * Either pair may be NULL (not both). M % 64 == 0 and N % 64 == 0 (weights.py:52-53).
 * Replaces the caller-side dual-axis weight quantisation the reference expects roots to carry
 * (npu_dynamic_mx_quant_with_dual_axis, tests/torch/_replay_mega_moe_arch35.py:55).
 */
int mi355moe_mx_quantize_weight(const uint16_t* w, int32_t groups, int32_t rows, int32_t cols, uint8_t* col_data,
                                uint8_t* col_scale, uint8_t* row_data, uint8_t* row_scale, void* stream);

/* ---------------------------------------------------------------------------------------------
 * MX weight re-layout for the GEMM (no reference counterpart: a one-time weight preparation, like
 * a pre-shuffled weight, that leaves every value and scale unchanged). Takes the forward MX weight
 * root (col_data [G, Kd, N] e4m3, col_scale [G, Kd/64, N, 2]) and writes the same weight with K
 * contiguous: data [G, N, Kd] e4m3 and scale [G, N, ld] e8m0, ld = mi355moe_mx_weight_scale_ld(Kd)
 * (Kd/32 codes per row, zero padded to a multiple of 16). The GEMM then reads weight fragments with
 * plain 16-byte LDS loads instead of transposing byte loads.
 */
int64_t mi355moe_mx_weight_scale_ld(int32_t kdim);
int mi355moe_mx_weight_to_eoi(const uint8_t* col_data, const uint8_t* col_scale, int32_t groups, int32_t kdim,
                              int32_t cols, uint8_t* data, uint8_t* scale, void* stream);

/* ---------------------------------------------------------------------------------------------
 * Gate/up interleave of the GMM1 weight for MI355MOE_LAYOUT_EIO_GU (no reference counterpart: a
 * one-time weight preparation that moves columns and changes no value). src holds `rows` rows of
 * 2I elements of elem_bytes bytes each, gate columns [0, I) then up columns [I, 2I); dst gets, for
 * each 64-column block b, gate columns 64 b ..+63 then up columns 64 b ..+63. Use
 * rows = E * H with elem_bytes 2 (bf16 w1) or 1 (e4m3 col_data), and rows = E * H / 64 with
 * elem_bytes 2 for the MXFP8 col_scale [E, H/64, 2I, 2] (one 2-byte pair per column).
 * I % 128 == 0; src and dst must not overlap. A SwiGLU tile then reads its gate and up columns as
 * one contiguous run per weight row instead of two runs 2I apart.
 */
int mi355moe_interleave_gate_up(const void* src, int64_t rows, int32_t intermediate_size, int32_t elem_bytes,
                                void* dst, void* stream);

/* ---------------------------------------------------------------------------------------------
 * Grouped GEMM over consecutive row segments (one segment per group):
 *   out[r, :] = x[r, :] @ W_g        for rows r of group g,
 * group_list is the int64 inclusive cumulative row count per group (the grouped_matmul
 * group_list convention, tests/common/multicore/moe_reference.py:185-200).
 * bf16 weights: layout EIO -> W_g stored [K, N]; EOI -> stored [N, K].
 * Output bf16 (rounded once from the fp32 accumulator).
 * Replaces the per-expert GMM tasks (ops/hyper_mega_moe/op_kernel/worker_kernel.cpp:225-299).
 */
size_t mi355moe_grouped_gemm_workspace_size(int32_t num_groups);
int mi355moe_grouped_gemm_bf16(const uint16_t* x, int64_t rows, int32_t kdim,
                               const uint16_t* w, int32_t layout, int32_t num_groups,
                               int32_t ndim, const int64_t* group_list, uint16_t* out, int32_t gemm_variant,
                               void* workspace, size_t workspace_size, void* stream);

/* ---------------------------------------------------------------------------------------------
 * mi355moe_grouped_gemm_bf16 without a workspace, for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). No
 * counterpart in the reference. Same arguments and results as mi355moe_grouped_gemm_bf16 (bit-
 * identical), minus the workspace: the tile plan lives in a static device array of
 * MI355MOE_NOALLOC_MAX_GROUPS + 1 int32 per GPU (16 KB, held until the process ends; each call
 * writes all of the plan it reads, so no state carries over). num_groups above the maximum answers
 * MI355MOE_EWORKSPACE_CODE. Calls no hipMalloc / hipFree. Every call on one GPU shares that GPU's
 * array: calls that overlap on one GPU (other streams, other host threads) race and must be
 * ordered by the caller. The first call on a device looks the array's address up (hipGetSymbolAddress)
 * with that device current.
 */
#define MI355MOE_NOALLOC_MAX_GROUPS 4096
int mi355moe_grouped_gemm_bf16_noalloc(const uint16_t* x, int64_t rows, int32_t kdim,
                                       const uint16_t* w, int32_t layout, int32_t num_groups,
                                       int32_t ndim, const int64_t* group_list, uint16_t* out,
                                       int32_t gemm_variant, void* stream);

/* ---------------------------------------------------------------------------------------------
 * MXFP8 grouped GEMM: out[r, :] = dequant(xq[r, :]) @ dequant(W_g), bf16 output, fp32 accumulate.
 * xq [rows, K] e4m3 with x_scale [rows, K/32] e8m0 (blocks along K). Weights by layout:
 *   EIO: w_data = col_data [G, K, N] e4m3, w_scale = col_scale [G, K/64, N, 2] (the forward MX
 *        weight root);
 *   EOI: w_data [G, N, K], w_scale [G, N, mi355moe_mx_weight_scale_ld(K)] (mi355moe_mx_weight_to_eoi).
 * K % 512 == 0, N % 16 == 0.
 * Replaces the MX GMM task (ops/common/mega_moe/adapters/arch35/gmm/mxfp8_worker.h:15-159, NN
 * layout, contracts/mx_gmm_descriptor.h:18-87).
 */
int mi355moe_grouped_gemm_mxfp8(const uint8_t* xq, const uint8_t* x_scale, int64_t rows, int32_t kdim,
                                const uint8_t* w_data, const uint8_t* w_scale, int32_t layout, int32_t num_groups,
                                int32_t ndim, const int64_t* group_list, uint16_t* out, int32_t gemm_variant,
                                void* workspace, size_t workspace_size, void* stream);

/* ---------------------------------------------------------------------------------------------
 * MegaMoE expert forward at EP=1: dispatch -> (MX quant) -> GMM1 + fused SwiGLU (+ MX requant)
 * -> GMM2 -> combine.  Replaces the MegaMoeExperts.forward launch chain
 * (modules/mega_moe/module.py:497-535 -> backends/bf16/autograd.py:398-443 -> hyper_multicore::
 * mega_moe, torch/csrc/registration.cpp:30-60; backends/mxfp8/execution.py:64-117 ->
 * hyper_multicore::mega_moe_mxfp8, torch/csrc/mega_moe_mxfp8.cpp:7-46).
 * SwiGLU: gate = left half of the 2I projection, act = bf16(silu(g) * u) with g, u the bf16
 * GMM1 outputs (tests/common/multicore/fp32_expert_reference.py:22-26).
 * MXFP8: w1/w2 are col_data e4m3 EIO [E,H,2I] / [E,I,H] with col_scale [E,H/64,2I,2] /
 * [E,I/64,H,2] (docs: MXFP8 weight contract), or, with weight_layout EOI, the same weights after
 * mi355moe_mx_weight_to_eoi: [E,2I,H] / [E,H,I] with row scales [E,2I,ld(H)] / [E,H,ld(I)].
 * weight_layout EIO_GU (bf16 and MXFP8): w1 and w1_scale after mi355moe_interleave_gate_up, w2 and
 * w2_scale EIO; results are those of EIO on the original weights, bit for bit.
 * H and I must be multiples of 128.
 * tokens_per_expert (optional) is a trusted int32 histogram of topk_ids; when NULL it is
 * computed. Workspace: mi355moe_moe_forward_workspace_size(args) bytes.
 * BF16 numerics options (MegaMoeNumericsOptions, modules/mega_moe/numerics.py; docs/mega_moe.md
 * "numerics"): swiglu_limit L > 0 clamps the SwiGLU inputs, up to [-L, L] and gate to <= L before
 * SiLU, or SiLU(gate) to <= L after it with MI355MOE_NUMERICS_CLAMP_AFTER_SILU;
 * MI355MOE_NUMERICS_PROBS_BEFORE_FC2 feeds FC2 with bf16(bf16(act) * p) and combines unweighted.
 * MXFP8 rejects both (module.py:132).
 */
enum { MI355MOE_NUMERICS_CLAMP_AFTER_SILU = 1, MI355MOE_NUMERICS_PROBS_BEFORE_FC2 = 2 };
typedef struct MI355MoeForwardArgs {
  const uint16_t* hidden;     /* [T, H] bf16 */
  int64_t num_tokens;
  int32_t hidden_size;
  int32_t intermediate_size;
  int32_t num_experts;
  int32_t top_k;
  const void* topk_ids;       /* [T, K] */
  int32_t ids_dtype;
  int32_t precision;          /* MI355MOE_PRECISION_* */
  const float* topk_weights;  /* [T, K] fp32 */
  int32_t weight_layout;      /* MI355MOE_LAYOUT_* */
  int32_t numerics_flags;     /* MI355MOE_NUMERICS_* bits (BF16 only; MegaMoeNumericsOptions) */
  const void* w1;
  const void* w2;
  const uint8_t* w1_scale;
  const uint8_t* w2_scale;
  const int32_t* tokens_per_expert; /* optional [E] int32 */
  uint16_t* out;              /* [T, H] bf16 */
  int32_t* error_flag;        /* optional: set to 1 for ids outside [0, E) */
  /* Optional timing hooks (no reference counterpart): hipEvent_t handles recorded on `stream`
   * at the stage boundaries [0] start, [1] after dispatch + MX activation quant, [2] after the GMM1
   * kernel, [3] after GMM2 (including the MX quantisation of its input when that is a kernel of its
   * own), [4] after combine. num_stage_events may be 0..5. */
  void* const* stage_events;
  int32_t num_stage_events;
  float swiglu_limit;         /* > 0: SwiGLU clamp limit L (BF16 only); 0: no clamp */
  int32_t gemm_variant;       /* MI355MOE_GEMM_* of both expert GEMMs (0: the default) */
} MI355MoeForwardArgs;
size_t mi355moe_moe_forward_workspace_size(const MI355MoeForwardArgs* args);
int mi355moe_moe_forward(const MI355MoeForwardArgs* args, void* workspace, size_t workspace_size,
                         void* stream);

/* ---------------------------------------------------------------------------------------------
 * MegaMoE expert backward at EP=1, BF16 (the gradients of mi355moe_moe_forward with the default
 * numerics). Replaces MegaMoeFunction.backward (modules/mega_moe/backends/bf16/autograd.py:672-760,
 * the hyper_multicore::mega_moe_grad launch) together with the backward of the combine
 * (restore_topk_output, route.py:1029-1051) and of the permutation (moe_token_permute_grad).
 * The forward intermediates are recomputed. Rounding points follow the reference's fp32 expert
 * reference (tests/common/multicore/fp32_expert_reference.py:27-35):
 *   dY[r] = bf16(p[t,k] * dOut[t]), dp[t,k] = sum_h y[r,h] * dOut[t,h] (fp32),
 *   gA = bf16(dY W2^T), dU = [bf16(gA u s (1 + g (1 - s))) | bf16(gA silu(g))], s = sigmoid(g),
 *   dW2_e = act_e^T dY_e, dW1_e = X_e^T dU_e (fp32 accumulate, stored in weight_grad_dtype),
 *   dX[t] = bf16(sum_k bf16(dU W1^T)[r]).
 * Gradients have the weights' layout. grad_topk_weights may be NULL.
 *
 * precision MXFP8 (EIO weights only, the reference's MX roots): w1 / w2 are the forward axis
 * col_data with w1_scale / w2_scale col_scale (as for mi355moe_moe_forward), and w1_row / w2_row
 * with w1_row_scale / w2_row_scale the backward axis row_data [E, M, N] / row_scale [E, M, N/64, 2]
 * (mi355moe_mx_quantize_weight). The graph follows the reference's MX backward
 * (modules/mega_moe/backends/mxfp8/graph.py:147-154, execution.py:119-164): forward recompute
 * (U bf16, act fp32 quantised along I and along the routed rows, y bf16), dY and dp as above,
 * dY quantised along H and along the routed rows (32-row blocks from each expert's first row),
 * dW2 = Q_rows(act)^T Q_rows(dY), gA = bf16(Q_H(dY) W2_row^T), the SwiGLU gradient kept in fp32
 * and quantised along 2I and along the routed rows, dW1 = Q_rows(X)^T Q_rows(dU),
 * dX_routed = bf16(Q_2I(dU) W1_row^T), dX = bf16(sum_k dX_routed). H % 512 == 0, I % 256 == 0.
 */
enum { MI355MOE_GRAD_BF16 = 0, MI355MOE_GRAD_FP32 = 1 };
typedef struct MI355MoeBackwardArgs {
  const uint16_t* hidden;     /* [T, H] bf16 */
  int64_t num_tokens;
  int32_t hidden_size;
  int32_t intermediate_size;
  int32_t num_experts;
  int32_t top_k;
  const void* topk_ids;       /* [T, K] */
  int32_t ids_dtype;
  int32_t weight_layout;      /* MI355MOE_LAYOUT_* */
  const float* topk_weights;  /* [T, K] fp32 */
  const uint16_t* w1;         /* bf16 EIO [E, H, 2I] or EOI [E, 2I, H] */
  const uint16_t* w2;         /* bf16 EIO [E, I, H] or EOI [E, H, I] */
  const uint16_t* grad_out;   /* [T, H] bf16 */
  uint16_t* grad_hidden;      /* [T, H] bf16 */
  void* grad_w1;              /* like w1, weight_grad_dtype */
  void* grad_w2;              /* like w2, weight_grad_dtype */
  float* grad_topk_weights;   /* optional [T, K] fp32 */
  int32_t weight_grad_dtype;  /* MI355MOE_GRAD_* (partial_weight_grad_dtype native / float32) */
  int32_t precision;          /* MI355MOE_PRECISION_* (0 = BF16) */
  const uint8_t* w1_scale;    /* MXFP8: col_scale [E, H/64, 2I, 2] */
  const uint8_t* w2_scale;    /* MXFP8: col_scale [E, I/64, H, 2] */
  const uint8_t* w1_row;      /* MXFP8: row_data [E, H, 2I] e4m3 */
  const uint8_t* w2_row;      /* MXFP8: row_data [E, I, H] e4m3 */
  const uint8_t* w1_row_scale; /* MXFP8: row_scale [E, H, 2I/64, 2] */
  const uint8_t* w2_row_scale; /* MXFP8: row_scale [E, I, H/64, 2] */
  int32_t* error_flag;        /* optional [1] int32: set to 1 when an id lies outside [0, E) (ABI 4) */
} MI355MoeBackwardArgs;
size_t mi355moe_moe_backward_workspace_size(const MI355MoeBackwardArgs* args);
int mi355moe_moe_backward(const MI355MoeBackwardArgs* args, void* workspace, size_t workspace_size,
                          void* stream);

#ifdef __cplusplus
}
#endif
#endif /* MI355MOE_H_ */
