"""Torch operator layer: ``torch.ops.hyper_multicore_mi355.*``.

The reference registers its path as out-of-tree torch operators in the ``hyper_multicore``
namespace (hyper_multicore/torch/csrc/registration.cpp:14-16, mega_gate_registration.cpp:9-42) with
Meta implementations for shape inference. This module registers the gfx950 path the same way, in
its own ``hyper_multicore_mi355`` namespace, on top of the functional operators of
:mod:`hyper_multicore_amd.ops` (which call the C ABI). Every operator has a fake (Meta) kernel, so
shapes and dtypes propagate under ``FakeTensorMode`` / ``torch.compile`` tracing without the
library or a GPU; the real kernels validate their inputs on the host and raise ``TypeError`` /
``ValueError`` like the reference's ``TORCH_CHECK``s, and fail loudly on CPU tensors (there is no
CPU path).

Operators (schema differences from the reference are noted per operator):

* ``moe_token_permute_out(tokens, indices, output!, mapping!, num_experts=-1)`` — the reference's
  out-variant permute (registration.cpp:15-16); ``num_experts`` is an extra, optional argument
  (-1: ``indices.max() + 1``, which synchronises the host with the stream once).
* ``token_permute(tokens, indices, num_experts) -> (routed, mapping)``.
* ``gate_logits(x, weight, weight_vision?, image_mask?) -> logits`` (fp32 projection).
* ``mega_gate_route(logits, text_bias, vision_bias?, image_mask?, top_k, routed_scaling_factor,
  use_vision_bias, scoring_func, num_groups, topk_groups) -> (weights, indices, route_scores,
  selected_scores, normalization_denominator)`` — the reference's ``mega_gate_route``
  (mega_gate_registration.cpp:19-30) with the scoring function and group limits as arguments instead
  of its ``runtime_config`` bytes (and no diagnostic buffer).
* ``mega_gate_route_grad(logits, route_scores, selected_scores, normalization_denominator,
  expert_indices, grad_routing_weights, top_k, routed_scaling_factor, scoring_func) -> grad_logits``
  (mega_gate_registration.cpp:31-41).
* ``dispatch(topk_ids, num_experts) -> (counts, expert_offsets, group_list, mapping,
  gather_index, error_flag)``.
* ``combine(values, mapping, probs?, top_k) -> out`` (the unpermute) and
  ``mega_moe_unpermute_grad_out(permuted_tokens, grad_output, sorted_indices, probs, grad_permuted!,
  grad_probs!)``, its gradient (registration.cpp:17-20; returns nothing instead of the aliases).
* ``mx_quantize_rows(x) -> (data, scale)``.
* ``grouped_gemm_bf16(x, weights, group_list, layout) -> out``.
* ``grouped_gemm_mxfp8(xq, x_scale, w_data, w_scale, group_list, layout) -> out``.
* ``moe_forward(hidden, topk_ids, topk_weights, w1, w2, w1_scale?, w2_scale?, num_experts,
  intermediate_size, precision, layout, swiglu_limit, clamp_after_silu, apply_probs_before_fc2)
  -> out`` and ``moe_forward_out(..., out!)`` (the reference's ``mega_moe`` writes caller-owned
  buffers, registration.cpp:30-60).
* ``moe_backward(hidden, topk_ids, topk_weights, w1, w2, grad_out, num_experts, intermediate_size,
  layout, fp32_weight_grad) -> (grad_hidden, grad_w1, grad_w2, grad_topk_weights)`` — the bf16
  ``mega_moe_grad`` (registration.cpp:62-107) at EP=1, with its buffers internal.
"""
from __future__ import annotations

from typing import Optional

import torch

from . import _lib, ops

NAMESPACE = "hyper_multicore_mi355"
OPERATORS = ("moe_token_permute_out", "token_permute", "gate_logits", "mega_gate_route", "mega_gate_route_grad",
             "mega_moe_unpermute_grad_out", "dispatch", "combine", "mx_quantize_rows", "grouped_gemm_bf16",
             "grouped_gemm_mxfp8", "moe_forward", "moe_forward_out", "moe_backward")


def _name(op: str) -> str:
    return f"{NAMESPACE}::{op}"


def _check_permute_out(tokens: torch.Tensor, indices: torch.Tensor, output: torch.Tensor,
                       mapping: torch.Tensor) -> tuple[int, int, int]:
    if tokens.dtype != torch.bfloat16 or tokens.ndim != 2:
        raise TypeError("tokens must be bf16 [T, H]")
    if indices.ndim != 2 or indices.dtype not in (torch.int32, torch.int64):
        raise TypeError("indices must be int32/int64 [T, K]")
    T, K = indices.shape
    H = tokens.shape[1]
    if tokens.shape[0] != T:
        raise ValueError("tokens and indices disagree on the token count")
    if output.dtype != torch.bfloat16 or tuple(output.shape) != (T * K, H) or not output.is_contiguous():
        raise ValueError(f"output must be contiguous bf16 [{T * K}, {H}]")
    if mapping.dtype != torch.int32 or tuple(mapping.shape) != (T * K,) or not mapping.is_contiguous():
        raise ValueError(f"mapping must be contiguous int32 [{T * K}]")
    return T, K, H


# ---- permute --------------------------------------------------------------------------------------
@torch.library.custom_op(_name("moe_token_permute_out"), mutates_args=("output", "mapping"))
def moe_token_permute_out(tokens: torch.Tensor, indices: torch.Tensor, output: torch.Tensor, mapping: torch.Tensor,
                          num_experts: int = -1) -> None:
    """routed[mapping[t*K+k]] = tokens[t]; stable by expert id (moe_token_permute_out.cpp:50-60)."""
    lib = _lib.load()
    device = ops._require_gpu(tokens, indices, output, mapping)
    T, K, H = _check_permute_out(tokens, indices, output, mapping)
    ids = indices.contiguous()
    if num_experts < 0:
        num_experts = int(ids.max().item()) + 1 if ids.numel() else 1
    ws = ops._workspace(lib.mi355moe_dispatch_workspace_size(T, K, num_experts), device)
    rc = lib.mi355moe_token_permute(ops._ptr(tokens.contiguous()), T, H, ops._ptr(ids), ops._ids_dtype(ids), K,
                                    num_experts, ops._ptr(output), ops._ptr(mapping), ops._ptr(ws), ws.numel(),
                                    ops._stream(device))
    _lib.check(rc, "mi355moe_token_permute")


@moe_token_permute_out.register_fake
def _(tokens, indices, output, mapping, num_experts=-1):
    _check_permute_out(tokens, indices, output, mapping)


@torch.library.custom_op(_name("token_permute"), mutates_args=())
def token_permute(tokens: torch.Tensor, indices: torch.Tensor, num_experts: int) -> tuple[torch.Tensor, torch.Tensor]:
    return ops.token_permute(tokens, indices, num_experts)


@token_permute.register_fake
def _(tokens, indices, num_experts):
    R = indices.shape[0] * indices.shape[1]
    return tokens.new_empty((R, tokens.shape[1])), tokens.new_empty((R,), dtype=torch.int32)


# ---- MegaGate -------------------------------------------------------------------------------------
@torch.library.custom_op(_name("gate_logits"), mutates_args=())
def gate_logits(x: torch.Tensor, weight: torch.Tensor, weight_vision: Optional[torch.Tensor] = None,
                image_mask: Optional[torch.Tensor] = None) -> torch.Tensor:
    return ops.gate_logits(x, weight, weight_vision, image_mask)


@gate_logits.register_fake
def _(x, weight, weight_vision=None, image_mask=None):
    if x.ndim != 2 or weight.ndim != 2 or weight.shape[1] != x.shape[1]:
        raise ValueError(f"bad router shapes x{tuple(x.shape)} w{tuple(weight.shape)}")
    return x.new_empty((x.shape[0], weight.shape[0]), dtype=torch.float32)


def _selected_and_denominator(scores: torch.Tensor, indices: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """The unbiased scores of the selected experts [T, K] and sum_k of them + 1e-20 [T, 1], summed in
    ascending k from 0 in fp32 as the route kernel normalises (route_pipeline.h:424-466: Sum, then
    Adds 1e-20)."""
    selected = scores.gather(1, indices)
    den = torch.zeros((scores.shape[0], 1), dtype=torch.float32, device=scores.device)
    for k in range(indices.shape[1]):
        den = den + selected[:, k:k + 1]
    return selected, den + 1.0e-20


@torch.library.custom_op(_name("mega_gate_route"), mutates_args=())
def mega_gate_route(logits: torch.Tensor, text_bias: torch.Tensor, vision_bias: Optional[torch.Tensor],
                    image_mask: Optional[torch.Tensor], top_k: int, routed_scaling_factor: float,
                    use_vision_bias: bool, scoring_func: str = "sigmoid", num_groups: int = 1,
                    topk_groups: int = 1) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor,
                                                   torch.Tensor]:
    """(routing weights fp32 [T, K], expert indices int64 [T, K], unbiased route scores fp32 [T, E],
    selected scores fp32 [T, K], normalization denominator fp32 [T, 1]) like the reference's five
    outputs (mega_gate.cpp:65-82)."""
    if use_vision_bias and (vision_bias is None or image_mask is None):
        raise ValueError("use_vision_bias needs vision_bias and image_mask")
    w, ids, scores = ops.gate_route(logits, text_bias, top_k=top_k, scoring_func=scoring_func,
                                    routed_scaling_factor=routed_scaling_factor,
                                    bias_vl=vision_bias if use_vision_bias else None,
                                    image_mask=image_mask if use_vision_bias else None, num_groups=num_groups,
                                    topk_groups=topk_groups, return_scores=True)
    selected, den = _selected_and_denominator(scores, ids)
    return w, ids, scores, selected, den


@mega_gate_route.register_fake
def _(logits, text_bias, vision_bias, image_mask, top_k, routed_scaling_factor, use_vision_bias,
      scoring_func="sigmoid", num_groups=1, topk_groups=1):
    if logits.ndim != 2:
        raise TypeError("logits must be fp32 [tokens, experts]")
    T = logits.shape[0]
    f = torch.float32
    return (logits.new_empty((T, top_k), dtype=f), logits.new_empty((T, top_k), dtype=torch.int64),
            logits.new_empty(tuple(logits.shape), dtype=f), logits.new_empty((T, top_k), dtype=f),
            logits.new_empty((T, 1), dtype=f))


def _check_route_grad(logits, route_scores, selected_scores, normalization_denominator, expert_indices,
                      grad_routing_weights) -> None:
    T = logits.shape[0]
    if (route_scores.shape != logits.shape or selected_scores.shape != grad_routing_weights.shape
            or tuple(normalization_denominator.shape) != (T, 1) or expert_indices.shape != grad_routing_weights.shape):
        raise ValueError("route gradient shapes must match the forward's outputs")


@torch.library.custom_op(_name("mega_gate_route_grad"), mutates_args=())
def mega_gate_route_grad(logits: torch.Tensor, route_scores: torch.Tensor, selected_scores: torch.Tensor,
                         normalization_denominator: torch.Tensor, expert_indices: torch.Tensor,
                         grad_routing_weights: torch.Tensor, top_k: int, routed_scaling_factor: float,
                         scoring_func: str = "sigmoid") -> torch.Tensor:
    """Gradient of the routing weights with respect to the logits (mega_gate_registration.cpp:31-41).
    The selected scores and the denominator are consumed as given, like the reference's RouteGrad."""
    _check_route_grad(logits, route_scores, selected_scores, normalization_denominator, expert_indices,
                      grad_routing_weights)
    return ops.gate_route_grad(logits, route_scores, expert_indices, grad_routing_weights, top_k=top_k,
                               scoring_func=scoring_func, routed_scaling_factor=routed_scaling_factor,
                               selected_scores=selected_scores, denominator=normalization_denominator)


@mega_gate_route_grad.register_fake
def _(logits, route_scores, selected_scores, normalization_denominator, expert_indices, grad_routing_weights, top_k,
      routed_scaling_factor, scoring_func="sigmoid"):
    _check_route_grad(logits, route_scores, selected_scores, normalization_denominator, expert_indices,
                      grad_routing_weights)
    return logits.new_empty(tuple(logits.shape), dtype=torch.float32)


# ---- dispatch / combine ---------------------------------------------------------------------------
@torch.library.custom_op(_name("dispatch"), mutates_args=())
def dispatch(topk_ids: torch.Tensor, num_experts: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor,
                                                                 torch.Tensor, torch.Tensor, torch.Tensor]:
    d = ops.dispatch(topk_ids, num_experts)
    return d.counts, d.expert_offsets, d.group_list, d.mapping, d.gather_index, d.error_flag


@dispatch.register_fake
def _(topk_ids, num_experts):
    if topk_ids.ndim != 2:
        raise ValueError("topk_ids must be [tokens, top_k]")
    R = topk_ids.shape[0] * topk_ids.shape[1]
    e = topk_ids.new_empty
    return (e((num_experts,), dtype=torch.int32), e((num_experts,), dtype=torch.int64),
            e((num_experts,), dtype=torch.int64), e((R,), dtype=torch.int32), e((R,), dtype=torch.int32),
            e((1,), dtype=torch.int32))


@torch.library.custom_op(_name("combine"), mutates_args=())
def combine(values: torch.Tensor, mapping: torch.Tensor, probs: Optional[torch.Tensor], top_k: int) -> torch.Tensor:
    return ops.token_unpermute(values, mapping, probs, top_k)


@combine.register_fake
def _(values, mapping, probs, top_k):
    if mapping.numel() % top_k:
        raise ValueError("mapping must be int32 [T*K]")
    return values.new_empty((mapping.numel() // top_k, values.shape[1]))


def _check_unpermute_grad(permuted_tokens, grad_output, sorted_indices, probs, grad_permuted, grad_probs) -> None:
    if permuted_tokens.ndim != 2 or grad_output.ndim != 2 or probs.ndim != 2 or sorted_indices.ndim != 1:
        raise ValueError("unpermute requires matrix tokens, gradients and probabilities, and flat indices")
    if grad_permuted.shape != permuted_tokens.shape or grad_probs.shape != probs.shape:
        raise ValueError("unpermute output shapes must match tokens and probabilities")
    if (permuted_tokens.shape[1] != grad_output.shape[1] or grad_output.shape[0] != probs.shape[0]
            or permuted_tokens.shape[0] != probs.numel() or sorted_indices.numel() != permuted_tokens.shape[0]):
        raise ValueError("unpermute requires all top-k rows without padding or dropped tokens")


@torch.library.custom_op(_name("mega_moe_unpermute_grad_out"), mutates_args=("grad_permuted", "grad_probs"))
def mega_moe_unpermute_grad_out(permuted_tokens: torch.Tensor, grad_output: torch.Tensor,
                                sorted_indices: torch.Tensor, probs: torch.Tensor, grad_permuted: torch.Tensor,
                                grad_probs: torch.Tensor) -> None:
    """The reference's out-variant unpermute gradient (registration.cpp:17-20,
    mega_moe_unpermute.cpp:16-62); ``sorted_indices`` is the slot -> routed-row mapping."""
    _check_unpermute_grad(permuted_tokens, grad_output, sorted_indices, probs, grad_permuted, grad_probs)
    ops.token_unpermute_grad(permuted_tokens, grad_output, sorted_indices, probs, probs.shape[1],
                             grad_values=grad_permuted, grad_probs=grad_probs)


@mega_moe_unpermute_grad_out.register_fake
def _(permuted_tokens, grad_output, sorted_indices, probs, grad_permuted, grad_probs):
    _check_unpermute_grad(permuted_tokens, grad_output, sorted_indices, probs, grad_permuted, grad_probs)


# ---- MX quantisation and grouped GEMMs ------------------------------------------------------------
@torch.library.custom_op(_name("mx_quantize_rows"), mutates_args=())
def mx_quantize_rows(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    return ops.mx_quantize_rows(x)


@mx_quantize_rows.register_fake
def _(x):
    if x.ndim != 2 or x.shape[1] % 32:
        raise ValueError("mx_quantize_rows takes bf16 [M, N] with N % 32 == 0")
    M, N = x.shape
    return x.new_empty((M, N), dtype=torch.uint8), x.new_empty((M, N // 32), dtype=torch.uint8)


def _gemm_n(weights: torch.Tensor, layout: str) -> int:
    if layout == "EIO":
        return weights.shape[2]
    if layout == "EOI":
        return weights.shape[1]
    raise ValueError(f"unknown layout {layout!r}")


@torch.library.custom_op(_name("grouped_gemm_bf16"), mutates_args=())
def grouped_gemm_bf16(x: torch.Tensor, weights: torch.Tensor, group_list: torch.Tensor,
                      layout: str = "EIO") -> torch.Tensor:
    return ops.grouped_gemm_bf16(x, weights, group_list, layout)


@grouped_gemm_bf16.register_fake
def _(x, weights, group_list, layout="EIO"):
    return x.new_empty((x.shape[0], _gemm_n(weights, layout)), dtype=torch.bfloat16)


@torch.library.custom_op(_name("grouped_gemm_mxfp8"), mutates_args=())
def grouped_gemm_mxfp8(xq: torch.Tensor, x_scale: torch.Tensor, w_data: torch.Tensor, w_scale: torch.Tensor,
                       group_list: torch.Tensor, layout: str = "EIO") -> torch.Tensor:
    return ops.grouped_gemm_mxfp8(xq, x_scale, w_data, w_scale, group_list, layout)


@grouped_gemm_mxfp8.register_fake
def _(xq, x_scale, w_data, w_scale, group_list, layout="EIO"):
    return xq.new_empty((xq.shape[0], _gemm_n(w_data, layout)), dtype=torch.bfloat16)


# ---- expert forward -------------------------------------------------------------------------------
def _check_forward(hidden: torch.Tensor, topk_ids: torch.Tensor, topk_weights: torch.Tensor, precision: str,
                   layout: str) -> None:
    if hidden.dtype != torch.bfloat16 or hidden.ndim != 2:
        raise TypeError("hidden must be bf16 [T, H]")
    if topk_ids.ndim != 2 or topk_ids.shape[0] != hidden.shape[0]:
        raise ValueError("topk_ids must be [T, K] with the hidden states' T")
    if tuple(topk_weights.shape) != tuple(topk_ids.shape):
        raise ValueError("topk_weights must be [T, K] like topk_ids")
    if precision not in _lib.PRECISION:
        raise ValueError(f"unknown precision {precision!r}")
    if layout not in _lib.LAYOUT:
        raise ValueError(f"unknown layout {layout!r}")


@torch.library.custom_op(_name("moe_forward"), mutates_args=())
def moe_forward(hidden: torch.Tensor, topk_ids: torch.Tensor, topk_weights: torch.Tensor, w1: torch.Tensor,
                w2: torch.Tensor, w1_scale: Optional[torch.Tensor], w2_scale: Optional[torch.Tensor],
                num_experts: int, intermediate_size: int, precision: str = "bf16", layout: str = "EIO",
                swiglu_limit: float = 0.0, clamp_after_silu: bool = False,
                apply_probs_before_fc2: bool = False) -> torch.Tensor:
    """bf16 [T, H]; ``swiglu_limit`` 0 = no clamp (the numerics options of MegaMoeNumericsOptions)."""
    _check_forward(hidden, topk_ids, topk_weights, precision, layout)
    return ops.moe_forward(hidden, topk_ids, topk_weights, w1, w2, num_experts=num_experts,
                           intermediate_size=intermediate_size, precision=precision, layout=layout,
                           w1_scale=w1_scale, w2_scale=w2_scale, swiglu_limit=swiglu_limit or None,
                           clamp_after_silu=clamp_after_silu, apply_probs_before_fc2=apply_probs_before_fc2)


@moe_forward.register_fake
def _(hidden, topk_ids, topk_weights, w1, w2, w1_scale, w2_scale, num_experts, intermediate_size, precision="bf16",
      layout="EIO", swiglu_limit=0.0, clamp_after_silu=False, apply_probs_before_fc2=False):
    _check_forward(hidden, topk_ids, topk_weights, precision, layout)
    return hidden.new_empty(tuple(hidden.shape))


@torch.library.custom_op(_name("moe_forward_out"), mutates_args=("out",))
def moe_forward_out(hidden: torch.Tensor, topk_ids: torch.Tensor, topk_weights: torch.Tensor, w1: torch.Tensor,
                    w2: torch.Tensor, w1_scale: Optional[torch.Tensor], w2_scale: Optional[torch.Tensor],
                    num_experts: int, intermediate_size: int, out: torch.Tensor, precision: str = "bf16",
                    layout: str = "EIO", swiglu_limit: float = 0.0, clamp_after_silu: bool = False,
                    apply_probs_before_fc2: bool = False) -> None:
    """As ``moe_forward``, written into the caller's contiguous bf16 ``out`` [T, H]."""
    _check_forward(hidden, topk_ids, topk_weights, precision, layout)
    if out.dtype != torch.bfloat16 or out.shape != hidden.shape or not out.is_contiguous():
        raise ValueError("out must be contiguous bf16 shaped like hidden")
    ops._require_gpu(hidden, out)
    ops.moe_forward(hidden, topk_ids, topk_weights, w1, w2, num_experts=num_experts,
                    intermediate_size=intermediate_size, precision=precision, layout=layout, w1_scale=w1_scale,
                    w2_scale=w2_scale, out=out, swiglu_limit=swiglu_limit or None,
                    clamp_after_silu=clamp_after_silu, apply_probs_before_fc2=apply_probs_before_fc2)


@moe_forward_out.register_fake
def _(hidden, topk_ids, topk_weights, w1, w2, w1_scale, w2_scale, num_experts, intermediate_size, out,
      precision="bf16", layout="EIO", swiglu_limit=0.0, clamp_after_silu=False, apply_probs_before_fc2=False):
    _check_forward(hidden, topk_ids, topk_weights, precision, layout)
    if out.shape != hidden.shape:
        raise ValueError("out must be shaped like hidden")


@torch.library.custom_op(_name("moe_backward"), mutates_args=())
def moe_backward(hidden: torch.Tensor, topk_ids: torch.Tensor, topk_weights: torch.Tensor, w1: torch.Tensor,
                 w2: torch.Tensor, grad_out: torch.Tensor, num_experts: int, intermediate_size: int,
                 layout: str = "EIO", fp32_weight_grad: bool = False
                 ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """Gradients of the bf16 ``moe_forward`` (default numerics): (grad_hidden bf16 [T, H], grad_w1,
    grad_w2 in the weights' layout, fp32 when ``fp32_weight_grad`` else bf16, grad_topk_weights fp32
    [T, K]); the reference's ``mega_moe_grad`` (registration.cpp:62-107) at EP=1. Needs the expert
    backward switched on in the library."""
    _check_forward(hidden, topk_ids, topk_weights, "bf16", layout)
    gx, g1, g2, gp = ops.moe_backward(hidden, topk_ids, topk_weights, w1, w2, grad_out, num_experts=num_experts,
                                      intermediate_size=intermediate_size, layout=layout,
                                      weight_grad_dtype=torch.float32 if fp32_weight_grad else torch.bfloat16,
                                      need_topk_grad=True)
    return gx, g1, g2, gp


@moe_backward.register_fake
def _(hidden, topk_ids, topk_weights, w1, w2, grad_out, num_experts, intermediate_size, layout="EIO",
      fp32_weight_grad=False):
    _check_forward(hidden, topk_ids, topk_weights, "bf16", layout)
    if grad_out.shape != hidden.shape:
        raise ValueError("grad_out must be shaped like hidden")
    wd = torch.float32 if fp32_weight_grad else torch.bfloat16
    return (hidden.new_empty(tuple(hidden.shape)), w1.new_empty(tuple(w1.shape), dtype=wd),
            w2.new_empty(tuple(w2.shape), dtype=wd), hidden.new_empty(tuple(topk_ids.shape), dtype=torch.float32))
