"""Functional torch-level operators over the gfx950 C ABI (``include/mi355moe.h``).

Every operator validates dtype / device / shape on the host (raising ``ValueError`` or
``TypeError`` like the reference's torch op layer, torch/csrc/*.cpp ``TORCH_CHECK``s), allocates
its outputs and workspace with torch's caching allocator and enqueues the HIP kernels on the
current stream. Nothing here synchronises the host and nothing falls back to a CPU path.
"""
from __future__ import annotations

import contextvars
import ctypes
import math
import os
from dataclasses import dataclass

import torch

from . import _lib


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _require_gpu(*tensors: torch.Tensor) -> torch.device:
    device = None
    for t in tensors:
        if t is None:
            continue
        if not isinstance(t, torch.Tensor):
            raise TypeError("expected a torch.Tensor")
        if t.device.type != "cuda":
            raise TypeError(f"gfx950 operators need tensors on the GPU, got {t.device}")
        if device is None:
            device = t.device
        elif t.device != device:
            raise ValueError("all tensors must be on the same GPU")
    return device


def _workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


def _ids_dtype(ids: torch.Tensor) -> int:
    if ids.dtype == torch.int32:
        return _lib.IDS_INT32
    if ids.dtype == torch.int64:
        return _lib.IDS_INT64
    raise TypeError("topk_ids must be int32 or int64")


# ------------------------------------------------------------------------------------------------
# MegaGate
# ------------------------------------------------------------------------------------------------
def gate_logits(x: torch.Tensor, weight: torch.Tensor, weight_vision: torch.Tensor | None = None,
                image_mask: torch.Tensor | None = None) -> torch.Tensor:
    """fp32 logits [T, E] = x [T, H] (bf16) @ weight[E, H]^T (bf16), fp32 accumulation.

    With ``weight_vision`` and ``image_mask`` ([T] bool), masked tokens use ``weight_vision``.
    """
    lib = _lib.load()
    device = _require_gpu(x, weight, weight_vision, image_mask)
    if x.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise TypeError("router projection takes bf16 hidden states and bf16 weights")
    if x.ndim != 2 or weight.ndim != 2 or weight.shape[1] != x.shape[1]:
        raise ValueError(f"bad router shapes x{tuple(x.shape)} w{tuple(weight.shape)}")
    if (weight_vision is None) != (image_mask is None):
        raise ValueError("weight_vision and image_mask go together")
    if weight_vision is not None:
        if weight_vision.shape != weight.shape or weight_vision.dtype != torch.bfloat16:
            raise ValueError("weight_vision must match weight")
        if image_mask.dtype != torch.bool or image_mask.numel() != x.shape[0]:
            raise ValueError("image_mask must be bool [T]")
        weight_vision = weight_vision.contiguous()
        image_mask = image_mask.reshape(-1).contiguous()
    x = x.contiguous()
    weight = weight.contiguous()
    T, H = x.shape
    E = weight.shape[0]
    out = torch.empty((T, E), dtype=torch.float32, device=device)
    ws = _workspace(lib.mi355moe_gate_logits_workspace_size(T, H, E), device)
    rc = lib.mi355moe_gate_logits(_ptr(x), T, H, _ptr(weight), _ptr(weight_vision), _ptr(image_mask), E,
                                  _ptr(out), _ptr(ws), ws.numel(), _stream(device))
    _lib.check(rc, "mi355moe_gate_logits")
    return out


def gate_route(logits: torch.Tensor, bias: torch.Tensor, *, top_k: int, scoring_func: str,
               routed_scaling_factor: float, bias_vl: torch.Tensor | None = None,
               image_mask: torch.Tensor | None = None, num_groups: int = 1, topk_groups: int = 1,
               return_scores: bool = False):
    """Route fp32 logits [T, E]: returns (weights fp32 [T,K], indices int64 [T,K][, scores [T,E]]).

    Mirrors hyper_multicore::mega_gate_route (torch/csrc/mega_gate.cpp:65-82) for all three
    scoring functions, plus the group-limited selection when ``num_groups > 1``.
    """
    lib = _lib.load()
    device = _require_gpu(logits, bias, bias_vl, image_mask)
    if logits.dtype != torch.float32 or logits.ndim != 2:
        raise TypeError("logits must be fp32 [tokens, experts]")
    T, E = logits.shape
    if bias.dtype != torch.float32 or bias.shape != (E,):
        raise ValueError("bias must be fp32 [num_experts]")
    if bias_vl is not None and (bias_vl.dtype != torch.float32 or bias_vl.shape != (E,)):
        raise ValueError("bias_vl must be fp32 [num_experts]")
    if image_mask is not None:
        if image_mask.dtype != torch.bool or image_mask.numel() != T:
            raise ValueError("image_mask must be bool with one entry per token")
        image_mask = image_mask.reshape(-1).contiguous()
    if scoring_func not in _lib.SCORE:
        raise ValueError(f"unsupported scoring_func: {scoring_func!r}")
    if logits.stride(1) != 1:
        logits = logits.contiguous()
    weights = torch.empty((T, top_k), dtype=torch.float32, device=device)
    indices = torch.empty((T, top_k), dtype=torch.int64, device=device)
    scores = torch.empty((T, E), dtype=torch.float32, device=device) if return_scores else None
    args = _lib.RouteArgs(
        logits=_ptr(logits), logits_row_stride=logits.stride(0), bias=_ptr(bias.contiguous()),
        bias_vl=_ptr(bias_vl.contiguous() if bias_vl is not None else None), image_mask=_ptr(image_mask),
        weights_out=_ptr(weights), indices_out=_ptr(indices), indices32_out=None, scores_out=_ptr(scores),
        num_tokens=T, num_experts=E, top_k=top_k, scoring=_lib.SCORE[scoring_func], num_groups=num_groups,
        topk_groups=topk_groups, routed_scaling_factor=float(routed_scaling_factor))
    rc = lib.mi355moe_gate_route(ctypes.byref(args), _stream(device))
    _lib.check(rc, "mi355moe_gate_route")
    return (weights, indices, scores) if return_scores else (weights, indices)


def gate_route_grad(logits: torch.Tensor, scores: torch.Tensor, indices: torch.Tensor, grad_weights: torch.Tensor, *,
                    top_k: int, scoring_func: str, routed_scaling_factor: float,
                    grad_logits: torch.Tensor | None = None, selected_scores: torch.Tensor | None = None,
                    denominator: torch.Tensor | None = None) -> torch.Tensor:
    """Gradient of the routing weights w.r.t. the fp32 logits (RouteGrad), fp32 [T, E].

    Mirrors hyper_multicore::mega_gate_route_grad (torch/csrc/mega_gate.cpp:182-197) for the three
    scoring functions; ``scores`` are the forward's unbiased scores (``gate_route(...,
    return_scores=True)``). When ``grad_logits`` is given the route gradient is added to it in place
    (the gradient the logits output already carries) and it is returned. ``selected_scores`` fp32
    [T, K] and ``denominator`` fp32 [T, 1] (the forward's diagnostics) are used as given; without them
    both are recomputed from ``scores`` and ``indices`` in the forward's order.
    """
    lib = _lib.load()
    device = _require_gpu(logits, scores, indices, grad_weights, grad_logits, selected_scores, denominator)
    if logits.dtype != torch.float32 or logits.ndim != 2 or logits.stride(1) != 1:
        raise TypeError("logits must be fp32 [tokens, experts] with contiguous rows")
    T, E = logits.shape
    if scores.dtype != torch.float32 or scores.shape != (T, E) or not scores.is_contiguous():
        raise ValueError("scores must be contiguous fp32 [tokens, experts]")
    if indices.shape != (T, top_k) or indices.dtype not in (torch.int64, torch.int32):
        raise ValueError("indices must be int32/int64 [tokens, top_k]")
    if grad_weights.shape != (T, top_k):
        raise ValueError("grad_weights must be [tokens, top_k]")
    if scoring_func not in _lib.SCORE:
        raise ValueError(f"unsupported scoring_func: {scoring_func!r}")
    indices = indices.contiguous()
    grad_weights = grad_weights.to(torch.float32).contiguous()
    accumulate = grad_logits is not None
    if accumulate:
        if grad_logits.dtype != torch.float32 or grad_logits.shape != (T, E) or not grad_logits.is_contiguous():
            raise ValueError("grad_logits must be contiguous fp32 [tokens, experts]")
        out = grad_logits
    else:
        out = torch.empty((T, E), dtype=torch.float32, device=device)
    if selected_scores is not None:
        if selected_scores.dtype != torch.float32 or selected_scores.shape != (T, top_k):
            raise ValueError("selected_scores must be fp32 [tokens, top_k]")
        selected_scores = selected_scores.contiguous()
    if denominator is not None:
        if denominator.dtype != torch.float32 or denominator.numel() != T or denominator.shape[0] != T:
            raise ValueError("denominator must be fp32 [tokens, 1]")
        denominator = denominator.contiguous()
    i64 = indices.dtype == torch.int64
    args = _lib.RouteGradArgs(
        logits=_ptr(logits), logits_row_stride=logits.stride(0), scores=_ptr(scores),
        indices=_ptr(indices) if i64 else None, indices32=None if i64 else _ptr(indices),
        grad_weights=_ptr(grad_weights), grad_logits=_ptr(out), accumulate=int(accumulate),
        scoring=_lib.SCORE[scoring_func], num_tokens=T, num_experts=E, top_k=top_k,
        routed_scaling_factor=float(routed_scaling_factor), reserved=0,
        selected_scores=_ptr(selected_scores), denominator=_ptr(denominator))
    rc = lib.mi355moe_gate_route_grad(ctypes.byref(args), _stream(device))
    _lib.check(rc, "mi355moe_gate_route_grad")
    return out


# ------------------------------------------------------------------------------------------------
# Dispatch / permute / combine
# ------------------------------------------------------------------------------------------------
@dataclass
class DispatchResult:
    """Route metadata at EP=1 (modules/mega_moe/route.py RouteMetadata fields that survive EP=1)."""

    counts: torch.Tensor          # int32 [E]
    expert_offsets: torch.Tensor  # int64 [E] exclusive prefix (dispatch_src_off)
    group_list: torch.Tensor      # int64 [E] inclusive prefix
    mapping: torch.Tensor         # int32 [T*K] slot -> routed row
    gather_index: torch.Tensor    # int32 [T*K] routed row -> slot
    error_flag: torch.Tensor      # int32 [1], 1 if an id was outside [0, E)


def dispatch(topk_ids: torch.Tensor, num_experts: int) -> DispatchResult:
    """Histogram + scan + stable permutation of the routed slots of ``topk_ids`` [T, K]."""
    lib = _lib.load()
    device = _require_gpu(topk_ids)
    if topk_ids.ndim != 2:
        raise ValueError("topk_ids must be [tokens, top_k]")
    ids = topk_ids.contiguous()
    T, K = ids.shape
    R = T * K
    counts = torch.empty(num_experts, dtype=torch.int32, device=device)
    offsets = torch.empty(num_experts, dtype=torch.int64, device=device)
    group_list = torch.empty(num_experts, dtype=torch.int64, device=device)
    mapping = torch.empty(R, dtype=torch.int32, device=device)
    gather = torch.empty(R, dtype=torch.int32, device=device)
    err = torch.zeros(1, dtype=torch.int32, device=device)
    ws = _workspace(lib.mi355moe_dispatch_workspace_size(T, K, num_experts), device)
    args = _lib.DispatchArgs(topk_ids=_ptr(ids), ids_dtype=_ids_dtype(ids), top_k=K, num_tokens=T,
                             num_experts=num_experts, counts=_ptr(counts), expert_offsets=_ptr(offsets),
                             group_list=_ptr(group_list), mapping=_ptr(mapping), gather_index=_ptr(gather),
                             error_flag=_ptr(err))
    rc = lib.mi355moe_dispatch(ctypes.byref(args), _ptr(ws), ws.numel(), _stream(device))
    _lib.check(rc, "mi355moe_dispatch")
    return DispatchResult(counts, offsets, group_list, mapping, gather, err)


def token_permute(tokens: torch.Tensor, topk_ids: torch.Tensor, num_experts: int):
    """(routed bf16 [T*K, H], mapping int32 [T*K]) like npu_moe_token_permute (route.py:281-295)."""
    lib = _lib.load()
    device = _require_gpu(tokens, topk_ids)
    if tokens.dtype != torch.bfloat16 or tokens.ndim != 2:
        raise TypeError("tokens must be bf16 [T, H]")
    ids = topk_ids.contiguous()
    T, K = ids.shape
    if tokens.shape[0] != T:
        raise ValueError("tokens and topk_ids disagree on the token count")
    H = tokens.shape[1]
    x = tokens.contiguous()
    routed = torch.empty((T * K, H), dtype=torch.bfloat16, device=device)
    mapping = torch.empty(T * K, dtype=torch.int32, device=device)
    ws = _workspace(lib.mi355moe_dispatch_workspace_size(T, K, num_experts), device)
    rc = lib.mi355moe_token_permute(_ptr(x), T, H, _ptr(ids), _ids_dtype(ids), K, num_experts, _ptr(routed),
                                    _ptr(mapping), _ptr(ws), ws.numel(), _stream(device))
    _lib.check(rc, "mi355moe_token_permute")
    return routed, mapping


def token_unpermute(values: torch.Tensor, mapping: torch.Tensor, probs: torch.Tensor | None,
                    top_k: int) -> torch.Tensor:
    """out[t] = bf16(sum_k probs[t,k] * values[mapping[t*K+k]]) in ascending k, fp32 accumulate."""
    lib = _lib.load()
    device = _require_gpu(values, mapping, probs)
    if values.dtype != torch.bfloat16 or values.ndim != 2:
        raise TypeError("values must be bf16 [rows, H]")
    if mapping.dtype != torch.int32 or mapping.numel() % top_k:
        raise ValueError("mapping must be int32 [T*K]")
    T = mapping.numel() // top_k
    H = values.shape[1]
    if probs is not None:
        if probs.shape != (T, top_k):
            raise ValueError("probs must be [T, K]")
        probs = probs.to(torch.float32).contiguous()
    out = torch.empty((T, H), dtype=torch.bfloat16, device=device)
    rc = lib.mi355moe_token_unpermute(_ptr(values.contiguous()), _ptr(mapping.contiguous()), _ptr(probs), T,
                                      top_k, H, _ptr(out), _stream(device))
    _lib.check(rc, "mi355moe_token_unpermute")
    return out


def _overlaps(a: torch.Tensor | None, b: torch.Tensor | None) -> bool:
    """Whether the memory of two tensors intersects (their element spans)."""
    if a is None or b is None or a.numel() == 0 or b.numel() == 0:
        return False
    def span(t):  # [first byte, one past the last byte) of the elements
        last = sum((n - 1) * st for n, st in zip(t.shape, t.stride()))
        return t.data_ptr(), t.data_ptr() + (last + 1) * t.element_size()
    (a0, a1), (b0, b1) = span(a), span(b)
    return a0 < b1 and b0 < a1


def token_unpermute_grad(values: torch.Tensor, grad_out: torch.Tensor, mapping: torch.Tensor, probs: torch.Tensor,
                         top_k: int, *, grad_values: torch.Tensor | None = None,
                         grad_probs: torch.Tensor | None = None):
    """Gradient of :func:`token_unpermute` with probabilities: (grad_values bf16 [T*K, H] with
    grad_values[mapping[t*K+k]] = bf16(p[t,k] * grad_out[t]), grad_probs fp32 [T, K] with
    grad_probs[t,k] = <values[mapping[t*K+k]], grad_out[t]>), like hyper_multicore::
    mega_moe_unpermute_grad_out (torch/csrc/mega_moe_unpermute.cpp:16-62). Written into
    ``grad_values`` / ``grad_probs`` when given (contiguous, shaped as above); rows of grad_values that
    no slot maps to are zero in a freshly allocated result and left as they are in a given one. The
    outputs may not overlap the inputs or each other (mega_moe_unpermute.cpp:47-52)."""
    lib = _lib.load()
    device = _require_gpu(values, grad_out, mapping, probs, grad_values, grad_probs)
    if values.dtype != torch.bfloat16 or grad_out.dtype != torch.bfloat16 or values.ndim != 2 or grad_out.ndim != 2:
        raise TypeError("values and grad_out must be bf16 matrices")
    if mapping.dtype != torch.int32 or mapping.ndim != 1 or probs.dtype != torch.float32:
        raise TypeError("mapping must be int32 [T*K] and probs float32 [T, K]")
    T, H = grad_out.shape
    if probs.shape != (T, top_k) or mapping.numel() != T * top_k or values.shape != (T * top_k, H):
        raise ValueError("unpermute gradient needs all top-k rows: values [T*K, H], probs [T, K], mapping [T*K]")
    for out_t, name in ((grad_values, "grad_values"), (grad_probs, "grad_probs")):
        if any(_overlaps(out_t, t) for t in (values, grad_out, mapping, probs)):
            raise ValueError(f"{name} must not overlap the inputs")
    if _overlaps(grad_values, grad_probs):
        raise ValueError("grad_values and grad_probs must not overlap")
    if grad_values is None:
        grad_values = torch.zeros((T * top_k, H), dtype=torch.bfloat16, device=device)
    if grad_probs is None:
        grad_probs = torch.empty((T, top_k), dtype=torch.float32, device=device)
    if (grad_values.shape != values.shape or grad_values.dtype != torch.bfloat16 or not grad_values.is_contiguous()
            or grad_probs.shape != probs.shape or grad_probs.dtype != torch.float32 or not grad_probs.is_contiguous()):
        raise ValueError("grad_values / grad_probs must be contiguous and shaped like values / probs")
    rc = lib.mi355moe_token_unpermute_grad(_ptr(values.contiguous()), _ptr(grad_out.contiguous()),
                                           _ptr(mapping.contiguous()), _ptr(probs.contiguous()), T, top_k, H,
                                           _ptr(grad_values), _ptr(grad_probs), _stream(device))
    _lib.check(rc, "mi355moe_token_unpermute_grad")
    return grad_values, grad_probs


# ------------------------------------------------------------------------------------------------
# MX quantisation
# ------------------------------------------------------------------------------------------------
def mx_quantize_rows(x: torch.Tensor):
    """bf16 [M, N] -> (e4m3 data uint8 [M, N], e8m0 scale uint8 [M, N/32]); blocks along N."""
    lib = _lib.load()
    device = _require_gpu(x)
    if x.dtype != torch.bfloat16 or x.ndim != 2 or x.shape[1] % 32:
        raise ValueError("mx_quantize_rows takes bf16 [M, N] with N % 32 == 0")
    x = x.contiguous()
    M, N = x.shape
    q = torch.empty((M, N), dtype=torch.uint8, device=device)
    s = torch.empty((M, N // 32), dtype=torch.uint8, device=device)
    _lib.check(lib.mi355moe_mx_quantize_rows(_ptr(x), M, N, _ptr(q), _ptr(s), _stream(device)),
               "mi355moe_mx_quantize_rows")
    return q, s


def mx_quantize_cols(w: torch.Tensor):
    """bf16 [G, K, N] -> (col_data e4m3fn [G, K, N], col_scale uint8 [G, K/64, N, 2])."""
    lib = _lib.load()
    device = _require_gpu(w)
    if w.dtype != torch.bfloat16 or w.ndim != 3 or w.shape[1] % 64:
        raise ValueError("mx_quantize_cols takes bf16 [G, K, N] with K % 64 == 0")
    w = w.contiguous()
    G, K, N = w.shape
    data = torch.empty((G, K, N), dtype=torch.float8_e4m3fn, device=device)
    scale = torch.empty((G, K // 64, N, 2), dtype=torch.uint8, device=device)
    _lib.check(lib.mi355moe_mx_quantize_cols(_ptr(w), G, K, N, _ptr(data), _ptr(scale), _stream(device)),
               "mi355moe_mx_quantize_cols")
    return data, scale


def mx_quantize_weight(w: torch.Tensor, *, col: bool = True, row: bool = True):
    """Dual-axis MX weight quantisation of bf16 [G, M, N] (the MXFP8 weight root's physical fields,
    modules/mega_moe/backends/mxfp8/weights.py:24-97): returns (col_data e4m3fn [G, M, N], col_scale
    uint8 [G, M/64, N, 2], row_data e4m3fn [G, M, N], row_scale uint8 [G, M, N/64, 2]), None for an
    axis not asked for. M and N must be multiples of 64."""
    lib = _lib.load()
    device = _require_gpu(w)
    if w.dtype != torch.bfloat16 or w.ndim != 3 or w.shape[1] % 64 or w.shape[2] % 64:
        raise ValueError("mx_quantize_weight takes bf16 [G, M, N] with M % 64 == 0 and N % 64 == 0")
    if not (col or row):
        raise ValueError("ask for at least one axis")
    w = w.contiguous()
    G, M, N = w.shape
    cd = torch.empty((G, M, N), dtype=torch.float8_e4m3fn, device=device) if col else None
    cs = torch.empty((G, M // 64, N, 2), dtype=torch.uint8, device=device) if col else None
    rd = torch.empty((G, M, N), dtype=torch.float8_e4m3fn, device=device) if row else None
    rs = torch.empty((G, M, N // 64, 2), dtype=torch.uint8, device=device) if row else None
    _lib.check(lib.mi355moe_mx_quantize_weight(_ptr(w), G, M, N, _ptr(cd), _ptr(cs), _ptr(rd), _ptr(rs),
                                               _stream(device)), "mi355moe_mx_quantize_weight")
    return cd, cs, rd, rs


# ------------------------------------------------------------------------------------------------
# Grouped GEMM and the full expert forward
# ------------------------------------------------------------------------------------------------
def grouped_gemm_bf16(x: torch.Tensor, weights: torch.Tensor, group_list: torch.Tensor,
                      layout: str = "EIO", *, gemm_variant: str | None = None) -> torch.Tensor:
    """Concatenated per-group ``x[seg_g] @ W_g``; group_list = int64 inclusive row cumsum.

    layout "EIO": weights [G, K, N]; "EOI": weights [G, N, K].
    """
    lib = _lib.load()
    device = _require_gpu(x, weights, group_list)
    if x.dtype != torch.bfloat16 or weights.dtype != torch.bfloat16:
        raise TypeError("grouped_gemm_bf16 takes bf16 operands")
    G = weights.shape[0]
    if layout == "EIO":
        K, N = weights.shape[1], weights.shape[2]
    elif layout == "EOI":
        N, K = weights.shape[1], weights.shape[2]
    else:
        raise ValueError(f"unknown layout {layout!r}")
    if x.shape[1] != K or group_list.shape != (G,) or group_list.dtype != torch.int64:
        raise ValueError("shape mismatch in grouped_gemm_bf16")
    rows = x.shape[0]
    out = torch.empty((rows, N), dtype=torch.bfloat16, device=device)
    ws = _workspace(lib.mi355moe_grouped_gemm_workspace_size(G), device)
    rc = lib.mi355moe_grouped_gemm_bf16(_ptr(x.contiguous()), rows, K, _ptr(weights.contiguous()),
                                        _lib.LAYOUT[layout], G, N, _ptr(group_list.contiguous()), _ptr(out),
                                        _variant_code(gemm_variant), _ptr(ws), ws.numel(), _stream(device))
    _lib.check(rc, "mi355moe_grouped_gemm_bf16")
    return out


def features() -> int:
    """Bit set of the optional paths the loaded library has switched on (``_lib.FEATURE_*``)."""
    return int(_lib.load().mi355moe_features())


# Measurement default of the grouped-GEMM configuration for calls that do not name one: set with
# set_gemm_variant (per thread / asyncio context), initially the MI355MOE_GG_VARIANT environment
# variable, else "default". The library itself keeps no variant state; every call passes its own.
_GEMM_VARIANT: contextvars.ContextVar[str | None] = contextvars.ContextVar("mi355moe_gemm_variant", default=None)


def _check_variant(name: str) -> str:
    if name not in _lib.GEMM_VARIANT:
        raise ValueError(f"unknown GEMM variant {name!r}; expected one of {sorted(_lib.GEMM_VARIANT)}")
    return name


def gemm_variant() -> str:
    """The grouped-GEMM configuration used by calls that do not name one."""
    name = _GEMM_VARIANT.get()
    return name if name is not None else os.environ.get("MI355MOE_GG_VARIANT", "default") or "default"


def _variant_code(name: str | None) -> int:
    return _lib.GEMM_VARIANT[_check_variant(gemm_variant() if name is None else name)]


def set_gemm_variant(name: str) -> str:
    """Make ``name`` the grouped-GEMM configuration of the following calls in this thread / context
    that do not pass ``gemm_variant`` (a measurement control) and return the previous one. Raises
    ``ValueError`` for an unknown name and ``RuntimeError`` when the library has the variant switched
    off."""
    prev = gemm_variant()
    _GEMM_VARIANT.set(_check_variant(name))
    return prev


def mx_weight_to_eoi(col_data: torch.Tensor, col_scale: torch.Tensor):
    """Re-layout an MX weight root (col_data [G, K, N], col_scale [G, K/64, N, 2]) with K contiguous:
    (data e4m3fn [G, N, K], scale uint8 [G, N, ld]), ld = K/32 padded to a multiple of 16. Values
    and scales are unchanged; the GEMM reads this layout without transposing LDS loads."""
    lib = _lib.load()
    device = _require_gpu(col_data, col_scale)
    if col_data.ndim != 3 or col_data.shape[1] % 64:
        raise ValueError("mx_weight_to_eoi takes col_data [G, K, N] with K % 64 == 0")
    G, K, N = col_data.shape
    if col_scale.shape != (G, K // 64, N, 2):
        raise ValueError("col_scale must be [G, K/64, N, 2]")
    ld = lib.mi355moe_mx_weight_scale_ld(K)
    data = torch.empty((G, N, K), dtype=torch.float8_e4m3fn, device=device)
    scale = torch.empty((G, N, ld), dtype=torch.uint8, device=device)
    _lib.check(lib.mi355moe_mx_weight_to_eoi(_ptr(col_data.contiguous()), _ptr(col_scale.contiguous()), G, K, N,
                                             _ptr(data), _ptr(scale), _stream(device)), "mi355moe_mx_weight_to_eoi")
    return data, scale


def interleave_gate_up(w1: torch.Tensor, w1_scale: torch.Tensor | None = None):
    """The GMM1 weight in layout ``"EIO_GU"``: w1 [E, H, 2I] (bf16, or MX col_data e4m3) with its gate
    columns [0, I) and up columns [I, 2I) interleaved in 64-column blocks (gate 64 b ..+63, then up
    64 b ..+63), and the MX col_scale [E, H/64, 2I, 2] the same way. Values are unchanged; the
    forward with ``layout="EIO_GU"`` on these equals ``"EIO"`` on the originals bit for bit, and reads
    each tile's gate and up columns as one run. Returns (w1, w1_scale or None); w2 stays EIO."""
    lib = _lib.load()
    device = _require_gpu(w1, w1_scale)
    if w1.ndim != 3 or w1.shape[2] % 256 or w1.element_size() not in (1, 2):
        raise ValueError("interleave_gate_up takes w1 [E, H, 2I] with I % 128 == 0")
    E, H, I = w1.shape[0], w1.shape[1], w1.shape[2] // 2
    out = torch.empty_like(w1, memory_format=torch.contiguous_format)
    _lib.check(lib.mi355moe_interleave_gate_up(_ptr(w1.contiguous()), E * H, I, w1.element_size(), _ptr(out),
                                               _stream(device)), "mi355moe_interleave_gate_up")
    scale = None
    if w1_scale is not None:
        if w1_scale.shape != (E, H // 64, 2 * I, 2) or w1_scale.element_size() != 1:
            raise ValueError("w1_scale must be the MX col_scale [E, H/64, 2I, 2]")
        scale = torch.empty_like(w1_scale, memory_format=torch.contiguous_format)
        _lib.check(lib.mi355moe_interleave_gate_up(_ptr(w1_scale.contiguous()), E * (H // 64), I, 2, _ptr(scale),
                                                   _stream(device)), "mi355moe_interleave_gate_up")
    return out, scale


def grouped_gemm_mxfp8(xq: torch.Tensor, x_scale: torch.Tensor, w_data: torch.Tensor, w_scale: torch.Tensor,
                       group_list: torch.Tensor, layout: str = "EIO", *,
                       gemm_variant: str | None = None) -> torch.Tensor:
    """MX grouped GEMM: xq e4m3 [rows, K] (+ e8m0 [rows, K/32]) times the group weight, per group
    segment; bf16 [rows, N] out. layout "EIO": w_data = col_data [G, K, N], w_scale = col_scale
    [G, K/64, N, 2]; "EOI": the :func:`mx_weight_to_eoi` form [G, N, K] + [G, N, ld]."""
    lib = _lib.load()
    device = _require_gpu(xq, x_scale, w_data, w_scale, group_list)
    G = w_data.shape[0]
    if layout == "EIO":
        K, N = w_data.shape[1], w_data.shape[2]
        scale_ok = w_scale.shape == (G, K // 64, N, 2)
    elif layout == "EOI":
        N, K = w_data.shape[1], w_data.shape[2]
        scale_ok = w_scale.shape == (G, N, lib.mi355moe_mx_weight_scale_ld(K))
    else:
        raise ValueError(f"unknown layout {layout!r}")
    rows = xq.shape[0]
    if xq.shape != (rows, K) or x_scale.shape != (rows, K // 32) or not scale_ok:
        raise ValueError("shape mismatch in grouped_gemm_mxfp8")
    if group_list.shape != (G,) or group_list.dtype != torch.int64:
        raise ValueError("group_list must be int64 [G]")
    out = torch.empty((rows, N), dtype=torch.bfloat16, device=device)
    ws = _workspace(lib.mi355moe_grouped_gemm_workspace_size(G), device)
    rc = lib.mi355moe_grouped_gemm_mxfp8(_ptr(xq.contiguous()), _ptr(x_scale.contiguous()), rows, K,
                                         _ptr(w_data.contiguous()), _ptr(w_scale.contiguous()), _lib.LAYOUT[layout],
                                         G, N, _ptr(group_list.contiguous()), _ptr(out),
                                         _variant_code(gemm_variant), _ptr(ws), ws.numel(), _stream(device))
    _lib.check(rc, "mi355moe_grouped_gemm_mxfp8")
    return out


def moe_forward(hidden: torch.Tensor, topk_ids: torch.Tensor, topk_weights: torch.Tensor, w1: torch.Tensor,
                w2: torch.Tensor, *, num_experts: int, intermediate_size: int, precision: str = "bf16",
                layout: str = "EIO", w1_scale: torch.Tensor | None = None, w2_scale: torch.Tensor | None = None,
                tokens_per_expert: torch.Tensor | None = None, out: torch.Tensor | None = None,
                error_flag: torch.Tensor | None = None, stage_events=None, swiglu_limit: float | None = None,
                clamp_after_silu: bool = False, apply_probs_before_fc2: bool = False,
                gemm_variant: str | None = None) -> torch.Tensor:
    """Expert forward at EP=1 through ``mi355moe_moe_forward``; returns bf16 [T, H].

    BF16 numerics options as ``MegaMoeNumericsOptions`` (``swiglu_limit``, ``clamp_after_silu``,
    ``apply_probs_before_fc2``).

    ``stage_events``: optional list of up to 5 ``torch.cuda.Event(enable_timing=True)`` recorded
    at the stage boundaries (start, after dispatch, after GMM1, after GMM2, after combine).

    ``gemm_variant``: grouped-GEMM configuration of both expert GEMMs (``_lib.GEMM_VARIANT``; None:
    :func:`gemm_variant`).
    """
    lib = _lib.load()
    device = _require_gpu(hidden, topk_ids, topk_weights, w1, w2, w1_scale, w2_scale, tokens_per_expert)
    if hidden.dtype != torch.bfloat16 or hidden.ndim != 2:
        raise TypeError("hidden must be bf16 [T, H]")
    T, H = hidden.shape
    K = topk_ids.shape[1]
    hidden = hidden.contiguous()
    ids = topk_ids.contiguous()
    probs = topk_weights.to(torch.float32).contiguous()
    if out is None:
        out = torch.empty((T, H), dtype=torch.bfloat16, device=device)
    args = _lib.ForwardArgs(
        hidden=_ptr(hidden), num_tokens=T, hidden_size=H, intermediate_size=intermediate_size,
        num_experts=num_experts, top_k=K, topk_ids=_ptr(ids), ids_dtype=_ids_dtype(ids),
        precision=_lib.PRECISION[precision], topk_weights=_ptr(probs), weight_layout=_lib.LAYOUT[layout],
        numerics_flags=(_lib.NUMERICS_CLAMP_AFTER_SILU if clamp_after_silu else 0)
        | (_lib.NUMERICS_PROBS_BEFORE_FC2 if apply_probs_before_fc2 else 0),
        swiglu_limit=0.0 if swiglu_limit is None else float(swiglu_limit),
        w1=_ptr(w1), w2=_ptr(w2), w1_scale=_ptr(w1_scale), w2_scale=_ptr(w2_scale),
        tokens_per_expert=_ptr(tokens_per_expert), out=_ptr(out), error_flag=_ptr(error_flag),
        gemm_variant=_variant_code(gemm_variant))
    if stage_events:
        handles = []
        for ev in stage_events:
            if ev.cuda_event == 0:  # events are created lazily on first record
                ev.record()
            handles.append(ev.cuda_event)
        arr = (ctypes.c_void_p * len(handles))(*handles)
        args.stage_events = ctypes.cast(arr, ctypes.POINTER(ctypes.c_void_p))
        args.num_stage_events = len(handles)
    need = lib.mi355moe_moe_forward_workspace_size(ctypes.byref(args))
    if need == 0 and T > 0:
        _lib.check(lib.mi355moe_moe_forward(ctypes.byref(args), None, 0, _stream(device)), "mi355moe_moe_forward")
    ws = _workspace(need, device)
    rc = lib.mi355moe_moe_forward(ctypes.byref(args), _ptr(ws), ws.numel(), _stream(device))
    _lib.check(rc, "mi355moe_moe_forward")
    return out


def moe_backward(hidden: torch.Tensor, topk_ids: torch.Tensor, topk_weights: torch.Tensor, w1: torch.Tensor,
                 w2: torch.Tensor, grad_out: torch.Tensor, *, num_experts: int, intermediate_size: int,
                 layout: str = "EIO", weight_grad_dtype: torch.dtype = torch.bfloat16,
                 need_topk_grad: bool = True, error_flag: torch.Tensor | None = None):
    """Gradients of :func:`moe_forward` (bf16, default numerics) through ``mi355moe_moe_backward``:
    returns (grad_hidden bf16 [T, H], grad_w1, grad_w2 in the weights' layout and
    ``weight_grad_dtype``, grad_topk_weights fp32 [T, K] or None)."""
    lib = _lib.load()
    device = _require_gpu(hidden, topk_ids, topk_weights, w1, w2, grad_out)
    if hidden.dtype != torch.bfloat16 or hidden.ndim != 2 or grad_out.shape != hidden.shape:
        raise TypeError("hidden and grad_out must be bf16 [T, H]")
    if w1.dtype != torch.bfloat16 or w2.dtype != torch.bfloat16:
        raise TypeError("expert weights must be bf16")
    if weight_grad_dtype not in (torch.bfloat16, torch.float32):
        raise ValueError("weight_grad_dtype must be bfloat16 or float32")
    T, H = hidden.shape
    K = topk_ids.shape[1]
    hidden = hidden.contiguous()
    ids = topk_ids.contiguous()
    probs = topk_weights.to(torch.float32).contiguous()
    dout = grad_out.to(torch.bfloat16).contiguous()
    w1 = w1.contiguous()
    w2 = w2.contiguous()
    grad_hidden = torch.empty((T, H), dtype=torch.bfloat16, device=device)
    grad_w1 = torch.empty(w1.shape, dtype=weight_grad_dtype, device=device)
    grad_w2 = torch.empty(w2.shape, dtype=weight_grad_dtype, device=device)
    grad_p = torch.empty((T, K), dtype=torch.float32, device=device) if need_topk_grad else None
    args = _lib.BackwardArgs(
        hidden=_ptr(hidden), num_tokens=T, hidden_size=H, intermediate_size=intermediate_size,
        num_experts=num_experts, top_k=K, topk_ids=_ptr(ids), ids_dtype=_ids_dtype(ids),
        weight_layout=_lib.LAYOUT[layout], topk_weights=_ptr(probs), w1=_ptr(w1), w2=_ptr(w2),
        grad_out=_ptr(dout), grad_hidden=_ptr(grad_hidden), grad_w1=_ptr(grad_w1), grad_w2=_ptr(grad_w2),
        grad_topk_weights=_ptr(grad_p), weight_grad_dtype=1 if weight_grad_dtype == torch.float32 else 0,
        error_flag=_ptr(error_flag))
    need = lib.mi355moe_moe_backward_workspace_size(ctypes.byref(args))
    if need == 0 and T > 0:
        _lib.check(lib.mi355moe_moe_backward(ctypes.byref(args), None, 0, _stream(device)), "mi355moe_moe_backward")
    ws = _workspace(need, device)
    rc = lib.mi355moe_moe_backward(ctypes.byref(args), _ptr(ws), ws.numel(), _stream(device))
    _lib.check(rc, "mi355moe_moe_backward")
    return grad_hidden, grad_w1, grad_w2, grad_p


def moe_backward_mxfp8(hidden: torch.Tensor, topk_ids: torch.Tensor, topk_weights: torch.Tensor,
                       w1: tuple, w2: tuple, grad_out: torch.Tensor, *, num_experts: int, intermediate_size: int,
                       weight_grad_dtype: torch.dtype = torch.bfloat16, need_topk_grad: bool = True,
                       error_flag: torch.Tensor | None = None):
    """Gradients of the MXFP8 :func:`moe_forward` (mxfp8/graph.py:147-154) through
    ``mi355moe_moe_backward``. ``w1`` / ``w2`` are (col_data, col_scale, row_data, row_scale) of the
    EIO MX roots: col_data [E, M, N] e4m3, col_scale [E, M/64, N, 2], row_data [E, M, N] e4m3,
    row_scale [E, M, N/64, 2]. Returns (grad_hidden bf16 [T, H], grad_w1 [E, H, 2I], grad_w2
    [E, I, H] in ``weight_grad_dtype``, grad_topk_weights fp32 [T, K] or None)."""
    lib = _lib.load()
    device = _require_gpu(hidden, topk_ids, topk_weights, grad_out, *w1, *w2)
    if hidden.dtype != torch.bfloat16 or hidden.ndim != 2 or grad_out.shape != hidden.shape:
        raise TypeError("hidden and grad_out must be bf16 [T, H]")
    if weight_grad_dtype not in (torch.bfloat16, torch.float32):
        raise ValueError("weight_grad_dtype must be bfloat16 or float32")
    T, H = hidden.shape
    K = topk_ids.shape[1]
    E, I = num_experts, intermediate_size
    shapes = (((E, H, 2 * I), (E, H // 64, 2 * I, 2), (E, H, 2 * I), (E, H, 2 * I // 64, 2)),
              ((E, I, H), (E, I // 64, H, 2), (E, I, H), (E, I, H // 64, 2)))
    fields = []
    for root, want in zip((w1, w2), shapes):
        if len(root) != 4:
            raise ValueError("MX weights must be (col_data, col_scale, row_data, row_scale)")
        for t, shape in zip(root, want):
            if t.numel() != math.prod(shape) or t.element_size() != 1 or not t.is_contiguous():
                raise ValueError(f"MX weight field must be a contiguous 1-byte tensor of shape {shape}")
        fields.append([t.view(torch.uint8) for t in root])
    hidden = hidden.contiguous()
    ids = topk_ids.contiguous()
    probs = topk_weights.to(torch.float32).contiguous()
    dout = grad_out.to(torch.bfloat16).contiguous()
    grad_hidden = torch.empty((T, H), dtype=torch.bfloat16, device=device)
    grad_w1 = torch.empty((E, H, 2 * I), dtype=weight_grad_dtype, device=device)
    grad_w2 = torch.empty((E, I, H), dtype=weight_grad_dtype, device=device)
    grad_p = torch.empty((T, K), dtype=torch.float32, device=device) if need_topk_grad else None
    (c1, s1, r1, rs1), (c2, s2, r2, rs2) = fields
    args = _lib.BackwardArgs(
        hidden=_ptr(hidden), num_tokens=T, hidden_size=H, intermediate_size=I, num_experts=E, top_k=K,
        topk_ids=_ptr(ids), ids_dtype=_ids_dtype(ids), weight_layout=_lib.LAYOUT["EIO"], topk_weights=_ptr(probs),
        w1=_ptr(c1), w2=_ptr(c2), grad_out=_ptr(dout), grad_hidden=_ptr(grad_hidden), grad_w1=_ptr(grad_w1),
        grad_w2=_ptr(grad_w2), grad_topk_weights=_ptr(grad_p),
        weight_grad_dtype=1 if weight_grad_dtype == torch.float32 else 0, precision=_lib.PRECISION["mxfp8"],
        w1_scale=_ptr(s1), w2_scale=_ptr(s2), w1_row=_ptr(r1), w2_row=_ptr(r2), w1_row_scale=_ptr(rs1),
        w2_row_scale=_ptr(rs2), error_flag=_ptr(error_flag))
    need = lib.mi355moe_moe_backward_workspace_size(ctypes.byref(args))
    if need == 0 and T > 0:
        _lib.check(lib.mi355moe_moe_backward(ctypes.byref(args), None, 0, _stream(device)), "mi355moe_moe_backward")
    ws = _workspace(need, device)
    rc = lib.mi355moe_moe_backward(ctypes.byref(args), _ptr(ws), ws.numel(), _stream(device))
    _lib.check(rc, "mi355moe_moe_backward")
    return grad_hidden, grad_w1, grad_w2, grad_p
