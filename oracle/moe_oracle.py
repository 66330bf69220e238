"""TEST INFRASTRUCTURE ONLY - torch-CPU restatement of the MegaGate -> MegaMoE forward path.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use this module; the
product package never imports it. Each function cites the reference code it restates.

Pinning (see tests/test_oracle.py and tests/test_oracle_mx_closed_form.py): the route against the
closed torch forms and the DeepSeek-V3 grouped form; route metadata and the permutation against the
reference tests' known answers (tests/golden/*.json); MX quantisation against torch's own
float8_e4m3fn cast, known-answer blocks and an independent brute-force quantiser; the bf16 expert
math against the TorchExperts loop and closed forms, the MXFP8 expert math against an independent
single-expert closed form with mutation checks. Parity unpinned: the MX backward's rounding point
noted at expert_backward_reference_mx.
"""
from __future__ import annotations

import ctypes
import math

import numpy as np
import torch
import torch.nn.functional as F

from . import build_oracle

_router_lib = None


def _router():
    global _router_lib
    if _router_lib is None:
        _router_lib = build_oracle.load()
    return _router_lib


SCORING = {"softmax": 0, "sigmoid": 1, "sqrtsoftplus": 2}


# ------------------------------------------------------------------------------------------------
# Router
# ------------------------------------------------------------------------------------------------
def det_expf(x: float) -> float:
    return _router().oracle_det_expf(float(x))


def det_logf(x: float) -> float:
    return _router().oracle_det_logf(float(x))


def route_c(logits: np.ndarray, bias: np.ndarray, *, top_k: int, scoring_func: str, routed_scaling_factor: float,
            bias_vl: np.ndarray | None = None, image_mask: np.ndarray | None = None, num_groups: int = 1,
            topk_groups: int = 1):
    """C oracle of the route (router_ref.c): returns (weights f32 [T,K], indices i64 [T,K], scores f32 [T,E]).

    Restates module.py:199-227 / route_pipeline.h:73-562 with the gfx950 kernel's fp32 order.
    """
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    T, E = logits.shape
    bias = np.ascontiguousarray(bias, dtype=np.float32)
    bvl = None if bias_vl is None else np.ascontiguousarray(bias_vl, dtype=np.float32)
    mask = None if image_mask is None else np.ascontiguousarray(image_mask, dtype=np.uint8).reshape(-1)
    weights = np.empty((T, top_k), np.float32)
    indices = np.empty((T, top_k), np.int64)
    scores = np.empty((T, E), np.float32)
    p = lambda a: None if a is None else a.ctypes.data_as(ctypes.c_void_p)
    rc = _router().oracle_route(p(logits), T, E, p(bias), p(bvl), p(mask), top_k, SCORING[scoring_func],
                                num_groups, topk_groups, ctypes.c_float(routed_scaling_factor), p(weights),
                                p(indices), p(scores))
    if rc != 0:
        raise ValueError(f"oracle_route rejected the arguments ({rc})")
    return weights, indices, scores


def route_grad_c(logits: np.ndarray, scores: np.ndarray, indices: np.ndarray, grad_weights: np.ndarray, *,
                 top_k: int, scoring_func: str, routed_scaling_factor: float,
                 accumulate_into: np.ndarray | None = None) -> np.ndarray:
    """C oracle of RouteGrad (router_ref.c: oracle_route_grad): d(routing weights)/d(logits) applied to
    grad_weights [T,K], as fp32 [T,E] (added to ``accumulate_into`` when given).

    Restates route_grad_pipeline.h:138-189 and op_api/hyper_mega_gate_route_grad.cpp:109-120 (the
    torch-autograd operation order of module.py:199-227) for sqrt-softplus, and torch autograd of the
    sigmoid / softmax scores.
    """
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    T, E = logits.shape
    scores = np.ascontiguousarray(scores, dtype=np.float32)
    indices = np.ascontiguousarray(indices, dtype=np.int64)
    grad_weights = np.ascontiguousarray(grad_weights, dtype=np.float32)
    if scores.shape != (T, E) or indices.shape != (T, top_k) or grad_weights.shape != (T, top_k):
        raise ValueError("route_grad_c: shape mismatch")
    out = (np.array(accumulate_into, dtype=np.float32, copy=True) if accumulate_into is not None
           else np.zeros((T, E), np.float32))
    p = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    rc = _router().oracle_route_grad(p(logits), p(scores), p(indices), p(grad_weights), T, E, top_k,
                                     SCORING[scoring_func], ctypes.c_float(routed_scaling_factor),
                                     1 if accumulate_into is not None else 0, p(out))
    if rc != 0:
        raise ValueError(f"oracle_route_grad rejected the arguments ({rc})")
    return out


def route_grad_torch(logits: torch.Tensor, indices: torch.Tensor, grad_weights: torch.Tensor, *,
                     top_k: int, scoring_func: str, routed_scaling_factor: float) -> torch.Tensor:
    """torch autograd of the routing weights w.r.t. fp32 logits (the expression of module.py:199-227 /
    _test_mega_gate.py:752-777) for fixed indices."""
    logits = logits.detach().float().clone().requires_grad_(True)
    if scoring_func == "sqrtsoftplus":
        scores = F.softplus(logits).sqrt()
    elif scoring_func == "softmax":
        scores = logits.softmax(dim=-1)
    else:
        scores = logits.sigmoid()
    selected = scores.gather(1, indices)
    weights = selected / (selected.sum(dim=-1, keepdim=True) + 1.0e-20) if top_k > 1 else selected
    weights = weights * routed_scaling_factor
    return torch.autograd.grad(weights, logits, grad_outputs=grad_weights.float())[0]


def gate_logits_reference(x: torch.Tensor, weight: torch.Tensor, weight_vl: torch.Tensor | None = None,
                          image_mask: torch.Tensor | None = None) -> torch.Tensor:
    """F.linear(x.float(), W.float()) (module.py:195-198); per-modality weights select by mask."""
    x = x.reshape(-1, x.shape[-1]).float()
    logits = F.linear(x, weight.float())
    if weight_vl is not None:
        vis = F.linear(x, weight_vl.float())
        logits = torch.where(image_mask.reshape(-1, 1), vis, logits)
    return logits


def route_reference(logits: torch.Tensor, bias: torch.Tensor, *, top_k: int, scoring_func: str,
                    routed_scaling_factor: float, bias_vl: torch.Tensor | None = None,
                    image_mask: torch.Tensor | None = None, num_groups: int = 1, topk_groups: int = 1):
    """Torch-op form of MegaGate._torch_forward (module.py:199-227) after the projection.

    num_groups > 1 applies the DeepSeek-V3 group-limited selection in its published torch form
    (group score = topk(2).sum per group, topk of groups, masked_fill, topk) - the build's
    extension; with num_groups == 1 this is exactly the reference's plain biased top-k.
    Returns (weights [T,K], indices [T,K] from topk(sorted=False), scores [T,E]).
    """
    logits = logits.float()
    if scoring_func == "sqrtsoftplus":
        scores = F.softplus(logits).sqrt()
    elif scoring_func == "softmax":
        scores = logits.softmax(dim=-1)
    elif scoring_func == "sigmoid":
        scores = logits.sigmoid()
    else:
        raise ValueError(scoring_func)
    correction = bias
    if image_mask is not None and bias_vl is not None:
        correction = torch.where(image_mask.reshape(-1, 1), bias_vl.unsqueeze(0), bias.unsqueeze(0))
    biased = scores + correction
    if num_groups > 1:
        T, E = biased.shape
        group_scores = biased.view(T, num_groups, -1).topk(2, dim=-1).values.sum(dim=-1)
        group_idx = group_scores.topk(topk_groups, dim=-1, sorted=False).indices
        group_mask = torch.zeros_like(group_scores).scatter_(1, group_idx, 1.0)
        expert_mask = group_mask.unsqueeze(-1).expand(T, num_groups, E // num_groups).reshape(T, E)
        biased = biased.masked_fill(expert_mask == 0, float("-inf"))
    indices = torch.topk(biased, top_k, dim=-1, sorted=False).indices
    weights = scores.gather(1, indices)
    if top_k > 1:
        weights = weights / (weights.sum(dim=-1, keepdim=True) + 1.0e-20)
    return weights * routed_scaling_factor, indices, scores


# ------------------------------------------------------------------------------------------------
# Dispatch metadata and permutation
# ------------------------------------------------------------------------------------------------
def expert_counts(ids: torch.Tensor, num_experts: int) -> torch.Tensor:
    """bincount(ids.flatten(), minlength=E) as int32 (route.py:186-211)."""
    return torch.bincount(ids.reshape(-1).to(torch.int64), minlength=num_experts).to(torch.int32)


def route_metadata(counts_by_source: torch.Tensor, *, rank: int, ep_size: int, dispatch_mode: str = "push",
                   received_counts: torch.Tensor | None = None, counts: torch.Tensor | None = None) -> dict:
    """Restatement of _compute_route_metadata's tensor path (route.py:309-390).

    counts_by_source is [EP, E]: row p = the expert histogram of source rank p.
    """
    E = counts_by_source.shape[1]
    local = E // ep_size
    if counts is None:
        counts = counts_by_source[rank]
    if received_counts is None:
        received_counts = counts_by_source[:, rank * local:(rank + 1) * local]
    source_prefix = counts_by_source.cumsum(dim=1, dtype=torch.int64) - counts_by_source
    dest = counts_by_source.reshape(ep_size, ep_size, local).permute(1, 2, 0).contiguous()
    dest_flat = dest.reshape(ep_size, -1)
    dest_prefix = (dest_flat.cumsum(dim=1, dtype=torch.int64) - dest_flat).reshape(ep_size, local, ep_size)
    local_dest_prefix = dest_prefix[rank]
    local_dest_counts = dest[rank]
    lo, hi = rank * local, (rank + 1) * local
    pull = dispatch_mode == "pull"
    return {
        "dispatch_src_off": (source_prefix[:, lo:hi].reshape(-1) if pull else source_prefix[rank]).to(torch.int64),
        "dispatch_target_off": (local_dest_prefix.T.reshape(-1) if pull
                                else dest_prefix[:, :, rank].reshape(-1)).to(torch.int64),
        "dispatch_size": (received_counts.reshape(-1) if pull else counts).to(torch.int32),
        "combine_src_off": local_dest_prefix.T.reshape(-1).to(torch.int64),
        "combine_target_off": source_prefix[:, lo:hi].reshape(-1).to(torch.int64),
        "combine_size": received_counts.reshape(-1).to(torch.int32),
        "group_list": (local_dest_prefix[:, -1] + local_dest_counts[:, -1]).to(torch.int64),
    }


def stable_permutation(ids: torch.Tensor, num_experts: int):
    """Stable sort of flat slots s = t*K + k by expert id (npu_moe_token_permute convention,
    route.py:281-295; utilities.asc:176-204). Returns (mapping [R] slot->row, gather [R] row->slot),
    both int32. Ids outside [0, E) get mapping -1 and no row."""
    flat = ids.reshape(-1).to(torch.int64)
    valid = (flat >= 0) & (flat < num_experts)
    key = torch.where(valid, flat, torch.full_like(flat, num_experts))
    order = torch.sort(key, stable=True).indices
    n_valid = int(valid.sum())
    gather = order[:n_valid].to(torch.int32)
    mapping = torch.full((flat.numel(),), -1, dtype=torch.int32)
    mapping[gather.long()] = torch.arange(n_valid, dtype=torch.int32)
    return mapping, gather


def permute_tokens(x: torch.Tensor, ids: torch.Tensor, num_experts: int):
    """routed[mapping[s]] = x[s // K] (moe_token_permute_out, moe_token_permute_out.cpp:50-60)."""
    K = ids.shape[1]
    mapping, gather = stable_permutation(ids, num_experts)
    return x[(gather.long() // K)], mapping


def unpermute_tokens(values: torch.Tensor, mapping: torch.Tensor, probs: torch.Tensor | None, top_k: int):
    """Build contract of the combine: fp32 sum over k ascending of p * bf16 row, one bf16 round."""
    T = mapping.numel() // top_k
    out = torch.zeros((T, values.shape[1]), dtype=torch.float32)
    m = mapping.reshape(T, top_k).long()
    for k in range(top_k):
        rows = values.float()[m[:, k].clamp(min=0)]
        p = torch.ones(T) if probs is None else probs[:, k].float()
        contrib = rows * p[:, None]
        contrib[m[:, k] < 0] = 0.0
        out = out + contrib
    return out.to(torch.bfloat16)


def unpermute_grad_reference(values: torch.Tensor, grad_out: torch.Tensor, mapping: torch.Tensor,
                             probs: torch.Tensor, top_k: int):
    """Gradient of the weighted unpermute (mega_moe_unpermute_grad_out -> aclnnMoeTokenUnpermuteGrad,
    non-padded; torch/csrc/mega_moe_unpermute.cpp:56-62): for slot s = t*K + k and row r = mapping[s],
    grad_values[r] = bf16(fp32(grad_out[t]) * p[s]) and grad_probs[s] = sum_h fp32(values[r, h]) *
    fp32(grad_out[t, h]) (fp32 accumulation; the order is not part of the contract). Returns
    (grad_values bf16 [T*K, H], grad_probs fp32 [T, K]); rows no slot maps to stay zero."""
    T = mapping.numel() // top_k
    m = mapping.reshape(-1).long()
    g = grad_out.float()[torch.arange(T * top_k) // top_k]  # [T*K, H], the token row of each slot
    p = probs.reshape(-1).float()
    grad_values = torch.zeros((values.shape[0], values.shape[1]), dtype=torch.bfloat16)
    grad_values[m] = (g * p[:, None]).to(torch.bfloat16)
    grad_probs = (values.float()[m] * g).sum(dim=1).reshape(T, top_k)
    return grad_values, grad_probs


# ------------------------------------------------------------------------------------------------
# MX (e4m3fn + e8m0 per 32)
# ------------------------------------------------------------------------------------------------
def mx_shared_exponent(amax: torch.Tensor, scale_alg: int = 1) -> torch.Tensor:
    """e8m0 exponent of 32-element blocks with maxima ``amax`` (int32, clamped to [-127, 127]; -127 for
    all-zero blocks).

    scale_alg 1 (the reference's MX quantisers: dual_axis_mxfp8_worker.h:44 sets ``tiling.scaleAlg = 1``
    and instantiates the SwiGLU quantiser with the same algorithm, :79-80; the weight roots use
    ``npu_dynamic_mx_quant_with_dual_axis(scale_alg=1)``, _replay_mega_moe_arch35.py:55): the smallest
    e with amax <= 448 * 2^e, i.e. ceil(log2(amax / 448)), so no element saturates. With amax = M * 2^E,
    M in [1, 2): 448 * 2^(E-8) = 1.75 * 2^E, hence e = E - 8 for M <= 1.75 and E - 7 above.
    scale_alg 0 (OCP MX v1.0): floor(log2(amax)) - 8 = E - 8; elements above 448 * 2^e saturate."""
    m, exp = torch.frexp(amax)  # amax = m * 2^exp, m in [0.5, 1): E = exp - 1, M = 2 m
    e = exp - 1 - 8
    if scale_alg == 1:
        e = e + (m > 0.875).to(e.dtype)
    elif scale_alg != 0:
        raise ValueError(f"unknown MX scale algorithm {scale_alg}")
    return torch.where(amax > 0, e, torch.full_like(e, -127)).clamp(-127, 127)


def mx_quantize(x: torch.Tensor, dim: int = -1, scale_alg: int = 1):
    """Quantise fp32/bf16 x in 32-element blocks along ``dim``: shared exponent from
    :func:`mx_shared_exponent` (scale algorithm 1 by default, as the reference), elements cast with
    torch's float8_e4m3fn RNE after saturation to +-448 (which only scale algorithm 0 reaches).
    Returns (e4m3 codes uint8 like x, e8m0 codes uint8 with dim/32)."""
    x = x.float().movedim(dim, -1)
    shape = x.shape
    blocks = x.reshape(*shape[:-1], shape[-1] // 32, 32)
    amax = blocks.abs().amax(dim=-1)
    shared = mx_shared_exponent(amax, scale_alg)
    scaled = torch.ldexp(blocks, (-shared).unsqueeze(-1).to(torch.float32))
    scaled = scaled.clamp(-448.0, 448.0)
    q = scaled.to(torch.float8_e4m3fn).view(torch.uint8).reshape(shape)
    codes = (shared + 127).to(torch.uint8)
    return q.movedim(-1, dim), codes.movedim(-1, dim)


def mx_dequantize(q: torch.Tensor, codes: torch.Tensor, dim: int = -1) -> torch.Tensor:
    """Inverse of mx_quantize: e4m3 value * 2^(code - 127), fp32."""
    q = q.movedim(dim, -1)
    codes = codes.movedim(dim, -1)
    vals = q.contiguous().view(torch.float8_e4m3fn).float()
    shape = vals.shape
    blocks = vals.reshape(*shape[:-1], shape[-1] // 32, 32)
    out = torch.ldexp(blocks, (codes.to(torch.float32) - 127.0).unsqueeze(-1))
    return out.reshape(shape).movedim(-1, dim)


def col_scale_to_blocks(col_scale: torch.Tensor) -> torch.Tensor:
    """[G, K/64, N, 2] packed e8m0 (weights.py:61-86) -> [G, K/32, N] one code per 32-block."""
    G, K64, N, _ = col_scale.shape
    return col_scale.permute(0, 1, 3, 2).reshape(G, K64 * 2, N)


def mx_quantize_weight_cols(w: torch.Tensor, scale_alg: int = 1):
    """bf16 [G, K, N] -> (col_data codes uint8 [G,K,N], col_scale uint8 [G,K/64,N,2])."""
    q, codes = mx_quantize(w.float(), dim=1, scale_alg=scale_alg)  # codes [G, K/32, N]
    G, K32, N = codes.shape
    col_scale = codes.reshape(G, K32 // 2, 2, N).permute(0, 1, 3, 2).contiguous()
    return q, col_scale


def mx_dequantize_weight_cols(col_data: torch.Tensor, col_scale: torch.Tensor) -> torch.Tensor:
    codes = col_scale_to_blocks(col_scale)
    return mx_dequantize(col_data.view(torch.uint8), codes, dim=1)


# ------------------------------------------------------------------------------------------------
# Expert math
# ------------------------------------------------------------------------------------------------
def _bf16(t: torch.Tensor) -> torch.Tensor:
    return t.to(torch.bfloat16).float()


def swiglu_reference(g: torch.Tensor, u: torch.Tensor, swiglu_limit: float | None = None,
                     clamp_after_silu: bool = False) -> torch.Tensor:
    """fp32 SwiGLU activation of the bf16 GMM1 halves (docs/mega_moe.md:253-262, numerics.py):
    no limit: silu(g) * u; limit L before SiLU: silu(min(g, L)) * clamp(u, -L, L); after SiLU:
    min(silu(g), L) * clamp(u, -L, L)."""
    gate, up = g.float(), u.float()
    if swiglu_limit is None:
        return F.silu(gate) * up
    L = float(swiglu_limit)
    up = up.clamp(-L, L)
    if clamp_after_silu:
        return F.silu(gate).clamp(max=L) * up
    return F.silu(gate.clamp(max=L)) * up


def expert_forward_reference(hidden: torch.Tensor, ids: torch.Tensor, probs: torch.Tensor, w1: torch.Tensor,
                             w2: torch.Tensor, *, layout: str = "EIO", precision: str = "bf16",
                             w1_scale: torch.Tensor | None = None, w2_scale: torch.Tensor | None = None,
                             num_experts: int | None = None, swiglu_limit: float | None = None,
                             clamp_after_silu: bool = False, apply_probs_before_fc2: bool = False) -> torch.Tensor:
    """fp32-accumulate expert forward with the reference's bf16 rounding points
    (fp32_expert_reference.py:22-26): U = bf16(x @ W1), act = bf16(silu(g) * u) with g the left
    half, y = bf16(act @ W2); combine = fp32 sum over k ascending of p * y, one bf16 rounding.

    precision "mxfp8": x quantised per 32 along H, W1/W2 given as col_data/col_scale (EIO),
    act = silu(g) * u quantised per 32 along I before the down projection (mxfp8/graph.py:140-146).

    bf16 numerics options (docs/mega_moe.md:218-270; module.py:132 rejects them for MXFP8):
    ``swiglu_limit`` / ``clamp_after_silu`` as in :func:`swiglu_reference`;
    ``apply_probs_before_fc2``: the FC2 input is bf16(fp32(bf16(act)) * p) with p the routed row's
    probability, and the combine sums the K rows unweighted (execution.py:75-77,
    autograd.py:124-126).
    """
    if precision != "bf16" and (swiglu_limit is not None or apply_probs_before_fc2):
        raise ValueError("MXFP8 does not support clamp or before-FC2 probability weighting")
    T, H = hidden.shape
    K = ids.shape[1]
    E = num_experts if num_experts is not None else w1.shape[0]
    if precision == "bf16":
        W1 = w1.float() if layout == "EIO" else w1.float().transpose(1, 2)
        W2 = w2.float() if layout == "EIO" else w2.float().transpose(1, 2)
        xin = hidden.float()
    else:
        W1 = mx_dequantize_weight_cols(w1, w1_scale)
        W2 = mx_dequantize_weight_cols(w2, w2_scale)
        q, s = mx_quantize(hidden.float(), dim=-1)
        xin = mx_dequantize(q, s, dim=-1)
    I = W1.shape[2] // 2
    mapping, gather = stable_permutation(ids, E)
    y = torch.zeros((gather.numel(), H), dtype=torch.float32)
    flat = ids.reshape(-1).long()
    start = 0
    for e in range(E):
        n = int((flat == e).sum())
        if n == 0:
            continue
        slots = gather[start:start + n].long()
        rows = slots // K
        u = _bf16(xin[rows] @ W1[e])
        g, up = u[:, :I], u[:, I:]
        act = swiglu_reference(g, up, swiglu_limit, clamp_after_silu)
        if precision == "bf16":
            act = _bf16(act)
            if apply_probs_before_fc2:
                act = _bf16(act * probs.reshape(-1)[slots].float()[:, None])
        else:
            aq, asc = mx_quantize(act, dim=-1)
            act = mx_dequantize(aq, asc, dim=-1)
        y[start:start + n] = _bf16(act @ W2[e])
        start += n
    return unpermute_tokens(y.to(torch.bfloat16), mapping, None if apply_probs_before_fc2 else probs, K)


def expert_forward_reference_tokens(hidden: torch.Tensor, ids: torch.Tensor, probs: torch.Tensor,
                                    tokens: torch.Tensor, expert_weights, *, precision: str = "bf16",
                                    scale_alg: int = 1) -> torch.Tensor:
    """:func:`expert_forward_reference` restricted to the token rows ``tokens`` (same rounding points,
    fp32 accumulate; fp32_expert_reference.py:22-26, moe_reference.py:170-181), for layers whose
    weights are too large to expand at once. ``expert_weights(e)`` returns the fp32 weights of expert
    e as (W1 [H, 2I], W2 [I, H]); for MXFP8 they are the dequantised roots and the activations are
    MX-quantised per row (a routed row's quantisation depends on that row only). Returns bf16
    [len(tokens), H]: out[i] = bf16(sum over k ascending of p[t, k] * y[t, k]) for t = tokens[i]."""
    tok = tokens.long()
    K = ids.shape[1]
    x = hidden.float()[tok]
    if precision != "bf16":
        q, s = mx_quantize(x, dim=-1, scale_alg=scale_alg)
        x = mx_dequantize(q, s, dim=-1)
    sel = ids[tok].long()                      # [n, K]
    p = probs[tok].float()
    n, H = x.shape
    y = torch.zeros((n, K, H), dtype=torch.float32)
    for e in torch.unique(sel).tolist():
        if e < 0:
            continue
        rows, ks = (sel == e).nonzero(as_tuple=True)
        W1, W2 = expert_weights(e)
        I = W1.shape[1] // 2
        u = _bf16(x[rows] @ W1)
        act = swiglu_reference(u[:, :I], u[:, I:])
        if precision == "bf16":
            act = _bf16(act)
        else:
            aq, asc = mx_quantize(act, dim=-1, scale_alg=scale_alg)
            act = mx_dequantize(aq, asc, dim=-1)
        y[rows, ks] = _bf16(act @ W2)
    out = torch.zeros((n, H), dtype=torch.float32)
    for k in range(K):
        contrib = y[:, k] * p[:, k:k + 1]
        contrib[sel[:, k] < 0] = 0.0
        out = out + contrib
    return out.to(torch.bfloat16)


def expert_backward_reference(hidden: torch.Tensor, ids: torch.Tensor, probs: torch.Tensor, w1: torch.Tensor,
                              w2: torch.Tensor, grad_out: torch.Tensor, *, layout: str = "EIO",
                              num_experts: int | None = None):
    """Backward of the bf16 expert forward (combine included) with the reference's rounding points.

    Expert part (fp32_expert_reference.py:27-35): with the recomputed bf16 projection U = [g | u],
    silu = silu(g) and act = bf16(silu * u) of the forward,
        gA = bf16(dY @ W2^T), gG = bf16(gA * u * s * (1 + g * (1 - s))) with s = sigmoid(g),
        gU = bf16(gA * silu), dU = [gG | gU], dW1_e = X_e^T dU_e, dW2_e = act_e^T dY_e (fp32),
        dX_routed = bf16(dU @ W1^T).
    Combine / permutation (restore_topk_output route.py:1029-1051 and moe_token_permute_grad;
    build contract, the torch_npu ops are closed): dY_r = bf16(fp32(dOut[t]) * p[t, k]) for the
    routed row r of slot (t, k); dp[t, k] = sum_h fp32(y_r[h]) * fp32(dOut[t, h]) with y the bf16
    expert output; dX[t] = bf16(sum_k fp32(dX_routed[r])).

    Returns (dX bf16 [T, H], dW1 fp32 in w1's layout, dW2 fp32 in w2's layout, dp fp32 [T, K]).
    """
    T, H = hidden.shape
    K = ids.shape[1]
    E = num_experts if num_experts is not None else w1.shape[0]
    W1 = w1.float() if layout == "EIO" else w1.float().transpose(1, 2)  # [E, H, 2I]
    W2 = w2.float() if layout == "EIO" else w2.float().transpose(1, 2)  # [E, I, H]
    I = W1.shape[2] // 2
    x = hidden.float()
    dout = grad_out.float()
    mapping, gather = stable_permutation(ids, E)
    flat = ids.reshape(-1).long()
    pflat = probs.reshape(-1).float()
    dW1 = torch.zeros(E, H, 2 * I)
    dW2 = torch.zeros(E, I, H)
    dxr = torch.zeros(gather.numel(), H)
    dp = torch.zeros(T * K)
    start = 0
    for e in range(E):
        n = int((flat == e).sum())
        if n == 0:
            continue
        slots = gather[start:start + n].long()
        rows = slots // K
        xe = x[rows]
        u_all = _bf16(xe @ W1[e])
        g, up = u_all[:, :I], u_all[:, I:]
        silu = F.silu(g)
        act = _bf16(silu * up)
        y = _bf16(act @ W2[e])
        dy = _bf16(dout[rows] * pflat[slots][:, None])
        dp[slots] = (y * dout[rows]).sum(1)
        ga = _bf16(dy @ W2[e].T)
        sg = torch.sigmoid(g)
        gg = _bf16(ga * up * sg * (1 + g * (1 - sg)))
        gu = _bf16(ga * silu)
        du = torch.cat([gg, gu], dim=1)
        dW1[e] = xe.T @ du
        dW2[e] = act.T @ dy
        dxr[start:start + n] = _bf16(du @ W1[e].T)
        start += n
    dx = unpermute_tokens(dxr.to(torch.bfloat16), mapping, None, K)
    if layout == "EOI":
        dW1, dW2 = dW1.transpose(1, 2).contiguous(), dW2.transpose(1, 2).contiguous()
    return dx, dW1, dW2, dp.reshape(T, K)


def mx_quantize_grouped_rows(x: torch.Tensor, counts: list[int]):
    """Column-axis MX quantisation of a routed-row matrix x [R, C] (rows grouped by expert, counts[e]
    rows each): every column in blocks of 32 rows that start at each expert's first row, a partial
    last block zero-padded (the grouped packed column axis of dual_axis_mxfp8_worker.h:24-33,
    x_col / a_col / dy_col / du_col of mxfp8/execution.py:28-35).

    Returns (codes uint8 [R, C], packed scales uint8 [(R + 63) // 64 + E, C, 2], dequantised fp32
    [R, C]). Expert e's scales start at 64-row group floor(start_e / 64) + e (its pairs cover 64 rows
    each); pair slots of 32-row blocks past the expert's rows hold code 0.
    """
    x = x.float()
    R, C = x.shape
    E = len(counts)
    codes = torch.zeros((R, C), dtype=torch.uint8)
    deq = torch.zeros((R, C), dtype=torch.float32)
    packed = torch.zeros(((R + 63) // 64 + E, C, 2), dtype=torch.uint8)
    start = 0
    for e, n in enumerate(counts):
        if n == 0:
            continue
        nb = (n + 31) // 32
        blk = torch.zeros((nb * 32, C), dtype=torch.float32)
        blk[:n] = x[start:start + n]
        q, sc = mx_quantize(blk, dim=0)  # q [nb*32, C], sc [nb, C]
        codes[start:start + n] = q[:n]
        deq[start:start + n] = mx_dequantize(q, sc, dim=0)[:n]
        base = start // 64 + e
        for b in range(nb):
            packed[base + b // 2, :, b % 2] = sc[b]
        start += n
    return codes, packed, deq


def mx_dequantize_weight_rows(row_data: torch.Tensor, row_scale: torch.Tensor) -> torch.Tensor:
    """Backward axis of an MX root: row_data [E, M, N] e4m3 codes, row_scale [E, M, N/64, 2] (blocks of
    32 along N) -> fp32 [E, M, N]."""
    E, M, N = row_data.shape
    return mx_dequantize(row_data.view(torch.uint8), row_scale.reshape(E, M, N // 32), dim=-1)


def expert_backward_reference_mx(hidden: torch.Tensor, ids: torch.Tensor, probs: torch.Tensor,
                                 w1_col: tuple[torch.Tensor, torch.Tensor], w2_col: tuple[torch.Tensor, torch.Tensor],
                                 w1_row: tuple[torch.Tensor, torch.Tensor], w2_row: tuple[torch.Tensor, torch.Tensor],
                                 grad_out: torch.Tensor, *, num_experts: int | None = None):
    """MXFP8 expert backward (mxfp8/graph.py:147-154, mxfp8/execution.py:119-164), fp32 accumulation of
    the dequantised operands, in the EIO weight layout:
      forward recompute   U = bf16(Q_H(x) W1c), act = silu(g) u (fp32), y = bf16(Q_I(act) W2c)
      combine backward    dY = bf16(p dOut), dp = <y, dOut>
      quant_dy            dy_row = Q_H(dY) (blocks along H), dy_col = Q_rows(dY) (blocks of 32 routed
                          rows from each expert's start)
      dw2 (TN)            dW2_e = Q_rows(act)_e^T dy_col_e
      da (NT)             da = bf16(dy_row W2r_e^T), W2r the root's row axis (blocks along H)
      swiglu_grad_quant   dU = [da u s (1 + g (1 - s)) | da silu(g)] in fp32 (no bf16 rounding: the
                          gradient is quantised straight away), du_row = Q_2I(dU), du_col = Q_rows(dU)
      dw1 (TN)            dW1_e = Q_rows(x)_e^T du_col_e
      dx (NT)             dXr = bf16(du_row W1r_e^T), W1r blocks along 2I
      permute backward    dX[t] = bf16(sum_k dXr[mapping[t, k]])
    w*_col = (col_data, col_scale) as mx_quantize_weight_cols returns; w*_row = (row_data [E, M, N],
    row_scale [E, M, N/64, 2]). Whether the fused SwiGLU-gradient quantisation rounds dU to bf16
    first is not visible in the reference (ops-nn source absent): parity unpinned at that point.
    Returns (dX bf16 [T, H], dW1 fp32 [E, H, 2I], dW2 fp32 [E, I, H], dp fp32 [T, K]).
    """
    T, H = hidden.shape
    K = ids.shape[1]
    E = num_experts if num_experts is not None else w1_col[0].shape[0]
    W1c = mx_dequantize_weight_cols(*w1_col)       # [E, H, 2I]
    W2c = mx_dequantize_weight_cols(*w2_col)       # [E, I, H]
    W1r = mx_dequantize_weight_rows(*w1_row)       # [E, H, 2I]
    W2r = mx_dequantize_weight_rows(*w2_row)       # [E, I, H]
    I = W1c.shape[2] // 2
    q, s = mx_quantize(hidden.float(), dim=-1)
    xq = mx_dequantize(q, s, dim=-1)
    dout = grad_out.float()
    mapping, gather = stable_permutation(ids, E)
    flat = ids.reshape(-1).long()
    pflat = probs.reshape(-1).float()
    counts = [int((flat == e).sum()) for e in range(E)]
    R = gather.numel()
    rows_all = gather.long() // K
    x_r = hidden.float()[rows_all]
    U = torch.zeros(R, 2 * I)
    act = torch.zeros(R, I)
    y = torch.zeros(R, H)
    start = 0
    for e, n in enumerate(counts):
        if n:
            sl = slice(start, start + n)
            U[sl] = _bf16(xq[rows_all[sl]] @ W1c[e])
            act[sl] = F.silu(U[sl, :I]) * U[sl, I:]
            aq, asc = mx_quantize(act[sl], dim=-1)
            y[sl] = _bf16(mx_dequantize(aq, asc, dim=-1) @ W2c[e])
        start += n
    dy = _bf16(dout[rows_all] * pflat[gather.long()][:, None])
    dp = torch.zeros(T * K)
    dp[gather.long()] = (y * dout[rows_all]).sum(1)
    dq, dsc = mx_quantize(dy, dim=-1)
    dy_row = mx_dequantize(dq, dsc, dim=-1)
    _, _, dy_col = mx_quantize_grouped_rows(dy, counts)
    _, _, a_col = mx_quantize_grouped_rows(act, counts)
    _, _, x_col = mx_quantize_grouped_rows(x_r, counts)
    dW1 = torch.zeros(E, H, 2 * I)
    dW2 = torch.zeros(E, I, H)
    da = torch.zeros(R, I)
    start = 0
    for e, n in enumerate(counts):
        if n:
            sl = slice(start, start + n)
            dW2[e] = a_col[sl].T @ dy_col[sl]
            da[sl] = _bf16(dy_row[sl] @ W2r[e].T)
        start += n
    g, u = U[:, :I], U[:, I:]
    sg = torch.sigmoid(g)
    dU = torch.cat([da * u * sg * (1 + g * (1 - sg)), da * (g * sg)], dim=1)
    uq, usc = mx_quantize(dU, dim=-1)
    du_row = mx_dequantize(uq, usc, dim=-1)
    _, _, du_col = mx_quantize_grouped_rows(dU, counts)
    dxr = torch.zeros(R, H)
    start = 0
    for e, n in enumerate(counts):
        if n:
            sl = slice(start, start + n)
            dW1[e] = x_col[sl].T @ du_col[sl]
            dxr[sl] = _bf16(du_row[sl] @ W1r[e].T)
        start += n
    dx = unpermute_tokens(dxr.to(torch.bfloat16), mapping, None, K)
    return dx, dW1, dW2, dp.reshape(T, K)


def torch_experts_reference(hidden: torch.Tensor, ids: torch.Tensor, probs: torch.Tensor, gate_w: torch.Tensor,
                            up_w: torch.Tensor, down_w: torch.Tensor) -> torch.Tensor:
    """The TorchExperts CPU loop (tests/common/multicore/moe_reference.py:170-181): weights are
    [E, I, H] gate / up and [E, H, I] down; bf16 F.linear, bf16 weighted rows, bf16 index_add in
    expert-major order."""
    output = torch.zeros_like(hidden)
    for expert in range(gate_w.shape[0]):
        rows, slots = torch.where(ids == expert)
        if rows.numel() == 0:
            continue
        source = hidden.index_select(0, rows)
        gate = F.linear(source, gate_w[expert])
        up = F.linear(source, up_w[expert])
        activation = (F.silu(gate.float()) * up.float()).to(hidden.dtype)
        value = F.linear(activation, down_w[expert])
        weighted = (value.float() * probs[rows, slots, None]).to(hidden.dtype)
        output = output.index_add(0, rows, weighted)
    return output


def rel_l2(a: torch.Tensor, b: torch.Tensor) -> float:
    a = a.double().reshape(-1)
    b = b.double().reshape(-1)
    return float(torch.linalg.vector_norm(a - b) / max(float(torch.linalg.vector_norm(b)), 1e-30))


def moe_flops(tokens: int, top_k: int, hidden: int, inter: int, experts: int) -> float:
    """Algorithmic FLOPs: expert GEMMs 6*R*H*I plus router 2*T*H*E."""
    return 6.0 * tokens * top_k * hidden * inter + 2.0 * tokens * hidden * experts


def ulp_distance(a: float, b: float) -> int:
    ai = np.array([a], np.float32).view(np.int32)[0]
    bi = np.array([b], np.float32).view(np.int32)[0]
    return abs(int(ai) - int(bi))


__all__ = [n for n in dir() if not n.startswith("_") and n not in ("annotations", "ctypes", "math", "np", "torch", "F")]
