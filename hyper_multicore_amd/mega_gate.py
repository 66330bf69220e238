"""MegaGate router module on the gfx950 route kernels (drop-in for the single-GPU case).

Public surface mirrors hyper_multicore/modules/mega_gate/module.py:71-289: constructor
arguments, parameters ``weight [E, H]``, fp32 ``bias [E]`` and optional fp32 ``bias_vl [E]``
(kept fp32 under ``.to()``), ``from_module`` and ``forward(hidden, image_mask=None) ->
(logits fp32 [T, E], weights fp32 [T, K], indices int64 [T, K])``.

All three scoring functions run on the GPU kernels (the reference runs softmax / sigmoid through
its torch path, module.py:266-271). Extensions over the reference, all off by default:
``num_expert_groups`` / ``topk_groups`` select the DeepSeek-V3 group-limited top-k, and
``vision_router=True`` adds a separate projection ``weight_vl [E, H]`` used for tokens whose
``image_mask`` is set.

Training: when the library reports RouteGrad on (``ops.features()``), outputs computed with grad
enabled carry an autograd function (the reference's ``_MegaGateRouteFunction`` plus the projection's
autograd, modules/mega_gate/function.py:96-207): the routing-weight gradient reaches the fp32 logits
through the RouteGrad kernel (added to the gradient of the returned logits), and the projection
backward ``dX = dL @ W``, ``dW = dL^T @ X`` runs as fp32 GEMMs, per modality. The ranking biases get
no gradient. Otherwise the outputs are forward-only.
"""
from __future__ import annotations

import math
from collections.abc import Callable
from typing import Any

import torch
from torch.autograd.function import once_differentiable

from . import _lib, ops

__all__ = ["MegaGate"]


def _keep_fp32(module: torch.nn.Module, fn: Callable, names: tuple[str, ...]) -> Callable:
    """Wrap an ``_apply`` function so the named parameters keep fp32 dtype
    (modules/_precision.py preserve_fp32_parameters)."""
    ids = {id(getattr(module, n)) for n in names if getattr(module, n, None) is not None}

    def apply(t: torch.Tensor) -> torch.Tensor:
        out = fn(t)
        if id(t) in ids and isinstance(out, torch.Tensor) and out.is_floating_point() and out.dtype != torch.float32:
            out = out.to(torch.float32)
        return out

    return apply


class _MegaGateFunction(torch.autograd.Function):  # pylint: disable=abstract-method,arguments-differ
    """Projection + route with the RouteGrad backward (modules/mega_gate/function.py:96-160)."""

    @staticmethod
    def forward(ctx, flat, weight, weight_vl, mask, bias, bias_vl, cfg):
        ctx.set_materialize_grads(False)
        logits = ops.gate_logits(flat, weight, weight_vl, mask if weight_vl is not None else None)
        weights, indices, scores = ops.gate_route(
            logits, bias, top_k=cfg["top_k"], scoring_func=cfg["scoring_func"],
            routed_scaling_factor=cfg["routed_scaling_factor"], bias_vl=bias_vl,
            image_mask=mask if bias_vl is not None else None, num_groups=cfg["num_groups"],
            topk_groups=cfg["topk_groups"], return_scores=True)
        ctx.save_for_backward(flat, weight, weight_vl, mask, logits, scores, indices)
        ctx.cfg = cfg
        ctx.mark_non_differentiable(indices)
        return logits, weights, indices

    @staticmethod
    @once_differentiable
    def backward(ctx, grad_logits, grad_weights, _grad_indices):
        flat, weight, weight_vl, mask, logits, scores, indices = ctx.saved_tensors
        cfg = ctx.cfg
        grad = None
        if grad_logits is not None:
            grad = grad_logits.to(torch.float32).contiguous().clone()
        if grad_weights is not None:
            grad = ops.gate_route_grad(logits, scores, indices, grad_weights, top_k=cfg["top_k"],
                                       scoring_func=cfg["scoring_func"],
                                       routed_scaling_factor=cfg["routed_scaling_factor"], grad_logits=grad)
        if grad is None:
            return None, None, None, None, None, None, None
        need_x, need_w, need_wvl = ctx.needs_input_grad[0], ctx.needs_input_grad[1], ctx.needs_input_grad[2]
        # logits = X.float() @ W.float()^T per modality (function.py:176-178)
        rows = [(None, weight, need_w)] if weight_vl is None else [(~mask, weight, need_w), (mask, weight_vl, need_wvl)]
        dx = torch.empty(flat.shape, dtype=torch.float32, device=flat.device) if need_x else None
        dws = []
        for sel, w, need in rows:
            g = grad if sel is None else grad[sel]
            x = flat if sel is None else flat[sel]
            if need_x:
                part = g @ w.to(torch.float32)
                if sel is None:
                    dx = part
                else:
                    dx[sel] = part
            dws.append((g.t() @ x.to(torch.float32)).to(w.dtype) if need else None)
        dw = dws[0]
        dwvl = dws[1] if len(dws) > 1 else None
        return (dx.to(flat.dtype) if dx is not None else None), dw, dwvl, None, None, None, None


class MegaGate(torch.nn.Module):
    """Project hidden states and select experts with MegaGate routing on gfx950."""

    def __init__(self, *, hidden_size: int, num_experts: int, top_k: int, scoring_func: str,
                 routed_scaling_factor: float, vision_enabled: bool = False, initializer_range: float = 0.02,
                 num_expert_groups: int = 1, topk_groups: int = 1, vision_router: bool = False) -> None:
        super().__init__()
        if hidden_size <= 0 or num_experts <= 0:
            raise ValueError("hidden_size and num_experts must be positive")
        if top_k <= 0 or top_k > num_experts:
            raise ValueError("top_k must be in [1, num_experts]")
        if scoring_func not in ("sqrtsoftplus", "softmax", "sigmoid"):
            raise ValueError(f"unsupported scoring_func: {scoring_func!r}")
        if not math.isfinite(routed_scaling_factor):
            raise ValueError("routed_scaling_factor must be finite")
        if not math.isfinite(initializer_range) or initializer_range < 0.0:
            raise ValueError("initializer_range must be finite and nonnegative")
        if num_expert_groups < 1 or num_experts % num_expert_groups:
            raise ValueError("num_expert_groups must divide num_experts")
        if num_expert_groups > 1:
            if not 1 <= topk_groups <= num_expert_groups:
                raise ValueError("topk_groups must be in [1, num_expert_groups]")
            if topk_groups * (num_experts // num_expert_groups) < top_k:
                raise ValueError("the kept groups must hold at least top_k experts")
            if num_experts // num_expert_groups < 2:
                raise ValueError("group-limited routing needs at least two experts per group")
        if num_experts > 1024 or top_k > 64:
            raise ValueError("the gfx950 route kernel supports num_experts <= 1024 and top_k <= 64")
        self.hidden_size = int(hidden_size)
        self.num_experts = int(num_experts)
        self.top_k = int(top_k)
        self.scoring_func = scoring_func
        self.routed_scaling_factor = float(routed_scaling_factor)
        self.initializer_range = float(initializer_range)
        self.num_expert_groups = int(num_expert_groups)
        self.topk_groups = int(topk_groups) if num_expert_groups > 1 else 1
        self.weight = torch.nn.Parameter(torch.empty(num_experts, hidden_size))
        self.bias = torch.nn.Parameter(torch.empty(num_experts, dtype=torch.float32))
        if vision_enabled:
            self.bias_vl = torch.nn.Parameter(torch.empty(num_experts, dtype=torch.float32))
        else:
            self.register_parameter("bias_vl", None)
        if vision_router:
            self.weight_vl = torch.nn.Parameter(torch.empty(num_experts, hidden_size))
        else:
            self.register_parameter("weight_vl", None)
        self.reset_parameters()

    def reset_parameters(self) -> None:
        """Reset projection and correction-bias parameters (module.py:35-44)."""
        torch.nn.init.normal_(self.weight, mean=0.0, std=self.initializer_range)
        torch.nn.init.zeros_(self.bias)
        if self.bias_vl is not None:
            torch.nn.init.zeros_(self.bias_vl)
        if self.weight_vl is not None:
            torch.nn.init.normal_(self.weight_vl, mean=0.0, std=self.initializer_range)

    @classmethod
    def from_module(cls, module: torch.nn.Module, **configuration: Any) -> "MegaGate":
        """Bind an existing router's projection and correction-bias Parameters (module.py:142-179)."""
        weight = getattr(module, "weight", None)
        if not isinstance(weight, torch.nn.Parameter) or weight.ndim != 2:
            raise ValueError("source router requires a weight Parameter shaped [num_experts, hidden_size]")
        options = {}
        for name in ("top_k", "scoring_func", "routed_scaling_factor"):
            value = configuration.pop(name, getattr(module, name, None))
            if value is None:
                raise ValueError(f"Provide {name} or expose it on the source router")
            options[name] = value
        bias_vl = getattr(module, "bias_vl", None)
        vision_enabled = configuration.pop("vision_enabled", bias_vl is not None)
        if bias_vl is not None and not vision_enabled:
            raise ValueError("source bias_vl requires vision_enabled=True")
        result = cls(hidden_size=weight.shape[1], num_experts=weight.shape[0], top_k=options["top_k"],
                     scoring_func=options["scoring_func"],
                     routed_scaling_factor=options["routed_scaling_factor"], vision_enabled=vision_enabled,
                     **configuration).to(device=weight.device)
        result.weight = weight
        for name in ("bias", "bias_vl"):
            value = getattr(module, name, None)
            if value is not None:
                if (not isinstance(value, torch.nn.Parameter) or value.shape != (weight.shape[0],)
                        or value.dtype != torch.float32 or value.device != weight.device):
                    raise ValueError(f"source {name} must be an FP32 Parameter [num_experts] on the weight device")
                setattr(result, name, value)
        return result

    def _apply(self, fn: Callable, recurse: bool = True) -> "MegaGate":
        """Keep correction biases fp32 under enclosing model dtype conversion (module.py:181-183)."""
        return super()._apply(_keep_fp32(self, fn, ("bias", "bias_vl")), recurse=recurse)

    def forward(self, hidden_states: torch.Tensor, image_mask: torch.Tensor | None = None):
        """Return (logits fp32 [T, E], routing weights fp32 [T, K], indices int64 [T, K])."""
        if image_mask is not None and self.bias_vl is None and self.weight_vl is None:
            raise ValueError("image_mask requires vision_enabled=True when constructing MegaGate")
        if image_mask is not None and image_mask.shape != hidden_states.shape[:2]:
            raise ValueError("image_mask must have shape [batch, sequence]")
        if hidden_states.device.type != "cuda":
            raise RuntimeError("MegaGate (gfx950) runs on the GPU; move the module and inputs to a cuda device")
        flat = hidden_states.reshape(-1, self.hidden_size)
        if flat.dtype != torch.bfloat16:
            flat = flat.to(torch.bfloat16)
        weight = self.weight if self.weight.dtype == torch.bfloat16 else self.weight.to(torch.bfloat16)
        mask = None
        if image_mask is not None:
            if not image_mask.is_contiguous():
                raise ValueError("image_mask must be contiguous for native MegaGate")
            mask = image_mask.reshape(-1)
        weight_vl = None
        if self.weight_vl is not None and mask is not None:
            weight_vl = self.weight_vl if self.weight_vl.dtype == torch.bfloat16 else self.weight_vl.to(torch.bfloat16)
        if flat.shape[0] == 0:
            E, K = self.num_experts, self.top_k
            dev = hidden_states.device
            return (torch.empty((0, E), dtype=torch.float32, device=dev),
                    torch.empty((0, K), dtype=torch.float32, device=dev),
                    torch.empty((0, K), dtype=torch.int64, device=dev))
        use_vl = mask is not None and self.bias_vl is not None
        wants_grad = torch.is_grad_enabled() and (
            flat.requires_grad or weight.requires_grad or (weight_vl is not None and weight_vl.requires_grad))
        if wants_grad and ops.features() & _lib.FEATURE_ROUTE_GRAD:
            cfg = {"top_k": self.top_k, "scoring_func": self.scoring_func,
                   "routed_scaling_factor": self.routed_scaling_factor, "num_groups": self.num_expert_groups,
                   "topk_groups": self.topk_groups}
            return _MegaGateFunction.apply(
                flat, weight, weight_vl, mask, self.bias.detach().to(torch.float32),
                self.bias_vl.detach().to(torch.float32) if use_vl else None, cfg)
        logits = ops.gate_logits(flat, weight, weight_vl, mask if weight_vl is not None else None)
        weights, indices = ops.gate_route(
            logits, self.bias.detach().to(torch.float32), top_k=self.top_k, scoring_func=self.scoring_func,
            routed_scaling_factor=self.routed_scaling_factor,
            bias_vl=self.bias_vl.detach().to(torch.float32) if use_vl else None,
            image_mask=mask if use_vl else None, num_groups=self.num_expert_groups, topk_groups=self.topk_groups)
        return logits, weights, indices
