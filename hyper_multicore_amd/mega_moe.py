"""MegaMoeExperts executor on the gfx950 kernels (expert-parallel degree 1).

Public surface mirrors hyper_multicore/modules/mega_moe/module.py:141-535: the executor owns no
parameters; ``forward(hidden_states, topk_ids, topk_weights, *, expert_weights,
tokens_per_expert=None)`` returns bf16 in the input shape. BF16 weights are accepted in the EIO
``([E,H,2I], [E,I,H])`` or EOI ``([E,2I,H], [E,H,I])`` layout (inferred from the shapes and bound
on first use); MXFP8 weights are MX roots carrying ``col_data`` (e4m3fn, EIO) and ``col_scale``
(uint8 e8m0 ``[E, M/64, N, 2]``), see :func:`hyper_multicore_amd.mxfp8.quantize_expert_weight`.

Gradients: with the library's backward switched on (``ops.features()``), a bf16 forward under
autograd with default numerics records a function whose backward computes the gradients of the
hidden states, both expert weights and the routing weights on the GPU; otherwise the output carries
no autograd history. MXFP8 likewise once the library reports its MX backward on: the backward reads
the roots' ``row_data`` / ``row_scale`` axis (``quantize_expert_weight(w, backward_axis=True)``) and
returns the root gradients in the roots' dtype. The BF16 numerics options (``swiglu_limit``, ``clamp_after_silu``, ``apply_probs_before_fc2``) run
when the loaded library reports them switched on (``ops.features()``), otherwise the constructor
raises ``NotImplementedError``; MXFP8 rejects them as the reference does. ``ep_group`` must be
``None`` or a group of size 1.
"""
from __future__ import annotations

import math
import os
import struct
from dataclasses import dataclass
from typing import Any

import torch

from . import _lib, ops

__all__ = ["MegaMoeExperts", "MegaMoeNumericsOptions", "MegaMoeTuningOptions", "MegaMoeSchedulerOptions"]

_COMMUNICATION_SPLIT = 128


@dataclass(frozen=True)
class MegaMoeNumericsOptions:
    """Numerical semantics (modules/mega_moe/numerics.py:21-50)."""

    partial_weight_grad_dtype: str | None = None
    swiglu_limit: float | None = None
    clamp_after_silu: bool = False
    apply_probs_before_fc2: bool = False


@dataclass(frozen=True)
class MegaMoeSchedulerOptions:
    """Accepted for API compatibility (experimental/_mega_moe.py); the gfx950 work list is fixed."""

    policy: str | None = None
    queue_ready_lookahead: int | None = None
    batch_experts: bool = False
    nominal_schedule: bool = False
    lowering: str | None = None


@dataclass(frozen=True)
class MegaMoeTuningOptions:
    """Accepted for API compatibility (experimental/_mega_moe.py:22-100). The EP transport knobs
    (dispatch mode, capacity factors, splits) have no effect at EP=1 but are validated."""

    dispatch_mode: str = "push"
    initial_capacity_factor: float | None = None
    capacity_growth_factor: float | None = None
    dispatch_split: int = _COMMUNICATION_SPLIT
    combine_split: int = _COMMUNICATION_SPLIT
    scheduler: MegaMoeSchedulerOptions = MegaMoeSchedulerOptions()


def _check_swiglu_limit(limit: Any) -> None:
    """None, or a finite positive number whose float32 value is finite and positive (the kernel
    takes it as float32; module.py:55-79 applies the same rule)."""
    if limit is None:
        return
    ok = isinstance(limit, (int, float)) and not isinstance(limit, bool)
    if ok:
        try:
            as_f32 = struct.unpack("<f", struct.pack("<f", float(limit)))[0]
        except (OverflowError, ValueError):
            as_f32 = float("inf")
        ok = math.isfinite(float(limit)) and math.isfinite(as_f32) and as_f32 > 0.0
    if not ok:
        raise ValueError("swiglu_limit must be None or a finite positive float32-representable number, "
                         f"got {limit!r}.")


def _positive_int(name: str, value: Any) -> int:
    if not isinstance(value, int) or isinstance(value, bool) or value <= 0:
        raise ValueError(f"{name} must be a positive integer, got {value!r}.")
    return value


ROUTE_COUNT_ERROR = "MegaMoe counts must describe the actual distinct Top-K routes"
# Host-side route checks in MegaMoeExperts.forward (a debugging aid, off by default). Like the
# reference's static-token path (route.py:186-211), the forward trusts tokens_per_expert and checks only
# its shape, device and dtype; ids outside [0, E) are skipped on the device and reported through the
# library's error flag. With MI355MOE_CHECK_ROUTES=1 the forward also runs validate_routes, which
# waits for the device once per call.
CHECK_ROUTES = os.environ.get("MI355MOE_CHECK_ROUTES", "0") == "1"


def validate_routes(topk_ids: torch.Tensor, num_experts: int, tokens_per_expert: torch.Tensor | None = None) -> None:
    """Refuse routes whose counts cannot describe the actual Top-K routes (route.py:566-593 raises
    RuntimeError before any expert work): an id outside [0, E), or ``tokens_per_expert`` that is not
    the histogram of the ids. One reduction on the ids' device and one host read (the reference also
    reads its route summary on the host)."""
    ids = topk_ids.reshape(-1)
    bad = ((ids < 0) | (ids >= num_experts)).any()
    if tokens_per_expert is not None:
        hist = torch.bincount(ids.clamp(0, num_experts - 1).long(), minlength=num_experts)
        bad = bad | (hist != tokens_per_expert.reshape(-1).to(hist.dtype)).any()
    if bool(bad):
        raise RuntimeError(ROUTE_COUNT_ERROR)


class _MoeFunction(torch.autograd.Function):
    """bf16 expert forward with the library's backward (autograd.py:672-760 role); the forward
    intermediates are recomputed in the backward, so only the inputs are saved."""

    @staticmethod
    def forward(ctx, hidden, topk_weights, w1, w2, topk_ids, num_experts, intermediate_size, layout,
                weight_grad_dtype):
        ctx.save_for_backward(hidden, topk_weights, w1, w2, topk_ids)
        ctx.meta = (num_experts, intermediate_size, layout, weight_grad_dtype)
        return ops.moe_forward(hidden, topk_ids, topk_weights, w1, w2, num_experts=num_experts,
                               intermediate_size=intermediate_size, precision="bf16", layout=layout)

    @staticmethod
    def backward(ctx, grad_out):
        hidden, topk_weights, w1, w2, topk_ids = ctx.saved_tensors
        num_experts, inter, layout, grad_dtype = ctx.meta
        gx, g1, g2, gp = ops.moe_backward(hidden, topk_ids, topk_weights, w1, w2, grad_out, num_experts=num_experts,
                                          intermediate_size=inter, layout=layout, weight_grad_dtype=grad_dtype,
                                          need_topk_grad=ctx.needs_input_grad[1])
        gp = gp.to(topk_weights.dtype) if gp is not None else None
        return gx, gp, g1, g2, None, None, None, None, None


class _MxMoeFunction(torch.autograd.Function):
    """MXFP8 expert forward with the library's MX backward (mxfp8/autograd.py:35-86 role): the forward
    reads the roots' column axis; the backward resolves the roots again for their row axis (the
    reference re-resolves after its parameter hooks, so a root whose owner has replaced the row fields
    or released the column fields since the forward works, test_mxfp8_root_lifecycle.py:31-73). The
    forward intermediates are recomputed from the column axis the forward read, which the context
    keeps."""

    @staticmethod
    def forward(ctx, hidden, topk_weights, root1, root2, topk_ids, executor, weight_grad_dtype):
        from .mxfp8 import resolve_forward_weight
        layout, d1, s1, d2, s2 = executor._mx_weights(hidden, (root1, root2))
        ctx.save_for_backward(hidden, topk_weights, topk_ids)
        ctx.roots = (root1, root2)
        E, H, I = executor.num_experts, executor.hidden_size, executor.intermediate_size
        ctx.cols = (resolve_forward_weight(root1, (E, H, 2 * I), hidden.device),
                    resolve_forward_weight(root2, (E, I, H), hidden.device))
        ctx.meta = (executor.num_experts, executor.hidden_size, executor.intermediate_size, weight_grad_dtype)
        return ops.moe_forward(hidden, topk_ids, topk_weights, d1, d2, num_experts=executor.num_experts,
                               intermediate_size=executor.intermediate_size, precision="mxfp8", layout=layout,
                               w1_scale=s1, w2_scale=s2)

    @staticmethod
    def backward(ctx, grad_out):
        from .mxfp8 import resolve_backward_weight
        hidden, topk_weights, topk_ids = ctx.saved_tensors
        E, H, I, grad_dtype = ctx.meta
        r1, r2 = ctx.roots
        fields = []
        for root, shape, col in ((r1, (E, H, 2 * I), ctx.cols[0]), (r2, (E, I, H), ctx.cols[1])):
            row = resolve_backward_weight(root, shape, hidden.device)
            fields.append((*col, *row))
        ctx.cols = None
        gx, g1, g2, gp = ops.moe_backward_mxfp8(hidden, topk_ids, topk_weights, fields[0], fields[1], grad_out,
                                                num_experts=E, intermediate_size=I, weight_grad_dtype=grad_dtype,
                                                need_topk_grad=ctx.needs_input_grad[1])
        g1 = g1.reshape(r1.shape).to(r1.dtype) if ctx.needs_input_grad[2] else None
        g2 = g2.reshape(r2.shape).to(r2.dtype) if ctx.needs_input_grad[3] else None
        gp = gp.to(topk_weights.dtype) if gp is not None else None
        return gx, gp, g1, g2, None, None, None


class MegaMoeExperts(torch.nn.Module):
    """Execute router-selected experts with the gfx950 MegaMoE kernels on one GPU."""

    def __init__(self, *, hidden_size: int, intermediate_size: int, num_experts: int, top_k: int,
                 ep_group: Any | None = None, precision: str = "bf16",
                 numerics_options: MegaMoeNumericsOptions | None = None,
                 tuning_options: MegaMoeTuningOptions | None = None,
                 expert_placement: Any | None = None) -> None:
        super().__init__()
        for name, value in (("hidden_size", hidden_size), ("intermediate_size", intermediate_size),
                            ("num_experts", num_experts), ("top_k", top_k)):
            _positive_int(name, value)
        if top_k > num_experts:
            raise ValueError(f"top_k ({top_k}) cannot exceed num_experts ({num_experts}).")
        if precision not in ("bf16", "mxfp8"):
            raise ValueError("MegaMoE precision must be bf16 or mxfp8")
        if numerics_options is not None and not isinstance(numerics_options, MegaMoeNumericsOptions):
            raise TypeError("numerics_options must be MegaMoeNumericsOptions or None")
        if tuning_options is not None and not isinstance(tuning_options, MegaMoeTuningOptions):
            raise TypeError("tuning_options must be MegaMoeTuningOptions or None")
        numerics = numerics_options or MegaMoeNumericsOptions()
        tuning = tuning_options or MegaMoeTuningOptions()
        for name, value in (("apply_probs_before_fc2", numerics.apply_probs_before_fc2),
                            ("clamp_after_silu", numerics.clamp_after_silu)):
            if not isinstance(value, bool):
                raise TypeError(f"{name} must be a boolean")
        _check_swiglu_limit(numerics.swiglu_limit)
        if precision == "mxfp8" and (numerics.swiglu_limit is not None or numerics.apply_probs_before_fc2):
            raise ValueError("MXFP8 does not support clamp or before-FC2 probability weighting")
        if ((numerics.swiglu_limit is not None or numerics.apply_probs_before_fc2)
                and not ops.features() & _lib.FEATURE_NUMERICS):
            raise NotImplementedError("this build of the gfx950 library has the SwiGLU clamp and the "
                                      "before-FC2 probabilities switched off")
        if numerics.partial_weight_grad_dtype not in (None, "native", "float32"):
            raise ValueError("partial_weight_grad_dtype must be native, float32 or None")
        if tuning.dispatch_mode not in ("push", "pull"):
            raise ValueError("dispatch_mode must be push or pull")
        for name, split in (("dispatch_split", tuning.dispatch_split), ("combine_split", tuning.combine_split)):
            if not isinstance(split, int) or isinstance(split, bool) or split <= 0 or split % _COMMUNICATION_SPLIT:
                raise ValueError(f"{name} must be a positive integer multiple of {_COMMUNICATION_SPLIT}, got {split!r}.")
        if precision == "mxfp8" and (tuning.scheduler.batch_experts or tuning.scheduler.nominal_schedule
                                     or tuning.scheduler.lowering == "compact"):
            raise ValueError("MXFP8 requires dense per-expert lowering")
        ep_size = 1
        if ep_group is not None:
            size = getattr(ep_group, "size", None)
            ep_size = size() if callable(size) else 1
            if ep_size != 1:
                raise ValueError("this build runs every expert on one GPU: ep_group must have size 1")
        if expert_placement is not None and getattr(expert_placement, "strategy", "none") != "none":
            raise ValueError("adaptive expert placement requires an EP group with more than one rank")
        if precision == "mxfp8" and (hidden_size % 64 or intermediate_size % 64):
            raise ValueError("MXFP8 requires hidden_size and intermediate_size divisible by 64")
        self.hidden_size = hidden_size
        self.intermediate_size = intermediate_size
        self.num_experts = num_experts
        self.top_k = top_k
        self.ep_size = ep_size
        self.local_experts = num_experts
        self._precision = precision
        self._numerics = numerics
        self._tuning = tuning
        self._layout: str | None = None
        local, hidden, inter = num_experts, hidden_size, intermediate_size
        self._weight_shapes = {
            "EIO": ((local, hidden, inter * 2), (local, inter, hidden)),
            "EOI": ((local, inter * 2, hidden), (local, hidden, inter)),
        }

    @property
    def precision(self) -> str:
        return self._precision

    @property
    def swiglu_limit(self) -> float | None:
        return self._numerics.swiglu_limit

    @property
    def clamp_after_silu(self) -> bool:
        return self._numerics.clamp_after_silu

    @property
    def apply_probs_before_fc2(self) -> bool:
        return self._numerics.apply_probs_before_fc2

    def share_execution_resources(self, *others: "MegaMoeExperts") -> None:
        """No-op: each call allocates its workspace from torch's caching allocator."""

    def close(self) -> None:
        """No-op: the executor holds no device resources between calls."""

    def _infer_layout(self, shape1: tuple, shape2: tuple) -> str:
        actual = (shape1, shape2)
        if actual == self._weight_shapes["EIO"]:
            return "EIO"
        if actual == self._weight_shapes["EOI"]:
            return "EOI"
        raise ValueError(f"expert_weights must have EIO shapes {self._weight_shapes['EIO']} or "
                         f"EOI shapes {self._weight_shapes['EOI']}, got {actual}.")

    def _bf16_weights(self, hidden: torch.Tensor, expert_weights: tuple):
        try:
            w1, w2 = expert_weights
            shape1, shape2 = tuple(w1.shape), tuple(w2.shape)
        except (AttributeError, TypeError, ValueError) as error:
            raise ValueError("expert_weights must contain two tensors") from error
        layout = self._layout or self._infer_layout(shape1, shape2)
        expected1, expected2 = self._weight_shapes[layout]
        if shape1 != expected1:
            raise ValueError(f"gate_up_weight must have shape {expected1}, got {shape1}.")
        if shape2 != expected2:
            raise ValueError(f"down_weight must have shape {expected2}, got {shape2}.")
        if w1.device != hidden.device or w2.device != hidden.device:
            raise ValueError("expert weights and hidden states must be on the same GPU.")
        if w1.dtype != torch.bfloat16 or w2.dtype != torch.bfloat16:
            raise TypeError("expert weights and hidden states must all use BF16.")
        if layout == "EOI" and (not w1.is_contiguous() or not w2.is_contiguous()):
            raise ValueError("EOI expert weights must be contiguous for zero-copy execution.")
        self._layout = layout
        return layout, w1.contiguous(), w2.contiguous()

    def _mx_weights(self, hidden: torch.Tensor, expert_weights: tuple):
        """(layout, w1 data, w1 scales, w2 data, w2 scales): the roots' EIO fields, with W1's gate and
        up columns interleaved (layout EIO_GU, prepared once per root and cached on it): the same
        results bit for bit as the EIO fields, and the fastest layout measured for both the prefill
        and the decode shapes (a GMM1 tile reads one run per weight row)."""
        from .mxfp8 import prepared_gate_up_weight, resolve_forward_weight
        try:
            r1, r2 = expert_weights
        except (TypeError, ValueError) as error:
            raise ValueError("expert_weights must contain two MX roots") from error
        E, H, I = self.num_experts, self.hidden_size, self.intermediate_size
        d1, s1 = resolve_forward_weight(r1, (E, H, 2 * I), hidden.device)
        d2, s2 = resolve_forward_weight(r2, (E, I, H), hidden.device)
        g1, u1 = prepared_gate_up_weight(r1, d1, s1)
        return "EIO_GU", g1, u1, d2, s2

    def forward(self, hidden_states: torch.Tensor, topk_ids: torch.Tensor, topk_weights: torch.Tensor, *,
                expert_weights: tuple, tokens_per_expert: torch.Tensor | None = None) -> torch.Tensor:
        """Route token states through the configured experts (module.py:497-535)."""
        if hidden_states.ndim < 2 or hidden_states.shape[-1] != self.hidden_size:
            raise ValueError("hidden_states must have at least two dimensions and configured "
                             f"hidden size {self.hidden_size}, got {tuple(hidden_states.shape)}.")
        flat = hidden_states.reshape(-1, self.hidden_size)
        route_shape = (flat.shape[0], self.top_k)
        if tuple(topk_ids.shape) != route_shape:
            raise ValueError(f"topk_ids must have shape {route_shape}, got {tuple(topk_ids.shape)}.")
        if tuple(topk_weights.shape) != route_shape:
            raise ValueError(f"topk_weights must have shape {route_shape}, got {tuple(topk_weights.shape)}.")
        if tokens_per_expert is not None and tuple(tokens_per_expert.shape) != (self.num_experts,):
            raise ValueError(f"tokens_per_expert must have shape ({self.num_experts},), "
                             f"got {tuple(tokens_per_expert.shape)}.")
        if hidden_states.dtype != torch.bfloat16 or hidden_states.device.type != "cuda":
            raise TypeError("MegaMoeExperts requires BF16 GPU hidden states.")
        if topk_ids.dtype not in (torch.int32, torch.int64):
            raise TypeError("topk_ids must be int32 or int64")
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError("MegaMoeExperts runs eagerly; graph capture is not supported")
        if flat.shape[0] == 0:
            return torch.empty_like(hidden_states)
        if tokens_per_expert is not None:
            if tokens_per_expert.device != topk_ids.device:
                raise ValueError("tokens_per_expert must be on the route tensor device.")
            if tokens_per_expert.dtype not in (torch.int32, torch.int64):
                raise TypeError(f"tokens_per_expert must be int32 or int64, got {tokens_per_expert.dtype}.")
        if CHECK_ROUTES:
            validate_routes(topk_ids, self.num_experts, tokens_per_expert)
        if tokens_per_expert is not None:
            tokens_per_expert = tokens_per_expert.to(torch.int32)
        if self._precision == "bf16":
            layout, w1, w2 = self._bf16_weights(flat, expert_weights)
            nm = self._numerics
            default_numerics = nm.swiglu_limit is None and not nm.apply_probs_before_fc2
            wants_grad = torch.is_grad_enabled() and any(
                t.requires_grad for t in (flat, topk_weights, w1, w2))
            if wants_grad and default_numerics and ops.features() & _lib.FEATURE_BACKWARD:
                grad_dtype = torch.float32 if nm.partial_weight_grad_dtype == "float32" else torch.bfloat16
                out = _MoeFunction.apply(flat, topk_weights, w1, w2, topk_ids, self.num_experts,
                                         self.intermediate_size, layout, grad_dtype)
            else:
                out = ops.moe_forward(flat, topk_ids, topk_weights, w1, w2, num_experts=self.num_experts,
                                      intermediate_size=self.intermediate_size, precision="bf16", layout=layout,
                                      tokens_per_expert=tokens_per_expert, swiglu_limit=nm.swiglu_limit,
                                      clamp_after_silu=nm.clamp_after_silu,
                                      apply_probs_before_fc2=nm.apply_probs_before_fc2)
        else:
            roots = tuple(expert_weights) if isinstance(expert_weights, (tuple, list)) else ()
            wants_grad = torch.is_grad_enabled() and (
                flat.requires_grad or topk_weights.requires_grad
                or any(isinstance(r, torch.Tensor) and r.requires_grad for r in roots))
            if wants_grad and len(roots) == 2 and ops.features() & _lib.FEATURE_MX_BACKWARD:
                nm = self._numerics
                grad_dtype = torch.float32 if nm.partial_weight_grad_dtype == "float32" else torch.bfloat16
                out = _MxMoeFunction.apply(flat, topk_weights, roots[0], roots[1], topk_ids, self, grad_dtype)
                return out.reshape(hidden_states.shape)
            layout, d1, s1, d2, s2 = self._mx_weights(flat, expert_weights)
            out = ops.moe_forward(flat, topk_ids, topk_weights, d1, d2, num_experts=self.num_experts,
                                  intermediate_size=self.intermediate_size, precision="mxfp8", layout=layout,
                                  w1_scale=s1, w2_scale=s2, tokens_per_expert=tokens_per_expert)
        return out.reshape(hidden_states.shape)
