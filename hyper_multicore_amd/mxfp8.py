"""MXFP8 expert-weight roots (modules/mega_moe/backends/mxfp8/weights.py:21-86 convention).

A root is a tensor (or any object) carrying the forward physical fields
``col_data`` (``torch.float8_e4m3fn``, viewable as ``[E, M, N]``) and ``col_scale``
(``torch.uint8`` e8m0, viewable as ``[E, M/64, N, 2]``: the two 32-blocks of each 64-row group
along the reduction axis M, for every output column N). ``quantize_expert_weight`` builds such a
root from a bf16 ``[E, M, N]`` weight on the GPU.
"""
from __future__ import annotations

import torch

from . import _lib, ops

__all__ = ["quantize_expert_weight", "resolve_forward_weight", "resolve_backward_weight", "prepared_eoi_weight",
           "prepared_gate_up_weight"]


def quantize_expert_weight(weight: torch.Tensor, *, backward_axis: bool = False) -> torch.Tensor:
    """Return a root holding ``col_data`` / ``col_scale`` for a bf16 EIO weight ``[E, M, N]``.

    With ``backward_axis=True`` the root also carries the backward axis ``row_data`` / ``row_scale``
    (``[E, M, N]`` e4m3 and ``[E, M, N/64, 2]``: blocks of 32 along N), both axes quantised in one
    pass by the dual-axis kernel (needs the library's MX weight-preparation feature).
    The root is a one-element bf16 tensor expanded to the logical shape ``[E, M, N]`` on the
    weight's device; only the physical attributes are read by the executor.
    """
    if weight.ndim != 3:
        raise ValueError("expected an EIO expert weight [E, M, N]")
    E, M, N = weight.shape
    if M % 64 or N % 64:
        raise ValueError(f"MegaMoE MXFP8 expert shape requires M/N divisible by 64, got {tuple(weight.shape)}.")
    row_data = row_scale = None
    if backward_axis:
        if not ops.features() & _lib.FEATURE_MX_WEIGHT_PREP:
            raise NotImplementedError("the dual-axis MX weight quantisation is switched off in this build")
        data, scale, row_data, row_scale = ops.mx_quantize_weight(weight.to(torch.bfloat16))
    else:
        data, scale = ops.mx_quantize_cols(weight.to(torch.bfloat16))
    root = torch.empty((1, 1, 1), dtype=torch.bfloat16, device=weight.device).expand(E, M, N)
    root.col_data = data
    root.col_scale = scale
    root.row_data = row_data
    root.row_scale = row_scale
    root.logical_shape = (E, M, N)
    return root


def resolve_forward_weight(root, logical_shape: tuple[int, int, int], device: torch.device):
    """Validate and return (col_data uint8 view [E,M,N], col_scale uint8 [E,M/64,N,2])."""
    data = getattr(root, "col_data", None)
    scale = getattr(root, "col_scale", None)
    if data is None or scale is None:
        raise ValueError("MegaMoE MXFP8 current root is missing required col data/scale.")
    if data.dtype != torch.float8_e4m3fn or scale.dtype != torch.uint8:
        raise TypeError("MegaMoE MXFP8 physical storage requires E4M3FN data and packed uint8 E8M0 scales.")
    if not data.is_contiguous() or not scale.is_contiguous():
        raise ValueError("MX physical data and scale must be contiguous; implicit copies are forbidden")
    if data.device != device or scale.device != device:
        raise ValueError("MX physical data, scales and hidden states must share a device")
    E, M, N = logical_shape
    if data.numel() != E * M * N or scale.numel() != E * (M // 64) * N * 2:
        raise ValueError(f"MX root does not hold an [E, M, N] = {logical_shape} weight")
    return data.view(torch.uint8).view(E, M, N), scale.view(E, M // 64, N, 2)


def resolve_backward_weight(root, logical_shape: tuple[int, int, int], device: torch.device):
    """The backward axis of a root (weights.py:59-78 'row' pair): (row_data uint8 view [E, M, N],
    row_scale uint8 [E, M, N/64, 2]), blocks of 32 along N for every row."""
    data = getattr(root, "row_data", None)
    scale = getattr(root, "row_scale", None)
    if data is None or scale is None:
        raise ValueError("MegaMoE MXFP8 current root is missing required row data/scale.")
    if data.dtype != torch.float8_e4m3fn or scale.dtype != torch.uint8:
        raise TypeError("MegaMoE MXFP8 physical storage requires E4M3FN data and packed uint8 E8M0 scales.")
    if not data.is_contiguous() or not scale.is_contiguous():
        raise ValueError("MX physical data and scale must be contiguous; implicit copies are forbidden")
    if data.device != device or scale.device != device:
        raise ValueError("MX physical data, scales and hidden states must share a device")
    E, M, N = logical_shape
    if data.numel() != E * M * N or scale.numel() != E * M * (N // 64) * 2:
        raise ValueError(f"MX root does not hold an [E, M, N] = {logical_shape} weight")
    return data.view(torch.uint8).view(E, M, N), scale.view(E, M, N // 64, 2)


def _cached_on_root(root, attr: str, data: torch.Tensor, scale: torch.Tensor, prepare):
    """prepare(data, scale), built on first use and cached on the root under `attr`. The cache is keyed
    on the storage of the root's fields, so a root whose ``col_data`` / ``col_scale`` are replaced is
    prepared again; in-place writes into the same storage are not detected (roots are treated as
    immutable weights)."""
    key = (data.data_ptr(), scale.data_ptr(), tuple(data.shape), data.device)
    cached = getattr(root, attr, None)
    if cached is not None and cached[0] == key:
        return cached[1], cached[2]
    d, s = prepare(data, scale)
    d = d.view(torch.uint8)
    try:
        setattr(root, attr, (key, d, s))
    except AttributeError:  # roots without attribute storage are prepared per call
        pass
    return d, s


def prepared_eoi_weight(root, data: torch.Tensor, scale: torch.Tensor):
    """The K-contiguous re-layout of a root's (data, scale) for the GEMM (``ops.mx_weight_to_eoi``),
    cached on the root."""
    return _cached_on_root(root, "_mi355_eoi", data, scale, ops.mx_weight_to_eoi)


def prepared_gate_up_weight(root, data: torch.Tensor, scale: torch.Tensor):
    """The GMM1 root's (data, scale) with gate and up columns interleaved in 64-column blocks
    (``ops.interleave_gate_up``, layout ``"EIO_GU"``), cached on the root."""
    return _cached_on_root(root, "_mi355_gate_up", data, scale, ops.interleave_gate_up)
