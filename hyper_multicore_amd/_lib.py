"""ctypes binding of the C ABI declared in ``include/mi355moe.h``.

The library is loaded from the package's ``_lib/`` folder (built in-tree by ``build.py``).
There is no fallback: when the library is missing every operation raises, so a GPU run can
never silently take a CPU or PyTorch path.
"""
from __future__ import annotations

import ctypes
from ctypes import POINTER, Structure, c_float, c_int32, c_int64, c_size_t, c_uint8, c_uint16, c_void_p
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libmi355moe.so"
ABI_VERSION = 7

OK, EINVAL, ELAUNCH, EUNSUPPORTED, EWORKSPACE = 0, -1, -2, -3, -4
NOALLOC_MAX_GROUPS = 4096
SCORE = {"softmax": 0, "sigmoid": 1, "sqrtsoftplus": 2}
IDS_INT32, IDS_INT64 = 0, 1
PRECISION = {"bf16": 0, "mxfp8": 1}
FEATURE_MX_EOI = 1
FEATURE_NUMERICS = 2
FEATURE_DECODE_TILES = 4
FEATURE_BACKWARD = 8
FEATURE_ROUTE_GRAD = 16
FEATURE_MX_WEIGHT_PREP = 32
FEATURE_MX_BACKWARD = 64
GEMM_VARIANT = {"default": 0, "pp": 5, "w4": 6}
NUMERICS_CLAMP_AFTER_SILU = 1
NUMERICS_PROBS_BEFORE_FC2 = 2
LAYOUT = {"EIO": 0, "EOI": 1, "EIO_GU": 2}

_ERRORS = {
    EINVAL: "invalid argument",
    ELAUNCH: "HIP launch failure",
    EUNSUPPORTED: "shape or option not supported by the gfx950 kernels",
    EWORKSPACE: "workspace missing or too small",
}


class RouteArgs(Structure):
    _fields_ = [
        ("logits", c_void_p), ("logits_row_stride", c_int64),
        ("bias", c_void_p), ("bias_vl", c_void_p), ("image_mask", c_void_p),
        ("weights_out", c_void_p), ("indices_out", c_void_p), ("indices32_out", c_void_p),
        ("scores_out", c_void_p),
        ("num_tokens", c_int64), ("num_experts", c_int32), ("top_k", c_int32), ("scoring", c_int32),
        ("num_groups", c_int32), ("topk_groups", c_int32), ("routed_scaling_factor", c_float),
    ]


class RouteGradArgs(Structure):
    _fields_ = [
        ("logits", c_void_p), ("logits_row_stride", c_int64), ("scores", c_void_p), ("indices", c_void_p),
        ("indices32", c_void_p), ("grad_weights", c_void_p), ("grad_logits", c_void_p), ("accumulate", c_int32),
        ("scoring", c_int32), ("num_tokens", c_int64), ("num_experts", c_int32), ("top_k", c_int32),
        ("routed_scaling_factor", c_float), ("reserved", c_int32),
        ("selected_scores", c_void_p), ("denominator", c_void_p),
    ]


class DispatchArgs(Structure):
    _fields_ = [
        ("topk_ids", c_void_p), ("ids_dtype", c_int32), ("top_k", c_int32), ("num_tokens", c_int64),
        ("num_experts", c_int32), ("counts", c_void_p), ("expert_offsets", c_void_p),
        ("group_list", c_void_p), ("mapping", c_void_p), ("gather_index", c_void_p),
        ("error_flag", c_void_p),
    ]


class ForwardArgs(Structure):
    _fields_ = [
        ("hidden", c_void_p), ("num_tokens", c_int64), ("hidden_size", c_int32),
        ("intermediate_size", c_int32), ("num_experts", c_int32), ("top_k", c_int32),
        ("topk_ids", c_void_p), ("ids_dtype", c_int32), ("precision", c_int32),
        ("topk_weights", c_void_p), ("weight_layout", c_int32), ("numerics_flags", c_int32),
        ("w1", c_void_p), ("w2", c_void_p), ("w1_scale", c_void_p), ("w2_scale", c_void_p),
        ("tokens_per_expert", c_void_p), ("out", c_void_p), ("error_flag", c_void_p),
        ("stage_events", POINTER(c_void_p)), ("num_stage_events", c_int32), ("swiglu_limit", c_float),
        ("gemm_variant", c_int32),
    ]


class BackwardArgs(Structure):
    """MI355MoeBackwardArgs in include/mi355moe.h."""
    _fields_ = [
        ("hidden", c_void_p), ("num_tokens", c_int64), ("hidden_size", c_int32), ("intermediate_size", c_int32),
        ("num_experts", c_int32), ("top_k", c_int32), ("topk_ids", c_void_p), ("ids_dtype", c_int32),
        ("weight_layout", c_int32), ("topk_weights", c_void_p), ("w1", c_void_p), ("w2", c_void_p),
        ("grad_out", c_void_p), ("grad_hidden", c_void_p), ("grad_w1", c_void_p), ("grad_w2", c_void_p),
        ("grad_topk_weights", c_void_p), ("weight_grad_dtype", c_int32), ("precision", c_int32),
        ("w1_scale", c_void_p), ("w2_scale", c_void_p), ("w1_row", c_void_p), ("w2_row", c_void_p),
        ("w1_row_scale", c_void_p), ("w2_row_scale", c_void_p), ("error_flag", c_void_p),
    ]


# (name, restype, argtypes)
_SIGNATURES = [
    ("mi355moe_abi_version", c_int32, []),
    ("mi355moe_features", c_int32, []),
    ("mi355moe_gate_logits_workspace_size", c_size_t, [c_int64, c_int32, c_int32]),
    ("mi355moe_gate_logits", c_int32, [c_void_p, c_int64, c_int32, c_void_p, c_void_p, c_void_p, c_int32,
                                       c_void_p, c_void_p, c_size_t, c_void_p]),
    ("mi355moe_gate_route", c_int32, [POINTER(RouteArgs), c_void_p]),
    ("mi355moe_gate_route_grad", c_int32, [POINTER(RouteGradArgs), c_void_p]),
    ("mi355moe_dispatch_workspace_size", c_size_t, [c_int64, c_int32, c_int32]),
    ("mi355moe_dispatch", c_int32, [POINTER(DispatchArgs), c_void_p, c_size_t, c_void_p]),
    ("mi355moe_token_permute", c_int32, [c_void_p, c_int64, c_int32, c_void_p, c_int32, c_int32, c_int32,
                                         c_void_p, c_void_p, c_void_p, c_size_t, c_void_p]),
    ("mi355moe_token_unpermute", c_int32, [c_void_p, c_void_p, c_void_p, c_int64, c_int32, c_int32,
                                           c_void_p, c_void_p]),
    ("mi355moe_token_unpermute_grad", c_int32, [c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int32, c_int32,
                                                c_void_p, c_void_p, c_void_p]),
    ("mi355moe_mx_quantize_rows", c_int32, [c_void_p, c_int64, c_int32, c_void_p, c_void_p, c_void_p]),
    ("mi355moe_mx_quantize_cols", c_int32, [c_void_p, c_int32, c_int32, c_int32, c_void_p, c_void_p,
                                            c_void_p]),
    ("mi355moe_mx_quantize_weight", c_int32, [c_void_p, c_int32, c_int32, c_int32, c_void_p, c_void_p, c_void_p,
                                              c_void_p, c_void_p]),
    ("mi355moe_mx_weight_scale_ld", c_int64, [c_int32]),
    ("mi355moe_mx_weight_to_eoi", c_int32, [c_void_p, c_void_p, c_int32, c_int32, c_int32, c_void_p, c_void_p,
                                            c_void_p]),
    ("mi355moe_interleave_gate_up", c_int32, [c_void_p, c_int64, c_int32, c_int32, c_void_p, c_void_p]),
    ("mi355moe_grouped_gemm_workspace_size", c_size_t, [c_int32]),
    ("mi355moe_grouped_gemm_bf16", c_int32, [c_void_p, c_int64, c_int32, c_void_p, c_int32, c_int32, c_int32,
                                             c_void_p, c_void_p, c_int32, c_void_p, c_size_t, c_void_p]),
    ("mi355moe_grouped_gemm_bf16_noalloc", c_int32, [c_void_p, c_int64, c_int32, c_void_p, c_int32, c_int32,
                                                     c_int32, c_void_p, c_void_p, c_int32, c_void_p]),
    ("mi355moe_grouped_gemm_mxfp8", c_int32, [c_void_p, c_void_p, c_int64, c_int32, c_void_p, c_void_p, c_int32,
                                              c_int32, c_int32, c_void_p, c_void_p, c_int32, c_void_p, c_size_t,
                                              c_void_p]),
    ("mi355moe_moe_forward_workspace_size", c_size_t, [POINTER(ForwardArgs)]),
    ("mi355moe_moe_forward", c_int32, [POINTER(ForwardArgs), c_void_p, c_size_t, c_void_p]),
    ("mi355moe_moe_backward_workspace_size", c_size_t, [POINTER(BackwardArgs)]),
    ("mi355moe_moe_backward", c_int32, [POINTER(BackwardArgs), c_void_p, c_size_t, c_void_p]),
]
EXPORTED = [name for name, _, _ in _SIGNATURES]

_lib = None


def load() -> ctypes.CDLL:
    """Load (once) and return the native library; raise if it is missing or stale."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"native library {LIB_PATH} is missing; build it with `python -m hyper_multicore_amd.build`")
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, restype, argtypes in _SIGNATURES:
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    version = lib.mi355moe_abi_version()
    if version != ABI_VERSION:
        raise RuntimeError(f"libmi355moe ABI {version} does not match the Python binding ({ABI_VERSION})")
    _lib = lib
    return lib


def check(rc: int, what: str) -> None:
    """Raise the reference-style exception for a non-zero status code."""
    if rc == OK:
        return
    message = f"{what}: {_ERRORS.get(rc, 'error')} (status {rc})"
    if rc in (EINVAL, EUNSUPPORTED, EWORKSPACE):
        raise ValueError(message)
    raise RuntimeError(message)
