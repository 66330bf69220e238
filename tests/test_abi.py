"""CPU checks of the C-ABI library: it loads, exports every symbol declared in include/*.h, and
rejects bad arguments before touching the GPU (no compute calls are made here)."""
import ctypes
import os
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


def _declared_symbols():
    names = set()
    for header in (ROOT / "include").glob("*.h"):
        text = header.read_text()
        for m in re.finditer(r"^\s*(?:int|int64_t|size_t|void)\s+(mi355moe_\w+)\s*\(", text, re.M):
            names.add(m.group(1))
    return names


def test_library_exports_every_declared_symbol():
    from hyper_multicore_amd import _lib
    lib = _lib.load()
    declared = _declared_symbols()
    assert declared, "no declarations found"
    missing = [n for n in declared if not hasattr(lib, n)]
    assert not missing, missing
    assert set(_lib.EXPORTED) == declared
    assert lib.mi355moe_abi_version() == _lib.ABI_VERSION


def test_invalid_arguments_rejected_without_launch():
    from hyper_multicore_amd import _lib
    lib = _lib.load()
    args = _lib.RouteArgs(num_tokens=4, num_experts=0, top_k=1, scoring=0, num_groups=1, topk_groups=1)
    assert lib.mi355moe_gate_route(ctypes.byref(args), None) == _lib.EINVAL
    args = _lib.RouteArgs(num_tokens=4, num_experts=8, top_k=9, scoring=0, num_groups=1, topk_groups=1)
    assert lib.mi355moe_gate_route(ctypes.byref(args), None) == _lib.EINVAL
    args = _lib.RouteArgs(num_tokens=4, num_experts=256, top_k=8, scoring=1, num_groups=8, topk_groups=0)
    assert lib.mi355moe_gate_route(ctypes.byref(args), None) == _lib.EINVAL
    d = _lib.DispatchArgs(num_tokens=4, top_k=2, num_experts=8, ids_dtype=7)
    assert lib.mi355moe_dispatch(ctypes.byref(d), None, 0, None) == _lib.EINVAL
    d = _lib.DispatchArgs(num_tokens=4, top_k=2, num_experts=8, ids_dtype=0, topk_ids=1, mapping=1)
    assert lib.mi355moe_dispatch(ctypes.byref(d), None, 0, None) == _lib.EWORKSPACE
    f = _lib.ForwardArgs(num_tokens=16, hidden_size=1000, intermediate_size=512, num_experts=8, top_k=2,
                         ids_dtype=0, precision=1, weight_layout=0)
    assert lib.mi355moe_moe_forward_workspace_size(ctypes.byref(f)) == 0
    assert lib.mi355moe_moe_forward(ctypes.byref(f), None, 0, None) in (_lib.EINVAL, _lib.EUNSUPPORTED)
    f = _lib.ForwardArgs(num_tokens=16, hidden_size=1024, intermediate_size=512, num_experts=8, top_k=2,
                         ids_dtype=0, precision=1, weight_layout=3)  # no such layout
    assert lib.mi355moe_moe_forward(ctypes.byref(f), None, 0, None) == _lib.EINVAL
    f.weight_layout = 1  # MXFP8 EOI (re-laid-out weights): operands missing, or the path switched off
    assert lib.mi355moe_moe_forward(ctypes.byref(f), None, 0, None) in (_lib.EINVAL, _lib.EUNSUPPORTED)


def test_unpermute_grad_validation():
    from hyper_multicore_amd import _lib
    lib = _lib.load()
    f = lib.mi355moe_token_unpermute_grad
    assert f(16, 16, 16, 16, 4, 2, 1004, 16, 16, None) == _lib.EINVAL        # hidden % 8
    assert f(None, 16, 16, 16, 4, 2, 1024, 16, 16, None) == _lib.EINVAL      # missing rows
    assert f(24, 16, 16, 16, 4, 2, 1024, 16, 16, None) == _lib.EINVAL        # rows not 16-byte aligned
    assert f(16, 16, 16, 16, -1, 2, 1024, 16, 16, None) == _lib.EINVAL
    if not lib.mi355moe_features() & _lib.FEATURE_BACKWARD:  # nothing is launched while switched off
        assert f(16, 16, 16, 16, 4, 2, 1024, 16, 16, None) == _lib.EUNSUPPORTED


def test_numerics_options_validation():
    from hyper_multicore_amd import _lib
    lib = _lib.load()
    base = dict(num_tokens=16, hidden_size=1024, intermediate_size=512, num_experts=8, top_k=2, ids_dtype=0,
                precision=0, weight_layout=0)
    f = _lib.ForwardArgs(**base, numerics_flags=4)  # unknown bit
    assert lib.mi355moe_moe_forward(ctypes.byref(f), None, 0, None) == _lib.EINVAL
    for bad in (-1.0, float("nan"), float("inf")):
        f = _lib.ForwardArgs(**base, swiglu_limit=bad)
        assert lib.mi355moe_moe_forward(ctypes.byref(f), None, 0, None) == _lib.EINVAL
    f = _lib.ForwardArgs(**{**base, "precision": 1}, swiglu_limit=7.0)  # MXFP8 rejects the options
    assert lib.mi355moe_moe_forward(ctypes.byref(f), None, 0, None) == _lib.EINVAL
    f = _lib.ForwardArgs(**{**base, "precision": 1}, numerics_flags=2)
    assert lib.mi355moe_moe_forward(ctypes.byref(f), None, 0, None) == _lib.EINVAL
    f = _lib.ForwardArgs(**base, swiglu_limit=7.0)
    assert lib.mi355moe_moe_forward(ctypes.byref(f), None, 0, None) in (_lib.EINVAL, _lib.EUNSUPPORTED)


def test_backward_validation():
    from hyper_multicore_amd import _lib
    lib = _lib.load()
    base = dict(num_tokens=16, hidden_size=1024, intermediate_size=512, num_experts=8, top_k=2, ids_dtype=0,
                weight_layout=0)
    f = _lib.BackwardArgs(**base, weight_grad_dtype=2)
    assert lib.mi355moe_moe_backward(ctypes.byref(f), None, 0, None) == _lib.EINVAL
    f = _lib.BackwardArgs(**{**base, "weight_layout": 3})
    assert lib.mi355moe_moe_backward(ctypes.byref(f), None, 0, None) == _lib.EINVAL
    f = _lib.BackwardArgs(**{**base, "hidden_size": 1000})
    assert lib.mi355moe_moe_backward(ctypes.byref(f), None, 0, None) == _lib.EUNSUPPORTED
    f = _lib.BackwardArgs(**base)  # valid shape, operands missing (or the path switched off)
    assert lib.mi355moe_moe_backward(ctypes.byref(f), None, 0, None) in (_lib.EINVAL, _lib.EUNSUPPORTED)
    assert lib.mi355moe_moe_backward_workspace_size(ctypes.byref(f)) == 0 or lib.mi355moe_features() & 8


def test_route_grad_validation():
    """RouteGrad rejects bad shapes / missing operands before any launch; with valid (dummy) pointers it
    answers EUNSUPPORTED while the path is switched off."""
    from hyper_multicore_amd import _lib
    lib = _lib.load()
    base = dict(logits=1, logits_row_stride=64, scores=1, indices=1, grad_weights=1, grad_logits=1, scoring=2,
                num_tokens=16, num_experts=64, top_k=8, routed_scaling_factor=2.5)
    for bad in ({"num_experts": 1025}, {"top_k": 65}, {"top_k": 0}, {"scoring": 3}, {"scores": None},
                {"indices": None}, {"grad_weights": None}, {"grad_logits": None}, {"logits": None},
                {"logits_row_stride": 32}, {"num_tokens": -1}):
        a = _lib.RouteGradArgs(**{**base, **bad})
        assert lib.mi355moe_gate_route_grad(ctypes.byref(a), None) == _lib.EINVAL, bad
    # sigmoid / softmax gradients do not read the logits
    # (never with the path on: the dummy pointers would reach a kernel)
    if not lib.mi355moe_features() & _lib.FEATURE_ROUTE_GRAD:
        a = _lib.RouteGradArgs(**{**base, "scoring": 1, "logits": None})
        assert lib.mi355moe_gate_route_grad(ctypes.byref(a), None) == _lib.EUNSUPPORTED
    assert lib.mi355moe_gate_route_grad(None, None) == _lib.EINVAL


def test_mx_quantize_weight_validation():
    from hyper_multicore_amd import _lib
    lib = _lib.load()
    q = lib.mi355moe_mx_quantize_weight
    for args in ((1, 0, 64, 64, 1, 1, 1, 1), (1, 2, 96, 64, 1, 1, 1, 1), (1, 2, 64, 96, 1, 1, 1, 1),
                 (None, 2, 64, 64, 1, 1, 1, 1), (1, 2, 64, 64, None, None, None, None), (1, 2, 64, 64, 1, None, 1, 1),
                 (1, 2, 64, 64, 1, 1, None, 1)):
        assert q(*args, None) == _lib.EINVAL, args
    if not lib.mi355moe_features() & _lib.FEATURE_MX_WEIGHT_PREP:  # never launches with dummy pointers
        assert q(1, 2, 64, 64, 1, 1, None, None, None) == _lib.EUNSUPPORTED


def test_workspace_sizes():
    from hyper_multicore_amd import _lib
    lib = _lib.load()
    assert lib.mi355moe_dispatch_workspace_size(8192, 8, 256) >= 256 * 4
    f = _lib.ForwardArgs(num_tokens=8192, hidden_size=7168, intermediate_size=2048, num_experts=256, top_k=8,
                         ids_dtype=1, precision=0, weight_layout=1, hidden=1, topk_ids=1, topk_weights=1, w1=1, w2=1,
                         out=1)
    need = lib.mi355moe_moe_forward_workspace_size(ctypes.byref(f))
    R = 8192 * 8
    assert need >= R * 2048 * 2 + R * 7168 * 2  # act + expert outputs


def test_gpu_ops_refuse_cpu_tensors():
    import torch
    from hyper_multicore_amd import ops
    with pytest.raises(TypeError):
        ops.gate_route(torch.zeros(2, 8), torch.zeros(8), top_k=2, scoring_func="softmax", routed_scaling_factor=1.0)
    with pytest.raises(TypeError):  # the one-time weight preparation runs on the GPU only as well
        ops.interleave_gate_up(torch.zeros(2, 64, 256, dtype=torch.bfloat16))


def test_gemm_variant_is_per_call():
    """The GEMM configuration is an argument of each call: an unknown variant is refused before
    anything is enqueued (null pointers, so no launch is possible), a known one reaches the ordinary
    argument checks. The Python default is per thread and never reaches the library as state."""
    import threading
    from hyper_multicore_amd import _lib, ops
    lib = _lib.load()
    for bad in (-1, 1, 2, 3, 4, 7):  # 1-4: configurations retired with ABI 7
        assert lib.mi355moe_grouped_gemm_bf16(None, 4, 64, None, 0, 1, 8, None, None, bad, None, 0, None) \
            == _lib.EUNSUPPORTED
        assert lib.mi355moe_grouped_gemm_mxfp8(None, None, 4, 512, None, None, 0, 1, 16, None, None, bad, None, 0,
                                               None) == _lib.EUNSUPPORTED
        args = _lib.ForwardArgs(num_tokens=4, hidden_size=128, intermediate_size=128, num_experts=4, top_k=2,
                                ids_dtype=_lib.IDS_INT32, precision=_lib.PRECISION["bf16"], gemm_variant=bad)
        assert lib.mi355moe_moe_forward(ctypes.byref(args), None, 0, None) == _lib.EUNSUPPORTED
    # a valid variant passes the variant check and fails on the null operands instead
    assert lib.mi355moe_grouped_gemm_bf16(None, 4, 64, None, 0, 1, 8, None, None, _lib.GEMM_VARIANT["w4"], None, 0,
                                          None) == _lib.EINVAL
    with pytest.raises(ValueError):
        ops.set_gemm_variant("fastest")
    prev = ops.set_gemm_variant("w4")
    try:
        seen = []
        t = threading.Thread(target=lambda: seen.append(ops.gemm_variant()))
        t.start()
        t.join()
        # a new thread starts from the process default, not from this thread's setting
        assert ops.gemm_variant() == "w4" and seen == [os.environ.get("MI355MOE_GG_VARIANT") or "default"]
    finally:
        ops.set_gemm_variant(prev)


def test_interleave_gate_up_validation():
    """The gate/up interleave refuses bad sizes, element widths, misaligned or overlapping buffers
    before any launch; the backward refuses the forward-only interleaved layout."""
    from hyper_multicore_amd import _lib
    lib = _lib.load()
    f = lib.mi355moe_interleave_gate_up
    assert f(None, 0, 128, 1, None, None) == _lib.OK  # nothing to move
    assert f(16, 4, 192, 1, 4096, None) == _lib.EINVAL  # I % 128
    assert f(16, 4, 128, 4, 4096, None) == _lib.EINVAL  # element width
    assert f(None, 4, 128, 1, 4096, None) == _lib.EINVAL
    assert f(16, 4, 128, 1, 4104, None) == _lib.EINVAL  # dst not 16-byte aligned
    assert f(4096, 4, 128, 2, 4096 + 512, None) == _lib.EINVAL  # overlap (rows of 512 bytes)
    b = _lib.BackwardArgs(num_tokens=16, hidden_size=1024, intermediate_size=512, num_experts=8, top_k=2,
                          ids_dtype=0, weight_layout=_lib.LAYOUT["EIO_GU"])
    assert lib.mi355moe_moe_backward_workspace_size(ctypes.byref(b)) == 0
    assert lib.mi355moe_moe_backward(ctypes.byref(b), None, 0, None) == _lib.EUNSUPPORTED
