"""The no-allocation grouped GEMM entry point (mi355moe_grouped_gemm_bf16_noalloc): called through the
C ABI, it must give the same bytes as mi355moe_grouped_gemm_bf16 (the workspace form), on two calls in a
row of which the second is smaller (fewer groups and rows: the static tile plan keeps the first call's
tail, which the second must not read), in both weight layouts and for a decode shape (64-row tiles)."""
import numpy as np
import pytest
import torch

from oracle import moe_oracle as orc

pytestmark = pytest.mark.gpu


def _noalloc(x, w, gl, layout, variant="default"):
    from hyper_multicore_amd import _lib, ops
    lib = _lib.load()
    G = w.shape[0]
    K, N = (w.shape[1], w.shape[2]) if layout == "EIO" else (w.shape[2], w.shape[1])
    out = torch.full((x.shape[0], N), float("nan"), dtype=torch.bfloat16, device=x.device)
    rc = lib.mi355moe_grouped_gemm_bf16_noalloc(ops._ptr(x), x.shape[0], K, ops._ptr(w), _lib.LAYOUT[layout], G, N,
                                                ops._ptr(gl), ops._ptr(out), _lib.GEMM_VARIANT[variant],
                                                ops._stream(x.device))
    _lib.check(rc, "mi355moe_grouped_gemm_bf16_noalloc")
    return out


def _case(counts, K, N, layout, seed, gpu):
    g = torch.Generator().manual_seed(seed)
    G, rows = len(counts), sum(counts)
    x = torch.randn(rows, K, generator=g).to(torch.bfloat16).to(gpu)
    w = (torch.randn(G, K, N, generator=g) * 0.05).to(torch.bfloat16)
    w = (w if layout == "EIO" else w.transpose(1, 2).contiguous()).to(gpu)
    gl = torch.tensor(counts).cumsum(0).to(torch.int64).to(gpu)
    return x, w, gl


@pytest.mark.parametrize("variant", ["default", "w4"])
@pytest.mark.parametrize("layout", ["EIO", "EOI"])
def test_noalloc_matches_workspace_form_twice(gpu, layout, variant):
    """Both configurations: the default one (8-wave kernel, which builds its work list from group_list)
    and "w4" (the 4-wave kernel, which reads the tile plan from the static array, so the second,
    smaller call must not read the first call's longer plan)."""
    from hyper_multicore_amd import ops
    print(f"[no_alloc] layout {layout} variant {variant}", flush=True)
    first = _case([300, 0, 513, 77, 256, 1, 129, 40], 1024, 768, layout, 11, gpu)
    second = _case([5, 260, 0, 31], 512, 256, layout, 12, gpu)  # fewer groups and rows than the first
    for x, w, gl in (first, second):
        ref = ops.grouped_gemm_bf16(x, w, gl, layout, gemm_variant=variant)
        out = _noalloc(x, w, gl, layout, variant)
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16).cpu(), ref.view(torch.int16).cpu())
    # and against the fp32 product of the second case (the bytes compared above are the right ones)
    x, w, gl = second
    wf = (w if layout == "EIO" else w.transpose(1, 2)).float().cpu()
    starts = [0, *gl.cpu().tolist()]
    want = torch.cat([x[starts[i]:starts[i + 1]].float().cpu() @ wf[i] for i in range(len(starts) - 1)])
    assert orc.rel_l2(out.float().cpu(), want) < 2e-3


def test_noalloc_decode_shape_then_smaller(gpu):
    """Many small groups (the 64-row decode tiles where the library has them on), then fewer."""
    from hyper_multicore_amd import ops
    print("[no_alloc] decode shape", flush=True)
    rng = np.random.default_rng(5)
    for G, seed in ((96, 21), (40, 22)):
        counts = rng.integers(0, 30, G).tolist()
        x, w, gl = _case(counts, 512, 256, "EOI", seed, gpu)
        ref = ops.grouped_gemm_bf16(x, w, gl, "EOI")
        out = _noalloc(x, w, gl, "EOI")
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16).cpu(), ref.view(torch.int16).cpu())


def test_noalloc_rejects_too_many_groups(gpu):
    """Above the static plan's maximum the call answers the workspace error and launches nothing."""
    from hyper_multicore_amd import _lib
    lib = _lib.load()
    rc = lib.mi355moe_grouped_gemm_bf16_noalloc(None, 4, 64, None, 0, _lib.NOALLOC_MAX_GROUPS + 1, 8, None, None, 0,
                                                None)
    assert rc == _lib.EWORKSPACE
