"""GPU tests of the 8-wave ping-pong grouped-GEMM configuration (gemm_pp.hip, the default): it runs
the same MFMAs in the same K order per output element as the 4-wave configuration (variant "w4"),
so its outputs are bit-identical to it; and both match the fp32-accumulate oracle."""
import contextlib

import pytest
import torch

from oracle import moe_oracle as orc

pytestmark = pytest.mark.gpu

BF16_REL_L2 = 1e-2


@pytest.fixture(scope="module")
def gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from hyper_multicore_amd import _lib
    _lib.load()
    return torch.device("cuda:0")


def _seed(s):
    torch.manual_seed(s)
    return torch.Generator().manual_seed(s)


@contextlib.contextmanager
def _variant(name):
    from hyper_multicore_amd import ops
    prev = ops.set_gemm_variant(name)
    try:
        yield
    finally:
        ops.set_gemm_variant(prev)


VARIANTS = ["pp"]
COUNTS = [[100, 0, 300, 1, 129], [0, 0, 7], [256] * 4, [3, 40, 0, 513], [1], [600, 255, 257]]


@pytest.mark.parametrize("layout", ["EOI", "EIO"])
@pytest.mark.parametrize("Kd", [256, 2048])
@pytest.mark.parametrize("counts", COUNTS)
@pytest.mark.parametrize("variant", VARIANTS)
def test_grouped_gemm_bf16_pp_matches_default(gpu, variant, counts, Kd, layout):
    from hyper_multicore_amd import ops
    print(f"[pp] {variant} bf16 {layout} K={Kd} counts={counts}", flush=True)
    g = _seed(sum(counts) + Kd + (layout == "EIO"))
    G, N = len(counts), 768
    rows = sum(counts)
    x = torch.randn(rows, Kd, generator=g).to(torch.bfloat16)
    w = (torch.randn(G, Kd, N, generator=g) * 0.05).to(torch.bfloat16)  # [G, K, N]
    wd = (w if layout == "EIO" else w.transpose(1, 2).contiguous()).to(gpu)
    gl = torch.tensor(counts).cumsum(0).to(torch.int64).to(gpu)
    with _variant("w4"):
        out_def = ops.grouped_gemm_bf16(x.to(gpu), wd, gl, layout).cpu()
    with _variant(variant):
        out_pp = ops.grouped_gemm_bf16(x.to(gpu), wd, gl, layout).cpu()
    assert torch.equal(out_pp, out_def)
    starts = [0, *gl.cpu().tolist()]
    ref = torch.cat([x[starts[i]:starts[i + 1]].float() @ w[i].float() for i in range(G)]).to(torch.bfloat16)
    assert orc.rel_l2(out_pp, ref) < 2e-3


@pytest.mark.parametrize("layout", ["EOI", "EIO"])
@pytest.mark.parametrize("variant", VARIANTS)
def test_moe_forward_bf16_pp_matches_default(gpu, variant, layout):
    from hyper_multicore_amd import ops
    T, H, I, E, K = 700, 1024, 512, 16, 4
    print(f"[pp] moe_forward bf16 {layout}", flush=True)
    g = _seed(T + E + 3)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    ids = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(T)])
    probs = torch.rand(T, K, generator=g)
    probs = probs / probs.sum(1, keepdim=True)
    w1 = (torch.randn(E, H, 2 * I, generator=g) * 0.02).to(torch.bfloat16)
    w2 = (torch.randn(E, I, H, generator=g) * 0.02).to(torch.bfloat16)
    if layout == "EOI":
        w1d, w2d = w1.transpose(1, 2).contiguous().to(gpu), w2.transpose(1, 2).contiguous().to(gpu)
    else:
        w1d, w2d = w1.to(gpu), w2.to(gpu)
    args = dict(num_experts=E, intermediate_size=I, layout=layout)
    with _variant("w4"):
        out_def = ops.moe_forward(x.to(gpu), ids.to(gpu), probs.to(gpu), w1d, w2d, **args).cpu()
    with _variant(variant):
        out_pp = ops.moe_forward(x.to(gpu), ids.to(gpu), probs.to(gpu), w1d, w2d, **args).cpu()
    assert torch.equal(out_pp, out_def)
    ref = orc.expert_forward_reference(x, ids, probs, w1, w2, layout="EIO")
    assert orc.rel_l2(out_pp, ref) < BF16_REL_L2


@pytest.mark.parametrize("T,H,I,E,K", [(700, 1024, 512, 16, 4), (64, 1024, 256, 64, 8), (300, 2048, 384, 8, 2),
                                       (333, 1152, 256, 8, 4)])
@pytest.mark.parametrize("variant", VARIANTS)
def test_moe_forward_mxfp8_pp_matches_w4(gpu, variant, T, H, I, E, K):
    """MXFP8 forward on the 8-wave GEMMs (stage-major activation scales, col_data / col_scale weights)
    equals the 4-wave path bit for bit, and the MX-emulating oracle to the MX bar."""
    from hyper_multicore_amd import ops
    print(f"[pp] moe_forward mxfp8 T={T} H={H} I={I} E={E} K={K}", flush=True)
    g = _seed(T + E + 9)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    ids = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(T)])
    probs = torch.rand(T, K, generator=g)
    probs = probs / probs.sum(1, keepdim=True)
    w1 = (torch.randn(E, H, 2 * I, generator=g) * 0.02).to(torch.bfloat16)
    w2 = (torch.randn(E, I, H, generator=g) * 0.02).to(torch.bfloat16)
    d1, s1 = ops.mx_quantize_cols(w1.to(gpu))
    d2, s2 = ops.mx_quantize_cols(w2.to(gpu))
    args = dict(num_experts=E, intermediate_size=I, precision="mxfp8", w1_scale=s1, w2_scale=s2)
    ins = (x.to(gpu), ids.to(gpu), probs.to(gpu), d1.view(torch.uint8), d2.view(torch.uint8))
    with _variant("w4"):
        out_w4 = ops.moe_forward(*ins, **args).cpu()
    with _variant(variant):
        out_pp = ops.moe_forward(*ins, **args).cpu()
    assert torch.equal(out_pp, out_w4)
    ref = orc.expert_forward_reference(x, ids, probs, d1.cpu().view(torch.uint8), d2.cpu().view(torch.uint8),
                                       precision="mxfp8", w1_scale=s1.cpu(), w2_scale=s2.cpu())
    assert orc.rel_l2(out_pp, ref) < 3e-2


@pytest.mark.parametrize("precision", ["bf16", "mxfp8"])
@pytest.mark.parametrize("variant", VARIANTS)
def test_moe_forward_decode_shape_pp(gpu, variant, precision):
    """Decode shape (a few routed rows per expert, many empty experts) on the 8-wave GEMMs."""
    from hyper_multicore_amd import ops
    T, H, I, E, K = 16, 2048, 512, 64, 8
    g = _seed(77 + (precision == "mxfp8"))
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    ids = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(T)])
    probs = torch.rand(T, K, generator=g)
    w1 = (torch.randn(E, H, 2 * I, generator=g) * 0.02).to(torch.bfloat16)
    w2 = (torch.randn(E, I, H, generator=g) * 0.02).to(torch.bfloat16)
    if precision == "mxfp8":
        d1, s1 = ops.mx_quantize_cols(w1.to(gpu))
        d2, s2 = ops.mx_quantize_cols(w2.to(gpu))
        args = dict(num_experts=E, intermediate_size=I, precision="mxfp8", w1_scale=s1, w2_scale=s2)
        wts = (d1.view(torch.uint8), d2.view(torch.uint8))
    else:
        args = dict(num_experts=E, intermediate_size=I)
        wts = (w1.to(gpu), w2.to(gpu))
    ins = (x.to(gpu), ids.to(gpu), probs.to(gpu), *wts)
    with _variant("w4"):
        out_w4 = ops.moe_forward(*ins, **args).cpu()
    with _variant(variant):
        out_pp = ops.moe_forward(*ins, **args).cpu()
    assert torch.equal(out_pp, out_w4)
    if precision == "bf16":
        ref = orc.expert_forward_reference(x, ids, probs, w1, w2, layout="EIO")
        assert orc.rel_l2(out_pp, ref) < BF16_REL_L2


@pytest.mark.parametrize("T,H,I,E,K,gu", [(640, 1024, 384, 4, 2, False), (640, 1024, 384, 4, 2, True),
                                          (960, 512, 256, 12, 4, True), (700, 1024, 512, 16, 4, False)])
def test_moe_forward_mxfp8_skinny_tile_bit_identical(gpu, monkeypatch, T, H, I, E, K, gu):
    """The 384 x 128 MX tile (MI355MOE_PP_SKINNY=1: experts of 257..384 routed rows on it, one weight
    pass) runs the same MFMAs in the same K order per output element as the 256 x 256 tile, so the
    forward is bit-identical with it switched on and off (both GEMMs), and matches the oracle."""
    from hyper_multicore_amd import ops
    print(f"[pp] skinny mxfp8 T={T} H={H} I={I} E={E} K={K} gu={gu}", flush=True)
    g = _seed(T + E + 17)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    ids = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(T)])
    probs = torch.rand(T, K, generator=g)
    probs = probs / probs.sum(1, keepdim=True)
    w1 = (torch.randn(E, H, 2 * I, generator=g) * 0.02).to(torch.bfloat16)
    w2 = (torch.randn(E, I, H, generator=g) * 0.02).to(torch.bfloat16)
    d1, s1 = ops.mx_quantize_cols(w1.to(gpu))
    d2, s2 = ops.mx_quantize_cols(w2.to(gpu))
    a1, b1 = d1.view(torch.uint8), s1
    layout = "EIO"
    if gu:
        a1, b1 = ops.interleave_gate_up(d1.view(torch.uint8), s1)
        layout = "EIO_GU"
    counts = torch.bincount(ids.reshape(-1), minlength=E)
    assert bool(((counts > 256) & (counts <= 384)).any()) or T == 700
    args = dict(num_experts=E, intermediate_size=I, precision="mxfp8", layout=layout, w1_scale=b1, w2_scale=s2)
    ins = (x.to(gpu), ids.to(gpu), probs.to(gpu), a1, d2.view(torch.uint8))
    monkeypatch.delenv("MI355MOE_PP_SKINNY", raising=False)
    out = ops.moe_forward(*ins, **args).cpu()
    monkeypatch.setenv("MI355MOE_PP_SKINNY", "1")
    out_skinny = ops.moe_forward(*ins, **args).cpu()
    assert torch.equal(out_skinny, out)
    ref = orc.expert_forward_reference(x, ids, probs, d1.cpu().view(torch.uint8), d2.cpu().view(torch.uint8),
                                       precision="mxfp8", w1_scale=s1.cpu(), w2_scale=s2.cpu())
    assert orc.rel_l2(out_skinny, ref) < 3e-2


@pytest.mark.parametrize("layout", ["EOI", "EIO", "EIO_GU"])
@pytest.mark.parametrize("T,H,I,E,K", [(704, 1024, 384, 4, 2), (640, 1024, 384, 4, 2), (960, 512, 256, 12, 4)])
def test_moe_forward_bf16_skinny_tile_bit_identical(gpu, monkeypatch, T, H, I, E, K, layout):
    """bf16: the 384 x 128 tile for the experts above the other launch's tile height (320 when the
    rows average at most 320 per expert, else 256) and up to 384 rows gives the same forward bit for
    bit as without it, and matches the oracle."""
    from hyper_multicore_amd import ops
    print(f"[pp] skinny bf16 {layout} T={T} H={H} I={I} E={E} K={K}", flush=True)
    g = _seed(T + E + 23)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    ids = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(T)])
    probs = torch.rand(T, K, generator=g)
    probs = probs / probs.sum(1, keepdim=True)
    w1 = (torch.randn(E, H, 2 * I, generator=g) * 0.02).to(torch.bfloat16)
    w2 = (torch.randn(E, I, H, generator=g) * 0.02).to(torch.bfloat16)
    if layout == "EOI":
        wa, wb = w1.transpose(1, 2).contiguous().to(gpu), w2.transpose(1, 2).contiguous().to(gpu)
    else:
        wa, wb = w1.to(gpu), w2.to(gpu)
        if layout == "EIO_GU":
            wa, _ = ops.interleave_gate_up(wa)
    ins = (x.to(gpu), ids.to(gpu), probs.to(gpu), wa, wb)
    args = dict(num_experts=E, intermediate_size=I, layout=layout)
    monkeypatch.delenv("MI355MOE_PP_SKINNY", raising=False)
    out = ops.moe_forward(*ins, **args).cpu()
    monkeypatch.setenv("MI355MOE_PP_SKINNY", "1")
    out_skinny = ops.moe_forward(*ins, **args).cpu()
    assert torch.equal(out_skinny, out)
    ref = orc.expert_forward_reference(x, ids, probs, w1, w2)
    assert orc.rel_l2(out_skinny, ref) < BF16_REL_L2
