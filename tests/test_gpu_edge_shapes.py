"""Layer forward at edge shapes on the GPU, against the fp32-accumulate oracle (rel-L2 1e-2 bf16 /
3e-2 MXFP8) and, for MXFP8, the gate/up-interleaved weights bit for bit against the plain ones:
one token, top-1, a single expert, every token on one expert, the narrowest intermediate size (one
n-tile of GMM1), hidden sizes that are not multiples of 256, and decode-sized batches whose last round
of work items runs as column halves."""
import pytest
import torch

from oracle import moe_oracle as orc

pytestmark = pytest.mark.gpu

CASES = [
    # name, T, H, I, E, K, skew (all tokens routed to the first K experts)
    ("one_token", 1, 1024, 256, 8, 2, False),
    ("top1", 77, 1024, 256, 16, 1, False),
    ("single_expert", 40, 512, 128, 1, 1, False),
    ("all_on_one_expert", 300, 1024, 256, 32, 1, True),
    ("narrow_i", 200, 1024, 128, 8, 2, False),
    ("h_1152", 128, 1152, 256, 16, 4, False),
    ("decode_tail", 96, 2048, 512, 96, 8, False),
    ("decode_many_experts", 64, 1024, 256, 256, 8, False),
]


def _inputs(T, H, I, E, K, skew, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    if skew:
        ids = torch.arange(K).repeat(T, 1)
    else:
        ids = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(T)])
    probs = torch.rand(T, K, generator=g)
    probs = probs / probs.sum(1, keepdim=True)
    w1 = (torch.randn(E, H, 2 * I, generator=g) * 0.02).to(torch.bfloat16)
    w2 = (torch.randn(E, I, H, generator=g) * 0.02).to(torch.bfloat16)
    return x, ids.to(torch.int64), probs, w1, w2


@pytest.mark.parametrize("precision", ["bf16", "mxfp8"])
@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_layer_edge_shape(gpu, case, precision):
    from hyper_multicore_amd import ops
    name, T, H, I, E, K, skew = case
    print(f"[edge] {name} {precision} T={T} H={H} I={I} E={E} K={K}", flush=True)
    x, ids, probs, w1, w2 = _inputs(T, H, I, E, K, skew, T + H + I + E + K)
    xd, idsd, pd = x.to(gpu), ids.to(gpu), probs.to(gpu)
    args = dict(num_experts=E, intermediate_size=I, precision=precision)
    if precision == "bf16":
        out = ops.moe_forward(xd, idsd, pd, w1.to(gpu), w2.to(gpu), **args).cpu()
        ref = orc.expert_forward_reference(x, ids, probs, w1, w2)
        assert orc.rel_l2(out, ref) < 1e-2
        return
    d1, s1 = ops.mx_quantize_cols(w1.to(gpu))
    d2, s2 = ops.mx_quantize_cols(w2.to(gpu))
    d1, d2 = d1.view(torch.uint8), d2.view(torch.uint8)
    out = ops.moe_forward(xd, idsd, pd, d1, d2, w1_scale=s1, w2_scale=s2, **args)
    g1, t1 = ops.interleave_gate_up(d1, s1)
    out_gu = ops.moe_forward(xd, idsd, pd, g1, d2, w1_scale=t1, w2_scale=s2, layout="EIO_GU", **args)
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), out_gu.cpu())
    ref = orc.expert_forward_reference(x, ids, probs, d1.cpu(), d2.cpu(), precision="mxfp8", w1_scale=s1.cpu(),
                                       w2_scale=s2.cpu())
    assert orc.rel_l2(out.cpu(), ref) < 3e-2


@pytest.mark.parametrize("case", [c for c in CASES if c[0] in ("decode_tail", "decode_many_experts", "top1")],
                         ids=lambda c: c[0])
def test_decode_shapes_match_the_4wave_configuration(gpu, case):
    """The decode tiles (column halves included) against the 4-wave configuration, bit for bit."""
    from hyper_multicore_amd import ops
    name, T, H, I, E, K, skew = case
    x, ids, probs, w1, w2 = _inputs(T, H, I, E, K, skew, 7 * T + E)
    ins = (x.to(gpu), ids.to(gpu), probs.to(gpu), w1.to(gpu), w2.to(gpu))
    args = dict(num_experts=E, intermediate_size=I)
    out_default = ops.moe_forward(*ins, **args, gemm_variant="default").cpu()
    out_w4 = ops.moe_forward(*ins, **args, gemm_variant="w4").cpu()
    assert torch.equal(out_default, out_w4)
