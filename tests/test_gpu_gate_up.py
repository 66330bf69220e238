"""GPU checks of the gate/up-interleaved GMM1 weight layout (EIO_GU).

The preparation only moves columns: each 64-column block of the result is checked against the
matching slice of the original, element for element. The forward on the prepared weights reads the
same values into the same tile positions, so its output must equal the EIO forward on the original
weights bit for bit, for both precisions, every GEMM configuration, and the decode (64-row tiles),
prefill and empty-expert cases.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu

VARIANTS = ["default", "pp", "w4"]


def _blocks_of(w, I):
    """(gate blocks, up blocks) of the interleaved tensor's last axis, each [..., I]."""
    nb = I // 64
    gate = torch.cat([w[..., b * 128: b * 128 + 64] for b in range(nb)], dim=-1)
    up = torch.cat([w[..., b * 128 + 64: b * 128 + 128] for b in range(nb)], dim=-1)
    return gate, up


@pytest.mark.parametrize("I", [128, 384])
def test_interleave_gate_up_moves_blocks(gpu, I):
    from hyper_multicore_amd import ops
    g = torch.Generator().manual_seed(I)
    E, H = 3, 128
    w_bf16 = torch.randn(E, H, 2 * I, generator=g).to(torch.bfloat16).to(gpu)
    w_u8 = torch.randint(0, 256, (E, H, 2 * I), generator=g, dtype=torch.uint8).to(gpu)
    s_u8 = torch.randint(0, 256, (E, H // 64, 2 * I, 2), generator=g, dtype=torch.uint8).to(gpu)
    out_bf16, none = ops.interleave_gate_up(w_bf16)
    assert none is None
    out_u8, out_s = ops.interleave_gate_up(w_u8, s_u8)
    for src, dst in ((w_bf16, out_bf16), (w_u8, out_u8)):
        gate, up = _blocks_of(dst, I)
        assert torch.equal(gate, src[..., :I]) and torch.equal(up, src[..., I:])
    # scales: one 2-byte pair per column moves with its column
    gate, up = _blocks_of(out_s.transpose(-1, -2), I)
    assert torch.equal(gate, s_u8.transpose(-1, -2)[..., :I]) and torch.equal(up, s_u8.transpose(-1, -2)[..., I:])


def _inputs(T, H, I, E, K, seed, empty_expert):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    pool = E - 1 if empty_expert else E  # expert E-1 receives no rows
    ids = torch.stack([torch.randperm(pool, generator=g)[:K] for _ in range(T)]).to(torch.int32)
    probs = torch.rand(T, K, generator=g)
    probs = probs / probs.sum(1, keepdim=True)
    w1 = (torch.randn(E, H, 2 * I, generator=g) * 0.02).to(torch.bfloat16)
    w2 = (torch.randn(E, I, H, generator=g) * 0.02).to(torch.bfloat16)
    return x, ids, probs, w1, w2


@pytest.mark.parametrize("variant", VARIANTS)
@pytest.mark.parametrize("precision", ["bf16", "mxfp8"])
@pytest.mark.parametrize("T,H,I,E,K,empty", [(32, 1024, 256, 64, 8, True), (700, 1024, 512, 16, 4, True),
                                              (1024, 512, 384, 8, 2, False)])
def test_moe_forward_gate_up_matches_eio(gpu, variant, precision, T, H, I, E, K, empty):
    from hyper_multicore_amd import ops
    print(f"[gate_up] {precision} {variant} T={T} H={H} I={I} E={E} K={K}", flush=True)
    x, ids, probs, w1, w2 = _inputs(T, H, I, E, K, T + E + I, empty)
    x, ids, probs = x.to(gpu), ids.to(gpu), probs.to(gpu)
    args = dict(num_experts=E, intermediate_size=I, precision=precision, gemm_variant=variant)
    if precision == "bf16":
        w1d, w2d, s1, s2 = w1.to(gpu), w2.to(gpu), None, None
    else:
        d1, s1 = ops.mx_quantize_cols(w1.to(gpu))
        d2, s2 = ops.mx_quantize_cols(w2.to(gpu))
        w1d, w2d = d1.view(torch.uint8), d2.view(torch.uint8)
    w1i, s1i = ops.interleave_gate_up(w1d, s1)
    out_eio = ops.moe_forward(x, ids, probs, w1d, w2d, w1_scale=s1, w2_scale=s2, **args)
    out_gu = ops.moe_forward(x, ids, probs, w1i, w2d, w1_scale=s1i, w2_scale=s2, layout="EIO_GU", **args)
    torch.cuda.synchronize()
    assert torch.equal(out_eio.cpu(), out_gu.cpu())
