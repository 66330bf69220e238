"""GPU: the one-launch decode prologue (decode_prep.h: dispatch + MX token quantisation in one
launch) against the three-launch dispatch and the separate quantisation, through the C ABI.

The forward selects the prologue for decode shapes (64-row tiles) while MI355MOE_DECODE_PREP=1 is
set (read at each call). Both prologues write the same metadata, so the outputs must be bit-identical;
each is also checked against the oracle at the usual bars.
"""
import pytest
import torch

from oracle import moe_oracle as orc

pytestmark = pytest.mark.gpu


def _inputs(T, H, I, E, K, seed, id_dtype):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(T, H, generator=g) * 0.5).to(torch.bfloat16)
    ids = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(T)]).to(id_dtype)
    probs = torch.rand(T, K, generator=g)
    w1 = (torch.randn(E, H, 2 * I, generator=g) * H ** -0.5).to(torch.bfloat16)
    w2 = (torch.randn(E, I, H, generator=g) * I ** -0.5).to(torch.bfloat16)
    return x, ids, probs, w1, w2


@pytest.mark.parametrize("precision", ["bf16", "mxfp8"])
@pytest.mark.parametrize("T,K,E,id_dtype", [(128, 8, 256, torch.int64), (32, 8, 64, torch.int32),
                                            (5, 3, 40, torch.int64)])
def test_forward_one_launch_prologue_bit_identical(gpu, monkeypatch, precision, T, K, E, id_dtype):
    from hyper_multicore_amd import ops
    H, I = 1024, 512
    print(f"decode prologue {precision} T={T} K={K} E={E} ids={id_dtype}", flush=True)
    x, ids, probs, w1, w2 = _inputs(T, H, I, E, K, T * 7 + E, id_dtype)
    kw = dict(num_experts=E, intermediate_size=I)
    if precision == "mxfp8":
        d1, s1 = ops.mx_quantize_cols(w1.to(gpu))
        d2, s2 = ops.mx_quantize_cols(w2.to(gpu))
        wa, wb = d1.view(torch.uint8), d2.view(torch.uint8)
        kw.update(precision="mxfp8", w1_scale=s1, w2_scale=s2)
    else:
        wa, wb = w1.to(gpu), w2.to(gpu)
    args = (x.to(gpu), ids.to(gpu), probs.to(gpu), wa, wb)
    monkeypatch.delenv("MI355MOE_DECODE_PREP", raising=False)
    base = ops.moe_forward(*args, **kw).cpu()
    monkeypatch.setenv("MI355MOE_DECODE_PREP", "1")
    one = ops.moe_forward(*args, **kw).cpu()
    again = ops.moe_forward(*args, **kw).cpu()
    assert torch.equal(one, base)
    assert torch.equal(again, base)
    if precision == "mxfp8":
        ref = orc.expert_forward_reference(x, ids, probs, wa.cpu(), wb.cpu(), precision="mxfp8",
                                           w1_scale=s1.cpu(), w2_scale=s2.cpu())
        assert orc.rel_l2(one, ref) < 3e-2
    else:
        ref = orc.expert_forward_reference(x, ids, probs, w1, w2)
        assert orc.rel_l2(one, ref) < 1e-2
