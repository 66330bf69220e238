"""Every BASELINE.json config at its full shape on the GPU, with the bench's seeds (bench.Layer): the
router projection against an fp32 CPU projection; routing (indices and weights) and the dispatch
metadata (counts, offsets, group_list, permutation) bit-exact against the C oracle at full T; the
index sets of every row equal to the torch form of MegaGate._torch_forward (module.py:199-227,
torch.topk sets as _test_mega_gate.py:336-351 compares them) at full T, near ties below the
scorings' rounding difference apart (tests/route_ties.py); and the layer output
against the fp32-accumulate oracle (the MX-emulating one for MXFP8) - rel-L2 <= 1e-2 (bf16) / 3e-2
(MXFP8), the north-star bars (fp32_expert_reference.py:22-26 is the rounding contract) - on the
tokens of every expert's first and last routed row, of the rows on both sides of every 256- and
320-row tile boundary, and a seeded random sample."""
import numpy as np
import pytest
import torch

import bench
from oracle import moe_oracle as orc
from tests.route_ties import set_mismatches

pytestmark = pytest.mark.gpu

BAR = {"bf16": 1e-2, "mxfp8": 3e-2}
SAMPLE = 128  # random output tokens checked against the oracle, besides the boundary tokens
TILE_HEIGHTS = (256, 320)  # m-tile heights of the prefill grouped GEMMs


def boundary_tokens(counts: torch.Tensor, gather: torch.Tensor, top_k: int) -> torch.Tensor:
    """Tokens of each expert's first and last routed row and of the rows on both sides of every
    m-tile boundary inside an expert."""
    rows = []
    off = 0
    for n in counts.tolist():
        if n > 0:
            rows += [off, off + n - 1]
            for bm in TILE_HEIGHTS:
                for j in range(bm, n, bm):
                    rows += [off + j - 1, off + j]
        off += n
    return torch.unique(gather[torch.tensor(rows, dtype=torch.int64)].long() // top_k)


def _expert_weights(layer, e):
    """fp32 (W1 [H, 2I], W2 [I, H]) of expert e, expanded on the GPU, then moved to the CPU."""
    if layer.c["precision"] == "bf16":
        if layer.layout == "EOI":
            return layer.w1[e].float().t().contiguous().cpu(), layer.w2[e].float().t().contiguous().cpu()
        return layer.w1_root(e)[0].float().cpu(), layer.w2[e].float().cpu()
    w1r, s1r = layer.w1_root(slice(e, e + 1))
    w1 = orc.mx_dequantize_weight_cols(w1r, s1r)[0]
    w2 = orc.mx_dequantize_weight_cols(layer.w2[e:e + 1], layer.s2[e:e + 1])[0]
    return w1.cpu(), w2.cpu()


@pytest.mark.parametrize("name", ["small_bf16", "dsv3_bf16", "dsv3_mxfp8", "dsv3_decode_mxfp8", "multimodal_bf16"])
def test_layer_full_shape(gpu, name):
    from hyper_multicore_amd import ops
    c = bench.CONFIGS[name]
    print(f"[fullshape] {name}: T={c['T']} E={c['E']} K={c['K']} H={c['H']} I={c['I']} {c['precision']}",
          flush=True)
    layer = bench.Layer(name, gpu)
    T, E, K = c["T"], c["E"], c["K"]

    # router projection (fp32 logits) against the fp32 CPU projection
    logits = ops.gate_logits(layer.x, layer.wr, layer.wr_vl, layer.mask if layer.wr_vl is not None else None)
    ref = orc.gate_logits_reference(layer.x.cpu(), layer.wr.cpu(), None if layer.wr_vl is None else layer.wr_vl.cpu(),
                                    None if layer.mask is None else layer.mask.cpu())
    torch.testing.assert_close(logits.cpu(), ref, rtol=1e-5, atol=1e-5)
    if layer.skew is not None:
        logits = logits + layer.skew

    # routing: bit-exact against the C oracle at full T
    weights, ids = ops.gate_route(logits, layer.bias, top_k=K, scoring_func=c["scoring"],
                                  routed_scaling_factor=c["scale"], num_groups=c["groups"],
                                  topk_groups=c["topk_groups"])
    w_ref, i_ref, _ = orc.route_c(logits.cpu().numpy(), layer.bias.cpu().numpy(), top_k=K,
                                  scoring_func=c["scoring"], routed_scaling_factor=c["scale"],
                                  num_groups=c["groups"], topk_groups=c["topk_groups"])
    ids_cpu, w_cpu = ids.cpu(), weights.cpu()
    assert np.array_equal(ids_cpu.numpy(), i_ref)
    assert np.array_equal(w_cpu.numpy(), w_ref)

    # routing: every row's index set equals the torch form's (torch's own exp / sigmoid / softmax),
    # except rows whose selection is a near tie below the scorings' rounding difference
    w_t, i_t, s_t = orc.route_reference(logits.cpu(), layer.bias.cpu(), top_k=K, scoring_func=c["scoring"],
                                        routed_scaling_factor=c["scale"], num_groups=c["groups"],
                                        topk_groups=c["topk_groups"])
    near, other = set_mismatches(ids_cpu, i_t, s_t + layer.bias.cpu(), c["groups"], c["topk_groups"])
    print(f"[fullshape] {name}: torch-form index sets: {len(other)} rows differ, {len(near)} near-tie rows "
          f"{near[:8]} of {T}", flush=True)
    assert other == []
    assert len(near) <= max(1, T // 2000)
    same = torch.ones(T, dtype=torch.bool)
    same[near] = False
    got, want = torch.sort(ids_cpu, dim=1), torch.sort(i_t, dim=1)
    torch.testing.assert_close(w_cpu.gather(1, got.indices)[same], w_t.gather(1, want.indices)[same], rtol=1e-5,
                               atol=1e-7)

    # dispatch metadata: bit-exact
    d = ops.dispatch(ids, E)
    counts = orc.expert_counts(ids_cpu, E)
    mapping, gather = orc.stable_permutation(ids_cpu, E)
    assert torch.equal(d.counts.cpu(), counts)
    assert torch.equal(d.group_list.cpu(), counts.cumsum(0).to(torch.int64))
    assert torch.equal(d.expert_offsets.cpu(), counts.cumsum(0).to(torch.int64) - counts.to(torch.int64))
    assert torch.equal(d.mapping.cpu(), mapping)
    assert torch.equal(d.gather_index.cpu(), gather)
    assert int(d.error_flag.cpu()) == 0

    # the layer output on a seeded token sample
    out = ops.moe_forward(layer.x, ids, weights, layer.w1, layer.w2, num_experts=E, intermediate_size=c["I"],
                          precision=c["precision"], layout=layer.layout, w1_scale=layer.s1, w2_scale=layer.s2)
    torch.cuda.synchronize()
    g = torch.Generator().manual_seed(bench.SEED + c["idx"])
    rand = torch.randperm(T, generator=g)[:min(SAMPLE, T)]
    tokens = torch.unique(torch.cat([rand, boundary_tokens(counts, gather, K)]))
    ref_out = orc.expert_forward_reference_tokens(layer.x.cpu(), ids_cpu, w_cpu, tokens,
                                                  lambda e: _expert_weights(layer, e), precision=c["precision"])
    err = orc.rel_l2(out.cpu()[tokens], ref_out)
    print(f"[fullshape] {name}: output rel-L2 {err:.3e} on {len(tokens)} tokens "
          f"({int((counts > 0).sum())} active experts)", flush=True)
    assert err <= BAR[c["precision"]]
    # and token by token, so that one wrong tile cannot hide in the sample's average
    o, r = out.cpu()[tokens].float(), ref_out.float()
    per_tok = (o - r).norm(dim=1) / r.norm(dim=1).clamp_min(1e-30)
    worst = int(per_tok.argmax())
    print(f"[fullshape] {name}: worst token {int(tokens[worst])} rel-L2 {float(per_tok[worst]):.3e}", flush=True)
    assert float(per_tok.max()) <= 2 * BAR[c["precision"]]
