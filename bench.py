"""Benchmark of the MegaGate -> MegaMoE layer forward on one MI355X (synthetic data).

One step = one full MoE layer forward over one batch: router projection (bf16 MFMA, fp32 out),
route (scores, bias, group-limited top-k, renorm, scale), dispatch (histogram, scan, stable
permutation), [MX activation quant], GMM1 + fused SwiGLU [+ MX requant], GMM2 and the combine.
Inputs and weights are resident in HBM before the timed region.

Prints ONE JSON line: tokens/s for the workload, the roofline of the dominant kernel (GMM1,
timed with HIP events recorded by the library on its own stream), and a CPU baseline (the
oracle's restatement of the reference CPU path, on a bounded token prefix). Other configs are
reported under "extra" (``--extra none`` skips them).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--config dsv3_bf16] [--extra all]
                      [--gemm-variant default|pp|w4] [--gemm-shapes]
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import re
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK = {"bf16": 2.5e15, "mxfp8": 5.0e15, "hbm": 8.0e12}

# BASELINE.json configs (index in "configs")
CONFIGS = {
    "small_bf16": dict(idx=0, T=1024, E=8, K=2, H=1024, I=512, scoring="softmax", groups=1, topk_groups=1,
                       scale=1.0, precision="bf16", wstd=0.02, zipf=None, multimodal=False),
    "dsv3_bf16": dict(idx=1, T=8192, E=256, K=8, H=7168, I=2048, scoring="sigmoid", groups=8, topk_groups=4,
                      scale=2.5, precision="bf16", wstd=0.006, zipf=None, multimodal=False),
    "dsv3_mxfp8": dict(idx=2, T=8192, E=256, K=8, H=7168, I=2048, scoring="sigmoid", groups=8, topk_groups=4,
                       scale=2.5, precision="mxfp8", wstd=0.006, zipf=None, multimodal=False),
    "dsv3_decode_mxfp8": dict(idx=3, T=128, E=256, K=8, H=7168, I=2048, scoring="sigmoid", groups=8,
                              topk_groups=4, scale=2.5, precision="mxfp8", wstd=0.006, zipf=1.1, multimodal=False),
    "multimodal_bf16": dict(idx=4, T=16384, E=128, K=8, H=4096, I=1536, scoring="softmax", groups=1,
                            topk_groups=1, scale=1.0, precision="bf16", wstd=0.02, zipf=None, multimodal=True),
}
SEED = 1234


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


class Layer:
    """Synthetic inputs + weights of one config, resident on the GPU."""

    def __init__(self, name: str, device: torch.device, bf16_layout: str = "EOI", mx_layout: str = "EIO_GU"):
        from hyper_multicore_amd import _lib, ops
        self.ops = ops
        self._lib = _lib
        self.name = name
        c = self.c = CONFIGS[name]
        g = torch.Generator(device=device).manual_seed(SEED + c["idx"])
        T, E, H, I = c["T"], c["E"], c["H"], c["I"]
        self.x = torch.randn(T, H, device=device, generator=g).to(torch.bfloat16)
        self.wr = (torch.randn(E, H, device=device, generator=g) * 0.02).to(torch.bfloat16)
        self.bias = torch.zeros(E, device=device)
        self.wr_vl = None
        self.mask = None
        self.skew = None
        if c["multimodal"]:
            self.mask = torch.rand(T, device=device, generator=g) < 0.5
            self.x[self.mask] = (self.x[self.mask].float() * 0.5).to(torch.bfloat16)
            self.wr_vl = (torch.randn(E, H, device=device, generator=g) * 0.02).to(torch.bfloat16)
        else:
            self.bias = torch.randn(E, device=device, generator=g) * 0.01
        if c["zipf"] is not None:
            # Expert popularity ~ Zipf(s): a seeded rank per expert, and Gumbel-top-k logits
            # log p_e + G_te dominate the router logits, so top-k samples experts without
            # replacement in proportion to p_e (sigmoid is monotone).
            rank = torch.randperm(E, device=device, generator=g).float() + 1.0
            logp = -c["zipf"] * torch.log(rank)
            u = torch.rand(T, E, device=device, generator=g).clamp_(1e-9, 1 - 1e-9)
            self.skew = 8.0 * (logp - torch.log(-torch.log(u)))
        w1 = torch.randn(E, 2 * I, H, device=device, generator=g).mul_(c["wstd"]).to(torch.bfloat16)  # EOI
        w2 = torch.randn(E, H, I, device=device, generator=g).mul_(c["wstd"]).to(torch.bfloat16)      # EOI
        if c["precision"] == "bf16" and bf16_layout in ("EIO", "EIO_GU"):  # EIO: the reference module's default
            w1e, w2e = w1.transpose(1, 2).contiguous(), w2.transpose(1, 2).contiguous()
            del w1, w2
            self.w1, self.w2, self.s1, self.s2, self.layout = w1e, w2e, None, None, "EIO"
            if bf16_layout == "EIO_GU":
                self.w1, _ = ops.interleave_gate_up(w1e)
                del w1e
                self.layout = "EIO_GU"
        elif c["precision"] == "bf16":
            self.w1, self.w2, self.s1, self.s2, self.layout = w1, w2, None, None, "EOI"
        else:
            d1, s1 = ops.mx_quantize_cols(w1.transpose(1, 2).contiguous())  # EIO [E, H, 2I]
            del w1
            d2, s2 = ops.mx_quantize_cols(w2.transpose(1, 2).contiguous())  # EIO [E, I, H]
            del w2
            self.w1, self.w2, self.s1, self.s2, self.layout = d1.view(torch.uint8), d2.view(torch.uint8), s1, s2, "EIO"
            if mx_layout == "EOI":
                # one-time weight preparation (outside the timed region, like loading a checkpoint):
                # the same values and scales with K contiguous (the 4-wave GEMM configuration reads
                # them without transposing LDS loads; the default 8-wave one takes the EIO root)
                e1, t1 = ops.mx_weight_to_eoi(d1, s1)
                e2, t2 = ops.mx_weight_to_eoi(d2, s2)
                del d1, s1, d2, s2
                self.w1, self.w2, self.s1, self.s2, self.layout = e1.view(torch.uint8), e2.view(torch.uint8), t1, t2, "EOI"
            elif mx_layout == "EIO_GU":
                # one-time weight preparation: W1's gate and up columns interleaved in 64-column
                # blocks, so a GMM1 tile reads its gate and up columns as one run per weight row
                self.w1, self.s1 = ops.interleave_gate_up(d1, s1)
                del d1, s1
                self.w1 = self.w1.view(torch.uint8)
                self.layout = "EIO_GU"
        torch.cuda.synchronize()
        self.out = torch.empty(T, H, dtype=torch.bfloat16, device=device)

    def step(self, stage_events=None):
        c, ops = self.c, self.ops
        logits = ops.gate_logits(self.x, self.wr, self.wr_vl, self.mask if self.wr_vl is not None else None)
        if self.skew is not None:
            logits = logits + self.skew
        weights, ids = ops.gate_route(logits, self.bias, top_k=c["K"], scoring_func=c["scoring"],
                                      routed_scaling_factor=c["scale"], num_groups=c["groups"],
                                      topk_groups=c["topk_groups"])
        ops.moe_forward(self.x, ids, weights, self.w1, self.w2, num_experts=c["E"], intermediate_size=c["I"],
                        precision=c["precision"], layout=self.layout, w1_scale=self.s1, w2_scale=self.s2,
                        out=self.out, stage_events=stage_events)
        return ids

    def w1_root(self, experts=slice(None)):
        """W1 (and its MX col_scale) of the given experts with gate columns [0, I) then up columns
        [I, 2I), whatever layout the layer runs: the weights the CPU references take."""
        w1, s1 = self.w1[experts], None if self.s1 is None else self.s1[experts]
        if self.layout != "EIO_GU":
            return w1, s1
        I = self.c["I"]
        blocks = lambda t, half: torch.cat([t[..., b * 128 + half * 64: b * 128 + half * 64 + 64]
                                            for b in range(I // 64)], dim=-1)
        w1 = torch.cat([blocks(w1, 0), blocks(w1, 1)], dim=-1)
        if s1 is not None:
            s1 = torch.cat([blocks(s1.transpose(-1, -2), 0), blocks(s1.transpose(-1, -2), 1)],
                           dim=-1).transpose(-1, -2).contiguous()
        return w1, s1

    def counts(self):
        ids = self.step()
        torch.cuda.synchronize()
        return torch.bincount(ids.reshape(-1), minlength=self.c["E"]).cpu()


def gmm_work(c: dict, counts: torch.Tensor) -> dict:
    """Algorithmic FLOPs and bytes of GMM1 (the dominant kernel) and of the whole layer."""
    T, E, K, H, I = c["T"], c["E"], c["K"], c["H"], c["I"]
    R = T * K
    active = int((counts > 0).sum())
    mx = c["precision"] == "mxfp8"
    wbytes = 1.0 + 1.0 / 32 if mx else 2.0        # weight bytes per element (e4m3 + e8m0 / 32)
    abytes = 1.0 + 1.0 / 32 if mx else 2.0
    g1_flops = 2.0 * R * H * 2 * I
    g1_bytes = active * H * 2 * I * wbytes + T * H * abytes + R * I * abytes
    layer_flops = 6.0 * R * H * I + 2.0 * T * H * E
    layer_bytes = (active * 3 * H * I * wbytes + T * H * 2 * 2 + E * H * 2 + T * K * 16)
    return dict(active=active, g1_flops=g1_flops, g1_bytes=g1_bytes, layer_flops=layer_flops,
                layer_bytes=layer_bytes)


def m_tiles(c: dict, counts: torch.Tensor, variant: str = "default", decode_tiles: bool = True) -> dict:
    """Row tiles the expert GEMMs run (per column block) against the ideal R / BM, and the fraction
    of tile rows that are padding: the M-tail waste of ragged groups. BM is the library's choice: 64
    on the decode tiles (routed rows <= 32 per expert under the default variant), 320 for bf16 when
    groups average at most 320 rows, else 256."""
    R = c["T"] * c["K"]
    if decode_tiles and variant == "default" and R <= c["E"] * 32:
        bm = 64
    elif c["precision"] == "bf16" and variant in ("default", "pp") and R <= c["E"] * 320:
        bm = 320  # the 8-wave configuration's tall bf16 tiles (groups averaging at most 320 rows)
    else:
        bm = 256
    active = max(1, int((counts > 0).sum()))
    # the 384 x 128 tile (MI355MOE_PP_SKINNY=1): the groups above the other tile's height and up to 384
    # rows in one m-tile of 384 rows
    skinny = (bm in (256, 320) and variant in ("default", "pp")
              and os.environ.get("MI355MOE_PP_SKINNY") == "1" and c["E"] * 128 <= R <= c["E"] * 512)
    in_range = ((counts > bm) & (counts <= 384)) if skinny else torch.zeros_like(counts, dtype=torch.bool)
    tiles = int(((counts[~in_range] + bm - 1) // bm).sum())
    n_skinny = int(in_range.sum())
    res = {"bm": bm, "tiles": tiles, "ideal": -(-R // bm),
           "padded_row_frac": round(1 - R / (tiles * bm + n_skinny * 384), 4),
           "weight_passes_per_expert": round((tiles + n_skinny) / active, 3)}
    if skinny:
        res["skinny_tiles"] = n_skinny
    return res


def measure(layer: Layer, steps: int, warmup: int) -> dict:
    for _ in range(warmup):
        layer.step()
    torch.cuda.synchronize()
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(5)] for _ in range(steps)]
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record()
    for s in range(steps):
        layer.step(stage_events=ev[s])
    end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    total_ms = start.elapsed_time(end)
    stage = {"dispatch": [], "gmm1": [], "gmm2": [], "combine": []}
    for e in ev:
        stage["dispatch"].append(e[0].elapsed_time(e[1]))
        stage["gmm1"].append(e[1].elapsed_time(e[2]))
        stage["gmm2"].append(e[2].elapsed_time(e[3]))
        stage["combine"].append(e[3].elapsed_time(e[4]))
    avg = {k: sum(v) / len(v) for k, v in stage.items()}
    return dict(ms_per_step=total_ms / steps, wall_s=wall, stage_ms=avg)


def targets(results: dict) -> dict:
    """The measured figures beside BASELINE.json's bars, for the configs this run measured: C3's layer
    at >= 55 % of dense FP8 MFMA peak, C4's decode at >= 65 % of HBM bandwidth (as the GMM1 kernel's
    roofline and as the whole layer's weight and activation bytes over its time)."""
    out = {}
    if "dsv3_mxfp8" in results:
        out["dsv3_mxfp8_layer_mfma_frac"] = {"measured": results["dsv3_mxfp8"]["layer_mfma_frac"], "bar": 0.55}
    if "dsv3_decode_mxfp8" in results:
        r = results["dsv3_decode_mxfp8"]
        out["dsv3_decode_mxfp8_gmm1_hbm_frac"] = {"measured": r["roofline"]["frac"], "bar": 0.65}
        out["dsv3_decode_mxfp8_layer_hbm_frac"] = {"measured": r["layer_hbm_frac"], "bar": 0.65}
    return out


def measure_graph(layer: Layer, steps: int) -> dict:
    """The same step captured once into a HIP graph (torch.cuda.CUDAGraph) and replayed `steps` times:
    the eager step's kernels without the host launch path between them (what a serving loop that
    replays a captured decode step runs). The replay's output must equal the eager step's bit for bit."""
    layer.step()
    torch.cuda.synchronize()
    eager_out = layer.out.clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up on a side stream before capture (torch's capture recipe)
        layer.step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        layer.step()
    layer.out.zero_()
    graph.replay()
    torch.cuda.synchronize()
    matches = bool(torch.equal(layer.out, eager_out))
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    del graph
    return {"ms_per_step": round(ms, 4), "tokens_per_s": round(layer.c["T"] / (ms * 1e-3), 1),
            "matches_eager": matches}


def measured_traffic(workload: str, variant: str, layout: str, root: str = ROOT):
    """HBM bytes per GMM1 launch from the committed rocprofv3 counter passes of the same workload,
    GEMM variant and weight layout (profiles/traffic_<workload>_<variant>_<layout>.json, written by
    ``--summarize``: FETCH_SIZE and WRITE_SIZE in KiB per dispatch, each scaled by the factor the same
    counter reads for a plain copy kernel of known size), and the record's state:
      "current"  the record's kernel has the same machine code in the library this run loaded
                 (``code_digest`` of hyper_multicore_amd/codeobj.py);
      "stale"    the kernel's code changed since the counter runs: no traffic is reported;
      "none"     no record (no traffic)."""
    path = os.path.join(root, "profiles", f"traffic_{workload}_{variant}_{layout}.json")
    if not os.path.exists(path):
        return None, "none"
    with open(path) as f:
        rec = json.load(f)
    from hyper_multicore_amd import _lib, codeobj
    syms = rec.get("symbols", [rec.get("symbol")])
    digests = rec.get("code_digests", [rec.get("code_digest")])
    have = codeobj.kernel_digests(str(_lib.LIB_PATH))
    if not syms or any(s is None or d is None or have.get(s) != d for s, d in zip(syms, digests)):
        return None, "stale"
    return round((rec["fetch_kib"] * rec["fetch_factor"] + rec["write_kib"] * rec["write_factor"]) * 1024.0), "current"


def roofline(c: dict, work: dict, gmm1_ms: float, traffic=None, traffic_record: str = "none") -> dict:
    """Roofline of the GMM1 kernel (grouped GEMM + SwiGLU epilogue): algorithmic bytes or flops per
    launch over its average launch duration (HIP events around that one kernel on the library's
    stream). traffic = measured HBM bytes per launch (None without a current counter record);
    traffic_record = the record's state (measured_traffic)."""
    mx = c["precision"] == "mxfp8"
    peak_flops = PEAK["mxfp8" if mx else "bf16"]
    t_mfma = work["g1_flops"] / peak_flops
    t_hbm = work["g1_bytes"] / PEAK["hbm"]
    sec = gmm1_ms * 1e-3
    common = {"traffic": traffic, "traffic_record": traffic_record, "algorithmic_bytes": round(work["g1_bytes"]),
              "traffic_ratio": None if traffic is None else round(traffic / work["g1_bytes"], 3),
              "kernel": "grouped_gemm GMM1+SwiGLU", "launch_ms": round(gmm1_ms, 4)}
    if t_hbm > t_mfma:
        achieved = work["g1_bytes"] / sec / 1e9
        return {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK["hbm"] / 1e9, "unit": "GB/s",
                "frac": round(achieved / (PEAK["hbm"] / 1e9), 4), **common,
                "mfma_frac": round(work["g1_flops"] / sec / peak_flops, 4)}
    achieved = work["g1_flops"] / sec / 1e12
    return {"bound": "mfma", "achieved": round(achieved, 1), "peak": peak_flops / 1e12, "unit": "TFLOP/s",
            "frac": round(achieved / (peak_flops / 1e12), 4), **common,
            "hbm_frac": round(work["g1_bytes"] / sec / PEAK["hbm"], 4)}


def _library_features() -> int:
    from hyper_multicore_amd import ops
    return ops.features()


def cpu_model() -> str:
    """The host CPU's model string (/proc/cpuinfo), else what platform reports."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def cpu_baseline(name: str, layer: Layer, budget_s: float = 20.0) -> dict:
    """The oracle's restatement of the reference CPU path (MegaGate._torch_forward + the
    TorchExperts CPU loop, bf16 F.linear) on a prefix of the same synthetic batch."""
    from oracle import moe_oracle as orc
    c = layer.c
    threads = torch.get_num_threads()
    T = c["T"]
    sample = min(T, 1024 if c["H"] <= 1024 else 4096)
    x = layer.x[:sample].cpu()
    wr = layer.wr.cpu()
    bias = layer.bias.cpu()
    if c["precision"] == "bf16":
        w1 = layer.w1_root()[0].cpu()   # EOI [E, 2I, H] (EIO [E, H, 2I] transposed back below)
        w2 = layer.w2.cpu()             # EOI [E, H, I]
        if layer.layout in ("EIO", "EIO_GU"):
            w1, w2 = w1.transpose(1, 2).contiguous(), w2.transpose(1, 2).contiguous()
    else:
        w1r, s1r = layer.w1_root()
        w1 = orc.mx_dequantize_weight_cols(w1r.cpu(), s1r.cpu()).to(torch.bfloat16).transpose(1, 2).contiguous()
        del w1r, s1r
        w2 = orc.mx_dequantize_weight_cols(layer.w2.cpu(), layer.s2.cpu()).to(torch.bfloat16).transpose(1, 2).contiguous()
    I = c["I"]
    gate_w, up_w = w1[:, :I], w1[:, I:]
    mask = layer.mask[:sample].cpu() if layer.mask is not None else None
    wvl = layer.wr_vl.cpu() if layer.wr_vl is not None else None
    skew = layer.skew[:sample].cpu() if layer.skew is not None else None

    def run():
        logits = orc.gate_logits_reference(x, wr, wvl, mask)
        if skew is not None:
            logits = logits + skew
        w, ids, _ = orc.route_reference(logits, bias, top_k=c["K"], scoring_func=c["scoring"],
                                        routed_scaling_factor=c["scale"], num_groups=c["groups"],
                                        topk_groups=c["topk_groups"])
        return orc.torch_experts_reference(x, ids, w, gate_w, up_w, w2)

    ref = run()  # warm-up
    agree = None
    try:  # the GPU output of the same tokens (the last timed step) against the CPU path's output
        agree = round(orc.rel_l2(layer.out[:sample].float().cpu(), ref.float()), 6)
    except Exception as e:  # a reported figure, never a reason to lose the bench line
        log(f"[bench] sample agreement not computed: {e}")
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < 3 and (not times or time.perf_counter() < t_end):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    times.sort()
    med = times[len(times) // 2]
    return {"value": round(sample / med, 2), "unit": "tokens/s", "cores": threads, "kind": "port",
            "gpu_rel_l2": agree,
            "sample": f"first {sample} of {T} tokens of the {name} batch, median of {len(times)} after 1 warm-up; "
                      f"torch CPU {torch.__version__}, os.cpu_count()={os.cpu_count()}",
            "cpu_model": cpu_model()}


def run_config(name: str, device, steps: int, warmup: int, variant: str = "default",
               bf16_layout: str = "EOI", mx_layout: str = "EIO_GU") -> dict:
    layer = Layer(name, device, bf16_layout, mx_layout)
    counts = layer.counts()
    work = gmm_work(layer.c, counts)
    m = measure(layer, steps, warmup)
    c = layer.c
    ms = m["ms_per_step"]
    res = {
        "tokens_per_s": round(c["T"] / (ms * 1e-3), 1),
        "ms_per_step": round(ms, 4),
        "layer_tflops": round(work["layer_flops"] / (ms * 1e-3) / 1e12, 1),
        "layer_mfma_frac": round(work["layer_flops"] / (ms * 1e-3) / PEAK[c["precision"]], 4),
        "layer_hbm_frac": round(work["layer_bytes"] / (ms * 1e-3) / PEAK["hbm"], 4),
        "active_experts": work["active"],
        "m_tiles": m_tiles(c, counts, variant, bool(layer.ops.features() & layer._lib.FEATURE_DECODE_TILES)),
        "weight_layout": layer.layout,
        "stage_ms": {k: round(v, 4) for k, v in m["stage_ms"].items()},
        "roofline": roofline(c, work, m["stage_ms"]["gmm1"], *measured_traffic(name, variant, layer.layout)),
        "graph": measure_graph(layer, steps),
    }
    return res, layer


# ------------------------------------------------------------------------------------------------
# Profiles: the rocprofv3 commands behind profiles/ and their reduction to the committed summaries
# ------------------------------------------------------------------------------------------------
COPY_BYTES = 1 << 31  # calibration copy: reads and writes exactly this many bytes
# SwiGLU epilogues (2..5): the 8-wave kernel's third template argument, the 4-wave kernels' last
GMM1_KERNEL = re.compile(r"gg_pp_kernel<\w+, \w+, [2-5][,>]|grouped_gemm\w*_kernel<.*, [2-5]>\(")


def profile_commands(workload: str, out: str = "$GRAFT_REPO_ROOT/gpurun_out/prof") -> dict:
    """The commands (run from anywhere on the GPU box) whose output --summarize reduces; each counter
    pass runs on its own, as rocprofv3 does not split counters over passes."""
    root = "$GRAFT_REPO_ROOT"
    pre = "cd /tmp && export TMPDIR=/tmp && "
    bench = f"python3 {root}/bench.py --config {workload} --extra none --no-cpu"
    d = f"{out}/{workload}"
    cmds = {"kernel_trace": f"mkdir -p {d} && {pre}timeout -s KILL 300 rocprofv3 --kernel-trace --stats --output-format csv -d {d}/kt "
                            f"-o run -- {bench} --steps 10 --warmup 3 > {d}/bench.json"}
    for tag, counters in (("fetch", "FETCH_SIZE"), ("write", "WRITE_SIZE"), ("mfma", "MfmaUtil")):
        cmds[tag] = (f"{pre}timeout -s KILL 300 rocprofv3 --pmc {counters} --output-format csv -d {d}/{tag} -o pmc -- "
                     f"{bench} --steps 2 --warmup 1 > /dev/null")
    return cmds


def calibration_commands(out: str = "$GRAFT_REPO_ROOT/gpurun_out/prof") -> dict:
    copy = (f"python3 -c \"import torch; a = torch.empty({COPY_BYTES}, dtype=torch.uint8, device='cuda'); "
            f"b = torch.empty_like(a); b.copy_(a); torch.cuda.synchronize()\"")
    return {tag: f"cd /tmp && export TMPDIR=/tmp && timeout -s KILL 120 rocprofv3 --pmc {c} --output-format csv "
                 f"-d {out}/copy/{tag} -o pmc -- {copy}"
            for tag, c in (("fetch", "FETCH_SIZE"), ("write", "WRITE_SIZE"))}


def _csv_rows(folder: str, suffix: str) -> list:
    import csv
    import glob
    rows = []
    for path in sorted(glob.glob(os.path.join(folder, "**", f"*{suffix}"), recursive=True)):
        with open(path) as f:
            rows += list(csv.DictReader(f))
    if not rows:
        raise FileNotFoundError(f"no *{suffix} under {folder}")
    return rows


def _counter_mean(folder: str, counter: str, match) -> float:
    vals = [float(r["Counter_Value"]) for r in _csv_rows(folder, "counter_collection.csv")
            if r["Counter_Name"] == counter and match(r["Kernel_Name"])]
    if not vals:
        raise ValueError(f"no {counter} samples of the kernel in {folder}")
    return sum(vals) / len(vals)


def summarize(workload: str, out: str, dest: str = os.path.join(ROOT, "profiles")) -> str:
    """Reduce the outputs of profile_commands(workload) and calibration_commands() under ``out`` to
    profiles/grouped_gemm_<workload>.txt and profiles/traffic_<workload>_<variant>_<layout>.json."""
    d = os.path.join(out, workload)
    with open(os.path.join(d, "bench.json")) as f:
        line = json.loads([x for x in f.read().splitlines() if x.startswith("{")][-1])
    stats = _csv_rows(os.path.join(d, "kt"), "kernel_stats.csv")
    stats.sort(key=lambda r: -float(r["TotalDurationNs"]))
    gmm1 = [r for r in stats if GMM1_KERNEL.search(r["Name"])]
    if not gmm1:
        raise ValueError("no GMM1 (SwiGLU-epilogue grouped GEMM) kernel in the trace")
    # GMM1 may be more than one launch per step (the 384 x 128 MX tile beside the 256 x 256 one): the
    # SwiGLU-epilogue kernels launched as often as the most frequent one, each counted per step
    calls = max(int(r["Calls"]) for r in gmm1)
    g1s = [r["Name"] for r in gmm1 if int(r["Calls"]) == calls]
    g1 = g1s[0]
    copy_kib = COPY_BYTES / 1024.0
    is_copy = lambda name: "copyBuffer" in name  # noqa: E731
    fetch_factor = copy_kib / _counter_mean(os.path.join(out, "copy", "fetch"), "FETCH_SIZE", is_copy)
    write_factor = copy_kib / _counter_mean(os.path.join(out, "copy", "write"), "WRITE_SIZE", is_copy)
    fetch = sum(_counter_mean(os.path.join(d, "fetch"), "FETCH_SIZE", lambda n, k=k: n == k) for k in g1s)
    write = sum(_counter_mean(os.path.join(d, "write"), "WRITE_SIZE", lambda n, k=k: n == k) for k in g1s)
    traffic = (fetch * fetch_factor + write * write_factor) * 1024.0
    cfg = line["config"]
    variant, layout = cfg.get("gemm_variant", "default"), cfg.get("weight_layout", "EIO")
    rf = line["roofline"]
    avg_of = {r["Name"]: float(r["AverageNs"]) / 1e3 for r in gmm1}
    avg_us = sum(avg_of[k] for k in g1s)
    # the launches of the timed steps: the run's GMM1 launches in order are the routing-count step,
    # the warm-up steps, the timed steps, then those of the graph-replay measurement (the average
    # above holds them all)
    timed = dict(avg_of)
    try:
        trace = _csv_rows(os.path.join(d, "kt"), "kernel_trace.csv")
        n, skip = int(line.get("steps", 0)), 1 + int(line.get("warmup", 0))
        for k in g1s:
            durs = sorted((int(r["Start_Timestamp"]), (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
                          for r in trace if r["Kernel_Name"] == k)
            if n > 0 and len(durs) >= skip + n:
                timed[k] = sum(v for _, v in durs[skip:skip + n]) / n
    except FileNotFoundError:
        pass
    timed_us = sum(timed[k] for k in g1s)
    # MfmaUtil of the launches, weighted by their time
    mfma = sum(_counter_mean(os.path.join(d, "mfma"), "MfmaUtil", lambda n, k=k: n == k) * timed[k] for k in g1s)
    mfma /= timed_us
    cmds = profile_commands(workload)
    cal = calibration_commands()
    lines = [f"# rocprofv3 summary: MoE layer forward, workload {workload} (GEMM variant {variant}, {layout} weights)",
             "# commands (GPU box; $GRAFT_REPO_ROOT = the repository root there):"]
    lines += [f"#   {k}: {v}" for k, v in cmds.items()]
    lines += [f"#   copy calibration {k}: {v}" for k, v in cal.items()]
    lines += [f"# reduced with: python3 bench.py --summarize {workload} --profile-dir <prof dir>", "",
              "kernel trace (durations in microseconds; top 14 by total time)",
              f"{'kernel':<90} {'calls':>6} {'avg_us':>10} {'min_us':>10} {'max_us':>10} {'total_ms':>10}"]
    for r in stats[:14]:
        lines.append(f"{r['Name'][:90]:<90} {int(r['Calls']):>6} {float(r['AverageNs']) / 1e3:>10.1f} "
                     f"{float(r['MinNs']) / 1e3:>10.1f} {float(r['MaxNs']) / 1e3:>10.1f} "
                     f"{float(r['TotalDurationNs']) / 1e6:>10.3f}")
    alg = rf.get("algorithmic_bytes")
    lines += ["", f"GMM1 kernel: {' + '.join(g1s)}",
              f"  rocprofv3 duration of the timed steps' launches: {timed_us:.1f} us (all {int(gmm1[0]['Calls'])} "
              f"launches, warm-up included: {avg_us:.1f} us); bench HIP-event launch time: "
              f"{rf.get('launch_ms', float('nan')) * 1e3:.1f} us",
              f"  FETCH_SIZE {fetch:.0f} KiB/dispatch x {fetch_factor:.3f} (copy calibration: {COPY_BYTES} B copy reads "
              f"{copy_kib / fetch_factor:.0f} KiB) ; WRITE_SIZE {write:.0f} KiB/dispatch x {write_factor:.3f}",
              f"  HBM traffic per launch: {traffic / 1e9:.3f} GB; algorithmic bytes: "
              f"{(alg or 0) / 1e9:.3f} GB; ratio {traffic / alg if alg else float('nan'):.3f}",
              f"  MfmaUtil (MFMA busy / (GPU active cycles x SIMDs)): {mfma:.1f} %",
              f"  roofline from the rocprofv3 duration of the timed launches: "
              f"{(alg or 0) / (timed_us * 1e-6) / 1e9:.1f} GB/s = {(alg or 0) / (timed_us * 1e-6) / PEAK['hbm']:.4f} of HBM peak",
              "", f"bench line of the kernel-trace run: {json.dumps({k: line[k] for k in ('value', 'ms_per_step')})}",
              f"roofline: {json.dumps(rf)}"]
    os.makedirs(dest, exist_ok=True)
    txt = os.path.join(dest, f"grouped_gemm_{workload}.txt")
    with open(txt, "w") as f:
        f.write("\n".join(lines) + "\n")
    from hyper_multicore_amd import _lib, codeobj
    # the library this summary runs beside is the one the counter runs loaded (the same tree)
    founds = []
    for k in g1s:
        found = codeobj.find_kernel(str(_lib.LIB_PATH), k) if _lib.LIB_PATH.exists() else None
        if found is None:
            print(f"[summarize] {k} is not in {_lib.LIB_PATH}: the record gets no code digest and reads as stale",
                  file=sys.stderr)
            found = (None, None)
        founds.append(found)
    found = founds[0]
    with open(os.path.join(dest, f"traffic_{workload}_{variant}_{layout}.json"), "w") as f:
        json.dump({"kernel": g1, "symbol": found[0], "code_digest": found[1],
                   **({"kernels": g1s, "symbols": [f[0] for f in founds], "code_digests": [f[1] for f in founds]}
                      if len(g1s) > 1 else {}),
                   "fetch_kib": round(fetch, 1), "fetch_factor": round(fetch_factor, 4),
                   "write_kib": round(write, 1), "write_factor": round(write_factor, 4),
                   "mfma_util_pct": round(mfma, 2), "rocprof_avg_us": round(avg_us, 1),
                   "rocprof_timed_us": round(timed_us, 1),
                   "source": os.path.basename(txt)}, f, indent=1)
        f.write("\n")
    return txt


def gemm_shapes(device, reps: int) -> dict:
    """Grouped GEMMs of the DSv3 expert shapes on their own (256 experts x 256 rows; GMM1 shape
    N = 4096, K = 7168 and GMM2 shape N = 7168, K = 2048), per weight layout and precision, timed
    with events on the stream the library launches on, for every GEMM variant the library has on."""
    from hyper_multicore_amd import _lib, ops
    g = torch.Generator(device=device).manual_seed(SEED)
    G, rows = 256, 256
    gl = torch.full((G,), rows, dtype=torch.int64, device=device).cumsum(0)
    feats = ops.features()
    variants = ["default", "w4"]
    out = {}
    for name, N, K in (("gmm1_shape", 4096, 7168), ("gmm2_shape", 7168, 2048)):
        x = torch.randn(G * rows, K, device=device, generator=g).to(torch.bfloat16)
        w = (torch.randn(G, N, K, device=device, generator=g) * 0.006).to(torch.bfloat16)  # EOI
        w_eio = w.transpose(1, 2).contiguous()  # [G, K, N]
        runs = {"bf16_EOI": lambda: ops.grouped_gemm_bf16(x, w, gl, "EOI"),
                "bf16_EIO": lambda: ops.grouped_gemm_bf16(x, w_eio, gl, "EIO")}
        xq, xs = ops.mx_quantize_rows(x)
        d, sc = ops.mx_quantize_cols(w_eio)  # EIO col_data
        runs["mxfp8_EIO"] = lambda: ops.grouped_gemm_mxfp8(xq, xs, d.view(torch.uint8), sc, gl)
        if feats & _lib.FEATURE_MX_EOI:
            de, se = ops.mx_weight_to_eoi(d, sc)
            runs["mxfp8_EOI"] = lambda: ops.grouped_gemm_mxfp8(xq, xs, de.view(torch.uint8), se, gl, layout="EOI")
        flops = 2.0 * G * rows * N * K
        for key, fn in runs.items():
            mx = key.startswith("mxfp8")
            wbytes = G * N * K * ((1 + 1 / 32) if mx else 2)
            for v in variants:
                prev = ops.set_gemm_variant(v)
                try:
                    fn()
                    torch.cuda.synchronize()
                    t0 = torch.cuda.Event(enable_timing=True)
                    t1 = torch.cuda.Event(enable_timing=True)
                    t0.record()
                    for _ in range(reps):
                        fn()
                    t1.record()
                    torch.cuda.synchronize()
                    ms = t0.elapsed_time(t1) / reps
                finally:
                    ops.set_gemm_variant(prev)
                peak = PEAK["mxfp8" if mx else "bf16"]
                out[f"{name}/{key}/{v}"] = {"ms": round(ms, 4), "tflops": round(flops / ms / 1e9, 1),
                                           "mfma_frac": round(flops / (ms * 1e-3) / peak, 4),
                                           "weight_tb_s": round(wbytes / (ms * 1e-3) / 1e12, 3)}
                log(f"[bench] {name}/{key}/{v}: {out[f'{name}/{key}/{v}']}")
        del x, w, w_eio, xq, xs, d, sc
        torch.cuda.empty_cache()
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="dsv3_bf16", choices=sorted(CONFIGS))
    ap.add_argument("--extra", default="all", help="'all', 'none' or comma list of extra configs")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--gemm-variant", default=None, choices=["default", "pp", "w4"],
                    help="forward grouped-GEMM configuration (default: MI355MOE_GG_VARIANT or the library default)")
    ap.add_argument("--bf16-layout", default="EOI", choices=["EOI", "EIO", "EIO_GU"],
                    help="expert-weight layout of the bf16 configs (EIO: the reference module's default)")
    ap.add_argument("--mx-layout", default="EIO_GU", choices=["EIO", "EOI", "EIO_GU"],
                    help="MX expert-weight layout (EIO: the reference's col_data root; EOI: re-laid out once with "
                         "K contiguous; EIO_GU: the root with W1's gate and up columns interleaved once, as the "
                         "MegaMoE module prepares it)")
    ap.add_argument("--gemm-shapes", action="store_true",
                    help="time the DSv3-shape grouped GEMMs on their own per layout and variant (one JSON line)")
    ap.add_argument("--profile-commands", metavar="WORKLOAD", default=None,
                    help="print the rocprofv3 commands behind profiles/ for WORKLOAD ('copy': the calibration)")
    ap.add_argument("--summarize", metavar="WORKLOAD", default=None,
                    help="reduce the rocprofv3 output of --profile-commands WORKLOAD into profiles/")
    ap.add_argument("--profile-dir", default=os.path.join(ROOT, "gpurun_out", "prof"))
    args = ap.parse_args()
    if args.profile_commands is not None:
        cmds = calibration_commands() if args.profile_commands == "copy" else profile_commands(args.profile_commands)
        print("\n".join(cmds.values()))
        return 0
    if args.summarize is not None:
        print(summarize(args.summarize, args.profile_dir))
        return 0
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one MI355X only: this build runs every expert on one GPU (EP=1) and has no "
              "multi-GPU path; run with --gpus 1.", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("no GPU visible", file=sys.stderr)
        return 1
    from hyper_multicore_amd import _lib
    _lib.load()
    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    from hyper_multicore_amd import ops
    if args.gemm_shapes:
        print(json.dumps({"gemm_shapes": gemm_shapes(device, max(3, args.steps // 2)),
                          "library_features": _library_features()}), flush=True)
        return 0
    if args.gemm_variant is not None:
        ops.set_gemm_variant(args.gemm_variant)
    gemm_variant = ops.gemm_variant()
    log(f"[bench] workload {args.config}: steps={args.steps} warmup={args.warmup}")
    res, layer = run_config(args.config, device, args.steps, args.warmup, gemm_variant, args.bf16_layout,
                            args.mx_layout)
    c = layer.c
    cpu = None if args.no_cpu else cpu_baseline(args.config, layer)
    del layer
    torch.cuda.empty_cache()
    extra = {}
    names = [] if args.extra == "none" else (sorted(CONFIGS) if args.extra == "all" else args.extra.split(","))
    for name in names:
        if name == args.config:
            continue
        log(f"[bench] extra {name}")
        r, lyr = run_config(name, device, max(5, args.steps // 2), max(2, args.warmup // 2), gemm_variant,
                            args.bf16_layout, args.mx_layout)
        extra[name] = r
        del lyr
        torch.cuda.empty_cache()
    line = {
        "metric": "MoE layer tokens/s + achieved TFLOP/s (% MFMA peak), DSv3 shape, 1 MI355X",
        "value": res["tokens_per_s"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": res["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if c["precision"] == "bf16" else "mxfp8(e4m3+e8m0/32)",
        "data": "synthetic (seeded normal activations / random-init weights of the config's shapes)",
        "config": {"workload": args.config, "baseline_config_index": c["idx"], "tokens": c["T"], "experts": c["E"],
                   "top_k": c["K"], "hidden": c["H"], "intermediate": c["I"], "router": c["scoring"],
                   "groups": f"{c['groups']}/{c['topk_groups']}", "parallelism": "ep1",
                   "weight_layout": res["weight_layout"],
                   "gemm_variant": gemm_variant,
                   "library_features": _library_features()},
        "layer_tflops": res["layer_tflops"],
        "layer_mfma_frac": res["layer_mfma_frac"],
        "active_experts": res["active_experts"],
        "m_tiles": res["m_tiles"],
        "stage_ms": res["stage_ms"],
        "roofline": res["roofline"],
        "graph": res["graph"],
        "cpu_baseline": cpu,
        "extra": extra,
    }
    line["targets"] = targets({args.config: res, **extra})
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
