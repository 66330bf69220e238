"""Host-side logic of the drop-in modules (CPU only; no kernel launches)."""
import os
import pytest
import torch

import hyper_multicore_amd as hm
from hyper_multicore_amd import ops


def test_megagate_validation_mirrors_reference():
    kw = dict(hidden_size=16, num_experts=8, top_k=2, scoring_func="softmax", routed_scaling_factor=1.0)
    hm.MegaGate(**kw)
    for bad in (dict(top_k=9), dict(hidden_size=0), dict(scoring_func="relu"),
                dict(routed_scaling_factor=float("inf")), dict(initializer_range=-1.0),
                dict(num_expert_groups=3), dict(num_expert_groups=4, topk_groups=5),
                dict(num_expert_groups=4, topk_groups=1, top_k=3)):
        with pytest.raises(ValueError):
            hm.MegaGate(**{**kw, **bad})


def _small_gate(vision_enabled, initializer_range=0.02):
    return hm.MegaGate(hidden_size=128, num_experts=16, top_k=6, scoring_func="sqrtsoftplus",
                       routed_scaling_factor=1.5, vision_enabled=vision_enabled, initializer_range=initializer_range)


def test_megagate_parameter_initialization():
    """As the reference's unit test (tests/ut/modules/mega_gate/test_mega_gate_module.py:45-56): the
    projection from one Normal(0, initializer_range) draw, zero correction biases, exactly the
    parameters weight / bias / bias_vl."""
    from unittest.mock import patch
    with patch("torch.nn.init.normal_", wraps=torch.nn.init.normal_) as normal:
        gate = _small_gate(True, initializer_range=0.035)
    normal.assert_called_once_with(gate.weight, mean=0.0, std=0.035)
    assert set(gate.state_dict()) == {"weight", "bias", "bias_vl"}
    assert tuple(gate.weight.shape) == (16, 128)
    assert torch.isfinite(gate.weight).all() and torch.count_nonzero(gate.weight) > 0
    assert torch.count_nonzero(gate.bias) == 0 and torch.count_nonzero(gate.bias_vl) == 0


def test_megagate_meta_materialization_and_reset():
    """A module built on the meta device, materialised with to_empty and reset (the reference's
    test_mega_gate_module.py:58-69)."""
    with torch.device("meta"):
        gate = _small_gate(False)
    gate.to_empty(device="cpu")
    gate.reset_parameters()
    assert torch.isfinite(gate.weight).all() and torch.count_nonzero(gate.weight) > 0
    assert torch.count_nonzero(gate.bias) == 0
    assert gate.bias_vl is None


def test_megagate_keeps_fp32_biases_under_dtype_change():
    gate = hm.MegaGate(hidden_size=16, num_experts=8, top_k=2, scoring_func="sigmoid", routed_scaling_factor=1.0,
                       vision_enabled=True).to(torch.bfloat16)
    assert gate.weight.dtype == torch.bfloat16
    assert gate.bias.dtype == torch.float32 and gate.bias_vl.dtype == torch.float32
    assert torch.count_nonzero(gate.bias) == 0


def test_megagate_from_module_shares_parameters():
    src = torch.nn.Module()
    src.weight = torch.nn.Parameter(torch.randn(8, 16))
    src.bias = torch.nn.Parameter(torch.zeros(8))
    gate = hm.MegaGate.from_module(src, top_k=2, scoring_func="softmax", routed_scaling_factor=1.0)
    assert gate.weight is src.weight and gate.bias is src.bias
    with pytest.raises(ValueError):
        hm.MegaGate.from_module(src)  # top_k etc. missing


def test_megagate_forward_errors():
    gate = hm.MegaGate(hidden_size=16, num_experts=8, top_k=2, scoring_func="softmax", routed_scaling_factor=1.0)
    x = torch.randn(1, 4, 16)
    with pytest.raises(ValueError):
        gate(x, image_mask=torch.ones(1, 4, dtype=torch.bool))  # no vision bias
    with pytest.raises(RuntimeError):
        gate(x)  # the gfx950 path needs a GPU; there is no CPU fallback


def test_megamoe_options_and_validation():
    kw = dict(hidden_size=128, intermediate_size=64, num_experts=4, top_k=2)
    ex = hm.MegaMoeExperts(**kw)
    assert ex.precision == "bf16" and ex.swiglu_limit is None and not ex.apply_probs_before_fc2
    with pytest.raises(ValueError):
        hm.MegaMoeExperts(**kw, precision="fp16")
    with pytest.raises(ValueError):
        hm.MegaMoeExperts(**{**kw, "top_k": 5})
    with pytest.raises(ValueError):
        hm.MegaMoeExperts(**kw, precision="mxfp8",
                          numerics_options=hm.MegaMoeNumericsOptions(apply_probs_before_fc2=True))
    from hyper_multicore_amd import _lib, ops
    if ops.features() & _lib.FEATURE_NUMERICS:
        hm.MegaMoeExperts(**kw, numerics_options=hm.MegaMoeNumericsOptions(swiglu_limit=7.0))
    else:
        with pytest.raises(NotImplementedError):
            hm.MegaMoeExperts(**kw, numerics_options=hm.MegaMoeNumericsOptions(swiglu_limit=7.0))
    # swiglu_limit: finite, positive, and still finite and positive as float32 (module.py:55-79)
    for bad in (-1.0, 0.0, float("nan"), float("inf"), 1e39, 1e-50, True, "7"):
        with pytest.raises(ValueError):
            hm.MegaMoeExperts(**kw, numerics_options=hm.MegaMoeNumericsOptions(swiglu_limit=bad))
    with pytest.raises(TypeError):
        hm.MegaMoeExperts(**kw, numerics_options=dict(swiglu_limit=None))
    with pytest.raises(ValueError):
        hm.MegaMoeExperts(**kw, tuning_options=hm.MegaMoeTuningOptions(dispatch_split=100))

    class Group:
        def size(self):
            return 2
    with pytest.raises(ValueError):
        hm.MegaMoeExperts(**kw, ep_group=Group())


def test_megamoe_layout_inference_and_input_checks():
    ex = hm.MegaMoeExperts(hidden_size=128, intermediate_size=64, num_experts=4, top_k=2)
    assert ex._infer_layout((4, 128, 128), (4, 64, 128)) == "EIO"
    assert ex._infer_layout((4, 128, 128), (4, 128, 64)) == "EOI"
    with pytest.raises(ValueError):
        ex._infer_layout((4, 128, 64), (4, 64, 128))
    x = torch.randn(6, 128).to(torch.bfloat16)
    ids = torch.zeros(6, 2, dtype=torch.int64)
    w = torch.rand(6, 2)
    with pytest.raises(ValueError):
        ex(x, ids[:, :1], w, expert_weights=(None, None))
    with pytest.raises(TypeError):
        ex(x, ids, w, expert_weights=(None, None))  # CPU hidden states


def test_ops_reject_cpu_tensors():
    with pytest.raises(TypeError):
        ops.dispatch(torch.zeros(4, 2, dtype=torch.int64), 8)
    with pytest.raises(TypeError):
        ops.mx_quantize_rows(torch.zeros(4, 32, dtype=torch.bfloat16))


def _built_kernel():
    """(mangled symbol, code digest) of the bf16 prefill GMM1 kernel of the built library, or skip."""
    from hyper_multicore_amd import _lib, codeobj
    if not _lib.LIB_PATH.exists():
        pytest.skip("native library not built")
    found = codeobj.find_kernel(str(_lib.LIB_PATH), PP_BF16_GMM1)
    assert found is not None
    return found


PP_BF16_GMM1 = "void (anonymous namespace)::gg_pp_kernel<false, false, 2, true, 0>(GGParams)"


def test_bench_traffic_record(tmp_path):
    """roofline.traffic comes from a committed counter record of the same workload and GEMM variant:
    FETCH_SIZE / WRITE_SIZE KiB per dispatch, each times its copy-kernel calibration factor, and only
    while the record's kernel has the same machine code in the library (code digest)."""
    import json
    import bench
    sym, digest = _built_kernel()
    (tmp_path / "profiles").mkdir()
    rec = {"fetch_kib": 1000.0, "fetch_factor": 0.5, "write_kib": 10.0, "write_factor": 2.0, "symbol": sym,
           "code_digest": digest}
    (tmp_path / "profiles" / "traffic_dsv3_bf16_w4_EOI.json").write_text(json.dumps(rec))
    assert bench.measured_traffic("dsv3_bf16", "w4", "EOI", root=str(tmp_path)) == ((500 + 20) * 1024, "current")
    assert bench.measured_traffic("dsv3_bf16", "w4", "EIO", root=str(tmp_path)) == (None, "none")
    assert bench.measured_traffic("dsv3_bf16", "default", "EOI", root=str(tmp_path)) == (None, "none")
    for bad in ({"code_digest": "0" * 16}, {"symbol": sym + "x"}, {"symbol": None}):
        (tmp_path / "profiles" / "traffic_dsv3_bf16_w4_EOI.json").write_text(json.dumps({**rec, **bad}))
        assert bench.measured_traffic("dsv3_bf16", "w4", "EOI", root=str(tmp_path)) == (None, "stale")
    c = bench.CONFIGS["dsv3_bf16"]
    work = {"g1_flops": 1e12, "g1_bytes": 1e10}
    r = bench.roofline(c, work, 2.0, traffic=2e10, traffic_record="current")
    assert r["traffic"] == 2e10 and r["bound"] == "hbm" and r["unit"] == "GB/s"
    assert r["traffic_ratio"] == 2.0 and r["algorithmic_bytes"] == 1e10 and r["achieved"] == 5000.0
    assert r["traffic_record"] == "current"


def test_committed_traffic_records_are_current():
    """Every committed counter record names a kernel whose machine code in the built library is the
    code the counters were read from."""
    import glob
    import json
    from hyper_multicore_amd import _lib, codeobj
    if not _lib.LIB_PATH.exists():
        pytest.skip("native library not built")
    digests = codeobj.kernel_digests(str(_lib.LIB_PATH))
    paths = glob.glob(os.path.join(os.path.dirname(os.path.dirname(__file__)), "profiles", "traffic_*.json"))
    assert paths
    for path in paths:
        rec = json.load(open(path))
        assert digests.get(rec["symbol"]) == rec["code_digest"], path


def test_code_digests_cover_the_kernels():
    """The code-object reader finds every kernel of the library with a distinct digest per distinct
    body, and demangles the GEMM kernels' names."""
    from hyper_multicore_amd import _lib, codeobj
    if not _lib.LIB_PATH.exists():
        pytest.skip("native library not built")
    dig = codeobj.kernel_digests(str(_lib.LIB_PATH))
    assert len(dig) > 40
    assert all(len(v) == 16 for v in dig.values())
    names = codeobj.demangle(sorted(dig))
    assert PP_BF16_GMM1 in names
    assert any("decode_prep_kernel" in n for n in names)


def _write_csv(path, header, rows):
    import csv
    path.parent.mkdir(parents=True, exist_ok=True)
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(header)
        w.writerows(rows)


def test_bench_profile_summary(tmp_path):
    """--summarize picks the SwiGLU-epilogue grouped GEMM as GMM1, scales its counters by what the same
    counters read for the calibration copy, and writes the traffic record the bench line reads back."""
    import json
    import bench
    out = tmp_path / "prof"
    cnt = ["Kernel_Name", "Counter_Name", "Counter_Value"]
    copy_kib = bench.COPY_BYTES / 1024
    _write_csv(out / "copy" / "fetch" / "pmc_counter_collection.csv", cnt,
               [["__amd_rocclr_copyBuffer", "FETCH_SIZE", copy_kib / 2], ["other", "FETCH_SIZE", 1.0]])
    _write_csv(out / "copy" / "write" / "pmc_counter_collection.csv", cnt,
               [["__amd_rocclr_copyBuffer", "WRITE_SIZE", copy_kib]])
    g1 = "void (anonymous namespace)::gg_pp_kernel<false, false, 2, true, 0>(GGParams)"
    g2 = "void (anonymous namespace)::gg_pp_kernel<false, false, 0, true, 0>(GGParams)"
    for name, is_g1 in ((g1, True), (g2, False), ("void grouped_gemm_kernel<GGCfg<64, 1, 3, 3, 256, 2, 2, 2, false>, "
                                                   "true, true, 3>(GGParams)", True),
                        ("void grouped_gemm_kernel<false, false, 1>(GGParams)", False)):
        assert bool(bench.GMM1_KERNEL.search(name)) == is_g1, name
    d = out / "dsv3_bf16"
    _write_csv(d / "fetch" / "pmc_counter_collection.csv", cnt,
               [[g1, "FETCH_SIZE", 900.0], [g1, "FETCH_SIZE", 1100.0], [g2, "FETCH_SIZE", 5.0]])
    _write_csv(d / "write" / "pmc_counter_collection.csv", cnt, [[g1, "WRITE_SIZE", 100.0]])
    _write_csv(d / "mfma" / "pmc_counter_collection.csv", cnt, [[g1, "MfmaUtil", 40.0]])
    st = ["Name", "Calls", "TotalDurationNs", "AverageNs", "Percentage", "MinNs", "MaxNs"]
    _write_csv(d / "kt" / "run_kernel_stats.csv", st,
               [[g2, 10, 3e7, 3e6, 30, 3e6, 3e6], [g1, 10, 6e7, 6e6, 60, 6e6, 6e6]])
    line = {"value": 1.0, "ms_per_step": 9.0, "config": {"gemm_variant": "default", "weight_layout": "EOI"},
            "roofline": {"algorithmic_bytes": 2048 * 1024, "launch_ms": 6.1}}
    (d / "bench.json").write_text("[bench] noise\n" + json.dumps(line) + "\n")
    txt = bench.summarize("dsv3_bf16", str(out), dest=str(tmp_path / "profiles"))
    rec = json.loads((tmp_path / "profiles" / "traffic_dsv3_bf16_default_EOI.json").read_text())
    assert rec["kernel"] == g1 and rec["fetch_kib"] == 1000.0 and rec["fetch_factor"] == 2.0
    assert rec["write_factor"] == 1.0 and rec["rocprof_avg_us"] == 6000.0 and rec["mfma_util_pct"] == 40.0
    assert (rec["symbol"], rec["code_digest"]) == _built_kernel()
    assert bench.measured_traffic("dsv3_bf16", "default", "EOI", root=str(tmp_path)) == ((2000 + 100) * 1024,
                                                                                           "current")
    text = open(txt).read()
    assert "ratio 1.025" in text and "rocprofv3 --pmc FETCH_SIZE" in text
    assert rec["rocprof_timed_us"] == 6000.0  # no kernel trace: the all-launch average


def test_bench_profile_summary_times_the_timed_launches(tmp_path):
    """The rocprofv3 GMM1 duration the summary sets beside the HIP-event time is the mean over the timed
    steps' launches: after the routing-count step and the warm-up, before the graph replays."""
    import json
    import bench
    out = tmp_path / "prof"
    cnt = ["Kernel_Name", "Counter_Name", "Counter_Value"]
    copy_kib = bench.COPY_BYTES / 1024
    _write_csv(out / "copy" / "fetch" / "pmc_counter_collection.csv", cnt, [["__amd_rocclr_copyBuffer", "FETCH_SIZE", copy_kib]])
    _write_csv(out / "copy" / "write" / "pmc_counter_collection.csv", cnt, [["__amd_rocclr_copyBuffer", "WRITE_SIZE", copy_kib]])
    g1 = "void (anonymous namespace)::gg_pp_kernel<false, false, 2, true, 0>(GGParams)"
    d = out / "dsv3_bf16"
    for tag, c in (("fetch", "FETCH_SIZE"), ("write", "WRITE_SIZE"), ("mfma", "MfmaUtil")):
        _write_csv(d / tag / "pmc_counter_collection.csv", cnt, [[g1, c, 1.0]])
    # 1 routing-count + 2 warm-up launches at 9 us, 3 timed at 5, 6 and 7 us, then 4 replays at 20 us
    durations = [9, 9, 9, 5, 6, 7, 20, 20, 20, 20]
    trace, t = [], 1000
    for us in durations:
        trace.append([g1, t, t + us * 1000])
        t += 100000
    _write_csv(d / "kt" / "run_kernel_trace.csv", ["Kernel_Name", "Start_Timestamp", "End_Timestamp"], trace[::-1])
    avg = sum(durations) / len(durations) * 1000
    _write_csv(d / "kt" / "run_kernel_stats.csv", ["Name", "Calls", "TotalDurationNs", "AverageNs", "MinNs", "MaxNs"],
               [[g1, len(durations), avg * len(durations), avg, 5000, 20000]])
    line = {"value": 1.0, "ms_per_step": 1.0, "steps": 3, "warmup": 2,
            "config": {"gemm_variant": "default", "weight_layout": "EOI"},
            "roofline": {"algorithmic_bytes": 1 << 20, "launch_ms": 0.006}}
    (d / "bench.json").write_text(json.dumps(line) + "\n")
    bench.summarize("dsv3_bf16", str(out), dest=str(tmp_path / "profiles"))
    rec = json.loads((tmp_path / "profiles" / "traffic_dsv3_bf16_default_EOI.json").read_text())
    assert rec["rocprof_timed_us"] == 6.0 and rec["rocprof_avg_us"] == 12.5


def _physical(root, shape):
    """Attach packed column and row axes to an MX root (the reference's FSDP root fields)."""
    e, m, n = shape
    root.col_data = torch.empty(shape, dtype=torch.float8_e4m3fn)
    root.col_scale = torch.empty((e, m // 64, n, 2), dtype=torch.uint8)
    root.row_data = torch.empty(shape, dtype=torch.float8_e4m3fn)
    root.row_scale = torch.empty((e, m, n // 64, 2), dtype=torch.uint8)


def test_mx_backward_resolves_fresh_row_axis_and_keeps_forward_columns(monkeypatch):
    """The MX autograd function reads the row axis the owner materialised after the forward (fields
    replaced, column axis released), as test_mxfp8_root_lifecycle.py:31-73 requires of the reference;
    the recompute uses the column axis the forward read. The GPU calls are replaced by recorders."""
    from hyper_multicore_amd import mega_moe
    E, H, I, T, K = 2, 64, 64, 4, 1
    shapes = ((E, H, 2 * I), (E, I, H))
    roots = [torch.nn.Parameter(torch.empty(s, dtype=torch.bfloat16)) for s in shapes]
    for r, s in zip(roots, shapes):
        _physical(r, s)
    fwd_cols = [(r.col_data.data_ptr(), r.col_scale.data_ptr()) for r in roots]
    seen = {}

    def fake_forward(hidden, ids, probs, d1, d2, **kw):
        seen["forward"] = (d1.data_ptr(), kw["w1_scale"].data_ptr(), d2.data_ptr(), kw["w2_scale"].data_ptr())
        return hidden.clone()

    def fake_backward(hidden, ids, probs, w1, w2, grad_out, **kw):
        seen["backward"] = [tuple(t.data_ptr() for t in w) for w in (w1, w2)]
        return (grad_out.clone(), torch.zeros(E, H, 2 * I), torch.zeros(E, I, H),
                torch.zeros(T, K) if kw["need_topk_grad"] else None)

    from hyper_multicore_amd import mxfp8
    monkeypatch.setattr(ops, "features", lambda: 0)
    monkeypatch.setattr(ops, "moe_forward", fake_forward)
    monkeypatch.setattr(ops, "moe_backward_mxfp8", fake_backward)
    monkeypatch.setattr(mxfp8, "prepared_gate_up_weight", lambda root, d, s: (d, s))  # the GPU re-layout
    ex = hm.MegaMoeExperts(hidden_size=H, intermediate_size=I, num_experts=E, top_k=K, precision="mxfp8")
    x = torch.ones((T, H), dtype=torch.bfloat16, requires_grad=True)
    probs = torch.ones((T, K), requires_grad=True)
    ids = torch.zeros((T, K), dtype=torch.int64)
    y = mega_moe._MxMoeFunction.apply(x, probs, roots[0], roots[1], ids, ex, torch.float32)
    assert seen["forward"] == (*fwd_cols[0], *fwd_cols[1])
    for r, s in zip(roots, shapes):  # the owner gathers a fresh row axis and releases the column axis
        _physical(r, s)
        r.col_data = r.col_scale = None
    y.sum().backward()
    for got, r, cols in zip(seen["backward"], roots, fwd_cols):
        assert got == (*cols, r.row_data.data_ptr(), r.row_scale.data_ptr())
    assert torch.equal(x.grad, torch.ones_like(x))
    assert all(torch.equal(r.grad, torch.zeros_like(r)) for r in roots)
    for r, s in zip(roots, shapes):  # a root without its row axis is reported by name
        _physical(r, s)
        del r.row_data
    y = mega_moe._MxMoeFunction.apply(x, probs, roots[0], roots[1], ids, ex, torch.float32)
    with pytest.raises(ValueError, match="missing required row data/scale"):
        y.sum().backward()


def test_invalid_routes_raise_like_the_reference():
    """route.py:566-593: counts that do not describe the actual Top-K routes raise RuntimeError."""
    from hyper_multicore_amd.mega_moe import ROUTE_COUNT_ERROR, validate_routes
    ids = torch.tensor([[0, 1], [2, 3], [1, 2]])
    validate_routes(ids, 4)
    validate_routes(ids, 4, torch.tensor([1, 2, 2, 1]))
    for bad in (torch.tensor([[0, 1], [2, 4], [1, 2]]), torch.tensor([[0, -1], [2, 3], [1, 2]])):
        with pytest.raises(RuntimeError, match=ROUTE_COUNT_ERROR):
            validate_routes(bad, 4)
    with pytest.raises(RuntimeError, match=ROUTE_COUNT_ERROR):
        validate_routes(ids, 4, torch.tensor([1, 2, 1, 2]))  # not the histogram
    with pytest.raises(RuntimeError, match=ROUTE_COUNT_ERROR):
        validate_routes(ids.to(torch.int32), 3)  # id 3 outside [0, 3)


def test_output_overlap_check():
    """The no-overlap check of the unpermute gradient's outputs (mega_moe_unpermute.cpp:47-52): spans
    that share memory overlap, disjoint ones do not."""
    from hyper_multicore_amd.ops import _overlaps
    a = torch.zeros(100)
    assert _overlaps(a, a[50:]) and _overlaps(a[10:20], a[15:30])
    assert not _overlaps(a[:50], a[50:]) and not _overlaps(a, torch.zeros(10)) and not _overlaps(a, None)
    m = torch.zeros(64, 32)
    assert not _overlaps(m[:32], m[32:]) and _overlaps(m[:, :16], m[:, 16:])  # row blocks vs column halves
    assert not _overlaps(m, torch.zeros(64, 32))


def test_bench_targets_block():
    """The bench line's targets block sets the measured figures beside BASELINE.json's bars, for the
    configs the run measured only."""
    import bench
    t = bench.targets({"dsv3_decode_mxfp8": {"roofline": {"frac": 0.66}, "layer_hbm_frac": 0.61},
                       "dsv3_mxfp8": {"layer_mfma_frac": 0.19}})
    assert t["dsv3_mxfp8_layer_mfma_frac"] == {"measured": 0.19, "bar": 0.55}
    assert t["dsv3_decode_mxfp8_gmm1_hbm_frac"] == {"measured": 0.66, "bar": 0.65}
    assert t["dsv3_decode_mxfp8_layer_hbm_frac"]["measured"] == 0.61
    assert bench.targets({"small_bf16": {}}) == {}


def test_bench_profile_summary_two_gmm1_launches(tmp_path):
    """With the 384 x 128 MX tile GMM1 is two launches per step: the summary adds their counters and
    durations, and the traffic record names both kernels (each must be current for the bench to use it)."""
    import json
    import bench
    from hyper_multicore_amd import _lib
    if not _lib.LIB_PATH.exists():
        pytest.skip("native library not built")
    out = tmp_path / "prof"
    cnt = ["Kernel_Name", "Counter_Name", "Counter_Value"]
    copy_kib = bench.COPY_BYTES / 1024
    _write_csv(out / "copy" / "fetch" / "pmc_counter_collection.csv", cnt, [["__amd_rocclr_copyBuffer", "FETCH_SIZE", copy_kib]])
    _write_csv(out / "copy" / "write" / "pmc_counter_collection.csv", cnt, [["__amd_rocclr_copyBuffer", "WRITE_SIZE", copy_kib]])
    a = "void (anonymous namespace)::gg_pp_kernel<true, true, 5, false, 1>(GGParams)"
    b = "void (anonymous namespace)::gg_pp_kernel<true, true, 5, false, 2>(GGParams)"
    g2 = "void (anonymous namespace)::gg_pp_kernel<true, true, 0, false, 1>(GGParams)"
    d = out / "dsv3_mxfp8"
    _write_csv(d / "fetch" / "pmc_counter_collection.csv", cnt, [[a, "FETCH_SIZE", 3000.0], [b, "FETCH_SIZE", 1000.0],
                                                                 [g2, "FETCH_SIZE", 9.0]])
    _write_csv(d / "write" / "pmc_counter_collection.csv", cnt, [[a, "WRITE_SIZE", 30.0], [b, "WRITE_SIZE", 10.0]])
    _write_csv(d / "mfma" / "pmc_counter_collection.csv", cnt, [[a, "MfmaUtil", 30.0], [b, "MfmaUtil", 60.0]])
    st = ["Name", "Calls", "TotalDurationNs", "AverageNs", "Percentage", "MinNs", "MaxNs"]
    _write_csv(d / "kt" / "run_kernel_stats.csv", st,
               [[a, 10, 3e7, 3e6, 50, 3e6, 3e6], [b, 10, 1e7, 1e6, 20, 1e6, 1e6], [g2, 10, 2e7, 2e6, 30, 2e6, 2e6]])
    line = {"value": 1.0, "ms_per_step": 6.0, "config": {"gemm_variant": "default", "weight_layout": "EIO_GU"},
            "roofline": {"algorithmic_bytes": 4096 * 1024, "launch_ms": 4.0}}
    (d / "bench.json").write_text(json.dumps(line) + "\n")
    txt = bench.summarize("dsv3_mxfp8", str(out), dest=str(tmp_path / "profiles"))
    rec = json.loads((tmp_path / "profiles" / "traffic_dsv3_mxfp8_default_EIO_GU.json").read_text())
    assert rec["kernels"] == [a, b] and len(rec["symbols"]) == 2 and None not in rec["code_digests"]
    assert rec["fetch_kib"] == 4000.0 and rec["write_kib"] == 40.0
    assert rec["rocprof_avg_us"] == 4000.0 and rec["mfma_util_pct"] == 37.5  # (30 * 3 + 60 * 1) / 4
    assert bench.measured_traffic("dsv3_mxfp8", "default", "EIO_GU", root=str(tmp_path)) == ((4000 + 40) * 1024,
                                                                                           "current")
    assert f"GMM1 kernel: {a} + {b}" in open(txt).read()
    rec["code_digests"][1] = "0" * 16
    (tmp_path / "profiles" / "traffic_dsv3_mxfp8_default_EIO_GU.json").write_text(json.dumps(rec))
    assert bench.measured_traffic("dsv3_mxfp8", "default", "EIO_GU", root=str(tmp_path)) == (None, "stale")


def test_bench_m_tiles_weight_passes(monkeypatch):
    """m_tiles counts the expert weight passes: an expert of 257..511 rows takes two 256-row m-tiles,
    or one 384-row tile with MI355MOE_PP_SKINNY=1 when it has at most 384 rows."""
    import bench
    c = dict(bench.CONFIGS["dsv3_mxfp8"], T=256, K=4, E=4)  # R = 1024, 256 rows per expert on average
    counts = torch.tensor([100, 300, 384, 240])
    monkeypatch.delenv("MI355MOE_PP_SKINNY", raising=False)
    r = bench.m_tiles(c, counts)
    assert r["bm"] == 256 and r["tiles"] == 1 + 2 + 2 + 1 and r["weight_passes_per_expert"] == 1.5
    monkeypatch.setenv("MI355MOE_PP_SKINNY", "1")
    r = bench.m_tiles(c, counts)
    assert r["tiles"] == 2 and r["skinny_tiles"] == 2 and r["weight_passes_per_expert"] == 1.0
    assert r["padded_row_frac"] == round(1 - 1024 / (2 * 256 + 2 * 384), 4)


def test_bench_m_tiles_bf16_skinny(monkeypatch):
    """bf16: 320-row tiles when the groups average at most 320 rows; with the 384 x 128 tile the
    groups of 321..384 rows take one pass."""
    import bench
    c = dict(bench.CONFIGS["dsv3_bf16"], T=256, K=4, E=4)  # 256 rows per expert on average
    counts = torch.tensor([100, 330, 384, 210])
    monkeypatch.setenv("MI355MOE_PP_SKINNY", "1")
    r = bench.m_tiles(c, counts)
    assert r["bm"] == 320 and r["tiles"] == 2 and r["skinny_tiles"] == 2 and r["weight_passes_per_expert"] == 1.0
    monkeypatch.delenv("MI355MOE_PP_SKINNY")
    r = bench.m_tiles(c, counts)
    assert "skinny_tiles" not in r and r["tiles"] == 1 + 2 + 2 + 1
