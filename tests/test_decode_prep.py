"""The one-launch decode prologue (hyper_multicore_amd/csrc/decode_prep.h) on the CPU.

tests/native/prep_check runs the kernel's code under the host emulation of a workgroup
(tests/native/prep_sim.inc: 256 threads, the kernel's barriers, ballots and shuffles as lockstep
points, AddressSanitizer on every buffer, UndefinedBehaviorSanitizer). Its outputs are compared with the oracle: counts with
``expert_counts`` (route.py:186-211), group_list with the EP=1 ``route_metadata`` (route.py:309-390),
mapping / gather with ``stable_permutation`` (utilities.asc:176-204), the tile plan with its definition
(exclusive prefix of ceil(count / bm)), and the token quantisation with ``mx_quantize`` (scale algorithm
1). Deliberate faults of the emulation (ballot, shuffle, e4m3 rounding) must make the comparison fail.
"""
from __future__ import annotations

import shutil
import subprocess

import numpy as np
import pytest
import torch

from oracle import moe_oracle as orc
from tests.native import build_check

MAX_SLOTS = 8192
MAX_EXPERTS = 1024


@pytest.fixture(scope="module")
def prep(tmp_path_factory):
    if not (shutil.which("nm") and (build_check._rocm() / "bin" / "hipcc").exists()):
        pytest.skip("hipcc not available")
    exe = build_check.build_prep()
    d = tmp_path_factory.mktemp("prep")

    def run(ids: np.ndarray, E: int, bm: int, x: np.ndarray | None, flags: int = 31, mutation: int = 0):
        i64 = ids.dtype == np.int64
        slots = ids.size
        rows, cols = (0, 32) if x is None else x.shape
        head = np.array([int(i64), slots, E, bm, rows, cols, flags], dtype=np.int64)
        inp, out = d / "in.bin", d / "out.bin"
        xb = b"" if x is None else x.astype(np.uint16).tobytes()
        inp.write_bytes(head.tobytes() + ids.tobytes() + xb)
        r = subprocess.run([str(exe), str(inp), str(out), str(mutation)], capture_output=True, text=True,
                           timeout=300)
        if r.returncode == 3:
            return None
        assert r.returncode == 0, r.stderr
        b = out.read_bytes()
        o = 0

        def take(dtype, n):
            nonlocal o
            a = np.frombuffer(b, dtype=dtype, count=n, offset=o)
            o += a.nbytes
            return a

        st = take(np.int64, 2)
        res = {"ballots": int(st[0]), "workgroups": int(st[1]), "counts": take(np.int32, E),
               "group_list": take(np.int64, E), "mapping": take(np.int32, slots), "gather": take(np.int32, slots),
               "error": int(take(np.int32, 1)[0]), "tile_prefix": take(np.int32, E + 1),
               "q": take(np.uint8, rows * cols).reshape(rows, cols),
               "scale": take(np.uint8, rows * (cols // 32)).reshape(rows, cols // 32)}
        assert o == len(b)
        return res

    return run


def _expected(ids: np.ndarray, E: int, bm: int):
    t = torch.from_numpy(ids.astype(np.int64))
    valid = (t >= 0) & (t < E)
    counts = orc.expert_counts(t[valid], E)
    meta = orc.route_metadata(counts.reshape(1, E).to(torch.int64), rank=0, ep_size=1)
    mapping, gather = orc.stable_permutation(t, E)
    tiles = (counts.to(torch.int64) + bm - 1) // bm
    prefix = torch.cat([torch.zeros(1, dtype=torch.int64), tiles.cumsum(0)])
    return counts.numpy(), meta["group_list"].numpy(), mapping.numpy(), gather.numpy(), prefix.numpy(), \
        bool((~valid).any())


def _check_dispatch(res, ids, E, bm, flags=31):
    counts, group_list, mapping, gather, prefix, bad = _expected(ids, E, bm)
    np.testing.assert_array_equal(res["mapping"], mapping)
    if flags & 1:
        np.testing.assert_array_equal(res["counts"], counts)
    if flags & 2:
        np.testing.assert_array_equal(res["group_list"], group_list)
    if flags & 4:
        n = gather.size
        np.testing.assert_array_equal(res["gather"][:n], gather)
        # rows past the routed ones are not written
        assert (res["gather"][n:] == np.int32(-101058055)).all()
    if flags & 8:
        assert res["error"] == int(bad)
    if flags & 16:
        np.testing.assert_array_equal(res["tile_prefix"], prefix)


def _topk_ids(T, K, E, rng, dtype=np.int32):
    return np.stack([rng.choice(E, K, replace=False) for _ in range(T)]).astype(dtype)


def _bf16_rows(T, H, rng):
    x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32))
    x = x * torch.from_numpy(np.exp2(rng.integers(-20, 20, (T, H // 32))).astype(np.float32)).repeat_interleave(32, 1)
    x[0, :32] = 0.0  # an all-zero block
    x[1, 32:64] = 1e-40  # fp32 subnormals (zero in bf16 after rounding of the smallest ones)
    x[2, 64:96] = -448.0
    return x.to(torch.bfloat16)


def _check_quant(res, x_bf16):
    q, s = orc.mx_quantize(x_bf16.float())
    np.testing.assert_array_equal(res["q"], q.numpy())
    np.testing.assert_array_equal(res["scale"], s.numpy())


def test_decode_shape_mx(prep):
    """DSv3 decode: T=128, K=8, E=256, H=7168, the 64-row tile plan and the MX token quantisation."""
    rng = np.random.default_rng(0)
    ids = _topk_ids(128, 8, 256, rng)
    x = _bf16_rows(128, 7168, rng)
    res = prep(ids, 256, 64, x.view(torch.int16).numpy().view(np.uint16))
    _check_dispatch(res, ids, 256, 64)
    _check_quant(res, x)
    assert res["workgroups"] == 1 + (128 * 224 + 255) // 256
    assert res["ballots"] > 0


@pytest.mark.parametrize("T,K,E,bm,dtype", [
    (1, 1, 1, 64, np.int32), (3, 5, 7, 64, np.int32), (17, 3, 64, 64, np.int64), (33, 2, 65, 256, np.int32),
    (512, 8, 1024, 64, np.int64), (1024, 8, 384, 64, np.int32), (100, 6, 160, 320, np.int32)])
def test_dispatch_shapes(prep, T, K, E, bm, dtype):
    """Ragged slot counts (quarters not a multiple of 64, the last quarters empty), E not a multiple of
    64, the largest E and slot count, both id types."""
    rng = np.random.default_rng(T * 1000 + E)
    ids = _topk_ids(T, K, E, rng, dtype)
    res = prep(ids, E, bm, None)
    _check_dispatch(res, ids, E, bm)
    assert res["workgroups"] == 1


def test_dispatch_skewed_and_invalid(prep):
    """Every slot on one expert (ranks up to the slot limit) and invalid ids (negative, == E, beyond
    the int32 range for int64 ids): mapping -1, no row, the error flag set."""
    E = 300
    ids = np.full(MAX_SLOTS, 299, dtype=np.int32)
    _check_dispatch(prep(ids, E, 64, None), ids, E, 64)
    rng = np.random.default_rng(5)
    ids = rng.integers(0, E, 4000).astype(np.int64)
    ids[[0, 63, 64, 1999, 3999]] = [-1, E, 1 << 40, -(1 << 40), E + 7]
    res = prep(ids, E, 64, None)
    _check_dispatch(res, ids, E, 64)
    assert res["error"] == 1 and (res["mapping"][[0, 63, 64, 1999, 3999]] == -1).all()


@pytest.mark.parametrize("flags", [0, 1, 4, 16, 2 | 8])
def test_optional_outputs(prep, flags):
    """Outputs passed as null are not written; the mapping always is."""
    rng = np.random.default_rng(flags)
    ids = _topk_ids(64, 8, 96, rng)
    res = prep(ids, 96, 64, None, flags=flags)
    _check_dispatch(res, ids, 96, 64, flags)
    fill32 = np.int32(-101058055)  # 0xf9f9f9f9
    if not flags & 1:
        assert (res["counts"] == fill32).all()
    if not flags & 4:
        assert (res["gather"] == fill32).all()
    if not flags & 16:
        assert (res["tile_prefix"] == fill32).all()


def test_refused_sizes(prep):
    """Dispatches beyond the one-launch limits are refused (the forward then takes the three-launch
    dispatch)."""
    rng = np.random.default_rng(1)
    assert prep(rng.integers(0, 8, MAX_SLOTS + 1).astype(np.int32), 8, 64, None) is None
    assert prep(rng.integers(0, 8, 64).astype(np.int32), MAX_EXPERTS + 1, 64, None) is None


@pytest.mark.parametrize("mutation", [1, 2, 3])
def test_mutations_detected(prep, mutation):
    """1: ballots drop lane 0; 2: shuffles read one lane too far; 3: e4m3 rounding truncates."""
    rng = np.random.default_rng(2)
    ids = _topk_ids(128, 8, 256, rng)
    x = _bf16_rows(8, 256, rng)
    res = prep(ids, 256, 64, x.view(torch.int16).numpy().view(np.uint16), mutation=mutation)
    with pytest.raises(AssertionError):
        _check_dispatch(res, ids, 256, 64)
        _check_quant(res, x)


@pytest.mark.parametrize("seed", range(12))
def test_random_dispatches(prep, seed):
    """Seeded random shapes inside the limits: any slot count and expert count, both id types, skewed
    routing (a few hot experts), a sprinkle of invalid ids, any tile height."""
    rng = np.random.default_rng(100 + seed)
    E = int(rng.integers(1, MAX_EXPERTS + 1))
    slots = int(rng.integers(1, MAX_SLOTS + 1))
    dtype = np.int64 if seed % 2 else np.int32
    if seed % 3 == 0:  # hot experts
        hot = rng.integers(0, E, 3)
        ids = np.where(rng.random(slots) < 0.7, hot[rng.integers(0, 3, slots)], rng.integers(0, E, slots))
    else:
        ids = rng.integers(0, E, slots)
    ids = ids.astype(dtype)
    if seed % 4 == 1:
        bad = rng.choice(slots, max(1, slots // 500), replace=False)
        ids[bad] = E if dtype == np.int32 else (1 << 33)
    bm = int(rng.choice([1, 64, 256, 320]))
    _check_dispatch(prep(ids, E, bm, None), ids, E, bm)
