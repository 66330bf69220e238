"""Pin the MXFP8 branch of the expert-forward oracle (CPU only).

The closed form below is built without the oracle's MX code: e4m3fn values come from decoding the
format's bit fields, the shared exponent from a search for the smallest power of two with
amax <= 448 * 2^e (scale algorithm 1 of dual_axis_mxfp8_worker.h:44), elements from a nearest-value
search over the 127 finite positive codes with ties to the even code. The inputs are chosen so that
every fp64 matmul below is exact in fp32 (integer operands times powers of two, and a W2 with one
non-zero per output column), so the oracle's fp32 accumulation must reproduce it bit for bit.

Rounding points (fp32_expert_reference.py:22-26 and mxfp8/graph.py:140-146): x quantised per 32
along H; U = bf16(xq @ W1q); act = silu(g) * u in fp32 with g the left half; act quantised per 32
along I; y = bf16(actq @ W2q). Mutation checks: skipping the SwiGLU re-quantisation, quantising act
or x along the token axis, or dropping U's bf16 rounding each changes the closed form's output, so an
oracle with any of those mistakes fails the equality.
"""
import numpy as np
import torch

from oracle import moe_oracle as orc


def _e4m3_positive() -> np.ndarray:
    """Values of the e4m3fn codes 0..126 from their bit fields (exponent bias 7, subnormals at
    exponent field 0; 127 is NaN)."""
    vals = []
    for c in range(127):
        ef, m = (c >> 3) & 0xF, c & 7
        vals.append(m / 8 * 2.0 ** -6 if ef == 0 else (1 + m / 8) * 2.0 ** (ef - 7))
    return np.array(vals, np.float64)


_TABLE = _e4m3_positive()


def _shared_exp(amax: float) -> int:
    if amax == 0.0:
        return -127
    e = -127
    while amax > 448.0 * 2.0 ** e:
        e += 1
    return min(e, 127)


def _quant_block(v: np.ndarray) -> np.ndarray:
    """Dequantised values of one 32-element block."""
    e = _shared_exp(float(np.abs(v).max()))
    t = np.abs(v) / 2.0 ** e
    d = np.abs(t[:, None] - _TABLE[None, :])
    best = d.min(axis=1, keepdims=True)
    cand = d == best
    # ties: the even code (the lowest of at most two candidates that is even)
    codes = np.where(cand & (np.arange(127)[None, :] % 2 == 0), np.arange(127)[None, :], 999).min(axis=1)
    single = cand.sum(axis=1) == 1
    codes = np.where(single, cand.argmax(axis=1), codes)
    return np.sign(v) * _TABLE[codes] * 2.0 ** e


def _mx_roundtrip(a: np.ndarray, axis: int) -> np.ndarray:
    a = np.moveaxis(np.asarray(a, np.float64), axis, -1)
    out = np.empty_like(a)
    for idx in np.ndindex(*a.shape[:-1]):
        for b in range(0, a.shape[-1], 32):
            out[idx + (slice(b, b + 32),)] = _quant_block(a[idx + (slice(b, b + 32),)])
    return np.moveaxis(out, -1, axis)


def _bf16(a: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.asarray(a, np.float32)).bfloat16().double().numpy()


def _inputs(seed=5, T=64, H=64, I=64):
    g = torch.Generator().manual_seed(seed)
    x = torch.randint(-15, 16, (T, H), generator=g).double()
    x[0] *= 2.0 ** 10                       # one token far above the others (shifts token-axis scales)
    x[3, :32] *= 2.0 ** -12                 # a block far below the rest
    w1 = torch.randint(-7, 8, (H, 2 * I), generator=g).double() * 2.0 ** -5
    w2 = torch.zeros(I, H, dtype=torch.float64)
    pick = torch.randperm(I, generator=g)
    pick = torch.cat([pick, torch.randint(0, I, (H - I,), generator=g)])[:H]
    w2[pick, torch.arange(H)] = torch.randint(1, 4, (H,), generator=g).double() * 2.0 ** -2
    return x.numpy(), w1.numpy(), w2.numpy()


def _closed_form(x, w1, w2, *, requant=True, act_axis=1, x_axis=1, round_u=True):
    I = w1.shape[1] // 2
    xq = _mx_roundtrip(x, x_axis)
    w1q, w2q = _mx_roundtrip(w1, 0), _mx_roundtrip(w2, 0)
    u = xq @ w1q
    assert np.array_equal(u.astype(np.float32).astype(np.float64), u)  # exact in fp32
    if round_u:
        u = _bf16(u)
    else:
        u = u.astype(np.float32).astype(np.float64)
    g, up = u[:, :I], u[:, I:]
    with np.errstate(over="ignore"):
        act = (g / (1.0 + np.exp(-g)) * up).astype(np.float32).astype(np.float64)
    if requant:
        act = _mx_roundtrip(act, act_axis)
    y = act @ w2q  # one non-zero per output column: a single product, exact
    return _bf16(y)


def _oracle(x, w1, w2):
    T = x.shape[0]
    xb = torch.from_numpy(x).to(torch.bfloat16)
    assert torch.equal(xb.double(), torch.from_numpy(x))  # the inputs are exact in bf16
    d1, s1 = orc.mx_quantize_weight_cols(torch.from_numpy(w1).to(torch.bfloat16).unsqueeze(0))
    d2, s2 = orc.mx_quantize_weight_cols(torch.from_numpy(w2).to(torch.bfloat16).unsqueeze(0))
    ids = torch.zeros(T, 1, dtype=torch.int64)
    full = orc.expert_forward_reference(xb, ids, torch.ones(T, 1), d1, d2, precision="mxfp8", w1_scale=s1,
                                        w2_scale=s2)
    W1 = orc.mx_dequantize_weight_cols(d1, s1)
    W2 = orc.mx_dequantize_weight_cols(d2, s2)
    tok = orc.expert_forward_reference_tokens(xb, ids, torch.ones(T, 1), torch.arange(T),
                                              lambda e: (W1[e], W2[e]), precision="mxfp8")
    return full.double().numpy(), tok.double().numpy()


def test_independent_quantiser_matches_oracle_quantiser():
    """The brute-force block quantiser above and the oracle's mx_quantize agree on wide-range data,
    along both axes (subnormal elements, zero blocks and both sides of the 1.75 mantissa boundary)."""
    g = torch.Generator().manual_seed(12)
    a = torch.randn(64, 96, generator=g) * torch.logspace(-6, 6, 64).unsqueeze(1)
    a[5] = 0.0
    a[7, :32] = torch.tensor([1.75 * 2 ** 9] + [1e-3] * 31)
    a[9, :32] = torch.tensor([1.8 * 2 ** -3] + [-2 ** -20] * 31)
    a = a.float()
    for axis in (0, 1):
        q, c = orc.mx_quantize(a, dim=axis)
        ours = _mx_roundtrip(a.numpy(), axis)
        assert np.array_equal(orc.mx_dequantize(q, c, dim=axis).double().numpy(), ours), axis


def test_mxfp8_expert_reference_single_expert_closed_form():
    x, w1, w2 = _inputs()
    want = _closed_form(x, w1, w2)
    full, tok = _oracle(x, w1, w2)
    assert np.array_equal(full, want)
    assert np.array_equal(tok, want)


def test_mxfp8_closed_form_detects_plausible_mistakes():
    """Each plausible mistake in the MX branch changes the output of these inputs."""
    x, w1, w2 = _inputs()
    want = _closed_form(x, w1, w2)
    for mutation in (dict(requant=False), dict(act_axis=0), dict(x_axis=0), dict(round_u=False)):
        assert not np.array_equal(_closed_form(x, w1, w2, **mutation), want), mutation


def test_mxfp8_closed_form_second_seed():
    x, w1, w2 = _inputs(seed=9)
    full, tok = _oracle(x, w1, w2)
    assert np.array_equal(full, _closed_form(x, w1, w2))
