"""Index-set comparison of a router's output with the torch form of MegaGate._torch_forward
(module.py:199-227), the way _test_mega_gate.py:336-351 compares them: sorted index sets, exactly.

The router kernel computes its scores with its own exp / log (the C oracle reproduces them bit for
bit); torch's sigmoid / softmax / softplus differ from them by a few ulp, and differ between torch
builds and host CPUs too (vectorised exp). A row whose K-th and (K+1)-th candidates - or, for the
group-limited form, whose last kept and first dropped groups - are closer than those few ulp has no
rounding-independent index set; on every other row the sets must be identical. ``set_mismatches``
returns the rows whose sets differ, split into such near-tie rows and the rest (which a test asserts
to be empty)."""
from __future__ import annotations

import numpy as np
import torch

TIE_ULPS = 16  # score agreement of two correctly implemented exp-based scorings, with margin


def _ulp(x: float) -> float:
    return float(np.spacing(np.float32(abs(x))))


def set_mismatches(ids: torch.Tensor, ids_torch: torch.Tensor, biased: torch.Tensor, num_groups: int = 1,
                   topk_groups: int = 1):
    """Rows whose index sets differ: (near_tie_rows, other_rows). ``biased``: the torch form's biased
    scores [T, E] (scores + correction bias)."""
    a = torch.sort(ids.long(), dim=1).values
    b = torch.sort(ids_torch.long(), dim=1).values
    rows = torch.nonzero((a != b).any(dim=1)).flatten().tolist()
    near, other = [], []
    T, E = biased.shape
    for r in rows:
        sa, sb = set(a[r].tolist()), set(b[r].tolist())
        diff = sorted(sa ^ sb)
        vals = biased[r, diff].double()
        tol = TIE_ULPS * _ulp(float(vals.abs().max()))
        if float(vals.max() - vals.min()) <= tol:
            near.append(r)
            continue
        if num_groups > 1:
            # a flip of the last kept group: the groups' top-2 sums within the tolerance
            gs = biased[r].view(num_groups, -1).double().topk(2, dim=-1).values.sum(dim=-1)
            ga = {e // (E // num_groups) for e in sa}
            gb = {e // (E // num_groups) for e in sb}
            flip = sorted(ga ^ gb)
            if flip:
                gv = gs[flip]
                gtol = TIE_ULPS * _ulp(float(gv.abs().max()))
                if float(gv.max() - gv.min()) <= gtol:
                    near.append(r)
                    continue
        other.append(r)
    return near, other
