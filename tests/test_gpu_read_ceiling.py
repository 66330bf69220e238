"""The read-bandwidth ceiling for loads issued from the CUs (tests/native/read_ceiling.hip): every
configuration runs, reads the whole buffer once and stays below the HBM3E peak of 8 TB/s; the
best rate is the ceiling that the expert GEMMs' HBM fractions are read against."""
import pytest

pytestmark = pytest.mark.gpu


@pytest.mark.skip(reason="its first GPU run was part of a command that left the GPU faulted; the fault's cause "
                         "is not identified, so this measurement kernel stays off the GPU")
def test_read_ceiling_sweep(gpu):
    from tests.native import read_ceiling
    res = read_ceiling.sweep(gib=4.0, reps=10)
    best = max(res, key=lambda r: r["GBps"])
    print(f"[read_ceiling] best: {best['config']} {best['GBps']} GB/s = {best['GBps'] / 8000:.3f} of 8 TB/s",
          flush=True)
    for r in res:
        assert 0 < r["GBps"] < 8000 * 1.02, r
