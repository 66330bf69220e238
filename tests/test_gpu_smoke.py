"""The round-end smoke entry point (__graft_entry__.smoke) runs green on the GPU: one small MegaGate ->
MegaMoE forward, routing bit-exact against the C oracle and the expert output against the fp32 one."""
import pytest

import __graft_entry__

pytestmark = pytest.mark.gpu


def test_smoke_entry_point(gpu):
    __graft_entry__.smoke()
