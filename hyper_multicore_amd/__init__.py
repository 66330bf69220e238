"""MI355X (gfx950) MegaGate -> MegaMoE forward path, expert-parallel degree 1.

Drop-in for the single-GPU case of hyper_multicore's public modules
(hyper_multicore/__init__.py:31-63): ``MegaGate``, ``MegaMoeExperts``,
``MegaMoeNumericsOptions``; functional operators live in :mod:`hyper_multicore_amd.ops` and are
registered as ``torch.ops.hyper_multicore_mi355.*`` (:mod:`hyper_multicore_amd.torch_ops`).
The compute path is the C-ABI HIP library ``_lib/libmi355moe.so`` (``include/mi355moe.h``).
"""
from .mega_gate import MegaGate
from .mega_moe import MegaMoeExperts, MegaMoeNumericsOptions, MegaMoeSchedulerOptions, MegaMoeTuningOptions
from .mxfp8 import quantize_expert_weight
from . import torch_ops  # noqa: F401  (registers torch.ops.hyper_multicore_mi355)

__all__ = ["MegaGate", "MegaMoeExperts", "MegaMoeNumericsOptions", "MegaMoeSchedulerOptions",
           "MegaMoeTuningOptions", "quantize_expert_weight"]
