"""MI355X-native GRBeam shared-prefix beam decoding (drop-in for ``kadllm``'s GRBeam API).

Public names follow the reference package (src/kadllm/__init__.py:3-18):
``grbeam_search``, ``GRBeamAdapter``, ``PrefillResult``, ``GRBeamResult``,
the operators ``gated_delta``, ``causal_conv1d``, ``prefix_attention`` and the
adapter ``adapters.Qwen35GRBeamAdapter``; beyond them ``conditional_search``
(coarse levels, then per-coarse-beam quotas).  All numerics run in the HIP
kernels of ``libkadllm_hip.so`` (built by ``python -m kadllm_amd.csrc.build``).
"""

from .grbeam import (Constraint, GRBeamAdapter, GRBeamResult, PrefillResult, conditional_search,
                     grbeam_search)
from .ops import causal_conv1d, gated_delta, merge_attention, prefix_attention

__all__ = [
    "GRBeamResult",
    "PrefillResult",
    "GRBeamAdapter",
    "grbeam_search",
    "conditional_search",
    "Constraint",
    "causal_conv1d",
    "gated_delta",
    "prefix_attention",
    "merge_attention",
]
