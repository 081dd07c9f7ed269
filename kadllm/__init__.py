"""The reference's import name for the MI355X GRBeam path.

``import kadllm`` gives the public API of src/kadllm/__init__.py:3-18 for
GRBeam -- ``grbeam_search``, ``GRBeamAdapter``, ``PrefillResult``,
``GRBeamResult``, the operators and ``kadllm.adapters`` /
``kadllm.ops`` / ``kadllm.grbeam`` -- backed by ``kadllm_amd`` (HIP kernels
in libkadllm_hip.so).  WideTuning (``GatedMLPSpec``, ``WideTuningMLP``,
``install_widetuning``) is a training-time product outside this path and is
not provided.
"""

from kadllm_amd import (Constraint, GRBeamAdapter, GRBeamResult, PrefillResult,
                        causal_conv1d, conditional_search, gated_delta, grbeam_search,
                        merge_attention, prefix_attention)

from . import adapters, grbeam, ops  # noqa: E402  (the reference's submodules)

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
