"""``kadllm.adapters`` (src/kadllm/adapters/__init__.py) on the HIP path."""

from kadllm_amd.adapters import Qwen35GRBeamAdapter, Qwen35Prefix, ReferenceHybridLM, native_model

from . import qwen3_5, reference  # noqa: E402,F401

__all__ = ["ReferenceHybridLM", "Qwen35GRBeamAdapter", "Qwen35Prefix", "native_model"]
