"""Explicit GRBeam model adapters, separate from kernels and beam selection."""

from .qwen3_5 import Qwen35GRBeamAdapter, Qwen35Prefix, native_model
from .reference import ReferenceHybridLM

__all__ = ["ReferenceHybridLM", "Qwen35GRBeamAdapter", "Qwen35Prefix", "native_model"]
