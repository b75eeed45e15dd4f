"""MI355X-native (gfx950) reversible-training hot path.

Public surface mirrors src/reversibility/__init__.py: ``BaselineLM``,
``ModelConfig``, ``ReversibleLM``, ``build_model``.  The fused operators live in
``kernels`` (FusedSwiGLU, enable_swiglu), ``kernels_v3`` (FusedRMSNorm,
enable_rmsnorm) and ``optimized`` / ``optimized_v3`` (ReusedMidpoint,
SplitMidpoint, TiledMLP, install_v3); the HIP kernels behind them are reached
through the C ABI in include/reversibility_hip.h (``_hip``).
"""
from .model import BaselineLM, ModelConfig
from .reversible import ReversibleLM, build_model

__all__ = ["BaselineLM", "ModelConfig", "ReversibleLM", "build_model"]
