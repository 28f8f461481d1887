"""Parrot XL with an MI355X (gfx950) HIP inference path for its MoE layers."""
from .model import GenerationState, ModelConfig, ModelOutput, Parrot

__all__ = ["GenerationState", "ModelConfig", "ModelOutput", "Parrot"]
