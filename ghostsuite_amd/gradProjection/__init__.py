"""GradProjLoRA: per-sample gradients projected with a per-layer Kronecker sketch
P_o (.) P_i, computed in backward hooks by the gfx950 projection kernel."""
from .gradproj_engine import GradProjLoraEngine, GradProjLoRAEngine, create_gradproj_engine

__all__ = ["GradProjLoraEngine", "GradProjLoRAEngine", "create_gradproj_engine"]
