"""ghostsuite_amd -- GhostSuite's per-sample-gradient engines on MI355X (gfx950).

The public API mirrors the reference package ``ghostEngines``; the arithmetic of every
sampler runs in hand-written HIP kernels behind the C ABI of ``include/ghost_hip.h``
(libghost_hip.so, loaded through ctypes).  A drop-in replacement for code that imports
``ghostEngines`` is ``ghostsuite_amd.install_as_ghostEngines()``.
"""
import torch  # noqa: F401  (loads the HIP runtime that libghost_hip.so binds to)

from .graddotprod_engine import GradDotProdEngine
from .engine_manager import GhostEngineManager
from .gradProjection.gradproj_engine import GradProjLoraEngine, GradProjLoRAEngine

__all__ = ['GradDotProdEngine', 'GhostEngineManager', 'GradProjLoraEngine',
           'GradProjLoRAEngine', 'install_as_ghostEngines']


def install_as_ghostEngines() -> None:
    """Registers this package under the reference's module names (``ghostEngines`` and its
    submodules) so existing imports resolve to the MI355X implementation."""
    import sys
    from . import (autograd_grad_sample_dotprod, engine_manager, graddotprod_engine,
                   supported_layers_grad_samplers_dotprod, transformers_support)
    from .gradProjection import (autograd_gradproj, gradproj_engine, projection_utils,
                                 supported_layers_gradproj)
    from . import gradProjection
    pkg = sys.modules[__name__]
    sys.modules['ghostEngines'] = pkg
    for short, mod in {
        'autograd_grad_sample_dotprod': autograd_grad_sample_dotprod,
        'engine_manager': engine_manager,
        'graddotprod_engine': graddotprod_engine,
        'supported_layers_grad_samplers_dotprod': supported_layers_grad_samplers_dotprod,
        'transformers_support': transformers_support,
        'gradProjection': gradProjection,
        'gradProjection.autograd_gradproj': autograd_gradproj,
        'gradProjection.gradproj_engine': gradproj_engine,
        'gradProjection.projection_utils': projection_utils,
        'gradProjection.supported_layers_gradproj': supported_layers_gradproj,
    }.items():
        sys.modules['ghostEngines.' + short] = mod
