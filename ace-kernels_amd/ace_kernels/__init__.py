"""mL1-ACE calibration loss on MI355X (gfx950): the reference's API over HIP kernels.

Same public surface as the reference package (``src/ace_kernels/__init__.py``):
``ACEConfig``, ``ImplSpec``, ``ace_loss``, ``available_impls``, ``get_impl``.
Importing it registers ``hip_mi355x``; its kernels live in ``libace_hip.so``
(built by ``ace-kernels_amd/build.py``), loaded on first use.
"""

from ace_kernels import impls
from ace_kernels.config import ACEConfig
from ace_kernels.registry import ImplSpec, ace_loss, available_impls, get_impl

__all__ = ["ACEConfig", "ImplSpec", "ace_loss", "available_impls", "get_impl", "impls"]
