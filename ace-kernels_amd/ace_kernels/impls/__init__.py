"""Importing this package registers the HIP implementation (``hip_mi355x``)."""

from ace_kernels.impls import hip_mi355x

__all__ = ["hip_mi355x"]
