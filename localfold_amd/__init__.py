"""localfold-mi355x: the AF2 Evoformer / AF3 Pairformer pair-stack hot path on MI355X.

Hand-written gfx950 HIP kernels behind the C ABI of include/localfold.h
(localfold_amd/lib/liblocalfold.so).  `capi` mirrors the ABI in ctypes, `device` drives it
with torch device tensors, `js/` is the Node host that keeps the reference's classes.
"""
from . import capi  # noqa: F401

__all__ = ["capi"]
