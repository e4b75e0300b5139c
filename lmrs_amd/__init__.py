"""lmrs_amd -- MI355X-native batched token sampling for lmrs.

The product is the HIP library ``liblmrs_sampling.so`` (C-ABI in
``include/lmrs_sampling.h``); ``lmrs_amd.sampling`` is its Python binding and
the Python mirror of lmrs's ``crates/sampling`` API.
"""
from . import sampling  # noqa: F401

__all__ = ["sampling"]
