"""jacq_amd -- MI355X (gfx950) implementation of Jacq's int4-KIVI paged
KV-cache hot path: the cache writer and paged decode attention, behind the
reference's callable C launch contract (include/jacq_kivi.h).

The native library is ``jacq_amd/libjacq_kivi.so`` (``python -m jacq_amd.build``).
``jacq_amd.kivi`` binds it; there is no CPU fallback.  ``jacq_amd.torch_ops``
loads the torch custom ops built over it (``libjacq_kivi_torch.so``).
"""
from jacq_amd import abi, geometry  # noqa: F401

__all__ = ["abi", "geometry", "kivi", "cache_io", "torch_ops", "workloads"]
