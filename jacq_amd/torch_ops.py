"""The torch custom-op binding: ``torch.ops.jacq_kivi.*`` and
``torch.classes.jacq_kivi.ResidualSlots`` from ``libjacq_kivi_torch.so``
(``jacq_amd/csrc/kivi_torch_ops.cpp``, built by ``jacq_amd.build``).

It is the reference's vLLM op surface (integrations/vllm_kivi/
source_patch.py:2797-2870, validators :673-1495) compiled for ROCm: a vLLM
build that registers these ops in its own ``_C`` library would bind the same
C++ functions.  The ops take the same arguments as ``jacq_amd.kivi``'s Python
mirrors and fail with the same texts (as RuntimeError, torch's TORCH_CHECK).

    ops = torch_ops.load()
    ops.kivi_cache_write_dsl(k_code, k_scale, k_zero, v_code, v_scale, v_zero,
                             k_scr, v_scr, new_k, new_v, slot_mapping, table, seq_len)
    ops.kivi_decode_dsl(q, table, k_code, ..., v_scr, seq_len, out)

Every op has a ``<name>_check`` twin that runs the same checks except GPU
residency and the device architecture, on any backend, and launches nothing.
"""
from __future__ import annotations

import os

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
TORCH_LIB = os.path.join(HERE, "libjacq_kivi_torch.so")

OPS = ("kivi_decode_dsl", "kivi_decode_sparse_retained_dsl", "kivi_decode_batched_dsl",
       "kivi_cache_write_dsl", "kivi_cache_write_jac_dsl", "kivi_cache_write_batched_dsl",
       "kivi_cache_write_batched_jac_dsl")

_loaded = False


def load():
    """Load the op library once and return ``torch.ops.jacq_kivi``.  Raises
    when it has not been built (there is no Python fallback)."""
    global _loaded
    if not _loaded:
        from jacq_amd.kivi import NativeLibraryMissing, lib
        if not os.path.exists(TORCH_LIB):
            raise NativeLibraryMissing(
                f"{TORCH_LIB} is not built; run `python -m jacq_amd.build`")
        lib()  # the kernels library it links against, from the same folder
        torch.ops.load_library(TORCH_LIB)
        _loaded = True
    return torch.ops.jacq_kivi


def residual_slots(max_seqs: int):
    """A residual-slot allocator for a decode lane of ``max_seqs`` requests
    (source_patch.py:3047-3098): ``assign(req_ids, finished_req_ids,
    active_req_ids_or_None) -> [slot per request]``."""
    load()
    return torch.classes.jacq_kivi.ResidualSlots(max_seqs)
