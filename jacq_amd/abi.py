"""Versioned callable kernel ABI of the KIVI lane (restates
integrations/vllm_kivi/abi.py:29-201 for the MI355X build).

Fails closed: an unsupported GPU architecture, model geometry or sequence
length raises ``UnsupportedAbiError`` naming the violated boundary.  The v1
surface (``JACQ_KIVI_ABI_VERSION = 1``, 4096-token cap, 40/8/128 geometry)
is the reference's, unchanged; the runtime-geometry surface
(``JACQ_KIVI_EXT_VERSION``) lifts the geometry and the sequence cap.
"""
from __future__ import annotations

from jacq_amd import geometry as geo


class UnsupportedAbiError(Exception):
    """A GPU, geometry or length outside what this build's v1 surface serves;
    the message names the limit that was crossed."""


JACQ_KIVI_ABI_VERSION = 1   # abi.py:36 -- the reference launch contract
JACQ_KIVI_EXT_VERSION = 1   # additive jacq_kivi_* runtime-geometry surface

# The one validated architecture: MI355X (CDNA4).  abi.py:45 lists sm_80/sm_89.
SUPPORTED_GPU_ARCHES = ("gfx950",)

OLD_BLOCKS_CAP = geo.V1.max_pages_per_seq
BLOCK_SIZE = geo.V1.page_size
RESIDUAL_TOKENS = geo.V1.residual
MAX_SEQ_LEN = geo.V1_MAX_SEQ_LEN  # 4096

# C symbols a caller binds (include/jacq_kivi.h); abi.py:58-62 lists the
# torch ops that wrap them.
V1_SYMBOLS = (
    "jac_launch", "jac_launch_tp2_local", "jac_launch_batched", "jac_launch_batched_tp2_local",
    "jac_launch_cache_write", "jac_launch_cache_write_batched",
    "kivi_cache_write_launch", "kivi_cache_write_batched_launch",
)
EXT_SYMBOLS = (
    "jacq_kivi_abi_version", "jacq_kivi_ext_version", "jacq_kivi_last_error",
    "jacq_kivi_check_geometry", "jacq_kivi_max_seq_len", "jacq_kivi_check_block_table_width",
    "jacq_kivi_decode_workspace_size", "jacq_kivi_decode", "jacq_kivi_cache_append",
    "jacq_kivi_plan_batched_write",
)
REQUIRED_OPS = ("kivi_cache_write_dsl", "kivi_cache_write_jac_dsl", "kivi_decode_dsl")
CACHE_WRITE_KERNELS = ("hand_cuda", "jac_dsl")  # selector values kept for drop-in callers


def supported_geometry() -> geo.LaneGeometry:
    return geo.V1


def check_gpu_arch(arch: str) -> None:
    """Fail closed on architectures outside the validated set.  ``arch`` is
    e.g. ``torch.cuda.get_device_properties(0).gcnArchName``; feature suffixes
    (``gfx950:sramecc+:xnack-``) are ignored."""
    base = arch.split(":", 1)[0]
    if base not in SUPPORTED_GPU_ARCHES:
        raise UnsupportedAbiError(
            f"GPU arch {arch} is outside the validated set {SUPPORTED_GPU_ARCHES} (MI355X). "
            "Refusing to run.")


def check_geometry(g: geo.LaneGeometry) -> None:
    """v1 lane: only the 40/8/128 head geometry (abi.py:186-197)."""
    for attr in ("num_heads", "num_kv_heads", "head_dim"):
        got, want = getattr(g, attr), getattr(geo.V1, attr)
        if got != want:
            raise UnsupportedAbiError(
                f"{attr}={got}: the v1 symbols are built for {want} (40 query / 8 kv heads, "
                "head_dim 128); use the jacq_kivi_* runtime-geometry entry points")


def _check_seq_len(seq_len: int) -> None:
    if seq_len > MAX_SEQ_LEN:
        raise UnsupportedAbiError(
            f"seq_len {seq_len} is beyond the v1 limit of {MAX_SEQ_LEN} tokens "
            f"({OLD_BLOCKS_CAP} table entries x {BLOCK_SIZE} + {RESIDUAL_TOKENS} fp16 tokens); "
            "the jacq_kivi_* entry points take wider block tables")


WRITE_ORDER = ("K_CODE_PAGES", "K_SCALE_PAGES", "K_ZERO_PAGES", "V_CODE_PAGES", "V_SCALE_PAGES",
               "V_ZERO_PAGES", "K_RESIDUAL_SCRATCH", "V_RESIDUAL_SCRATCH", "NEW_K", "NEW_V",
               "BLOCK_TABLE", "SEQ_LEN", "hipStream_t stream")


def kernel_interface(seq_len: int = MAX_SEQ_LEN) -> dict:
    """The versioned callable surface for one decode step (abi.py:74-112)."""
    _check_seq_len(seq_len)
    return {
        "abi_version": JACQ_KIVI_ABI_VERSION,
        "ext_version": JACQ_KIVI_EXT_VERSION,
        "supported_gpu_arches": list(SUPPORTED_GPU_ARCHES),
        "required_ops": list(REQUIRED_OPS),
        "cache_write_kernels": list(CACHE_WRITE_KERNELS),
        "seq_len": seq_len,
        "old_pages": geo.V1.old_tokens(seq_len) // geo.V1.page_size,
        "symbols": {"v1": list(V1_SYMBOLS), "ext": list(EXT_SYMBOLS)},
        "kernels": [
            {"op": "kivi_decode_dsl", "symbol": "jac_launch",
             "launch_order": list(geo.JAC_LAUNCH_ORDER)},
            {"op": "kivi_cache_write_jac_dsl", "symbol": "jac_launch_cache_write",
             "launch_order": list(WRITE_ORDER)},
        ],
        "note": "describes the callable surface only; nothing is allocated or launched",
    }
