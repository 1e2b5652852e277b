"""Versioned callable kernel ABI of the KIVI lane (restates
integrations/vllm_kivi/abi.py:29-201 for the MI355X build).

Fails closed: an unsupported GPU architecture, model geometry or sequence
length raises ``UnsupportedAbiError`` naming the violated boundary.  The v1
surface (``JACQ_KIVI_ABI_VERSION = 1``, 4096-token cap, 40/8/128 geometry)
is the reference's, unchanged; the runtime-geometry surface
(``JACQ_KIVI_EXT_VERSION``) lifts the geometry and the sequence cap.
"""
from __future__ import annotations

from jacq_amd.bindings import KiviDecodeBindingAbi, default_qwen32b_binding_abi
from jacq_amd.layout import KiviModelGeometry


class UnsupportedAbiError(Exception):
    """Raised when a request or environment violates a hard ABI boundary."""


JACQ_KIVI_ABI_VERSION = 1   # abi.py:36 -- the reference launch contract
JACQ_KIVI_EXT_VERSION = 1   # additive jacq_kivi_* runtime-geometry surface

# The one validated architecture: MI355X (CDNA4).  abi.py:45 lists sm_80/sm_89.
SUPPORTED_GPU_ARCHES = ("gfx950",)

OLD_BLOCKS_CAP = 124
BLOCK_SIZE = 32
RESIDUAL_TOKENS = 128
MAX_SEQ_LEN = OLD_BLOCKS_CAP * BLOCK_SIZE + RESIDUAL_TOKENS  # 4096

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


def supported_geometry() -> KiviModelGeometry:
    return KiviModelGeometry.qwen25_coder_32b()


def check_gpu_arch(arch: str) -> None:
    """Fail closed on architectures outside the validated set.  ``arch`` is
    e.g. ``torch.cuda.get_device_properties(0).gcnArchName``; feature suffixes
    (``gfx950:sramecc+:xnack-``) are ignored."""
    base = arch.split(":", 1)[0]
    if base not in SUPPORTED_GPU_ARCHES:
        raise UnsupportedAbiError(
            f"GPU arch {arch} is outside the validated set {SUPPORTED_GPU_ARCHES} (MI355X). "
            "Refusing to run.")


def check_geometry(geometry: KiviModelGeometry) -> None:
    """v1 lane: only the 40/8/128 geometry (abi.py:186-197)."""
    expected = supported_geometry()
    for attr in ("num_attention_heads", "num_kv_heads", "head_dim"):
        got, want = getattr(geometry, attr), getattr(expected, attr)
        if got != want:
            raise UnsupportedAbiError(
                f"model geometry {attr}={got} does not match the supported lane "
                f"({expected.name}: {attr}={want}); fail closed.")


def _checked_binding(seq_len: int) -> KiviDecodeBindingAbi:
    if seq_len > MAX_SEQ_LEN:
        raise UnsupportedAbiError(
            f"seq_len {seq_len} exceeds the KIVI ABI v1 cap of {MAX_SEQ_LEN} "
            f"({OLD_BLOCKS_CAP} old pages x {BLOCK_SIZE} tokens + {RESIDUAL_TOKENS}-token "
            "residual). Use the runtime-geometry jacq_kivi_* surface for longer contexts.")
    return default_qwen32b_binding_abi(seq_len=seq_len)


def kernel_interface(seq_len: int = MAX_SEQ_LEN) -> dict:
    """The versioned callable surface for one decode step (abi.py:74-112)."""
    abi = _checked_binding(seq_len)
    return {
        "abi_version": JACQ_KIVI_ABI_VERSION,
        "ext_version": JACQ_KIVI_EXT_VERSION,
        "supported_gpu_arches": list(SUPPORTED_GPU_ARCHES),
        "required_ops": list(REQUIRED_OPS),
        "cache_write_kernels": list(CACHE_WRITE_KERNELS),
        "seq_len": abi.seq_len,
        "old_pages": abi.old_pages,
        "symbols": {"v1": list(V1_SYMBOLS), "ext": list(EXT_SYMBOLS)},
        "kernels": [
            {"op": "kivi_decode_dsl", "symbol": "jac_launch",
             "launch_order": abi.jac_launch_order()},
            {"op": "kivi_cache_write_jac_dsl", "symbol": "jac_launch_cache_write",
             "launch_order": ["K_CODE_PAGES", "K_SCALE_PAGES", "K_ZERO_PAGES", "V_CODE_PAGES",
                              "V_SCALE_PAGES", "V_ZERO_PAGES", "K_RESIDUAL_SCRATCH",
                              "V_RESIDUAL_SCRATCH", "NEW_K", "NEW_V", "BLOCK_TABLE", "SEQ_LEN",
                              "hipStream_t stream"]},
        ],
        "integrity_boundary": (
            "This describes the callable surface only; it allocates nothing and launches "
            "nothing. Numerical parity is established by the GPU tests against the CPU oracle."),
    }
