"""Host runtime of the KIVI lane: binds libjacq_kivi.so (include/jacq_kivi.h).

Two layers, both calling the native library through its C ABI:

* ``kivi_decode_dsl``, ``kivi_decode_batched_dsl``, ``kivi_cache_write_dsl``,
  ``kivi_cache_write_jac_dsl``, ``kivi_cache_write_batched_dsl`` -- the
  reference's torch-op surface (integrations/vllm_kivi/source_patch.py:768-1495)
  with the same argument meaning and the same fail-closed checks (dtype,
  contiguity, shapes, block-table width, SEQ_LEN range, one device of the
  validated architecture).  They dispatch to the v1 symbols.
* ``KiviGeometry`` / ``PagedKiviCache`` -- the runtime-geometry surface
  (``jacq_kivi_decode`` / ``jacq_kivi_cache_append``) for batches, 16-token
  pages and long contexts.

There is no fallback: if libjacq_kivi.so is missing the import of the native
layer raises ``NativeLibraryMissing``.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

import torch

from jacq_amd import abi as _abi

_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libjacq_kivi.so")

V1_NH, V1_NKV, V1_HD = 40, 8, 128
TP2_LOCAL_NH, TP2_LOCAL_NKV = 20, 4
OLD_BLOCKS, BLOCK_SIZE, RESIDUAL = 124, 32, 128
HD_PACKED, HD_GROUPS = V1_HD // 2, V1_HD // 32
RESIDUAL_SCRATCH = RESIDUAL + BLOCK_SIZE
MAX_QUERIES = 160


class NativeLibraryMissing(ImportError):
    pass


class KiviCheckError(RuntimeError):
    """A fail-closed argument check (the reference raises via TORCH_CHECK)."""


class KiviLaunchError(RuntimeError):
    pass


class KiviMergeTimeout(KiviLaunchError):
    """A split-K merge of an earlier decode timed out (JACQ_KIVI_ETIMEOUT)."""


ETIMEOUT = 4


class Geometry(ctypes.Structure):
    _fields_ = [
        ("num_heads", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("page_size", ctypes.c_int32),
        ("group_size", ctypes.c_int32),
        ("residual", ctypes.c_int32),
        ("max_pages_per_seq", ctypes.c_int32),
        ("num_pages", ctypes.c_int32),
    ]


class Subchunk(ctypes.Structure):
    _fields_ = [
        ("start_seq_len", ctypes.c_int32),
        ("num_new", ctypes.c_int32),
        ("scratch_start", ctypes.c_int32),
        ("age_out_page", ctypes.c_int32),
        ("post_shift_residual_len", ctypes.c_int32),
    ]


_lib: ctypes.CDLL | None = None
_vp = ctypes.c_void_p
_i32 = ctypes.c_int32


def library_path() -> str:
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    """Load libjacq_kivi.so (torch is imported first so both share one HIP
    runtime)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_LIB_PATH):
        raise NativeLibraryMissing(
            f"{_LIB_PATH} is not built; run `python -m jacq_amd.build` (hipcc, gfx950)")
    L = ctypes.CDLL(_LIB_PATH)
    dec10 = [_vp] * 10
    for name in ("jac_launch", "jac_launch_tp2_local"):
        f = getattr(L, name)
        f.argtypes = dec10 + [ctypes.c_int, _vp, _vp]
        f.restype = None
    for name in ("jac_launch_sparse_retained", "jac_launch_sparse_retained_tp2_local"):
        f = getattr(L, name)
        f.argtypes = dec10 + [ctypes.c_int, ctypes.c_int, _vp, _vp]
        f.restype = None
    for name in ("jac_launch_batched", "jac_launch_batched_tp2_local"):
        f = getattr(L, name)
        f.argtypes = [_vp] * 11 + [ctypes.c_int, _vp, _vp]
        f.restype = None
    L.jac_launch_cache_write.argtypes = [_vp] * 11 + [ctypes.c_int, _vp]
    L.jac_launch_cache_write.restype = None
    L.jac_launch_cache_write_batched.argtypes = [_vp] * 11 + [ctypes.c_int, ctypes.c_int, _vp]
    L.jac_launch_cache_write_batched.restype = None
    L.kivi_cache_write_launch.argtypes = [_vp] * 12 + [ctypes.c_int, ctypes.c_int, _vp]
    L.kivi_cache_write_launch.restype = None
    L.kivi_cache_write_batched_launch.argtypes = [_vp] * 12 + [ctypes.c_int] * 3 + [_vp]
    L.kivi_cache_write_batched_launch.restype = None
    L.jacq_kivi_abi_version.restype = ctypes.c_int
    L.jacq_kivi_ext_version.restype = ctypes.c_int
    L.jacq_kivi_last_error.restype = ctypes.c_char_p
    L.jacq_kivi_check_geometry.argtypes = [ctypes.POINTER(Geometry)]
    L.jacq_kivi_check_geometry.restype = ctypes.c_int
    L.jacq_kivi_max_seq_len.argtypes = [ctypes.POINTER(Geometry)]
    L.jacq_kivi_max_seq_len.restype = ctypes.c_int64
    L.jacq_kivi_check_block_table_width.argtypes = [ctypes.POINTER(Geometry), ctypes.c_int64,
                                                    ctypes.c_int64]
    L.jacq_kivi_check_block_table_width.restype = ctypes.c_int
    L.jacq_kivi_decode_workspace_size.argtypes = [ctypes.POINTER(Geometry), _i32]
    L.jacq_kivi_decode_workspace_size.restype = ctypes.c_size_t
    L.jacq_kivi_decode.argtypes = [ctypes.POINTER(Geometry)] + [_vp] * 11 + [
        _i32, _vp, _vp, ctypes.c_size_t, _vp]
    L.jacq_kivi_decode.restype = ctypes.c_int
    L.jacq_kivi_decode_noalloc.argtypes = [ctypes.POINTER(Geometry)] + [_vp] * 11 + [
        _i32, _vp, _vp]
    L.jacq_kivi_decode_noalloc.restype = ctypes.c_int
    L.jacq_kivi_decode_sparse_retained.argtypes = [ctypes.POINTER(Geometry), _vp, _i32, _vp,
                                                   _i32] + [_vp] * 9 + [_vp, ctypes.c_size_t,
                                                                        _vp]
    L.jacq_kivi_decode_sparse_retained.restype = ctypes.c_int
    L.jacq_kivi_cache_append.argtypes = [ctypes.POINTER(Geometry)] + [_vp] * 12 + [
        _i32, _i32, _vp]
    L.jacq_kivi_cache_append.restype = ctypes.c_int
    L.jacq_kivi_plan_batched_write.argtypes = [_i32, _i32, _i32, _i32, ctypes.POINTER(Subchunk),
                                               _i32]
    L.jacq_kivi_plan_batched_write.restype = _i32
    L.jacq_kivi_init.restype = ctypes.c_int
    L.jacq_kivi_decode_status.argtypes = [_vp, ctypes.c_size_t, _vp]
    L.jacq_kivi_decode_status.restype = ctypes.c_int
    L.jacq_kivi_write_decode.argtypes = [ctypes.POINTER(Geometry)] + [_vp] * 13 + [
        _i32, _vp, _vp, ctypes.c_size_t, _vp]
    L.jacq_kivi_write_decode.restype = ctypes.c_int
    L.jacq_kivi_write_decode_workspace_size.argtypes = [ctypes.POINTER(Geometry), _i32]
    L.jacq_kivi_write_decode_workspace_size.restype = ctypes.c_size_t
    L.jacq_kivi_release_workspaces.argtypes = []
    L.jacq_kivi_release_workspaces.restype = ctypes.c_int
    L.jacq_kivi_test_device_allocations.argtypes = []
    L.jacq_kivi_test_device_allocations.restype = ctypes.c_int64
    L.jacq_kivi_test_force_merge_timeout.argtypes = [ctypes.c_uint32]
    L.jacq_kivi_test_force_merge_timeout.restype = None
    L.jacq_kivi_profile_wave_stamps.argtypes = [_vp, _i32]
    L.jacq_kivi_profile_wave_stamps.restype = ctypes.c_int
    L.jacq_kivi_profile_start.argtypes = [_i32, _i32]
    L.jacq_kivi_profile_start.restype = ctypes.c_int
    L.jacq_kivi_profile_stop.argtypes = [ctypes.POINTER(ctypes.c_float),
                                         ctypes.POINTER(ctypes.c_float), _i32]
    L.jacq_kivi_profile_stop.restype = _i32
    L.jacq_kivi_profile_write_ms.argtypes = [ctypes.POINTER(ctypes.c_float), _i32]
    L.jacq_kivi_profile_write_ms.restype = _i32
    _lib = L
    return L


def last_error() -> str:
    return lib().jacq_kivi_last_error().decode()


def decode_status(workspace: torch.Tensor | None = None, device=None) -> None:
    """Raise KiviMergeTimeout (after resetting the workspaces) if a decode's
    split-K merge on the current device timed out since the last query."""
    dev = torch.device("cuda") if device is None else torch.device(device)
    st = lib().jacq_kivi_decode_status(
        _ptr(workspace), 0 if workspace is None else workspace.numel() * workspace.element_size(),
        _stream(dev))
    if st == ETIMEOUT:
        raise KiviMergeTimeout(last_error())
    if st != 0:
        raise KiviLaunchError(last_error())


def profile_start(max_calls: int, split: bool = True) -> None:
    """Record HIP events around the next max_calls decode calls.  With split,
    the matrix-core decode (one kernel) is launched with start / stop events
    stamped at the kernel's own start and end; the VALU decode records an event
    between its kernel and its merge."""
    if lib().jacq_kivi_profile_start(max_calls, int(split)) != 0:
        raise KiviLaunchError(last_error())


def profile_stop(cap: int = 4096):
    """(kernel ms, ms after the kernel until the decode's end event) per
    recorded decode call, in call order."""
    k = (ctypes.c_float * cap)()
    m = (ctypes.c_float * cap)()
    n = lib().jacq_kivi_profile_stop(k, m, cap)
    if n < 0:
        raise KiviLaunchError(last_error())
    return list(k[:n]), list(m[:n])


def profile_write_ms(cap: int = 4096):
    """Cache-write kernel ms per call recorded in the last profiling window."""
    w = (ctypes.c_float * cap)()
    n = lib().jacq_kivi_profile_write_ms(w, cap)
    if n < 0:
        raise KiviLaunchError(last_error())
    return list(w[:n])


def _raise(rc: int) -> None:
    if rc == ETIMEOUT:
        raise KiviMergeTimeout(last_error())
    raise KiviLaunchError(last_error())


def _ptr(t: torch.Tensor | None):
    return _vp(0 if t is None else t.data_ptr())


def _stream(device: torch.device):
    return _vp(torch.cuda.current_stream(device).cuda_stream)


# ---------------------------------------------------------------------------
# fail-closed checks (source_patch.py:673-742)
# ---------------------------------------------------------------------------

def _check(cond: bool, *msg) -> None:
    if not cond:
        raise KiviCheckError("".join(str(m) for m in msg))


def check_cuda_tensor(t: torch.Tensor, name: str) -> None:
    _check(t.is_cuda, name, " must be a CUDA tensor")
    _check(t.is_contiguous(), name, " must be contiguous for jac_launch")


def check_shape(t: torch.Tensor, expected, name: str) -> None:
    _check(t.dim() == len(expected), name, " rank mismatch for the KIVI DSL ABI")
    for axis, want in enumerate(expected):
        _check(t.size(axis) == want, name, " dim ", axis, " must be ", want,
               " for the KIVI DSL ABI, got ", t.size(axis))


def check_block_table_width(t: torch.Tensor, name: str, seq_len: int) -> None:
    """source_patch.py:692-707: 0 pages through seq_len=159, 1 at 160, 124 at 4096."""
    _check(t.dim() == 1, name, " rank mismatch for the KIVI DSL ABI")
    _check(1 <= seq_len <= OLD_BLOCKS * BLOCK_SIZE + RESIDUAL,
           "SEQ_LEN must be in [1, 4096] for KIVI BLOCK_TABLE validation")
    required = (seq_len - RESIDUAL) // BLOCK_SIZE if seq_len > RESIDUAL else 0
    _check(t.size(0) >= required, name, " dim 0 must be at least ", required,
           " for the KIVI DSL ABI, got ", t.size(0))


def check_launch_device(tensors, op_name: str) -> None:
    """source_patch.py:719-742: one device, of the validated architecture."""
    _check(len(tensors) > 0, op_name, " requires at least one tensor")
    device = tensors[0].device
    _check(device.type == "cuda", op_name, " tensors must be bound to a GPU device, got ", device)
    for t in tensors:
        _check(t.device == device, op_name, " tensors must all live on one GPU device; got ",
               t.device, " alongside ", device)
    arch = torch.cuda.get_device_properties(device).gcnArchName
    try:
        _abi.check_gpu_arch(arch)
    except _abi.UnsupportedAbiError as e:
        raise KiviCheckError(f"{op_name}: {e}") from None


def _validated(op: str, named, *args) -> None:
    """The op's checks before a launch: GPU residency and contiguity of the
    named tensors, then the op's fail-closed table -- run by the torch op's
    ``<op>_check`` twin (csrc/kivi_torch_ops.cpp, the one copy of the table:
    ranks, dtypes, shapes, geometry, lengths, table widths), its RuntimeError
    raised as KiviCheckError -- then one device of the validated
    architecture."""
    from jacq_amd import torch_ops
    for t, n in named:
        check_cuda_tensor(t, n)
    try:
        getattr(torch_ops.load(), op + "_check")(*args)
    except RuntimeError as e:
        raise KiviCheckError(str(e).splitlines()[0]) from None
    check_launch_device([t for t, _ in named], op)


POOL_NAMES = ("K_CODE_PAGES", "K_SCALE_PAGES", "K_ZERO_PAGES", "V_CODE_PAGES", "V_SCALE_PAGES",
              "V_ZERO_PAGES", "K_RESIDUAL_SCRATCH", "V_RESIDUAL_SCRATCH")


# ---------------------------------------------------------------------------
# reference op surface (source_patch.py:768-1495) -> v1 symbols
# ---------------------------------------------------------------------------

def kivi_decode_dsl(q, block_table, k_code_pages, k_scale_pages, k_zero_pages, v_code_pages,
                    v_scale_pages, v_zero_pages, k_residual_scratch, v_residual_scratch,
                    seq_len: int, out) -> None:
    """source_patch.py:768-869."""
    pool = (k_code_pages, k_scale_pages, k_zero_pages, v_code_pages, v_scale_pages, v_zero_pages,
            k_residual_scratch, v_residual_scratch)
    _validated("kivi_decode_dsl",
               [(q, "Q"), (block_table, "BLOCK_TABLE"), *zip(pool, POOL_NAMES), (out, "O")],
               q, block_table, *pool, int(seq_len), out)
    fn = lib().jac_launch_tp2_local if q.size(0) == TP2_LOCAL_NH else lib().jac_launch
    fn(_ptr(q), _ptr(block_table), *[_ptr(t) for t in pool], int(seq_len), _ptr(out),
       _stream(q.device))


def kivi_decode_sparse_retained_dsl(q, retained_block_table, k_code_pages, k_scale_pages,
                                    k_zero_pages, v_code_pages, v_scale_pages, v_zero_pages,
                                    k_residual_scratch, v_residual_scratch, seq_len: int,
                                    num_retained_pages: int, out) -> None:
    """source_patch.py:872-971: decode over the first NUM_RETAINED_PAGES
    entries of a compact retained-page table, residual at the dense SEQ_LEN."""
    pool = (k_code_pages, k_scale_pages, k_zero_pages, v_code_pages, v_scale_pages, v_zero_pages,
            k_residual_scratch, v_residual_scratch)
    _validated("kivi_decode_sparse_retained_dsl",
               [(q, "Q"), (retained_block_table, "RETAINED_BLOCK_TABLE"),
                *zip(pool, POOL_NAMES), (out, "O")],
               q, retained_block_table, *pool, int(seq_len), int(num_retained_pages), out)
    fn = (lib().jac_launch_sparse_retained_tp2_local if q.size(0) == TP2_LOCAL_NH
          else lib().jac_launch_sparse_retained)
    fn(_ptr(q), _ptr(retained_block_table), *[_ptr(t) for t in pool], int(seq_len),
       int(num_retained_pages), _ptr(out), _stream(q.device))


def kivi_decode_batched_dsl(q, seq_lens, block_table, k_code_pages, k_scale_pages, k_zero_pages,
                            v_code_pages, v_scale_pages, v_zero_pages, k_residual_scratch,
                            v_residual_scratch, num_queries: int, out) -> None:
    """source_patch.py:1268-1386 (one sequence, up to 160 causal queries)."""
    pool = (k_code_pages, k_scale_pages, k_zero_pages, v_code_pages, v_scale_pages, v_zero_pages,
            k_residual_scratch, v_residual_scratch)
    _validated("kivi_decode_batched_dsl",
               [(q, "Q"), (seq_lens, "SEQ_LENS"), (block_table, "BLOCK_TABLE"),
                *[(t, "KIVI cache tensor") for t in pool], (out, "O")],
               q, seq_lens, block_table, *pool, int(num_queries), out)
    fn = lib().jac_launch_batched_tp2_local if q.size(1) == TP2_LOCAL_NH else lib().jac_launch_batched
    fn(_ptr(q), _ptr(seq_lens), _ptr(block_table), *[_ptr(t) for t in pool], int(num_queries),
       _ptr(out), _stream(q.device))


def _writer_named(pool, new_k, new_v, slot_mapping, block_table):
    return [*[(t, "KIVI cache tensor") for t in pool], (new_k, "NEW_K"), (new_v, "NEW_V"),
            (slot_mapping, "SLOT_MAPPING"), (block_table, "BLOCK_TABLE")]


def kivi_cache_write_dsl(k_code_pages, k_scale_pages, k_zero_pages, v_code_pages, v_scale_pages,
                         v_zero_pages, k_residual_scratch, v_residual_scratch, new_k, new_v,
                         slot_mapping, block_table, seq_len: int) -> None:
    """source_patch.py:975-1078 -> kivi_cache_write_launch."""
    pool = (k_code_pages, k_scale_pages, k_zero_pages, v_code_pages, v_scale_pages, v_zero_pages,
            k_residual_scratch, v_residual_scratch)
    _validated("kivi_cache_write_dsl", _writer_named(pool, new_k, new_v, slot_mapping, block_table),
               *pool, new_k, new_v, slot_mapping, block_table, int(seq_len))
    lib().kivi_cache_write_launch(*[_ptr(t) for t in pool], _ptr(new_k), _ptr(new_v),
                                  _ptr(slot_mapping), _ptr(block_table), int(seq_len),
                                  int(k_code_pages.size(1)), _stream(new_k.device))


def kivi_cache_write_jac_dsl(k_code_pages, k_scale_pages, k_zero_pages, v_code_pages,
                             v_scale_pages, v_zero_pages, k_residual_scratch, v_residual_scratch,
                             new_k, new_v, slot_mapping, block_table, seq_len: int) -> None:
    """source_patch.py:1085-1180 -> jac_launch_cache_write (global geometry only)."""
    pool = (k_code_pages, k_scale_pages, k_zero_pages, v_code_pages, v_scale_pages, v_zero_pages,
            k_residual_scratch, v_residual_scratch)
    _validated("kivi_cache_write_jac_dsl",
               _writer_named(pool, new_k, new_v, slot_mapping, block_table),
               *pool, new_k, new_v, slot_mapping, block_table, int(seq_len))
    lib().jac_launch_cache_write(*[_ptr(t) for t in pool], _ptr(new_k), _ptr(new_v),
                                 _ptr(block_table), int(seq_len), _stream(new_k.device))


def kivi_cache_write_batched_dsl(k_code_pages, k_scale_pages, k_zero_pages, v_code_pages,
                                 v_scale_pages, v_zero_pages, k_residual_scratch,
                                 v_residual_scratch, new_k, new_v, slot_mapping, block_table,
                                 start_seq_len: int, num_new: int) -> None:
    """source_patch.py:1392-1495 -> kivi_cache_write_batched_launch."""
    pool = (k_code_pages, k_scale_pages, k_zero_pages, v_code_pages, v_scale_pages, v_zero_pages,
            k_residual_scratch, v_residual_scratch)
    _validated("kivi_cache_write_batched_dsl",
               _writer_named(pool, new_k, new_v, slot_mapping, block_table),
               *pool, new_k, new_v, slot_mapping, block_table, int(start_seq_len), int(num_new))
    lib().kivi_cache_write_batched_launch(*[_ptr(t) for t in pool], _ptr(new_k), _ptr(new_v),
                                          _ptr(slot_mapping), _ptr(block_table),
                                          int(start_seq_len), int(num_new),
                                          int(k_code_pages.size(1)), _stream(new_k.device))


def plan_batched_write(start_seq_len: int, num_new_tokens: int, residual: int = 128,
                       block_size: int = 32) -> list[tuple]:
    """source_patch.py:504-553, computed by the native library.  Returns
    (start_seq_len, num_new, scratch_start, age_out_page, post_shift_residual_len)
    tuples with None for absent values; raises ValueError like the reference."""
    cap = num_new_tokens + 8 if num_new_tokens > 0 else 1
    buf = (Subchunk * cap)()
    n = lib().jacq_kivi_plan_batched_write(start_seq_len, num_new_tokens, residual, block_size,
                                           buf, cap)
    if n < 0:
        raise ValueError(last_error())
    return [(s.start_seq_len, s.num_new, s.scratch_start,
             None if s.age_out_page < 0 else s.age_out_page,
             None if s.post_shift_residual_len < 0 else s.post_shift_residual_len)
            for s in buf[:n]]


# ---------------------------------------------------------------------------
# runtime-geometry surface
# ---------------------------------------------------------------------------

@dataclass(frozen=True)
class KiviGeometry:
    num_heads: int
    num_kv_heads: int
    head_dim: int
    page_size: int = 16
    group_size: int = 32
    residual: int = 128
    max_pages_per_seq: int = 124
    num_pages: int = 1

    @property
    def gqa(self) -> int:
        return self.num_heads // self.num_kv_heads

    @property
    def scratch_rows(self) -> int:
        return self.residual + self.group_size

    def c(self) -> Geometry:
        return Geometry(self.num_heads, self.num_kv_heads, self.head_dim, self.page_size,
                        self.group_size, self.residual, self.max_pages_per_seq, self.num_pages)

    def check(self) -> None:
        g = self.c()
        if lib().jacq_kivi_check_geometry(ctypes.byref(g)) != 0:
            raise KiviCheckError(last_error())

    def max_seq_len(self) -> int:
        return ((self.max_pages_per_seq * self.page_size) // self.group_size) * self.group_size \
            + self.residual


class PagedKiviCache:
    """Page pool + per-sequence fp16 residual scratch for ``batch`` sequences,
    allocated on one device.  Tensors use the v1 layouts (include/jacq_kivi.h)."""

    def __init__(self, geo: KiviGeometry, batch: int, device="cuda"):
        geo.check()
        self.geo, self.batch = geo, batch
        g = geo
        dev = torch.device(device)
        self.k_code = torch.zeros((g.num_pages, g.num_kv_heads, g.page_size, g.head_dim // 2),
                                  dtype=torch.uint8, device=dev)
        self.v_code = torch.zeros_like(self.k_code)
        self.k_scale = torch.zeros((g.num_pages, g.num_kv_heads, g.head_dim), dtype=torch.float16,
                                   device=dev)
        self.k_zero = torch.zeros_like(self.k_scale)
        self.v_scale = torch.zeros((g.num_pages, g.num_kv_heads, g.page_size,
                                    g.head_dim // g.group_size), dtype=torch.float16, device=dev)
        self.v_zero = torch.zeros_like(self.v_scale)
        self.k_scr = torch.zeros((batch, g.num_kv_heads, g.scratch_rows, g.head_dim),
                                 dtype=torch.float16, device=dev)
        self.v_scr = torch.zeros_like(self.k_scr)

    def sequence_view(self, b: int) -> "PagedKiviCache":
        """A one-sequence cache sharing this cache's pool and sequence b's scratch."""
        v = PagedKiviCache.__new__(PagedKiviCache)
        v.geo, v.batch = self.geo, 1
        (v.k_code, v.k_scale, v.k_zero, v.v_code, v.v_scale, v.v_zero) = (
            self.k_code, self.k_scale, self.k_zero, self.v_code, self.v_scale, self.v_zero)
        v.k_scr, v.v_scr = self.k_scr[b:b + 1], self.v_scr[b:b + 1]
        return v

    @classmethod
    def from_tensors(cls, geo: KiviGeometry, tensors: dict) -> "PagedKiviCache":
        """Wrap existing pool/scratch tensors (keys k_code ... v_scr)."""
        v = cls.__new__(cls)
        v.geo, v.batch = geo, tensors["k_scr"].shape[0]
        for k in ("k_code", "k_scale", "k_zero", "v_code", "v_scale", "v_zero", "k_scr", "v_scr"):
            setattr(v, k, tensors[k])
        return v

    def pool(self):
        return (self.k_code, self.k_scale, self.k_zero, self.v_code, self.v_scale, self.v_zero,
                self.k_scr, self.v_scr)

    def append(self, new_k: torch.Tensor, new_v: torch.Tensor, block_tables: torch.Tensor,
               start_lens: torch.Tensor) -> None:
        """new_k/new_v [batch, num_new, NKV, HD] fp16; start_lens [batch] int32."""
        g = self.geo
        _check(new_k.dim() == 4 and new_k.shape[0] == self.batch
               and new_k.shape[2:] == (g.num_kv_heads, g.head_dim), "NEW_K shape mismatch")
        _check(new_v.shape == new_k.shape, "NEW_V shape mismatch")
        _check(new_k.dtype == torch.float16 and new_v.dtype == torch.float16, "NEW_K/V must be fp16")
        _check(new_k.is_contiguous() and new_v.is_contiguous(), "NEW_K/V must be contiguous")
        check_shape(block_tables, (self.batch, g.max_pages_per_seq), "BLOCK_TABLES")
        _check(block_tables.dtype == torch.int32 and block_tables.is_contiguous(),
               "BLOCK_TABLES must be contiguous int32")
        check_shape(start_lens, (self.batch,), "START_LENS")
        _check(start_lens.dtype == torch.int32, "START_LENS must be int32")
        geo = g.c()
        rc = lib().jacq_kivi_cache_append(ctypes.byref(geo), *[_ptr(t) for t in self.pool()],
                                          _ptr(new_k), _ptr(new_v), _ptr(block_tables),
                                          _ptr(start_lens), int(new_k.shape[1]), self.batch,
                                          _stream(new_k.device))
        if rc != 0:
            raise KiviLaunchError(last_error())

    def decode(self, q: torch.Tensor, seq_lens: torch.Tensor, block_tables: torch.Tensor,
               out: torch.Tensor | None = None, workspace: torch.Tensor | None = None
               ) -> torch.Tensor:
        """q [batch, NH, HD] fp16 -> O [batch, NH, HD] fp32."""
        g = self.geo
        check_shape(q, (self.batch, g.num_heads, g.head_dim), "Q")
        _check(q.dtype == torch.float16 and q.is_contiguous(), "Q must be contiguous fp16")
        check_shape(seq_lens, (self.batch,), "SEQ_LENS")
        _check(seq_lens.dtype == torch.int32, "SEQ_LENS must be int32")
        check_shape(block_tables, (self.batch, g.max_pages_per_seq), "BLOCK_TABLES")
        _check(block_tables.dtype == torch.int32 and block_tables.is_contiguous(),
               "BLOCK_TABLES must be contiguous int32")
        if out is None:
            out = torch.empty((self.batch, g.num_heads, g.head_dim), dtype=torch.float32,
                              device=q.device)
        geo = g.c()
        ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
        rc = lib().jacq_kivi_decode(ctypes.byref(geo), _ptr(q), _ptr(seq_lens), _ptr(block_tables),
                                    *[_ptr(t) for t in self.pool()], self.batch, _ptr(out),
                                    _ptr(workspace), ws_bytes, _stream(q.device))
        if rc != 0:
            _raise(rc)
        return out

    def write_decode(self, q: torch.Tensor, new_k: torch.Tensor, new_v: torch.Tensor,
                     seq_lens: torch.Tensor, block_tables: torch.Tensor,
                     out: torch.Tensor | None = None, workspace: torch.Tensor | None = None
                     ) -> torch.Tensor:
        """One fused step (jacq_kivi_write_decode): append new_k/new_v
        [batch, NKV, HD] fp16 at position seq_lens - 1, then decode q
        [batch, NH, HD] over the new state -> O [batch, NH, HD] fp32."""
        g = self.geo
        check_shape(q, (self.batch, g.num_heads, g.head_dim), "Q")
        _check(q.dtype == torch.float16 and q.is_contiguous(), "Q must be contiguous fp16")
        for t, name in ((new_k, "NEW_K"), (new_v, "NEW_V")):
            check_shape(t, (self.batch, g.num_kv_heads, g.head_dim), name)
            _check(t.dtype == torch.float16 and t.is_contiguous(), name + " must be contiguous fp16")
        check_shape(seq_lens, (self.batch,), "SEQ_LENS")
        _check(seq_lens.dtype == torch.int32, "SEQ_LENS must be int32")
        check_shape(block_tables, (self.batch, g.max_pages_per_seq), "BLOCK_TABLES")
        _check(block_tables.dtype == torch.int32 and block_tables.is_contiguous(),
               "BLOCK_TABLES must be contiguous int32")
        if out is None:
            out = torch.empty((self.batch, g.num_heads, g.head_dim), dtype=torch.float32,
                              device=q.device)
        geo = g.c()
        ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
        rc = lib().jacq_kivi_write_decode(ctypes.byref(geo), _ptr(q), _ptr(new_k), _ptr(new_v),
                                          _ptr(seq_lens), _ptr(block_tables),
                                          *[_ptr(t) for t in self.pool()], self.batch, _ptr(out),
                                          _ptr(workspace), ws_bytes, _stream(q.device))
        if rc != 0:
            _raise(rc)
        return out

    def decode_sparse_retained(self, q: torch.Tensor, seq_len: int, retained_table: torch.Tensor,
                               num_retained_pages: int, out: torch.Tensor | None = None,
                               workspace: torch.Tensor | None = None) -> torch.Tensor:
        """One sequence (a batch-1 cache or sequence_view): q [NH, HD] fp16,
        retained_table [>= num_retained_pages] int32 -> O [NH, HD] fp32."""
        g = self.geo
        _check(self.batch == 1, "sparse-retained decode takes one sequence (use sequence_view)")
        check_shape(q, (g.num_heads, g.head_dim), "Q")
        _check(q.dtype == torch.float16 and q.is_contiguous(), "Q must be contiguous fp16")
        _check(retained_table.dtype == torch.int32 and retained_table.is_contiguous(),
               "RETAINED_BLOCK_TABLE must be contiguous int32")
        _check(retained_table.numel() >= num_retained_pages,
               "RETAINED_BLOCK_TABLE holds fewer than NUM_RETAINED_PAGES entries")
        if out is None:
            out = torch.empty((g.num_heads, g.head_dim), dtype=torch.float32, device=q.device)
        geo = g.c()
        ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
        rc = lib().jacq_kivi_decode_sparse_retained(
            ctypes.byref(geo), _ptr(q), int(seq_len), _ptr(retained_table),
            int(num_retained_pages), *[_ptr(t) for t in self.pool()], _ptr(out),
            _ptr(workspace), ws_bytes, _stream(q.device))
        if rc != 0:
            _raise(rc)
        return out
