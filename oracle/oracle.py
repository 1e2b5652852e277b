"""ctypes front end of the CPU oracle (oracle/kivi_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, ``__graft_entry__.smoke()`` and
``bench.py``'s cpu_baseline leg, never by the product package ``jacq_amd``.

Arrays are numpy; fp16 tensors are passed as their uint16 bit patterns.
Shapes follow the reference layouts (integrations/vllm_kivi/bindings.py:101-124)
with a leading batch axis on per-sequence tensors:

    k_code/v_code   [pages, NKV, P, HD/2]  uint8
    k_scale/k_zero  [pages, NKV, HD]       fp16
    v_scale/v_zero  [pages, NKV, P, HD/G]  fp16
    k_scr/v_scr     [B, NKV, R+G, HD]      fp16
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libkivi_oracle.so")


def build() -> str:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


class KiviGeo(ctypes.Structure):
    _fields_ = [
        ("nh", ctypes.c_int32),
        ("nkv", ctypes.c_int32),
        ("hd", ctypes.c_int32),
        ("page", ctypes.c_int32),
        ("group", ctypes.c_int32),
        ("residual", ctypes.c_int32),
        ("max_pages", ctypes.c_int32),
    ]


class KiviSubchunk(ctypes.Structure):
    _fields_ = [
        ("start_seq_len", ctypes.c_int32),
        ("num_new", ctypes.c_int32),
        ("scratch_start", ctypes.c_int32),
        ("age_out_page", ctypes.c_int32),
        ("post_shift_residual_len", ctypes.c_int32),
    ]


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _lib.kivi_f32_to_f16.restype = ctypes.c_uint16
        _lib.kivi_f32_to_f16.argtypes = [ctypes.c_float]
        _lib.kivi_f16_to_f32.restype = ctypes.c_float
        _lib.kivi_f16_to_f32.argtypes = [ctypes.c_uint16]
        for name in ("kivi_split_old_tokens",):
            getattr(_lib, name).restype = ctypes.c_int32
        _lib.kivi_ref_cache_write_batched.restype = ctypes.c_int32
        _lib.kivi_ref_plan_batched_write.restype = ctypes.c_int32
        _lib.kivi_ref_required_pages.restype = ctypes.c_int32
    return _lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return ctypes.c_void_p(a.ctypes.data)


@dataclass(frozen=True)
class Geometry:
    nh: int
    nkv: int
    hd: int
    page: int = 32
    group: int = 32
    residual: int = 128
    max_pages: int = 124

    @property
    def rs(self) -> int:
        return self.residual + self.group

    @property
    def hdg(self) -> int:
        return self.hd // self.group

    def c(self) -> KiviGeo:
        return KiviGeo(self.nh, self.nkv, self.hd, self.page, self.group, self.residual,
                       self.max_pages)


@dataclass
class Cache:
    """Page pool + per-sequence scratch, as numpy arrays (uint16 = fp16 bits)."""

    geo: Geometry
    k_code: np.ndarray
    k_scale: np.ndarray
    k_zero: np.ndarray
    v_code: np.ndarray
    v_scale: np.ndarray
    v_zero: np.ndarray
    k_scr: np.ndarray
    v_scr: np.ndarray

    @classmethod
    def empty(cls, geo: Geometry, num_pages: int, batch: int, fill: int = 0) -> "Cache":
        g = geo
        return cls(
            g,
            np.full((num_pages, g.nkv, g.page, g.hd // 2), fill, np.uint8),
            np.full((num_pages, g.nkv, g.hd), fill, np.uint16),
            np.full((num_pages, g.nkv, g.hd), fill, np.uint16),
            np.full((num_pages, g.nkv, g.page, g.hd // 2), fill, np.uint8),
            np.full((num_pages, g.nkv, g.page, g.hdg), fill, np.uint16),
            np.full((num_pages, g.nkv, g.page, g.hdg), fill, np.uint16),
            np.full((batch, g.nkv, g.rs, g.hd), fill, np.uint16),
            np.full((batch, g.nkv, g.rs, g.hd), fill, np.uint16),
        )

    def pool_args(self):
        return [_p(self.k_code), _p(self.k_scale), _p(self.k_zero), _p(self.v_code),
                _p(self.v_scale), _p(self.v_zero)]

    def scr(self, b: int):
        return [ctypes.c_void_p(self.k_scr[b].ctypes.data), ctypes.c_void_p(self.v_scr[b].ctypes.data)]

    def copy(self) -> "Cache":
        return Cache(self.geo, *[getattr(self, f).copy() for f in
                                 ("k_code", "k_scale", "k_zero", "v_code", "v_scale", "v_zero",
                                  "k_scr", "v_scr")])


def f32_to_f16_bits(x: float) -> int:
    return int(lib().kivi_f32_to_f16(ctypes.c_float(x)))


def f16_bits_to_f32(h: int) -> float:
    return float(lib().kivi_f16_to_f32(ctypes.c_uint16(h)))


def split_old_tokens(seq_len: int, residual: int, group: int) -> int:
    return int(lib().kivi_split_old_tokens(seq_len, residual, group))


def required_pages(seq_len: int, residual: int, group: int, page: int, max_seq_len: int) -> int:
    return int(lib().kivi_ref_required_pages(seq_len, residual, group, page, max_seq_len))


def cache_write(cache: Cache, b: int, new_k: np.ndarray, new_v: np.ndarray,
                block_table: np.ndarray, seq_len: int) -> None:
    """One token for sequence b; new_k/new_v [NKV,HD] uint16."""
    g = cache.geo.c()
    lib().kivi_ref_cache_write(ctypes.byref(g), *cache.pool_args(), *cache.scr(b),
                               _p(np.ascontiguousarray(new_k)), _p(np.ascontiguousarray(new_v)),
                               _p(np.ascontiguousarray(block_table, np.int32)), seq_len)


def cache_write_batched(cache: Cache, b: int, new_k: np.ndarray, new_v: np.ndarray,
                        block_table: np.ndarray, start_seq_len: int) -> int:
    """num_new tokens for sequence b; new_k/new_v [num_new,NKV,HD] uint16."""
    g = cache.geo.c()
    return int(lib().kivi_ref_cache_write_batched(
        ctypes.byref(g), *cache.pool_args(), *cache.scr(b), _p(np.ascontiguousarray(new_k)),
        _p(np.ascontiguousarray(new_v)), _p(np.ascontiguousarray(block_table, np.int32)),
        start_seq_len, new_k.shape[0]))


def plan_batched_write(start_seq_len: int, num_new: int, residual: int = 128,
                       group: int = 32) -> list[tuple]:
    cap = num_new + 8
    buf = (KiviSubchunk * cap)()
    n = lib().kivi_ref_plan_batched_write(start_seq_len, num_new, residual, group, buf, cap)
    if n < 0:
        raise ValueError(f"plan_batched_write error {n}")
    out = []
    for i in range(n):
        s = buf[i]
        out.append((s.start_seq_len, s.num_new, s.scratch_start,
                    None if s.age_out_page < 0 else s.age_out_page,
                    None if s.post_shift_residual_len < 0 else s.post_shift_residual_len))
    return out


def decode_online(cache: Cache, b: int, q: np.ndarray, block_table: np.ndarray,
                  seq_len: int) -> np.ndarray:
    g = cache.geo
    out = np.zeros((g.nh, g.hd), np.float32)
    lib().kivi_ref_decode_online(ctypes.byref(g.c()), _p(np.ascontiguousarray(q)),
                                 _p(np.ascontiguousarray(block_table, np.int32)),
                                 *cache.pool_args(), *cache.scr(b), seq_len, _p(out))
    return out


def decode_twopass(cache: Cache, b: int, q: np.ndarray, block_table: np.ndarray,
                   seq_len: int) -> np.ndarray:
    g = cache.geo
    out = np.zeros((g.nh, g.hd), np.float64)
    lib().kivi_ref_decode_twopass(ctypes.byref(g.c()), _p(np.ascontiguousarray(q)),
                                  _p(np.ascontiguousarray(block_table, np.int32)),
                                  *cache.pool_args(), *cache.scr(b), seq_len, _p(out))
    return out


def decode_sparse_retained(cache: Cache, b: int, q: np.ndarray, retained_table: np.ndarray,
                           seq_len: int, num_retained_pages: int,
                           twopass: bool = False) -> np.ndarray:
    """Sparse-retained decode (kivi_oracle.c, variants.rs:2620-2740): fp32
    online softmax, or the float64 two-pass attention with twopass."""
    g = cache.geo
    out = np.zeros((g.nh, g.hd), np.float64 if twopass else np.float32)
    fn = (lib().kivi_ref_decode_sparse_retained_twopass if twopass
          else lib().kivi_ref_decode_sparse_retained)
    fn(ctypes.byref(g.c()), _p(np.ascontiguousarray(q)),
       _p(np.ascontiguousarray(retained_table, np.int32)), *cache.pool_args(), *cache.scr(b),
       seq_len, num_retained_pages, _p(out))
    return out


def decode_splitk(cache: Cache, b: int, q: np.ndarray, block_table: np.ndarray,
                  seq_len: int, chunk: int) -> np.ndarray:
    g = cache.geo
    out = np.zeros((g.nh, g.hd), np.float32)
    lib().kivi_ref_decode_splitk(ctypes.byref(g.c()), _p(np.ascontiguousarray(q)),
                                 _p(np.ascontiguousarray(block_table, np.int32)),
                                 *cache.pool_args(), *cache.scr(b), seq_len, chunk, _p(out))
    return out


def decode_batch(cache: Cache, q: np.ndarray, seq_lens: np.ndarray, block_tables: np.ndarray,
                 nthreads: int = 1) -> np.ndarray:
    """q [B,NH,HD] uint16, block_tables [B,max_pages] int32 -> out [B,NH,HD] fp32."""
    g = cache.geo
    bsz = q.shape[0]
    assert block_tables.shape == (bsz, g.max_pages)
    out = np.zeros((bsz, g.nh, g.hd), np.float32)
    lib().kivi_ref_decode_batch(ctypes.byref(g.c()), _p(np.ascontiguousarray(q)),
                                _p(np.ascontiguousarray(seq_lens, np.int32)),
                                _p(np.ascontiguousarray(block_tables, np.int32)),
                                *cache.pool_args(), _p(cache.k_scr), _p(cache.v_scr), bsz,
                                _p(out), nthreads)
    return out


def lse_merge(m: np.ndarray, l: np.ndarray, acc: np.ndarray) -> np.ndarray:
    m = np.ascontiguousarray(m, np.float32)
    l = np.ascontiguousarray(l, np.float32)
    acc = np.ascontiguousarray(acc, np.float32)
    out = np.zeros(acc.shape[1], np.float32)
    lib().kivi_ref_lse_merge(len(m), acc.shape[1], _p(m), _p(l), _p(acc), _p(out))
    return out


def build_sequence(cache: Cache, b: int, k_hist: np.ndarray, v_hist: np.ndarray,
                   block_table: np.ndarray) -> None:
    """Feed a token history [L,NKV,HD] (uint16) through repeated single-token
    writes from an empty sequence -- the reference's served order."""
    for t in range(k_hist.shape[0]):
        cache_write(cache, b, k_hist[t], v_hist[t], block_table, t + 1)
