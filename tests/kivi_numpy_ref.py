"""Second, independent restatement of the KIVI cache read side in numpy
float64, used to cross-check the C oracle (oracle/) on the CPU.

It shares no code with the oracle: the layout formulas, the nibble order and
the dequantisation are re-derived here from the reference text, and the
attention is the textbook two-pass softmax on whole arrays.

  layout      integrations/vllm_kivi/source_patch.py:1565-1578, :1604
              (K_CODE/V_CODE byte ((page*NKV+h)*P+t)*(HD/2)+d/2,
               K_SCALE (page*NKV+h)*HD+d, V_SCALE ((page*NKV+h)*P+t)*HDG+g)
  unpack      crates/jac-codegen-cuda/src/variants.rs:2316-2327
              (channel 2j = low nibble of byte j)
  split rule  source_patch.py:1655-1659; decode window snapshot :74-83
"""
from __future__ import annotations

import numpy as np

GROUP = 32


def f16(bits: np.ndarray) -> np.ndarray:
    """uint16 fp16 bit patterns -> float64."""
    return np.asarray(bits, np.uint16).view(np.float16).astype(np.float64)


def decode_window(seq_len: int, residual: int, lq: int) -> tuple[int, int]:
    bounded = min(max(seq_len, 0), lq + residual)
    old = max(bounded - residual, 0) // GROUP * GROUP
    old = min(old, lq)
    res = min(max(bounded - old, 0), residual + GROUP)
    return old, res


def sparse_window(seq_len: int, residual: int, lq: int, page: int, max_pages: int,
                  retained: int) -> tuple[int, int]:
    """variants.rs:2667-2680: old tokens = the retained pages (clamped to
    [0, dense old pages] and the table width, whole groups), residual rows at
    the dense boundary."""
    dense_old, res = decode_window(seq_len, residual, lq)
    pages = min(max(retained, 0), dense_old // page, max_pages)
    return pages * page // GROUP * GROUP, res


def dequant_sequence(cache, b: int, block_table: np.ndarray, seq_len: int,
                     value_parts: bool = False, window: tuple[int, int] | None = None):
    """K, V [NKV, n, HD] float64 of the decode window of sequence b (or of an
    explicit (old, residual) window over block_table); with value_parts, V is
    returned as (code * scale, zero) of the quantised tokens (residual tokens:
    (value, 0))."""
    g = cache.geo
    page, hd, nkv = g.page, g.hd, g.nkv
    lq = (g.max_pages * page) // GROUP * GROUP
    old, res = window if window is not None else decode_window(seq_len, g.residual, lq)
    n = old + res
    K = np.zeros((nkv, n, hd))
    V = np.zeros((nkv, n, hd))
    VZ = np.zeros((nkv, n, hd))
    kc = cache.k_code.reshape(-1)
    vc = cache.v_code.reshape(-1)
    ks = cache.k_scale.reshape(-1)
    kz = cache.k_zero.reshape(-1)
    vs = cache.v_scale.reshape(-1)
    vz = cache.v_zero.reshape(-1)
    d = np.arange(hd)
    for h in range(nkv):
        for t in range(old):
            p = int(block_table[t // page])
            slot = t % page
            # K scales live once per 32-token group, in the group's first page
            p_grp = int(block_table[(t // GROUP * GROUP) // page])
            byte = kc[((p * nkv + h) * page + slot) * (hd // 2) + d // 2]
            code = np.where(d % 2 == 0, byte & 0xF, byte >> 4).astype(np.float64)
            base = (p_grp * nkv + h) * hd + d
            K[h, t] = code * f16(ks[base]) + f16(kz[base])
            byte = vc[((p * nkv + h) * page + slot) * (hd // 2) + d // 2]
            code = np.where(d % 2 == 0, byte & 0xF, byte >> 4).astype(np.float64)
            sidx = ((p * nkv + h) * page + slot) * (hd // GROUP) + d // GROUP
            V[h, t] = code * f16(vs[sidx]) + f16(vz[sidx])
            VZ[h, t] = f16(vz[sidx])
        K[h, old:n] = f16(cache.k_scr[b, h, :res])
        V[h, old:n] = f16(cache.v_scr[b, h, :res])
    if value_parts:
        return K, (V - VZ, VZ)
    return K, V


def attention(q_bits: np.ndarray, K: np.ndarray, V: np.ndarray) -> np.ndarray:
    """Two-pass softmax attention, GQA (query head qh reads kv head qh // G)."""
    q = f16(q_bits)
    nh, hd = q.shape
    nkv = K.shape[0]
    G = nh // nkv
    out = np.zeros((nh, hd))
    if K.shape[1] == 0:
        return out
    for qh in range(nh):
        h = qh // G
        s = K[h] @ q[qh] / np.sqrt(hd)
        p = np.exp(s - s.max())
        out[qh] = p @ V[h] / p.sum()
    return out
