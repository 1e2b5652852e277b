"""Geometry, argument table and byte math of the KIVI lane (no torch, no GPU).

Everything here is keyed on ``LaneGeometry``, the Python twin of the
library's ``jacq_kivi_geometry`` record (include/jacq_kivi.h): head counts,
head dim, page size, quantisation group, residual window, block-table width
and pool size.  From it follow

* ``launch_arguments`` -- one table row per argument of ``jac_launch``:
  name, element type and shape.  The order is the reference's launch order
  (tests/snapshots/kernels/decode_attention_kivi_paged_library_flash.cu:164-169,
  pinned by tests/test_launch_signature.py:37-57 of the reference);
* ``page_bytes`` / ``stored_bytes_per_token`` / ``capacity_vs_fp16`` -- the
  pool's storage accounting, whose values the reference pins at its lane
  geometry (tests/test_layout_and_scaffold.py:162-174: 40,960 bytes per page
  and layer, 2.99x the fp16 capacity at 4096 tokens);
* ``decode_step_bytes`` -- the algorithmic HBM bytes of one batched decode,
  the figure the benchmark's roofline divides by.
"""
from __future__ import annotations

from dataclasses import dataclass, replace

INT4_BITS = 4
PARAM_PAIR_BYTES = 4  # one fp16 scale + one fp16 zero


@dataclass(frozen=True)
class LaneGeometry:
    num_heads: int
    num_kv_heads: int
    head_dim: int
    page_size: int = 32
    group_size: int = 32
    residual: int = 128
    max_pages_per_seq: int = 124
    num_pages: int = 1

    # derived sizes -------------------------------------------------------
    @property
    def gqa(self) -> int:
        return self.num_heads // self.num_kv_heads

    @property
    def packed_dim(self) -> int:          # bytes of int4 codes per token and kv head
        return self.head_dim * INT4_BITS // 8

    @property
    def channel_groups(self) -> int:      # V scale/zero pairs per token and kv head
        return -(-self.head_dim // self.group_size)

    @property
    def scratch_rows(self) -> int:        # residual window + one group waiting to age out
        return self.residual + self.group_size

    def max_seq_len(self) -> int:
        whole_groups = self.max_pages_per_seq * self.page_size // self.group_size
        return whole_groups * self.group_size + self.residual

    def old_tokens(self, seq_len: int) -> int:
        """Tokens held quantised in pages (the split rule, source_patch.py:1655-1659)."""
        over = seq_len - self.residual
        return 0 if over < 0 else over // self.group_size * self.group_size

    # checks --------------------------------------------------------------
    def problems(self, lane: str = "runtime") -> list[str]:
        """Violations of the v1 lane (page == group == 32, the reference's only
        layout) or of the runtime lane the library accepts."""
        out = []
        if self.group_size != 32:
            out.append(f"group_size is {self.group_size}; the int4 lane quantises groups of 32")
        if lane == "v1":
            if self.page_size != self.group_size:
                out.append(f"page_size {self.page_size} differs from group_size "
                           f"{self.group_size}: a key group would straddle two pages, which "
                           "the v1 layout does not allow")
        elif self.page_size not in (16, 32):
            out.append(f"page_size is {self.page_size}; pages of 16 or 32 tokens are supported")
        if self.head_dim not in (64, 128):
            out.append(f"head_dim is {self.head_dim}; 64 or 128 are supported")
        if self.num_kv_heads < 1 or self.num_heads % self.num_kv_heads or self.gqa > 16:
            out.append(f"{self.num_heads} query heads over {self.num_kv_heads} kv heads: "
                       "need a whole ratio of at most 16")
        if self.residual <= 0 or self.residual % self.group_size:
            out.append(f"residual window {self.residual} is not a positive multiple of "
                       f"{self.group_size}")
        return out

    def require(self, lane: str = "runtime") -> "LaneGeometry":
        bad = self.problems(lane)
        if bad:
            raise ValueError(f"geometry not accepted by the {lane} lane: " + "; ".join(bad))
        return self


# The reference's fixed geometries (source_patch.py:660-671): the global
# symbols and the TP=2 local-rank ones.
V1 = LaneGeometry(40, 8, 128)
V1_TP2_LOCAL = replace(V1, num_heads=20, num_kv_heads=4)
V1_MAX_SEQ_LEN = V1.max_seq_len()   # 124 pages x 32 + 128 = 4096


# ---------------------------------------------------------------- arguments

def launch_arguments(g: LaneGeometry, pool_pages: int | None = None,
                     table_len: int | None = None) -> list[tuple[str, str, tuple]]:
    """(name, element type, shape) of each jac_launch argument, in launch
    order; the stream is the final argument and is not listed."""
    P = g.num_pages if pool_pages is None else pool_pages
    W = g.max_pages_per_seq if table_len is None else table_len
    H, D = g.num_kv_heads, g.head_dim
    codes = (P, H, g.page_size, g.packed_dim)
    return [
        ("Q", "fp16", (g.num_heads, D)),
        ("BLOCK_TABLE", "int32", (W,)),
        ("K_CODE_PAGES", "uint8", codes),
        ("K_SCALE_PAGES", "fp16", (P, H, D)),
        ("K_ZERO_PAGES", "fp16", (P, H, D)),
        ("V_CODE_PAGES", "uint8", codes),
        ("V_SCALE_PAGES", "fp16", (P, H, g.page_size, g.channel_groups)),
        ("V_ZERO_PAGES", "fp16", (P, H, g.page_size, g.channel_groups)),
        ("K_RESIDUAL_SCRATCH", "fp16", (H, g.scratch_rows, D)),
        ("V_RESIDUAL_SCRATCH", "fp16", (H, g.scratch_rows, D)),
        ("SEQ_LEN", "int32", ()),
        ("O", "fp32", (g.num_heads, D)),
    ]


JAC_LAUNCH_ORDER = tuple(a[0] for a in launch_arguments(V1)) + ("hipStream_t stream",)

ELEMENT_BYTES = {"fp16": 2, "fp32": 4, "int32": 4, "uint8": 1}


def argument_bytes(g: LaneGeometry, **kw) -> dict[str, int]:
    out = {}
    for name, dtype, shape in launch_arguments(g, **kw):
        n = 1
        for d in shape:
            n *= d
        out[name] = n * ELEMENT_BYTES[dtype]
    return out


# ---------------------------------------------------------------- storage

def page_bytes(g: LaneGeometry) -> dict[str, int]:
    """Bytes one physical page holds, per layer, for all kv heads."""
    tokens = g.page_size * g.num_kv_heads            # (token, kv head) rows in a page
    key_groups_in_page = -(-g.page_size // g.group_size)
    parts = {
        "k_codes": tokens * g.packed_dim,
        "v_codes": tokens * g.packed_dim,
        # one pair per channel per key group; a 32-token group over two
        # 16-token pages keeps its pairs on both
        "k_params": key_groups_in_page * g.num_kv_heads * g.head_dim * PARAM_PAIR_BYTES,
        "v_params": tokens * g.channel_groups * PARAM_PAIR_BYTES,
    }
    parts["total"] = sum(parts.values())
    parts["fp16_equivalent"] = 2 * tokens * g.head_dim * 2
    return parts


def stored_bytes_per_token(g: LaneGeometry, seq_len: int, num_layers: int) -> float:
    """Average storage per token over all layers for a sequence of seq_len
    tokens, counted in whole pages: the newest residual/page_size pages as
    fp16, the rest quantised (the accounting of the reference's layout
    report)."""
    pb = page_bytes(g)
    pages = -(-seq_len // g.page_size)
    fp16_pages = min(g.residual // g.page_size, pages)
    per_layer = (pages - fp16_pages) * pb["total"] + fp16_pages * pb["fp16_equivalent"]
    return per_layer * num_layers / seq_len


def capacity_vs_fp16(g: LaneGeometry, seq_len: int, num_layers: int) -> float:
    fp16_per_token = 2 * g.num_kv_heads * g.head_dim * 2 * num_layers
    return fp16_per_token / stored_bytes_per_token(g, seq_len, num_layers)


# ---------------------------------------------------------------- decode traffic

def decode_kv_bytes_per_token(head_dim: int, group_size: int = 32) -> float:
    """HBM bytes one decode reads per quantised token and kv head: K and V
    codes (head_dim bytes), the token's V pairs, and its share of the key
    group's pairs.  160 at head_dim 128, 80 at 64."""
    pairs_per_token = head_dim // group_size + head_dim / group_size
    return head_dim + PARAM_PAIR_BYTES * pairs_per_token


def decode_step_bytes(seq_lens, num_heads: int, num_kv_heads: int, head_dim: int,
                      page_size: int, residual: int, group_size: int = 32) -> int:
    """Algorithmic bytes of one batched decode: quantised tokens, fp16
    residual K and V, the block-table entries of the quantised pages, Q in
    fp16 and O in fp32."""
    g = LaneGeometry(num_heads, num_kv_heads, head_dim, page_size, group_size, residual)
    per_tok = decode_kv_bytes_per_token(head_dim, group_size)
    total = 0.0
    for n in seq_lens:
        old = g.old_tokens(int(n))
        total += num_kv_heads * (old * per_tok + (int(n) - old) * head_dim * 4)
        total += 4 * (old // page_size)
    total += len(seq_lens) * num_heads * head_dim * (2 + 4)
    return int(round(total))


def write_step_bytes(lens_before, num_kv_heads: int, head_dim: int, residual: int,
                     group_size: int = 32) -> int:
    """HBM bytes of one one-token write per sequence (the fused step's writer
    share, reported apart from the decode's bytes): the new K and V rows
    (fp16), and for a sequence whose group ages out, the group's 32 rows read,
    their codes and scale/zero pairs written, and the shift (the residual rows
    read and written again) -- per kv head."""
    g = LaneGeometry(num_kv_heads * 1, num_kv_heads, head_dim, 16, group_size, residual)
    total = 0
    for n in lens_before:
        n = int(n)
        total += num_kv_heads * 2 * head_dim * 2  # the new K and V rows
        if g.old_tokens(n + 1) > g.old_tokens(n):
            rows_in = 2 * group_size * head_dim * 2             # K and V rows of the group
            codes = 2 * group_size * head_dim // 2              # K and V int4 codes
            k_pairs = head_dim * PARAM_PAIR_BYTES               # per-channel K scale/zero
            v_pairs = group_size * (head_dim // group_size) * PARAM_PAIR_BYTES
            shift = 2 * 2 * residual * head_dim * 2             # K and V rows, read + write
            total += num_kv_heads * (rows_in + codes + k_pairs + v_pairs + shift)
    return total
