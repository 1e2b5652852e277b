"""KIVI page-layout byte math (restates integrations/vllm_kivi/layout.py:22-154).

Storage per layer, per the faithful KIVI layout the kernels read:

* keys: int4 codes grouped over 32 tokens per channel;
* values: int4 codes grouped over 32 channels per token;
* scale + zero are fp16 pairs (4 bytes per group);
* the newest ``residual_tokens`` stay fp16 in a per-sequence scratch of
  ``residual_tokens + group_size`` rows.

The reference lane requires ``block_size == group_size == 32``
(``validate_for_vllm_lane``, layout.py:51-74).  This build separates the page
size from the quantisation group: ``validate_for_mi355x_lane`` also accepts
16-token pages, where one 32-token key group spans two pages and its K
scale/zero is stored on both.
"""
from __future__ import annotations

import math
from dataclasses import asdict, dataclass


@dataclass(frozen=True)
class KiviModelGeometry:
    name: str
    num_layers: int
    num_attention_heads: int
    num_kv_heads: int
    head_dim: int
    dtype_bytes: int = 2

    @classmethod
    def qwen25_coder_32b(cls) -> "KiviModelGeometry":
        # layout.py:32-40 -- the reference lane's geometry
        return cls("Qwen2.5-Coder-32B-Instruct", 64, 40, 8, 128)

    @property
    def gqa(self) -> int:
        return self.num_attention_heads // self.num_kv_heads


@dataclass(frozen=True)
class KiviPageLayout:
    geometry: KiviModelGeometry
    block_size: int = 32
    group_size: int = 32
    nbits: int = 4
    residual_tokens: int = 128
    scale_zero_bytes: int = 4

    def validate_for_vllm_lane(self) -> None:
        """The reference's v1 lane rules (layout.py:51-74), unchanged."""
        if self.nbits != 4:
            raise ValueError(f"first KIVI lane is int4 only, got nbits={self.nbits}")
        if self.block_size != self.group_size:
            raise ValueError(
                "KIVI key grouping must not straddle vLLM pages in the first serving lane; "
                f"require block_size==group_size, got {self.block_size}!={self.group_size}")
        if self.block_size != 32:
            raise ValueError(f"first vLLM KIVI lane requires block_size=32, got {self.block_size}")
        self._common_checks()

    def validate_for_mi355x_lane(self) -> None:
        """Runtime-geometry lane: page 16 or 32, group 32, HD 64/128, G <= 16."""
        if self.nbits != 4:
            raise ValueError(f"KIVI lane is int4 only, got nbits={self.nbits}")
        if self.group_size != 32:
            raise ValueError(f"KIVI lane requires group_size=32, got {self.group_size}")
        if self.block_size not in (16, 32):
            raise ValueError(f"block_size must be 16 or 32, got {self.block_size}")
        if self.geometry.head_dim not in (64, 128):
            raise ValueError(f"head_dim must be 64 or 128, got {self.geometry.head_dim}")
        g = self.geometry
        if g.num_attention_heads % g.num_kv_heads or g.gqa > 16:
            raise ValueError("query heads must be a multiple (<= 16x) of kv heads")
        self._common_checks()

    def _common_checks(self) -> None:
        if self.geometry.head_dim % self.group_size != 0:
            raise ValueError(f"head_dim={self.geometry.head_dim} must be divisible by "
                             f"group_size={self.group_size}")
        if self.residual_tokens % self.group_size != 0 or self.residual_tokens <= 0:
            raise ValueError(f"residual_tokens={self.residual_tokens} must be a positive "
                             "multiple of the group")

    @property
    def elems_per_token(self) -> int:
        return self.geometry.num_kv_heads * self.geometry.head_dim

    @property
    def fp16_page_bytes_per_layer(self) -> int:
        return 2 * self.block_size * self.elems_per_token * self.geometry.dtype_bytes

    @property
    def code_page_bytes_per_component(self) -> int:
        return self.block_size * self.elems_per_token * self.nbits // 8

    @property
    def key_param_page_bytes(self) -> int:
        # one scale/zero pair per channel per page (a group spanning two
        # pages stores its pair on both)
        token_groups = math.ceil(self.block_size / self.group_size)
        return token_groups * self.elems_per_token * self.scale_zero_bytes

    @property
    def value_param_page_bytes(self) -> int:
        groups = self.geometry.num_kv_heads * math.ceil(self.geometry.head_dim / self.group_size)
        return self.block_size * groups * self.scale_zero_bytes

    @property
    def quantized_page_bytes_per_layer(self) -> int:
        return (2 * self.code_page_bytes_per_component + self.key_param_page_bytes
                + self.value_param_page_bytes)

    @property
    def residual_pages(self) -> int:
        return self.residual_tokens // self.block_size

    def effective_bytes_per_layer(self, seq_len: int) -> int:
        pages = math.ceil(seq_len / self.block_size)
        residual_pages = min(self.residual_pages, pages)
        quantized_pages = max(0, pages - residual_pages)
        return (quantized_pages * self.quantized_page_bytes_per_layer
                + residual_pages * self.fp16_page_bytes_per_layer)

    def effective_bytes_per_token_all_layers(self, seq_len: int) -> float:
        return self.effective_bytes_per_layer(seq_len) * self.geometry.num_layers / seq_len

    def fp16_bytes_per_token_all_layers(self) -> int:
        return 2 * self.elems_per_token * self.geometry.dtype_bytes * self.geometry.num_layers

    def capacity_ratio_vs_fp16(self, seq_len: int) -> float:
        return (self.fp16_bytes_per_token_all_layers()
                / self.effective_bytes_per_token_all_layers(seq_len))

    def to_abi_dict(self, seq_len: int = 4096) -> dict[str, object]:
        self.validate_for_vllm_lane()
        return {
            "geometry": asdict(self.geometry),
            "block_size": self.block_size,
            "group_size": self.group_size,
            "nbits": self.nbits,
            "residual_tokens": self.residual_tokens,
            "fp16_page_bytes_per_layer": self.fp16_page_bytes_per_layer,
            "quantized_page_bytes_per_layer": self.quantized_page_bytes_per_layer,
            "key_code_bytes": self.code_page_bytes_per_component,
            "value_code_bytes": self.code_page_bytes_per_component,
            "key_scale_zero_bytes": self.key_param_page_bytes,
            "value_scale_zero_bytes": self.value_param_page_bytes,
            "residual_pages": self.residual_pages,
            "effective_bytes_per_token_all_layers_at_seq_len":
                self.effective_bytes_per_token_all_layers(seq_len),
            "capacity_ratio_vs_fp16_at_seq_len": self.capacity_ratio_vs_fp16(seq_len),
        }


def decode_kv_bytes_per_token(head_dim: int, group_size: int = 32) -> float:
    """Algorithmic HBM bytes one decode step reads per old (quantised) token
    per kv head: K+V codes (HD bytes), V scale/zero (HD/group * 4), K
    scale/zero once per group (HD * 4 / group).  160 B for HD=128."""
    return head_dim + head_dim // group_size * 4 + head_dim * 4 / group_size


def decode_step_bytes(seq_lens, num_heads: int, num_kv_heads: int, head_dim: int,
                      page_size: int, residual: int, group_size: int = 32) -> int:
    """Algorithmic bytes of one batched decode step: quantised old tokens,
    fp16 residual K+V, Q fp16, O fp32 and the block-table entries read."""
    total = 0.0
    for n in seq_lens:
        q = n - residual
        old = (q // group_size) * group_size if q > 0 else 0
        res = n - old
        total += old * num_kv_heads * decode_kv_bytes_per_token(head_dim, group_size)
        total += res * num_kv_heads * head_dim * 4
        total += 4 * (old // page_size)
    total += len(seq_lens) * num_heads * head_dim * (2 + 4)
    return int(round(total))
