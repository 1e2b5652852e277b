"""Tensor binding ABI of the paged KIVI decode lane (restates
integrations/vllm_kivi/bindings.py:14-174).

Single source of truth for the shapes / dtypes / order a caller binds before
calling ``jac_launch`` (include/jacq_kivi.h).  Framework-light: it allocates
nothing and calls no GPU code.
"""
from __future__ import annotations

import math
from dataclasses import asdict, dataclass

from jacq_amd.layout import KiviModelGeometry, KiviPageLayout


@dataclass(frozen=True)
class TensorBinding:
    name: str
    dtype: str
    shape: tuple
    bytes_per_element: int
    role: str

    @property
    def numel_per_layer(self):
        prod = 1
        for dim in self.shape:
            if isinstance(dim, str):
                return "dynamic"
            prod *= dim
        return prod

    @property
    def bytes_per_layer(self):
        n = self.numel_per_layer
        return n if isinstance(n, str) else n * self.bytes_per_element

    def to_dict(self) -> dict:
        return {**asdict(self), "shape": list(self.shape), "numel_per_layer": self.numel_per_layer,
                "bytes_per_layer": self.bytes_per_layer}


# bindings.py:120-143 -- the order of the emitted jac_launch signature.
JAC_LAUNCH_ORDER = (
    "Q", "BLOCK_TABLE",
    "K_CODE_PAGES", "K_SCALE_PAGES", "K_ZERO_PAGES",
    "V_CODE_PAGES", "V_SCALE_PAGES", "V_ZERO_PAGES",
    "K_RESIDUAL_SCRATCH", "V_RESIDUAL_SCRATCH",
    "SEQ_LEN", "O", "hipStream_t stream",
)


@dataclass(frozen=True)
class KiviDecodeBindingAbi:
    layout: KiviPageLayout
    seq_len: int = 4096
    num_blocks: int | None = None
    max_blocks_per_seq: int | None = None

    def __post_init__(self) -> None:
        self.layout.validate_for_vllm_lane()
        if self.seq_len < self.layout.residual_tokens:
            raise ValueError("seq_len must cover the fp16 residual window in the first KIVI lane")
        if self.seq_len % self.layout.block_size != 0:
            raise ValueError("first KIVI binding ABI expects page-aligned seq_len")
        if self.num_blocks is not None and self.num_blocks <= 0:
            raise ValueError("num_blocks must be positive")
        if self.max_blocks_per_seq is not None and self.max_blocks_per_seq <= 0:
            raise ValueError("max_blocks_per_seq must be positive")

    @property
    def old_tokens(self) -> int:
        return max(0, self.seq_len - self.layout.residual_tokens)

    @property
    def old_pages(self) -> int:
        return self.old_tokens // self.layout.block_size

    @property
    def physical_blocks(self) -> int:
        return self.num_blocks if self.num_blocks is not None else self.old_pages

    @property
    def block_table_len(self) -> int:
        return self.max_blocks_per_seq if self.max_blocks_per_seq is not None else self.old_pages

    @property
    def geometry(self) -> KiviModelGeometry:
        return self.layout.geometry

    @property
    def hd_packed(self) -> int:
        return self.geometry.head_dim * self.layout.nbits // 8

    @property
    def hd_groups(self) -> int:
        return math.ceil(self.geometry.head_dim / self.layout.group_size)

    def tensor_bindings(self) -> list[TensorBinding]:
        g, b, bs = self.geometry, self.physical_blocks, self.layout.block_size
        rs = self.layout.residual_tokens + self.layout.group_size
        return [
            TensorBinding("Q", "torch.float16", (g.num_attention_heads, g.head_dim), 2,
                          "one decode query per attention head"),
            TensorBinding("BLOCK_TABLE", "torch.int32", (self.block_table_len,), 4,
                          "logical old-token page -> physical KIVI page"),
            TensorBinding("K_CODE_PAGES", "torch.uint8", (b, g.num_kv_heads, bs, self.hd_packed), 1,
                          "packed int4 key codes, two channels per byte"),
            TensorBinding("K_SCALE_PAGES", "torch.float16", (b, g.num_kv_heads, g.head_dim), 2,
                          "key scales grouped over the token group"),
            TensorBinding("K_ZERO_PAGES", "torch.float16", (b, g.num_kv_heads, g.head_dim), 2,
                          "key zeros grouped over the token group"),
            TensorBinding("V_CODE_PAGES", "torch.uint8", (b, g.num_kv_heads, bs, self.hd_packed), 1,
                          "packed int4 value codes, two channels per byte"),
            TensorBinding("V_SCALE_PAGES", "torch.float16", (b, g.num_kv_heads, bs, self.hd_groups),
                          2, "value scales grouped over head_dim channels per token"),
            TensorBinding("V_ZERO_PAGES", "torch.float16", (b, g.num_kv_heads, bs, self.hd_groups),
                          2, "value zeros grouped over head_dim channels per token"),
            TensorBinding("K_RESIDUAL_SCRATCH", "torch.float16", (g.num_kv_heads, rs, g.head_dim), 2,
                          "fp16 key residual tail with room for one group before age-out"),
            TensorBinding("V_RESIDUAL_SCRATCH", "torch.float16", (g.num_kv_heads, rs, g.head_dim), 2,
                          "fp16 value residual tail with room for one group before age-out"),
            TensorBinding("SEQ_LEN", "int", (), 8,
                          "runtime valid sequence length for old-page/residual bounds"),
            TensorBinding("O", "torch.float32", (g.num_attention_heads, g.head_dim), 4,
                          "decode output per attention head"),
        ]

    def jac_launch_order(self) -> list[str]:
        return list(JAC_LAUNCH_ORDER)

    def old_page_bytes_per_layer(self) -> int:
        return self.layout.quantized_page_bytes_per_layer * self.physical_blocks

    def residual_bytes_per_sequence_layer(self) -> int:
        g = self.geometry
        return 2 * g.num_kv_heads * self.layout.residual_tokens * g.head_dim * g.dtype_bytes

    def to_report(self) -> dict:
        return {
            "seq_len": self.seq_len,
            "old_tokens": self.old_tokens,
            "old_pages": self.old_pages,
            "physical_blocks_reported": self.physical_blocks,
            "block_table_len": self.block_table_len,
            "jac_launch_order": self.jac_launch_order(),
            "tensor_bindings": [b.to_dict() for b in self.tensor_bindings()],
            "old_page_bytes_per_layer": self.old_page_bytes_per_layer(),
            "residual_bytes_per_sequence_layer": self.residual_bytes_per_sequence_layer(),
        }


def default_qwen32b_binding_abi(seq_len: int = 4096) -> KiviDecodeBindingAbi:
    return KiviDecodeBindingAbi(KiviPageLayout(KiviModelGeometry.qwen25_coder_32b()),
                                seq_len=seq_len)
